"""GPU parity of the fp32 attention path (the drop-in for kernels::attention)
against the oracle and the reference kernels' golden outputs."""
import os

import numpy as np
import pytest

from common import assert_f32_parity, attention_fp64, errors
from gpu_util import dev_bf16, dev_f32, host, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_kernels.npz")


def test_cfg1_gpt2_mha_prefill_fp32(gpu):
    """batch 1, 12 heads, head_dim 64, seq 128, N(0,1) seed 0."""
    S, H, D = 128, 12, 64
    q = O.fill_normal((S, H, D), 0, "q")
    k = O.fill_normal((S, H, D), 0, "k")
    v = O.fill_normal((S, H, D), 0, "v")
    ref = O.attention(q, k, v, S, 0, H, H, D, D)
    say("cfg1 aigpu_attention", S, H, D)
    got = gpu.attention(q, k, v, S, 0, H, H, D, D)
    assert_f32_parity(ref, got, "cfg1")


@pytest.mark.parametrize("window", [0, 1, 7, 200])
def test_reference_unit_case_windows(gpu, window):
    """llm-testing.cpp:106-134: T=19 after S=11 cached, 4 heads over 2, D=48,
    qStride 96, against the reference kernel's own outputs."""
    g = np.load(GOLDEN)
    T, S, H, KV, D, ST = 19, 11, 4, 2, 48, 96
    say("llm-testing window", window)
    got = gpu.attention(g["llm_q"], g["llm_k"], g["llm_v"], T, S, H, KV, D, ST, window)
    assert_f32_parity(g[f"llm_out_serial_w{window}"], got, f"window {window}")
    # the reference test's own bar against the fp64 closed form
    ref64 = attention_fp64(g["llm_q"], g["llm_k"], g["llm_v"], T, S, H, KV, D, ST, window)
    assert np.abs(got - ref64).max() < 2e-6


def test_gqa_with_history_golden(gpu):
    g = np.load(GOLDEN)
    say("gqa history golden")
    got = gpu.attention(g["gqa_q"], g["gqa_k"], g["gqa_v"], 5, 7, 8, 2, 64, 64)
    assert_f32_parity(g["gqa_out"], got, "gqa")


def test_long_context_single_token(gpu):
    L, H, KV, D = 5000, 8, 2, 128
    q = O.fill_normal((1, H, D), 5, "q")
    k = O.fill_normal((L + 1, KV, D), 5, "k")
    v = O.fill_normal((L + 1, KV, D), 5, "v")
    ref = O.attention(q, k, v, 1, L, H, KV, D, D)
    say("long context single token", L)
    got = gpu.attention(q, k, v, 1, L, H, KV, D, D)
    assert_f32_parity(ref, got, "long")


@pytest.mark.parametrize("dim", [4, 32, 256, 36])
def test_value_row_groups(gpu, dim):
    """fp32 value rows read as 16-byte pieces, dim / 4 lanes per row (1, 8 and
    64 lanes; 9 lanes is not a power of two and takes the row-by-row path),
    with history so blocks of 64 keys are partly filled"""
    T, S, H, KV = 9, 70, 4, 2
    q = O.fill_normal((T, H, dim), 41, "q")
    k = O.fill_normal((S + T, KV, dim), 42, "k")
    v = O.fill_normal((S + T, KV, dim), 43, "v")
    ref = O.attention(q, k, v, T, S, H, KV, dim, dim)
    say("value row groups", dim)
    got = gpu.attention(q, k, v, T, S, H, KV, dim, dim)
    assert_f32_parity(ref, got, f"dim {dim}")


def test_device_form_head_major_bf16_cache(gpu):
    """one entry serves the head-major bf16 cache through explicit strides"""
    import torch
    cnt, start, H, KV, D, cap = 9, 40, 8, 4, 128, 64
    qbits = O.pack_bf16(O.fill_normal((cnt, H, D), 6, "q"))
    kbits = O.pack_bf16(O.fill_normal((KV, cap, D), 6, "k"))
    vbits = O.pack_bf16(O.fill_normal((KV, cap, D), 6, "v"))
    qf, kf, vf = O.unpack_bf16(qbits), O.unpack_bf16(kbits), O.unpack_bf16(vbits)
    ref = O.attention_strided(qf.reshape(-1), kf, vf, cnt, start, H, KV, D, D, D, cap * D)
    out = torch.zeros((cnt, H, D), dtype=torch.float32, device="cuda")
    say("device form head-major bf16")
    gpu.attention_device(dev_bf16(qbits), dev_bf16(kbits), dev_bf16(vbits), out, cnt, start, H, KV,
                         D, D, D, cap * D)
    assert_f32_parity(ref.reshape(cnt, H, D), host(out), "head-major")


def test_empty_and_invalid(gpu):
    q = np.zeros((1, 3, 8), np.float32)
    kv = np.zeros((1, 2, 8), np.float32)
    say("empty and invalid")
    out = gpu.attention(q, kv, kv, 0, 0, 3, 1, 8, 8)
    assert out.shape == (0, 3, 8)
    with pytest.raises(gpu.AiGpuError):
        gpu.attention(q, kv, kv, 1, 0, 3, 2, 8, 8)      # heads not a multiple of kvHeads
    assert "multiple" in gpu.last_error()


def test_counters_track_transfers(gpu):
    gpu.lib().aigpu_reset_counters()
    q = O.fill_normal((4, 2, 32), 7, "q")
    k = O.fill_normal((4, 2, 32), 7, "k")
    say("counters")
    gpu.attention(q, k, k, 4, 0, 2, 2, 32, 32)
    c = gpu.counters()
    assert c["launches"] >= 1 and c["hostToDeviceBytes"] >= q.nbytes + 2 * k.nbytes
    assert c["deviceToHostBytes"] == 4 * 2 * 32 * 4
    assert errors(np.zeros(1), np.zeros(1))["max_abs"] == 0


# The tiled fp32 form (fp32 q and KV, dim 64 or 128, 16-byte aligned rows):
# 128-token groups, 64-key tiles, key ranges split over workgroups whose
# records a merge launch combines when the groups alone leave CUs idle.
@pytest.mark.parametrize("count,start,H,KV,D,window,stride", [
    (300, 0, 8, 2, 128, 0, 128),     # three token groups, split, causal imbalance
    (200, 77, 4, 4, 64, 0, 64),      # history ending off a tile boundary, MHA
    (260, 40, 8, 2, 64, 100, 72),    # a window inside the tile range, qStride > dim
    (130, 500, 4, 1, 128, 33, 128),  # window 33, G = 4, a one-row second group
    (1, 4999, 2, 1, 64, 0, 64),      # one token against 5000 keys: many splits
    (33, 0, 2, 2, 128, 1, 128),      # window 1: every row sees only its own key
    (64, 0, 3, 1, 128, 0, 132),      # one tile, no split
])
def test_tiled_fp32_shapes(gpu, count, start, H, KV, D, window, stride):
    q = O.fill_normal((count, H, stride), 51, "q")
    k = O.fill_normal((start + count, KV, D), 52, "k")
    v = O.fill_normal((start + count, KV, D), 53, "v")
    ref = O.attention(q, k, v, count, start, H, KV, D, stride, window)
    say("tiled fp32", count, start, H, KV, D, window, stride)
    got = gpu.attention(q, k, v, count, start, H, KV, D, stride, window)
    assert_f32_parity(ref, got, f"tiled {count}/{start}/{D}/w{window}")


def test_tiled_fp32_head_major_strides(gpu):
    """the device form over an fp32 head-major cache (posStride = dim,
    headStride = capacity * dim), split, and called twice on one buffer"""
    cnt, start, H, KV, D, cap = 150, 90, 8, 2, 128, 256
    q = O.fill_normal((cnt, H, D), 54, "q")
    k = O.fill_normal((KV, cap, D), 55, "k")
    v = O.fill_normal((KV, cap, D), 56, "v")
    ref = O.attention_strided(q.reshape(-1), k, v, cnt, start, H, KV, D, D, D, cap * D)
    import torch
    out = torch.zeros((cnt, H, D), dtype=torch.float32, device="cuda")
    dq, dk, dv = dev_f32(q), dev_f32(k), dev_f32(v)
    for rep in range(2):
        say("tiled fp32 head-major", rep)
        gpu.attention_device(dq, dk, dv, out, cnt, start, H, KV, D, D, D, cap * D)
        assert_f32_parity(ref.reshape(cnt, H, D), host(out), f"head-major {rep}")


def test_tiled_fp32_unsplit_many_groups(gpu):
    """2048 tokens x 32 heads: enough workgroups that no key range is split;
    every head of 40 tokens (group edges, first, last) against the oracle"""
    cnt, H, KV, D = 2048, 32, 8, 128
    q = O.fill_normal((cnt, H, D), 57, "q")
    k = O.fill_normal((cnt, KV, D), 58, "k")
    v = O.fill_normal((cnt, KV, D), 59, "v")
    rows = sorted({0, 1, 31, 32, 127, 128, 129, 255, 256, 1023, 1024, 2046, 2047} |
                  set(range(3, 2048, 73)))
    ref = O.attention_strided(q.reshape(-1), k, v, cnt, 0, H, KV, D, D, KV * D, D, rows=rows, nthreads=0)
    say("tiled fp32 unsplit", cnt, H)
    got = gpu.attention(q, k, v, cnt, 0, H, KV, D, D)
    assert_f32_parity(ref, got[rows], "unsplit")
