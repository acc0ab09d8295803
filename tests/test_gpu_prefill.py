"""GPU parity of the prefill path (QK-RMSNorm -> RoPE -> KV append -> causal
GQA flash attention on fp16 MFMA) against the oracle restatement of
attentionMixer (LocalModel.hpp:2608-2659) + kernels::attention."""
import numpy as np
import pytest

from common import assert_bf16_parity, bf16_normal, errors, gammas
from gpu_util import dev_bf16, dev_f32, host, host_bits, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def run_case(gpu, count, start, H, KV, D, seed, norm=True, rope=True, window=0, dtype="bf16",
             rows=None, theta=1e6, q_stride=None, rot=None, gate=False):
    """Builds seeded inputs, runs the GPU prefill and the oracle; returns
    (oracle out, gpu out, oracle-normed keys, gpu caches)."""
    import torch
    qs = q_stride or D
    cap = start + count + 3
    if dtype == "bf16":
        qb, q = bf16_normal((count, H, qs), seed, "q")
        kb, k = bf16_normal((count, KV, D), seed, "k")
        vb, v = bf16_normal((count, KV, D), seed, "v")
        dq, dk, dv = dev_bf16(qb), dev_bf16(kb), dev_bf16(vb)
    else:
        q = O.fill_normal((count, H, qs), seed, "q")
        k = O.fill_normal((count, KV, D), seed, "k")
        v = O.fill_normal((count, KV, D), seed, "v")
        dq, dk, dv = dev_f32(q), dev_f32(k), dev_f32(v)
    gq = gammas(D, seed, "q_norm") if norm else None
    gk = gammas(D, seed, "k_norm") if norm else None
    rot = rot or D
    fr = O.rotary_frequencies(rot, theta) if rope else None
    # cached history [0, start): bf16 values in the head-major cache
    hkb, hk = bf16_normal((KV, start, D), seed, "k_cache")
    hvb, hv = bf16_normal((KV, start, D), seed, "v_cache")
    kc = np.zeros((KV, cap, D), np.uint16)
    vc = np.zeros((KV, cap, D), np.uint16)
    kc[:, :start] = hkb
    vc[:, :start] = hvb
    key_cache, value_cache = dev_bf16(kc), dev_bf16(vc)

    # oracle: norm + RoPE on fp32 (widened) inputs, then attention over history + new
    qn, kn = O.qk_norm_rope(q, k, count, start, H, KV, D, qs, gq, gk, 1e-6, fr, rot)
    keys = np.concatenate([hk.transpose(1, 0, 2), kn], 0)
    vals = np.concatenate([hv.transpose(1, 0, 2), v], 0)
    ref = O.attention_strided(qn, keys, vals, count, start, H, KV, D, qs, KV * D, D, window,
                              rows=rows, nthreads=0)
    if gate:   # attentionMixer's output gate: the raw second half of each q row
        assert rows is None
        ref = O.output_gate(ref, q, H, D, qs)

    out = torch.zeros((count, H, D), dtype=torch.float32, device="cuda")
    say("prefill", dict(count=count, start=start, H=H, KV=KV, D=D, window=window, dtype=dtype))
    gpu.prefill(dq, dk, dv, out, key_cache, value_cache, start, H, KV, D, q_stride=qs,
                q_norm=None if gq is None else dev_f32(gq),
                k_norm=None if gk is None else dev_f32(gk),
                freqs=None if fr is None else dev_f32(fr), rotary_dims=rot, window=window,
                output_gate=gate, check=True)
    got = host(out)
    if rows is not None:
        got = got[rows]
    return ref, got, kn, v, host(key_cache), host_bits(value_cache), vb if dtype == "bf16" else None


@pytest.mark.parametrize("D", [64, 128])
def test_small_gqa_norm_rope(gpu, D):
    ref, got, kn, v, kc, vcb, vb = run_case(gpu, 300, 0, 8, 2, D, 40)
    assert_bf16_parity(ref, got, f"D={D}")


def test_cache_append_layout(gpu):
    count, start, KV, D = 70, 25, 2, 128
    ref, got, kn, v, kc, vcb, vb = run_case(gpu, count, start, 4, KV, D, 41)
    assert_bf16_parity(ref, got, "history")
    # new keys land at [kv][start + t] as bf16 of the normed, rotated key
    new_k = kc[:, start:start + count].transpose(1, 0, 2)
    assert np.abs(new_k - kn).max() <= np.abs(kn).max() * 2 ** -8
    # values are appended unchanged
    assert np.array_equal(vcb[:, start:start + count].transpose(1, 0, 2), vb)


def test_fp32_inputs_mha_no_norm_no_rope(gpu):
    ref, got, *_ = run_case(gpu, 129, 0, 12, 12, 64, 42, norm=False, rope=False, dtype="f32")
    assert_bf16_parity(ref, got, "mha fp32 inputs")


@pytest.mark.parametrize("window", [1, 33, 100])
def test_sliding_window(gpu, window):
    ref, got, *_ = run_case(gpu, 250, 10, 4, 2, 128, 43, window=window)
    assert_bf16_parity(ref, got, f"window {window}")


def test_q_stride_with_gate_halves(gpu):
    # Qwen3.5-style q rows carry a gate after each head (qStride = 2D, LocalModel.hpp:2583)
    ref, got, *_ = run_case(gpu, 40, 0, 4, 2, 64, 44, q_stride=128)
    assert_bf16_parity(ref, got, "qStride 2D")


@pytest.mark.parametrize("rot", [32, 24])
def test_partial_rotary(gpu, rot):
    # rot % 16 == 0 takes the register-row prep kernel, other even widths the
    # LDS-row one
    ref, got, *_ = run_case(gpu, 90, 7, 4, 2, 128, 46, rot=rot)
    assert_bf16_parity(ref, got, f"rotary {rot} of 128")


@pytest.mark.parametrize("qs", [72, 68])
def test_q_stride_alignment(gpu, qs):
    # a 16-byte multiple row stride (72 bf16) and one that is not (68)
    ref, got, *_ = run_case(gpu, 60, 5, 4, 2, 64, 47, q_stride=qs)
    assert_bf16_parity(ref, got, f"qStride {qs}")


def test_fp32_inputs_gqa_norm_rope_history(gpu):
    ref, got, *_ = run_case(gpu, 70, 30, 8, 2, 128, 48, dtype="f32")
    assert_bf16_parity(ref, got, "fp32 inputs with history")


def test_single_token_and_ragged_tiles(gpu):
    for count in (1, 127, 128, 129):
        ref, got, *_ = run_case(gpu, count, 0, 4, 4, 128, 45 + count)
        assert_bf16_parity(ref, got, f"count {count}")


def test_cfg3_qwen3_8b_prefill_8k_sampled_rows(gpu):
    """32 q / 8 kv heads, D 128, seq 8192, QK-norm + RoPE theta 1e6,
    N(0,1) bf16 seed 2. Full GPU run; oracle on sampled rows (every row is an
    independent softmax, so a row subset checks the full-size kernel)."""
    rows = list(range(0, 64)) + list(range(64, 8128, 97)) + list(range(8128, 8192))
    ref, got, *_ = run_case(gpu, 8192, 0, 32, 8, 128, 2, rows=rows)
    e = assert_bf16_parity(ref, got, "cfg3")
    say("cfg3 errors", e)


@pytest.mark.parametrize("count,start,H,KV,window", [(4000, 300, 64, 8, 0), (4000, 300, 64, 8, 700),
                                                      (3600, 0, 40, 8, 0)])
def test_large_grids_sampled_rows(gpu, count, start, H, KV, window):
    """Grids of 600 to 1,024 workgroups (several per compute unit): a ragged
    last tile, history, a window that moves the first key tile of every
    query tile, and 5 query heads per kv head. Sampled rows cover every
    query tile's first and last rows and the call's last rows."""
    rows = sorted(set(list(range(0, count, 256)) + list(range(255, count, 256)) +
                      list(range(37, count, 211)) + list(range(count - 40, count))))
    ref, got, *_ = run_case(gpu, count, start, H, KV, 128, 60 + H + window, window=window, rows=rows)
    assert_bf16_parity(ref, got, f"count {count} H {H} window {window}")


def test_rejects_unsupported_dim(gpu):
    import torch
    x = torch.zeros((2, 2, 96), dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros((2, 4, 96), dtype=torch.bfloat16, device="cuda")
    out = torch.zeros((2, 2, 96), dtype=torch.float32, device="cuda")
    with pytest.raises(gpu.AiGpuError):
        gpu.prefill(x, x, x, out, kc, kc, 0, 2, 2, 96)
    assert "dim" in gpu.last_error()
    assert errors(np.ones(2), np.ones(2))["rel_l2"] == 0


@pytest.mark.parametrize("dtype,D", [("bf16", 128), ("f32", 64), ("bf16", 64)])
def test_output_gate(gpu, dtype, D):
    """Qwen3.5's attnOutputGate (LocalModel.hpp:2660-2665): q rows of 2 D,
    the second half gating the output through a sigmoid"""
    ref, got, *_ = run_case(gpu, 150, 20, 8, 2, D, 77, dtype=dtype, q_stride=2 * D, gate=True)
    assert_bf16_parity(ref, got, f"gate {dtype} D={D}")


def test_output_gate_needs_wide_rows(gpu):
    import aigpu
    with pytest.raises(aigpu.AiGpuError, match="output gate"):
        run_case(gpu, 4, 0, 2, 1, 64, 78, q_stride=64, gate=True)
