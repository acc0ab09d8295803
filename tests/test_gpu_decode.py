"""GPU parity of the batched decode (norm + RoPE on load, KV append, split-K
attention over a head-major bf16 cache) against the oracle restatement of
attentionMixer with count = 1 (LocalModel.hpp:2608-2659)."""
import numpy as np
import pytest

from common import assert_bf16_parity, bf16_normal, gammas
from gpu_util import dev_bf16, dev_f32, dev_u32, host, host_bits, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def run_decode(gpu, lengths, H, KV, D, seed, norm=True, rope=True, window=0, dtype="bf16",
               cap=None, theta=1e6, q_stride=None, check_cache=False, gate=False):
    import torch
    B = len(lengths)
    qs = q_stride or D
    cap = cap or (max(lengths) + 1)
    if dtype == "bf16":
        qb, q = bf16_normal((B, H, qs), seed, "q")
        kb, k = bf16_normal((B, KV, D), seed, "k")
        vb, v = bf16_normal((B, KV, D), seed, "v")
        dq, dk, dv = dev_bf16(qb), dev_bf16(kb), dev_bf16(vb)
    else:
        q = O.fill_normal((B, H, qs), seed, "q")
        k = O.fill_normal((B, KV, D), seed, "k")
        v = O.fill_normal((B, KV, D), seed, "v")
        dq, dk, dv = dev_f32(q), dev_f32(k), dev_f32(v)
    gq = gammas(D, seed, "q_norm") if norm else None
    gk = gammas(D, seed, "k_norm") if norm else None
    fr = O.rotary_frequencies(D, theta) if rope else None

    kc = np.zeros((B, KV, cap, D), np.uint16)
    vc = np.zeros((B, KV, cap, D), np.uint16)
    refs = []
    for b, L in enumerate(lengths):
        hkb, hk = bf16_normal((KV, L, D), seed, f"k_cache{b}")
        hvb, hv = bf16_normal((KV, L, D), seed, f"v_cache{b}")
        kc[b, :, :L] = hkb
        vc[b, :, :L] = hvb
        qn, kn = O.qk_norm_rope(q[b:b + 1], k[b:b + 1], 1, L, H, KV, D, qs, gq, gk, 1e-6, fr, D)
        keys = np.concatenate([hk.transpose(1, 0, 2), kn], 0)
        vals = np.concatenate([hv.transpose(1, 0, 2), v[b:b + 1]], 0)
        att = O.attention(qn, keys, vals, 1, L, H, KV, D, qs, window, nthreads=0)
        if gate:   # attentionMixer's output gate (LocalModel.hpp:2660-2665)
            att = O.output_gate(att, q[b:b + 1], H, D, qs)
        refs.append(att[0])
        refs[-1] = (refs[-1], kn[0])
    key_cache, value_cache = dev_bf16(kc), dev_bf16(vc)
    pos = dev_u32(np.array(lengths, np.uint32))
    out = torch.zeros((B, H, D), dtype=torch.float32, device="cuda")
    say("decode", dict(B=B, Lmax=max(lengths), H=H, KV=KV, D=D, window=window, dtype=dtype))
    gpu.decode(dq, dk, dv, out, key_cache, value_cache, pos, max(lengths), H, KV, D, q_stride=qs,
               q_norm=None if gq is None else dev_f32(gq),
               k_norm=None if gk is None else dev_f32(gk),
               freqs=None if fr is None else dev_f32(fr), rotary_dims=D, window=window,
               output_gate=gate)
    got = host(out)
    ref = np.stack([r[0] for r in refs])
    if check_cache:
        kcg = host(key_cache)
        vcg = host_bits(value_cache)
        for b, L in enumerate(lengths):
            kn = refs[b][1]
            assert np.abs(kcg[b, :, L] - kn).max() <= np.abs(kn).max() * 2 ** -8
            assert np.array_equal(vcg[b, :, L], vb[b] if dtype == "bf16" else O.pack_bf16(v[b]))
            # history untouched
            assert np.array_equal(host_bits(key_cache)[b, :, :L], kc[b, :, :L])
    return ref, got


def test_cfg2_qwen3_06b_decode(gpu):
    """16 q / 8 kv heads, D 128, cache 4096, QK-norm + RoPE at 4096, seed 1."""
    ref, got = run_decode(gpu, [4096], 16, 8, 128, 1, check_cache=True)
    say("cfg2 errors", assert_bf16_parity(ref, got, "cfg2"))


def test_cfg4_qwen3_30b_a3b_batched_ragged(gpu):
    """32 sequences, 32 q / 4 kv heads, D 128, lengths
    randInt(1024, 32768) drawn first from Random(3)."""
    r = O.Rng(3)
    lengths = [r.randint(1024, 32768) for _ in range(32)]
    ref, got = run_decode(gpu, lengths, 32, 4, 128, 3)
    say("cfg4 errors", assert_bf16_parity(ref, got, "cfg4"))


@pytest.mark.parametrize("L", [0, 1, 63, 64, 65, 511, 512, 513, 1000, 2049])
def test_chunk_boundaries(gpu, L):
    ref, got = run_decode(gpu, [L], 8, 1, 128, 50 + L, check_cache=True)
    assert_bf16_parity(ref, got, f"L={L}")


@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_group_sizes(gpu, G):
    ref, got = run_decode(gpu, [300, 5, 1500], 2 * G, 2, 128, 60 + G)
    assert_bf16_parity(ref, got, f"G={G}")


def test_dim64_fp32_inputs_no_norm(gpu):
    ref, got = run_decode(gpu, [700, 33, 1], 8, 4, 64, 70, norm=False, dtype="f32")
    assert_bf16_parity(ref, got, "D=64 fp32")


@pytest.mark.parametrize("window", [1, 7, 300])
def test_sliding_window(gpu, window):
    ref, got = run_decode(gpu, [1200, 5, 299], 8, 2, 128, 80, window=window)
    assert_bf16_parity(ref, got, f"window {window}")


def test_capacity_beyond_length(gpu):
    ref, got = run_decode(gpu, [100, 900], 4, 2, 128, 90, cap=4096)
    assert_bf16_parity(ref, got, "cap 4096")


def test_rejects_too_many_heads_per_group(gpu):
    import torch
    q = torch.zeros((1, 16, 128), dtype=torch.bfloat16, device="cuda")
    kv = torch.zeros((1, 1, 128), dtype=torch.bfloat16, device="cuda")
    cache = torch.zeros((1, 1, 8, 128), dtype=torch.bfloat16, device="cuda")
    out = torch.zeros((1, 16, 128), dtype=torch.float32, device="cuda")
    pos = dev_u32(np.array([3], np.uint32))
    with pytest.raises(gpu.AiGpuError):
        gpu.decode(q, kv, kv, out, cache, cache, pos, 3, 16, 1, 128)


def test_prefill_then_decode_shares_the_cache(gpu):
    """the cache a prefill writes is the cache decode reads (positions, layout)"""
    import torch
    P, H, KV, D, cap, seed = 600, 8, 2, 128, 1024, 95
    qb, q = bf16_normal((P + 1, H, D), seed, "q")
    kb, k = bf16_normal((P + 1, KV, D), seed, "k")
    vb, v = bf16_normal((P + 1, KV, D), seed, "v")
    gq, gk = gammas(D, seed, "qn"), gammas(D, seed, "kn")
    fr = O.rotary_frequencies(D, 1e6)
    key_cache = torch.zeros((KV, cap, D), dtype=torch.bfloat16, device="cuda")
    value_cache = torch.zeros_like(key_cache)
    out = torch.zeros((P, H, D), dtype=torch.float32, device="cuda")
    say("prefill then decode")
    gpu.prefill(dev_bf16(qb[:P]), dev_bf16(kb[:P]), dev_bf16(vb[:P]), out, key_cache, value_cache, 0,
                H, KV, D, q_norm=dev_f32(gq), k_norm=dev_f32(gk), freqs=dev_f32(fr), rotary_dims=D)
    hist_k = host(key_cache)[:, :P].transpose(1, 0, 2)
    hist_v = host(value_cache)[:, :P].transpose(1, 0, 2)
    out1 = torch.zeros((1, H, D), dtype=torch.float32, device="cuda")
    gpu.decode(dev_bf16(qb[P:]), dev_bf16(kb[P:]), dev_bf16(vb[P:]), out1, key_cache, value_cache,
               dev_u32(np.array([P], np.uint32)), P, H, KV, D, q_norm=dev_f32(gq),
               k_norm=dev_f32(gk), freqs=dev_f32(fr), rotary_dims=D)
    qn, kn = O.qk_norm_rope(q[P:], k[P:], 1, P, H, KV, D, D, gq, gk, 1e-6, fr, D)
    keys = np.concatenate([hist_k, kn], 0)
    vals = np.concatenate([hist_v, v[P:]], 0)
    ref = O.attention(qn, keys, vals, 1, P, H, KV, D, D)
    assert_bf16_parity(ref, host(out1), "prefill -> decode")


@pytest.mark.parametrize("lengths", [[40], [3000, 17, 700]])
def test_output_gate(gpu, lengths):
    """the output gate on both write paths: one-chunk sequences (attention
    kernel) and multi-chunk ones (merge kernel)"""
    ref, got = run_decode(gpu, lengths, 8, 2, 128, 91, q_stride=256, gate=True)
    assert_bf16_parity(ref, got, f"gate {lengths}")


def test_host_form_matches_device_form(gpu):
    """aigpu_decode_attention_host (host q/k/v, positions, norms, frequencies;
    device caches) against the device form on the same inputs: the same
    kernels run, so the outputs and both caches are bit-identical"""
    import torch
    lengths, H, KV, D, seed = [300, 1, 4096, 1500], 16, 8, 128, 61
    B, cap = len(lengths), 4097
    qb, _ = bf16_normal((B, H, D), seed, "q")
    kb, _ = bf16_normal((B, KV, D), seed, "k")
    vb, _ = bf16_normal((B, KV, D), seed, "v")
    gq, gk = gammas(D, seed, "q_norm"), gammas(D, seed, "k_norm")
    fr = O.rotary_frequencies(D, 1e6)
    kc = np.zeros((B, KV, cap, D), np.uint16)
    vc = np.zeros((B, KV, cap, D), np.uint16)
    for b, L in enumerate(lengths):
        kc[b, :, :L] = bf16_normal((KV, L, D), seed, f"k_cache{b}")[0]
        vc[b, :, :L] = bf16_normal((KV, L, D), seed, f"v_cache{b}")[0]
    pos = np.array(lengths, np.uint32)
    say("decode host form", dict(B=B, H=H, KV=KV, D=D))
    kd, vd = dev_bf16(kc), dev_bf16(vc)
    out = torch.zeros((B, H, D), dtype=torch.float32, device="cuda")
    gpu.decode(dev_bf16(qb), dev_bf16(kb), dev_bf16(vb), out, kd, vd, dev_u32(pos), max(lengths), H, KV, D,
               q_norm=dev_f32(gq), k_norm=dev_f32(gk), freqs=dev_f32(fr), rotary_dims=D)
    kh, vh = dev_bf16(kc), dev_bf16(vc)
    got = gpu.decode_host(qb, kb, vb, kh, vh, pos, H, KV, D, q_norm=gq, k_norm=gk, freqs=fr, rotary_dims=D)
    assert np.array_equal(got, host(out))
    assert np.array_equal(host_bits(kh), host_bits(kd))
    assert np.array_equal(host_bits(vh), host_bits(vd))
