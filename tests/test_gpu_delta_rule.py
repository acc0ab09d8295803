"""GPU parity of the gated delta rule (chunked scan) against the oracle's
sequential restatement of gatedDeltaNetMixer's recurrence
(LocalModel.hpp:2802-2830, deltaStep at Kernels.hpp:105-128)."""
import numpy as np
import pytest

from common import assert_bf16_parity, assert_f32_parity, bf16_normal
from gpu_util import dev_bf16, dev_f32, host, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def gates(S, hv, seed, decay_scale=1.0):
    g = -np.log1p(np.exp(O.fill_normal((S, hv), seed, "g").astype(np.float64)))
    g = (g * decay_scale).astype(np.float32)
    beta = (1.0 / (1.0 + np.exp(-O.fill_normal((S, hv), seed, "beta").astype(np.float64)))).astype(np.float32)
    return g, beta


def misaligned(t):
    """the same values in a view that starts 2 bytes past a 16-byte boundary"""
    import torch
    flat = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    flat[1:].copy_(t.reshape(-1))
    return flat[1:].view(t.shape)


def run_gdn(gpu, S, hk, hv, kd, vd, seed, dtype="f32", state0=None, raw_gates=False, unaligned=False,
            decay_scale=1.0):
    import torch
    if dtype == "bf16":
        qb, q = bf16_normal((S, hk, kd), seed, "q")
        kb, k = bf16_normal((S, hk, kd), seed, "k")
        vb, v = bf16_normal((S, hv, vd), seed, "v")
        dq, dk, dv = dev_bf16(qb), dev_bf16(kb), dev_bf16(vb)
        if unaligned:   # the register-staged scan instead of the DMA scan
            dq, dk, dv = misaligned(dq), misaligned(dk), misaligned(dv)
            assert dq.data_ptr() % 16 == 2
    else:
        q = O.fill_normal((S, hk, kd), seed, "q")
        k = O.fill_normal((S, hk, kd), seed, "k")
        v = O.fill_normal((S, hv, vd), seed, "v")
        dq, dk, dv = dev_f32(q), dev_f32(k), dev_f32(v)
    s0 = np.zeros((hv, kd, vd), np.float32) if state0 is None else state0
    state = dev_f32(s0)
    out = torch.zeros((S, hv, vd), dtype=torch.float32, device="cuda")
    say("delta rule", dict(S=S, hk=hk, hv=hv, kd=kd, vd=vd, dtype=dtype, raw=raw_gates))
    if raw_gates:
        a = O.fill_normal((S, hv), seed, "a")
        b = O.fill_normal((S, hv), seed, "b")
        alog = O.fill_normal((hv,), seed, "alog") * np.float32(0.5)
        dt = O.fill_normal((hv,), seed, "dt")
        g, beta = O.gdn_gates(a, b, alog, dt)
        gpu.gated_delta_rule(dq, dk, dv, state, out, a=dev_f32(a), b=dev_f32(b), a_log=dev_f32(alog),
                             dt_bias=dev_f32(dt))
    else:
        g, beta = gates(S, hv, seed, decay_scale)
        gpu.gated_delta_rule(dq, dk, dv, state, out, g=dev_f32(g), beta=dev_f32(beta))
    ref_out, ref_state = O.gated_delta_rule(q, k, v, g, beta, state=s0, nthreads=0)
    return ref_out, host(out), ref_state, host(state)


@pytest.mark.parametrize("S", [1, 63, 64, 65, 200])
def test_lengths_fp32(gpu, S):
    ro, go, rs, gs = run_gdn(gpu, S, 2, 4, 128, 128, 100 + S)
    assert_f32_parity(ro, go, f"out S={S}")
    assert_f32_parity(rs, gs, f"state S={S}")


# bf16 inputs take the bf16 hi/residual split kernel; fp32 inputs the fp32 one
@pytest.mark.parametrize("S", [1, 63, 64, 65, 200])
def test_lengths_bf16(gpu, S):
    ro, go, rs, gs = run_gdn(gpu, S, 2, 4, 128, 128, 200 + S, dtype="bf16")
    assert_bf16_parity(ro, go, f"out S={S}")
    assert_bf16_parity(rs, gs, f"state S={S}")


@pytest.mark.parametrize("kd", [128, 64])
def test_bf16_unaligned_inputs(gpu, kd):
    ro, go, rs, gs = run_gdn(gpu, 130, 2, 4, kd, 32, 300 + kd, dtype="bf16", unaligned=True)
    assert_bf16_parity(ro, go, f"out bf16 unaligned kd{kd}")
    assert_bf16_parity(rs, gs, f"state bf16 unaligned kd{kd}")


def test_bf16_raw_gates_initial_state_kd64(gpu):
    s0 = O.fill_normal((4, 64, 48), 17, "s0") * np.float32(0.1)
    ro, go, rs, gs = run_gdn(gpu, 300, 2, 4, 64, 48, 17, dtype="bf16", state0=s0, raw_gates=True)
    assert_bf16_parity(ro, go, "out bf16 kd64")
    assert_bf16_parity(rs, gs, "state bf16 kd64")


def test_raw_gates_and_initial_state(gpu):
    s0 = O.fill_normal((4, 128, 64), 7, "s0") * np.float32(0.1)
    ro, go, rs, gs = run_gdn(gpu, 150, 2, 4, 128, 64, 7, state0=s0, raw_gates=True)
    assert_f32_parity(ro, go, "out raw gates")
    assert_f32_parity(rs, gs, "state raw gates")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_eight_value_heads_per_key_head(gpu, dtype):
    """G = 8 value heads share each key head: the solve loads the first four
    heads' gates beside the q/k rows and the rest inside its head loop"""
    ro, go, rs, gs = run_gdn(gpu, 150, 2, 16, 128, 32, 21, dtype=dtype)
    check = assert_f32_parity if dtype == "f32" else assert_bf16_parity
    check(ro, go, f"out G=8 {dtype}")
    check(rs, gs, f"state G=8 {dtype}")


@pytest.mark.parametrize("scale", [0.02, 30.0])
def test_bf16_weak_and_strong_decays(gpu, scale):
    """log decays scaled to near 0 (the state barely forgets) and to ~-20 per
    token (in-chunk decays underflow to 0): the split records' base-2
    exponentials against the oracle's"""
    ro, go, rs, gs = run_gdn(gpu, 200, 2, 4, 128, 64, 23, dtype="bf16", decay_scale=scale)
    assert_bf16_parity(ro, go, f"out decay x{scale}")
    assert_bf16_parity(rs, gs, f"state decay x{scale}")


def test_key_dim_64(gpu):
    ro, go, rs, gs = run_gdn(gpu, 100, 4, 4, 64, 32, 8)
    assert_f32_parity(ro, go, "out kd64")
    assert_f32_parity(rs, gs, "state kd64")


def test_chunk_continuation(gpu):
    """a split call (state carried) equals one call: chunk continuity, the
    kernel-level form of llm-testing.cpp:853-890"""
    import torch
    S, hk, hv, kd, vd = 130, 2, 4, 128, 32
    q = O.fill_normal((S, hk, kd), 9, "q")
    k = O.fill_normal((S, hk, kd), 9, "k")
    v = O.fill_normal((S, hv, vd), 9, "v")
    g, beta = gates(S, hv, 9)
    whole_state = dev_f32(np.zeros((hv, kd, vd), np.float32))
    whole = torch.zeros((S, hv, vd), dtype=torch.float32, device="cuda")
    say("continuation")
    gpu.gated_delta_rule(dev_f32(q), dev_f32(k), dev_f32(v), whole_state, whole, g=dev_f32(g), beta=dev_f32(beta))
    split_state = dev_f32(np.zeros((hv, kd, vd), np.float32))
    parts = []
    for lo, hi in ((0, 64), (64, 100), (100, 130)):
        o = torch.zeros((hi - lo, hv, vd), dtype=torch.float32, device="cuda")
        gpu.gated_delta_rule(dev_f32(q[lo:hi]), dev_f32(k[lo:hi]), dev_f32(v[lo:hi]), split_state, o,
                             g=dev_f32(g[lo:hi]), beta=dev_f32(beta[lo:hi]))
        parts.append(host(o))
    assert_f32_parity(host(whole), np.concatenate(parts), "continuation out")
    assert_f32_parity(host(whole_state), host(split_state), "continuation state")


def test_cfg5_qwen3_next_16k(gpu):
    """16 qk / 32 v heads, D 128, seq 16384, chunk 64, bf16 inputs,
    l2-normalised q/k, beta = sigmoid(N(0,1)), g = -softplus(N(0,1)), seed 4."""
    ro, go, rs, gs = run_gdn(gpu, 16384, 16, 32, 128, 128, 4, dtype="bf16")
    say("cfg5 out", assert_bf16_parity(ro, go, "cfg5 out"))
    say("cfg5 state", assert_bf16_parity(rs, gs, "cfg5 state"))


def two_level_launches(fn):
    """runs fn with launch profiling on; the number of pass-C launches of the
    two-level scan it made"""
    import aigpu
    aigpu.profile(True)
    aigpu.profile_reset()
    try:
        result = fn()
        _, n = aigpu.profile_read("delta_seg_kernel<true>")
    finally:
        aigpu.profile(False)
    return result, n


# 128 x 128 heads over at least 8 chunks per segment take the two-level scan:
# P = 256 CUs / value heads segments (at most 16), cut as evenly as whole chunks
# allow; these shapes give P = 8 with L = 9 (segments 9 x 7 + 2 and a ragged
# last chunk), P = 4 with L = 9 (9, 9, 9, 6), and P = 15 with L = 9, with two
# value heads per key head, then four (P = 8) and one (P = 4); 20 value heads
# (P = 12, L = 10: a head count that is not a multiple of 8, so the join's
# workgroups of a head do not share an XCD)
@pytest.mark.parametrize("S,hk,hv", [(4100, 16, 32), (2085, 32, 64), (8292, 8, 16), (4100, 8, 32), (2085, 64, 64),
                                     (7323, 10, 20)])
def test_bf16_two_level_scan(gpu, S, hk, hv):
    s0 = O.fill_normal((hv, 128, 128), 31, "s0") * np.float32(0.1)
    (ro, go, rs, gs), n = two_level_launches(
        lambda: run_gdn(gpu, S, hk, hv, 128, 128, 31 + S, dtype="bf16", state0=s0))
    assert n == 1, "the two-level scan did not run"
    say(f"two-level S={S} hv={hv} out", assert_bf16_parity(ro, go, f"out two-level S={S}"))
    say(f"two-level S={S} hv={hv} state", assert_bf16_parity(rs, gs, f"state two-level S={S}"))


def test_bf16_two_level_scan_raw_gates(gpu):
    (ro, go, rs, gs), n = two_level_launches(
        lambda: run_gdn(gpu, 2085, 32, 64, 128, 128, 41, dtype="bf16", raw_gates=True))
    assert n == 1, "the two-level scan did not run"
    assert_bf16_parity(ro, go, "out two-level raw gates")
    assert_bf16_parity(rs, gs, "state two-level raw gates")


def test_bf16_two_level_continuation(gpu):
    """4,100 tokens in one call (65 chunks, P = 4, L = 17) against two calls of
    2,050 (33 chunks each, P = 4, L = 9) carrying the state: both take the
    two-level scan, and the split, unaligned to a chunk, must agree"""
    import torch
    S, hk, hv = 4100, 32, 64
    qb, _ = bf16_normal((S, hk, 128), 43, "q")
    kb, _ = bf16_normal((S, hk, 128), 43, "k")
    vb, _ = bf16_normal((S, hv, 128), 43, "v")
    g, beta = gates(S, hv, 43)
    s0 = O.fill_normal((hv, 128, 128), 43, "s0") * np.float32(0.1)

    def run(lo, hi, state):
        o = torch.zeros((hi - lo, hv, 128), dtype=torch.float32, device="cuda")
        gpu.gated_delta_rule(dev_bf16(qb[lo:hi]), dev_bf16(kb[lo:hi]), dev_bf16(vb[lo:hi]), state, o,
                             g=dev_f32(g[lo:hi]), beta=dev_f32(beta[lo:hi]))
        return host(o)

    say("two-level continuation")
    whole_state = dev_f32(s0)
    whole, n = two_level_launches(lambda: run(0, S, whole_state))
    assert n == 1
    split_state = dev_f32(s0)
    parts, n = two_level_launches(lambda: [run(0, 2050, split_state), run(2050, S, split_state)])
    assert n == 2
    assert_bf16_parity(whole, np.concatenate(parts), "two-level continuation out")
    assert_bf16_parity(host(whole_state), host(split_state), "two-level continuation state")


@pytest.mark.parametrize("dtype,S,hk,hv", [("f32", 200, 2, 4), ("bf16", 4100, 16, 32)])
def test_host_form(gpu, dtype, S, hk, hv):
    """aigpu_gated_delta_rule_host, the entry the reference's mixer binds
    (host arrays staged through the backend's scratch): the single-level fp32
    scan, and the two-level scan for bf16 rows that the staging leaves on
    16-byte boundaries"""
    import aigpu
    seed = 51 + S
    if dtype == "bf16":
        qb, q = bf16_normal((S, hk, 128), seed, "q")
        kb, k = bf16_normal((S, hk, 128), seed, "k")
        vb, v = bf16_normal((S, hv, 128), seed, "v")
        args = (qb, kb, vb)
    else:
        q = O.fill_normal((S, hk, 128), seed, "q")
        k = O.fill_normal((S, hk, 128), seed, "k")
        v = O.fill_normal((S, hv, 128), seed, "v")
        args = (q, k, v)
    g, beta = gates(S, hv, seed)
    s0 = O.fill_normal((hv, 128, 128), seed, "s0") * np.float32(0.1)
    state = s0.copy()
    say("delta rule host form", dict(S=S, hk=hk, hv=hv, dtype=dtype))
    out, n = two_level_launches(lambda: aigpu.gated_delta_rule_host(*args, state, g=g, beta=beta))
    assert n == (1 if dtype == "bf16" else 0)
    ref_out, ref_state = O.gated_delta_rule(q, k, v, g, beta, state=s0, nthreads=0)
    check = assert_f32_parity if dtype == "f32" else assert_bf16_parity
    check(ref_out, out, f"host form out {dtype}")
    check(ref_state, state, f"host form state {dtype}")
