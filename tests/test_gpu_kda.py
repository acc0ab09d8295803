"""GPU parity of Kimi Delta Attention's recurrence (chunked scan, one decay per
key channel) against the oracle's sequential restatement of kimiDeltaMixer
(LocalModel.hpp:2928-2947, deltaStep with perKeyDecay at Kernels.hpp:105-128).

Both input types compute in fp32 on the GPU (bf16 inputs are widened exactly),
so both are held to the fp32 bar."""
import numpy as np
import pytest

from common import assert_f32_parity, bf16_normal
from gpu_util import dev_bf16, dev_f32, host, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def decays(S, hv, kd, seed, scale=1.0):
    """log decays -softplus(x): every channel decays, some fast, some barely"""
    x = O.fill_normal((S, hv, kd), seed, "gk").astype(np.float64) * scale
    return (-np.log1p(np.exp(x))).astype(np.float32)


def run_kda(gpu, S, hk, hv, kd, vd, seed, dtype="f32", state0=None, normalize=True, gscale=1.0):
    import torch
    if dtype == "bf16":
        qb, q = bf16_normal((S, hk, kd), seed, "q")
        kb, k = bf16_normal((S, hk, kd), seed, "k")
        vb, v = bf16_normal((S, hv, vd), seed, "v")
        dq, dk, dv = dev_bf16(qb), dev_bf16(kb), dev_bf16(vb)
    else:
        q = O.fill_normal((S, hk, kd), seed, "q")
        k = O.fill_normal((S, hk, kd), seed, "k")
        v = O.fill_normal((S, hv, vd), seed, "v")
        if not normalize:   # unnormalised keys must stay small for the rule to stay bounded
            q = q * np.float32(1.0 / np.sqrt(kd))
            k = k * np.float32(1.0 / np.sqrt(kd))
        dq, dk, dv = dev_f32(q), dev_f32(k), dev_f32(v)
    g = decays(S, hv, kd, seed, gscale)
    beta = (1.0 / (1.0 + np.exp(-O.fill_normal((S, hv), seed, "beta").astype(np.float64)))).astype(np.float32)
    s0 = np.zeros((hv, kd, vd), np.float32) if state0 is None else state0
    state = dev_f32(s0)
    out = torch.zeros((S, hv, vd), dtype=torch.float32, device="cuda")
    say("kda", dict(S=S, hk=hk, hv=hv, kd=kd, vd=vd, dtype=dtype, normalize=normalize))
    gpu.kda_rule(dq, dk, dv, dev_f32(g), dev_f32(beta), state, out, normalize=normalize)
    ref_out, ref_state = O.kda_rule(q, k, v, g, beta, state=s0, normalize=normalize, nthreads=0)
    return ref_out, host(out), ref_state, host(state)


@pytest.mark.parametrize("S", [1, 63, 64, 65, 200])
def test_lengths_fp32(gpu, S):
    ro, go, rs, gs = run_kda(gpu, S, 2, 4, 128, 128, 500 + S)
    assert_f32_parity(ro, go, f"out S={S}")
    assert_f32_parity(rs, gs, f"state S={S}")


@pytest.mark.parametrize("S", [1, 65, 200])
def test_lengths_bf16_inputs(gpu, S):
    ro, go, rs, gs = run_kda(gpu, S, 2, 4, 128, 128, 600 + S, dtype="bf16")
    assert_f32_parity(ro, go, f"out bf16 S={S}")
    assert_f32_parity(rs, gs, f"state bf16 S={S}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_key_dim_64_and_initial_state(gpu, dtype):
    s0 = O.fill_normal((6, 64, 32), 7, "s0") * np.float32(0.5)
    ro, go, rs, gs = run_kda(gpu, 150, 3, 6, 64, 32, 700, dtype=dtype, state0=s0)
    assert_f32_parity(ro, go, f"out kd64 {dtype}")
    assert_f32_parity(rs, gs, f"state kd64 {dtype}")


def test_fast_decays(gpu):
    """decays near zero in a few tokens: exp(gc_t - gc_j) underflows across the
    chunk, which the factorisation through a block's first row must survive"""
    ro, go, rs, gs = run_kda(gpu, 130, 1, 2, 128, 64, 800, gscale=6.0)
    assert_f32_parity(ro, go, "out fast decay")
    assert_f32_parity(rs, gs, "state fast decay")


def test_unnormalised(gpu):
    ro, go, rs, gs = run_kda(gpu, 100, 2, 2, 64, 16, 900, normalize=False)
    assert_f32_parity(ro, go, "out raw")
    assert_f32_parity(rs, gs, "state raw")


def test_chunked_calls_carry_the_state(gpu):
    """one call over 150 tokens equals calls of 64 + 86 tokens with the state
    carried between them"""
    import torch
    S, hk, hv, kd, vd = 150, 1, 2, 64, 32
    q = O.fill_normal((S, hk, kd), 41, "q")
    k = O.fill_normal((S, hk, kd), 41, "k")
    v = O.fill_normal((S, hv, vd), 41, "v")
    g = decays(S, hv, kd, 41)
    beta = np.full((S, hv), 0.7, np.float32)
    say("kda split", dict(S=S))
    st1 = dev_f32(np.zeros((hv, kd, vd), np.float32))
    o1 = torch.zeros((S, hv, vd), dtype=torch.float32, device="cuda")
    gpu.kda_rule(dev_f32(q), dev_f32(k), dev_f32(v), dev_f32(g), dev_f32(beta), st1, o1)
    st2 = dev_f32(np.zeros((hv, kd, vd), np.float32))
    parts = []
    for a, b in ((0, 64), (64, S)):
        o = torch.zeros((b - a, hv, vd), dtype=torch.float32, device="cuda")
        gpu.kda_rule(dev_f32(q[a:b]), dev_f32(k[a:b]), dev_f32(v[a:b]), dev_f32(g[a:b]), dev_f32(beta[a:b]), st2, o)
        parts.append(host(o))
    assert_f32_parity(host(o1), np.concatenate(parts), "split out")
    assert_f32_parity(host(st1), host(st2), "split state")


def test_rejects_bad_shapes(gpu):
    import torch
    z = torch.zeros((4, 1, 96), dtype=torch.float32, device="cuda")
    v = torch.zeros((4, 1, 16), dtype=torch.float32, device="cuda")
    st = torch.zeros((1, 96, 16), dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError, match="keyDim"):
        gpu.kda_rule(z, z, v, torch.zeros((4, 1, 96), device="cuda"), torch.zeros((4, 1), device="cuda"), st, v)


@pytest.mark.parametrize("safe", [False, True])
def test_raw_gates(gpu, safe):
    """the gates computed in the solve from f, b, aLog, dtBias as kimiDeltaMixer
    does (LocalModel.hpp:2894-2905)"""
    import torch
    S, H, KD, VD = 140, 4, 128, 64
    q = O.fill_normal((S, H, KD), 51, "q")
    k = O.fill_normal((S, H, KD), 51, "k")
    v = O.fill_normal((S, H, VD), 51, "v")
    f = O.fill_normal((S, H, KD), 51, "f") * np.float32(2.0)
    b = O.fill_normal((S, H), 51, "b")
    a_log = O.fill_normal((H,), 51, "alog") * np.float32(0.5)
    dt = O.fill_normal((H, KD), 51, "dt")
    g, beta = O.kda_gates(f, b, a_log, dt, safe, -5.0)
    s0 = O.fill_normal((H, KD, VD), 51, "s0") * np.float32(0.3)
    state = dev_f32(s0)
    out = torch.zeros((S, H, VD), dtype=torch.float32, device="cuda")
    say("kda raw gates", dict(S=S, safe=safe))
    gpu.kda_rule(dev_f32(q), dev_f32(k), dev_f32(v), None, None, state, out, f=dev_f32(f), b=dev_f32(b),
                 a_log=dev_f32(a_log), dt_bias=dev_f32(dt), safe_gate=safe, lower_bound=-5.0)
    ro, rs = O.kda_rule(q, k, v, g, beta, state=s0, nthreads=0)
    assert_f32_parity(ro, host(out), f"out raw safe={safe}")
    assert_f32_parity(rs, host(state), f"state raw safe={safe}")
