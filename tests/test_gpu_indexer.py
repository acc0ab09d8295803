"""GPU parity of the sparse-attention indexer (aigpu_select_keys) against the
oracle's restatement of selectKeys (LocalModel.hpp:2971-3068: or_index_update,
or_select_keys) over the oracle's matmul_nt for its four projections.

Bars: the new index keys and pooled keys within 1e-5 of max(1, |x|), the
gates within 1e-4 (a projection's 1e-5 of sum |a w|); the scores of every
sparse token within 1e-4 of the magnitude they pass through,
A = sum_h |w_h| headScale (|q_h| . |pool|) dimScale, plus 1e-6 (their q and w
come from projections held to 1e-5 of sum |a w|); the selection key for
key, except for pools whose oracle score is within that bound of the keep-th
best one, which a different summation order may swap. Equal scores take the
lower pools on both sides."""
import numpy as np
import pytest

from gpu_util import dev_f32, host, say
from oracle import oracle as O
from test_gpu_matmul import to_device
from test_gpu_mixer import weight

pytestmark = pytest.mark.gpu


def run(gpu, count, start, kind="f32", hidden=128, q_rank=64, heads=4, dim=64, pool=4, top_k=16, tail=True,
        seed=5, zero_q=False, bias=True):
    import torch
    cap = start + count + pool
    r = np.random.default_rng(seed)
    shapes = {"k": (dim, hidden), "gate": (dim, hidden), "q": (heads * dim, q_rank), "w": (heads, hidden)}
    dev, ref = {}, {}
    for i, (name, (n, k)) in enumerate(shapes.items()):
        stored, scales, _ = weight(n, k, kind, seed + 7 * i, "ix" + name)
        if zero_q and name == "q":
            stored = np.zeros_like(stored)
        dev[name] = {"w": to_device(stored), "kind": kind, "out": n, "in": k,
                     "scales": None if scales is None else dev_f32(scales)}
        ref[name] = (stored, scales)

    def proj(a, name):
        stored, scales = ref[name]
        return O.matmul_nt(a, stored, kind, scales)

    k_norm = r.uniform(0.5, 1.5, dim).astype(np.float32)
    k_bias = (r.standard_normal(dim) * 0.1).astype(np.float32) if bias else None
    ape = r.standard_normal((pool, dim)).astype(np.float32)
    # history [0, start) through the oracle
    keys = np.zeros((cap, dim), np.float32)
    gates = np.zeros((cap, dim), np.float32)
    pools = np.zeros((cap // pool + 1, dim), np.float32)
    if start:
        hh = O.fill_normal((start, hidden), seed, "hist")
        gates[:start] = proj(hh, "gate")
        O.index_update(proj(hh, "k"), k_norm, k_bias, ape, keys, gates, pools, 0, pool)
    h = O.fill_normal((count, hidden), seed, "h")
    qr = O.fill_normal((count, q_rank), seed, "qr")
    d_keys, d_gates, d_pools = dev_f32(keys), dev_f32(gates), dev_f32(pools)
    want_keys, want_gates, want_pools = keys.copy(), gates.copy(), pools.copy()
    want_gates[start:start + count] = proj(h, "gate")
    O.index_update(proj(h, "k"), k_norm, k_bias, ape, want_keys, want_gates, want_pools, start, pool)
    q_o, w_o = proj(qr, "q"), proj(h, "w")
    sel, sc = O.select_keys(q_o, w_o, want_pools, start, heads, dim, pool, top_k, tail)

    stride = top_k // pool * pool + pool
    i32 = dict(dtype=torch.int32, device="cuda")
    ss, sn, sk = torch.zeros(count, **i32), torch.zeros(count, **i32), torch.zeros(count * stride, **i32)
    max_pools = (start + count) // pool
    scores = torch.zeros((count, max(1, max_pools)), dtype=torch.float32, device="cuda")
    say("select keys", dict(count=count, start=start, kind=kind, heads=heads, dim=dim, pool=pool, top_k=top_k,
                            tail=tail, zero_q=zero_q))
    gpu.select_keys(dev_f32(h), dev_f32(qr), dev, dev_f32(k_norm), None if k_bias is None else dev_f32(k_bias),
                    dev_f32(ape), d_keys, d_gates, d_pools, ss, sn, sk, start, heads, dim, top_k, pool, tail=tail,
                    scores=scores)
    gk, gg, gp = host(d_keys), host(d_gates), host(d_pools)
    np.testing.assert_allclose(gg, want_gates, rtol=0, atol=1e-4)
    np.testing.assert_allclose(gk, want_keys, rtol=0, atol=1e-5 * max(1.0, np.abs(want_keys).max()))
    np.testing.assert_allclose(gp, want_pools, rtol=0, atol=1e-5 * max(1.0, np.abs(want_pools).max()))
    st = host(ss).view(np.uint32)
    ct = host(sn).view(np.uint32)
    ks = host(sk).view(np.uint32)
    gsc = host(scores)
    budget = top_k // pool
    for t in range(count):
        pos = start + t
        complete = (pos + 1) // pool
        assert st[t] == t * stride
        if sel[t] is None:
            assert ct[t] == 0xFFFFFFFF, f"token {t} should see every key"
            continue
        got = ks[st[t]:st[t] + ct[t]]
        s = sc[t, :complete]
        mag = (np.abs(w_o[t])[:, None] / np.sqrt(heads) *
               (np.abs(q_o[t].reshape(heads, dim)) @ np.abs(want_pools[:complete]).T) / np.sqrt(dim)).sum(0)
        tol = 1e-4 * mag + 1e-6
        assert (np.abs(gsc[t, :complete] - s) <= tol).all(), f"token {t} scores"
        if list(got) == list(sel[t]):
            continue
        keep = min(budget, complete)
        boundary = np.sort(s)[::-1][keep - 1]
        diff = set(int(x) // pool for x in set(got.tolist()) ^ set(sel[t].tolist()))
        assert all(abs(s[p] - boundary) <= 2 * tol.max() for p in diff), f"token {t}: {sorted(diff)}"
        assert len(got) == len(sel[t]) and list(got) == sorted(got)


@pytest.mark.parametrize("kind", ["f32", "bf16", "q8"])
def test_prefill_from_empty(gpu, kind):
    run(gpu, 120, 0, kind)


@pytest.mark.parametrize("tail", [True, False])
def test_continuation_mid_pool(gpu, tail):
    run(gpu, 45, 37, tail=tail)


def test_decode_step_against_a_long_history(gpu):
    run(gpu, 1, 700, top_k=64, heads=8, dim=128, q_rank=96)


def test_pool_of_one_and_many_heads(gpu):
    run(gpu, 60, 20, pool=1, top_k=8, heads=16, dim=32)


def test_equal_scores_take_the_lower_pools(gpu):
    run(gpu, 30, 40, zero_q=True)


def test_rejects_bad_shapes(gpu):
    import torch
    z = torch.zeros((4, 64), dtype=torch.float32, device="cuda")
    w = {n: {"w": torch.zeros(64 * 64 * 4, dtype=torch.uint8, device="cuda"), "kind": "f32", "out": 64}
         for n in ("k", "gate", "q", "w")}
    i = torch.zeros(64, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="weight shapes"):
        gpu.select_keys(z, z, w, z[0], None, z, z, z, z, i, i, i, 0, 2, 32, 8, 4)


def test_more_than_8192_pools_per_token(gpu):
    """past 256 x 32 pools a token's scores are streamed rather than held in registers"""
    run(gpu, 3, 8300, pool=1, top_k=64, heads=2, dim=32)
