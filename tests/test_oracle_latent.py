"""Pins the oracle's restatement of latentAttentionMixer's attention
(LocalModel.hpp:3118-3158). The reference's LocalModel.hpp needs <format>,
absent from this image, so it is pinned by the identity the mixer's own
comment states (:3073-3084): folding q through Wk and pushing the weighted
latents through Wv equals ordinary attention over per-head keys Wk c and
values Wv c, computed here in fp64; plus the sparse selection and one-key
special cases."""
import numpy as np

from oracle import oracle as O


def setup(seed, count=5, start=6, heads=3, dn=8, dv=6, C=32):
    r = np.random.default_rng(seed)
    q = r.standard_normal((count, heads, dn)).astype(np.float32)
    latent = r.standard_normal((start + count, C)).astype(np.float32)
    wkv = (r.standard_normal((heads * (dn + dv), C)) / np.sqrt(C)).astype(np.float32)
    return q, latent, wkv


def explicit(q, latent, wkv, start, heads, dn, dv, scale, keys_of):
    """per-head keys Wk c and values Wv c, then softmax attention, in fp64"""
    count = q.shape[0]
    C = latent.shape[1]
    W = wkv.astype(np.float64).reshape(heads, dn + dv, C)
    out = np.zeros((count, heads, dv))
    for t in range(count):
        keys = keys_of(t)
        lat = latent[keys].astype(np.float64)
        for h in range(heads):
            K = lat @ W[h, :dn].T          # [n][dn]
            V = lat @ W[h, dn:].T          # [n][dv]
            s = K @ q[t, h].astype(np.float64) * scale
            p = np.exp(s - s.max())
            out[t, h] = (p / p.sum()) @ V
    return out


def test_dense_equals_explicit_per_head_attention():
    q, latent, wkv = setup(1)
    start, heads, dn, dv = 6, 3, 8, 6
    scale = 1.0 / np.sqrt(dn + 4)
    got = O.latent_attention(q, latent, wkv, start, heads, dn, dv, scale)
    want = explicit(q, latent, wkv, start, heads, dn, dv, scale, lambda t: np.arange(start + t + 1))
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-6)
    # keys and values taken from the wrong half of each head's rows must fail
    W = wkv.reshape(heads, dn + dv, -1)
    swapped = np.concatenate([W[:, dn:dn + dn] if dv >= dn else W[:, -dn:], W[:, :dv]], axis=1)
    bad = explicit(q, latent, np.ascontiguousarray(swapped.reshape(-1, W.shape[2])), start, heads, dn, dv, scale,
                   lambda t: np.arange(start + t + 1))
    assert np.max(np.abs(got - bad)) > 1e-2


def test_selection_equals_attention_over_the_chosen_keys():
    q, latent, wkv = setup(2)
    start, heads, dn, dv = 6, 3, 8, 6
    scale = 0.3
    sel = [[0, 2, 5], None, [1, 3, 4, 7, 8], [9], None]
    got = O.latent_attention(q, latent, wkv, start, heads, dn, dv, scale, selection=sel)
    want = explicit(q, latent, wkv, start, heads, dn, dv, scale,
                    lambda t: np.array(sel[t]) if sel[t] is not None else np.arange(start + t + 1))
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-6)


def test_one_key_returns_its_value():
    q, latent, wkv = setup(3, count=1, start=0)
    heads, dn, dv = 3, 8, 6
    got = O.latent_attention(q, latent, wkv, 0, heads, dn, dv, 1.0)
    W = wkv.astype(np.float64).reshape(heads, dn + dv, -1)
    want = np.stack([W[h, dn:] @ latent[0].astype(np.float64) for h in range(heads)])
    np.testing.assert_allclose(got[0], want, rtol=1e-5, atol=1e-6)


def test_empty_selection_leaves_the_context_zero():
    """LocalModel.hpp:3145-3156 sums nothing for a token with no selected key:
    its context, and so its output, stays zero (indexTail off, before the
    first full pool)"""
    q, latent, wkv = setup(4)
    start, heads, dn, dv = 6, 3, 8, 6
    sel = [[], None, [2], [], [0, 1]]
    got = O.latent_attention(q, latent, wkv, start, heads, dn, dv, 0.3, selection=sel)
    assert np.all(got[0] == 0.0) and np.all(got[3] == 0.0)
    assert np.isfinite(got).all() and np.abs(got[1]).max() > 0.0
