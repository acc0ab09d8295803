"""Pins the oracle's restatement of the sparse-attention indexer (selectKeys,
LocalModel.hpp:2971-3068: or_index_update, or_select_keys) where the
reference holds no tests or vectors of its own, by what the mathematics fixes:
layerNormRow's moments, the pooling softmax's special cases, the score's
closed form for one head, its linearity in the head weights, and the choice
against a brute-force sort of the same scores."""
import numpy as np
import pytest

from oracle import oracle as O


def rng(seed):
    return np.random.default_rng(seed)


def update(k, ape, gates, P, start=0, keys=None, pools=None, w=None, b=None):
    count, Di = k.shape
    cap = start + count + P
    keys = np.zeros((cap, Di), np.float32) if keys is None else keys
    pools = np.zeros((cap // P + 1, Di), np.float32) if pools is None else pools
    O.index_update(k, np.ones(Di, np.float32) if w is None else w, b, ape, keys, gates, pools, start, P)
    return keys, pools


def test_layer_norm_moments_and_affine():
    r = rng(1)
    Di, P = 64, 4
    k = (r.standard_normal((10, Di)) * 3 + 2).astype(np.float32)
    gates = np.zeros((20, Di), np.float32)
    keys, _ = update(k, np.zeros((P, Di), np.float32), gates, P)
    assert np.abs(keys[:10].mean(1)).max() < 1e-6
    assert np.abs(keys[:10].var(1) - 1).max() < 1e-4      # var / (var + 1e-6)
    w = r.uniform(0.5, 1.5, Di).astype(np.float32)
    b = r.standard_normal(Di).astype(np.float32)
    keys2, _ = update(k, np.zeros((P, Di), np.float32), gates, P, w=w, b=b)
    np.testing.assert_allclose(keys2[:10], keys[:10] * w + b, rtol=1e-6, atol=1e-6)


def test_pool_of_equal_weights_is_the_mean():
    r = rng(2)
    Di, P = 32, 4
    k = r.standard_normal((12, Di)).astype(np.float32)
    gates = np.full((16, Di), 0.7, np.float32)
    keys, pools = update(k, np.zeros((P, Di), np.float32), gates, P)
    want = keys[:12].reshape(3, P, Di).mean(1)
    np.testing.assert_allclose(pools[:3], want, rtol=1e-6, atol=1e-6)


def test_pool_follows_a_dominant_member_and_ape_shifts_it():
    r = rng(3)
    Di, P = 32, 4
    k = r.standard_normal((8, Di)).astype(np.float32)
    gates = np.zeros((12, Di), np.float32)
    gates[2] = 60.0                                  # member 2 of pool 0
    ape = np.zeros((P, Di), np.float32)
    ape[1] = 80.0                                    # member 1 of every pool
    keys, pools = update(k, ape, gates, P)
    np.testing.assert_allclose(pools[0], keys[1], rtol=1e-5, atol=1e-6)   # ape 80 beats the gate 60
    np.testing.assert_allclose(pools[1], keys[5], rtol=1e-5, atol=1e-6)


def test_pool_of_one_is_the_key_and_two_calls_equal_one():
    r = rng(4)
    Di = 16
    k = r.standard_normal((9, Di)).astype(np.float32)
    gates = r.standard_normal((12, Di)).astype(np.float32)
    keys, pools = update(k, np.zeros((1, Di), np.float32), gates, 1)
    np.testing.assert_array_equal(pools[:9], keys[:9])
    P = 3
    ape = r.standard_normal((P, Di)).astype(np.float32)
    keys_a, pools_a = update(k, ape, gates, P)
    keys_b, pools_b = np.zeros_like(keys_a), np.zeros_like(pools_a)   # sized for all 9 tokens
    update(k[:4], ape, gates, P, keys=keys_b, pools=pools_b)
    update(k[4:], ape, gates, P, start=4, keys=keys_b, pools=pools_b)
    np.testing.assert_array_equal(keys_a, keys_b)
    np.testing.assert_array_equal(pools_a, pools_b)


def test_single_head_score_is_relu_of_the_scaled_dot():
    r = rng(5)
    Di, P, count = 64, 2, 9
    pools = r.standard_normal((count // P + 1, Di)).astype(np.float32)
    q = r.standard_normal((count, Di)).astype(np.float32)
    w = np.ones((count, 1), np.float32)
    _, sc = O.select_keys(q, w, pools, 0, 1, Di, P, 2, tail=False)
    for t in range(count):
        for p in range((t + 1) // P):
            want = max(0.0, float(q[t].astype(np.float64) @ pools[p].astype(np.float64))) / np.sqrt(Di)
            assert abs(sc[t, p] - want) <= 1e-5 * max(1.0, abs(want))


def test_scores_are_linear_in_the_head_weights():
    r = rng(6)
    Di, P, H, count = 32, 4, 3, 24
    pools = r.standard_normal((count // P + 1, Di)).astype(np.float32)
    q = r.standard_normal((count, H * Di)).astype(np.float32)
    wa = r.standard_normal((count, H)).astype(np.float32)
    wb = r.standard_normal((count, H)).astype(np.float32)
    _, sa = O.select_keys(q, wa, pools, 0, H, Di, P, 4, tail=False)
    _, sb = O.select_keys(q, wb, pools, 0, H, Di, P, 4, tail=False)
    _, sab = O.select_keys(q, wa + wb, pools, 0, H, Di, P, 4, tail=False)
    np.testing.assert_allclose(sab, sa + sb, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("tail", [True, False])
def test_choice_is_the_brute_force_top_k(tail):
    r = rng(7)
    Di, P, H, top_k, start, count = 32, 4, 2, 12, 30, 50
    pools = r.standard_normal(((start + count) // P + 1, Di)).astype(np.float32)
    q = r.standard_normal((count, H * Di)).astype(np.float32)
    w = r.standard_normal((count, H)).astype(np.float32)
    sel, sc = O.select_keys(q, w, pools, start, H, Di, P, top_k, tail=tail)
    budget = top_k // P
    for t in range(count):
        pos = start + t
        complete = (pos + 1) // P
        if complete <= budget and tail:
            assert sel[t] is None
            continue
        keep = min(budget, complete)
        order = np.lexsort((np.arange(complete), -sc[t, :complete]))[:keep]
        want = [p * P + j for p in sorted(order) for j in range(P)]
        if tail:
            want += list(range(complete * P, pos + 1))
        assert list(sel[t]) == want, f"token {t}"
        assert all(a < b for a, b in zip(sel[t], sel[t][1:])) and (len(sel[t]) == 0 or sel[t][-1] <= pos)


def test_equal_scores_take_the_lower_pools():
    Di, P = 16, 2
    pools = np.ones((20, Di), np.float32)
    q = -np.ones((10, Di), np.float32)   # every logit negative: every score 0
    w = np.ones((10, 1), np.float32)
    sel, sc = O.select_keys(q, w, pools, 20, 1, Di, P, 4, tail=True)
    assert not sc.any()
    for t in range(10):
        pos = 20 + t
        assert list(sel[t]) == [0, 1, 2, 3] + list(range((pos + 1) // P * P, pos + 1))
