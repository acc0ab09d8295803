"""Pins the oracle's restatement of the Gated DeltaNet neighbours of the
recurrence (LocalModel.hpp:2678-2708 causalConvolution, :2739-2776 the fused
qkvz de-interleave, :2833-2841 the gated norm).

The reference's LocalModel.hpp needs <format>, which this image's libstdc++
lacks, so these functions cannot be compiled into oracle/_ref; they are pinned
by fp64 closed forms, special cases and the reference's own chunk-continuity
property (llm-testing.cpp:853-890) instead.
"""
import numpy as np

from oracle import oracle as O


def _rng(seed):
    return np.random.default_rng(seed)


def _conv_fp64(x, kernel, window):
    """per-channel causal convolution written independently: the history is
    the carried window followed by the inputs, and output t weights history
    rows t .. t+K-1 (the last one the current token) by taps 0 .. K-1"""
    hist = np.concatenate([window.astype(np.float64), x.astype(np.float64)])
    K = kernel.shape[1]
    count = x.shape[0]
    acc = np.stack([(hist[t:t + K] * kernel.T.astype(np.float64)).sum(axis=0) for t in range(count)])
    return acc / (1.0 + np.exp(-acc))


def test_conv_matches_fp64_with_window_and_asymmetric_taps():
    r = _rng(1)
    count, CW, K = 37, 24, 4
    x = r.standard_normal((count, CW)).astype(np.float32)
    kernel = r.standard_normal((CW, K)).astype(np.float32)
    window = r.standard_normal((K - 1, CW)).astype(np.float32)
    out, nw = O.gdn_conv(x, kernel, window)
    ref = _conv_fp64(x, kernel, window)
    assert np.max(np.abs(out - ref)) < 2e-6 * max(1.0, np.max(np.abs(ref)))
    np.testing.assert_array_equal(nw, x[-(K - 1):])
    # a reversed tap order is a plausible mistake; it must not pass
    bad = _conv_fp64(x, kernel[:, ::-1], window)
    assert np.max(np.abs(out - bad)) > 1e-2


def test_conv_one_hot_current_tap_is_silu():
    r = _rng(2)
    count, CW, K = 9, 16, 4
    x = r.standard_normal((count, CW)).astype(np.float32) * 4
    kernel = np.zeros((CW, K), np.float32)
    kernel[:, K - 1] = 1.0
    out, _ = O.gdn_conv(x, kernel, np.full((K - 1, CW), 7.0, np.float32))
    xd = x.astype(np.float64)
    np.testing.assert_allclose(out, xd / (1.0 + np.exp(-xd)), rtol=2e-6, atol=1e-7)


def test_conv_window_continuity_token_by_token():
    """one call over the prompt equals one call per token with the window
    carried (the property llm-testing.cpp:853-890 checks of the reference)"""
    r = _rng(3)
    count, CW, K = 11, 20, 4
    x = r.standard_normal((count, CW)).astype(np.float32)
    kernel = r.standard_normal((CW, K)).astype(np.float32)
    w0 = r.standard_normal((K - 1, CW)).astype(np.float32)
    whole, wend = O.gdn_conv(x, kernel, w0)
    w = w0
    parts = []
    for t in range(count):
        o, w = O.gdn_conv(x[t:t + 1], kernel, w)
        parts.append(o)
    np.testing.assert_array_equal(np.concatenate(parts), whole)
    np.testing.assert_array_equal(w, wend)


def test_conv_short_call_shifts_window():
    r = _rng(4)
    CW, K = 8, 4
    w0 = r.standard_normal((K - 1, CW)).astype(np.float32)
    x = r.standard_normal((1, CW)).astype(np.float32)
    _, nw = O.gdn_conv(x, r.standard_normal((CW, K)).astype(np.float32), w0)
    np.testing.assert_array_equal(nw, np.concatenate([w0[1:], x]))


def _fuse(q, k, v, z, b, a):
    """the fused projection rows as the reference's comment lays them out:
    per key head its q, then its k, then its group's v, then the same group's
    z; the ba rows: the group's b, then its a"""
    count, nK, KD = q.shape
    nV = v.shape[1]
    G = nV // nK
    rows, pairs = [], []
    for kh in range(nK):
        grp = slice(kh * G, (kh + 1) * G)
        rows.append(np.concatenate([q[:, kh], k[:, kh], v[:, grp].reshape(count, -1),
                                    z[:, grp].reshape(count, -1)], axis=1))
        pairs.append(np.concatenate([b[:, grp], a[:, grp]], axis=1))
    return np.stack(rows, axis=1), np.stack(pairs, axis=1)


def test_deinterleave_round_trip():
    r = _rng(5)
    count, nK, nV, KD, VD = 3, 2, 6, 4, 5
    q = r.standard_normal((count, nK, KD)).astype(np.float32)
    k = r.standard_normal((count, nK, KD)).astype(np.float32)
    v = r.standard_normal((count, nV, VD)).astype(np.float32)
    z = r.standard_normal((count, nV, VD)).astype(np.float32)
    b = r.standard_normal((count, nV)).astype(np.float32)
    a = r.standard_normal((count, nV)).astype(np.float32)
    fused, ba = _fuse(q, k, v, z, b, a)
    qkv, z2, b2, a2 = O.gdn_deinterleave(fused, ba, nK, nV, KD, VD)
    KW = nK * KD
    np.testing.assert_array_equal(qkv[:, :KW], q.reshape(count, -1))
    np.testing.assert_array_equal(qkv[:, KW:2 * KW], k.reshape(count, -1))
    np.testing.assert_array_equal(qkv[:, 2 * KW:], v.reshape(count, -1))
    np.testing.assert_array_equal(z2, z)
    np.testing.assert_array_equal(b2, b)
    np.testing.assert_array_equal(a2, a)


def test_gated_norm_fp64_and_constant_row():
    r = _rng(6)
    count, nV, VD = 4, 3, 32
    x = r.standard_normal((count, nV, VD)).astype(np.float32)
    z = r.standard_normal((count, nV, VD)).astype(np.float32) * 3
    gamma = r.uniform(0.5, 1.5, VD).astype(np.float32)
    out = O.gdn_gated_norm(x, z, gamma, 1e-6)
    xd, zd = x.astype(np.float64), z.astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean(-1, keepdims=True) + 1e-6) * gamma * (zd / (1 + np.exp(-zd)))
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
    # a constant row normalises to sign * gamma (eps negligible)
    c = np.full((1, 1, VD), -2.5, np.float32)
    zz = np.full((1, 1, VD), 30.0, np.float32)   # SiLU(30) = 30 to fp32 precision
    out = O.gdn_gated_norm(c, zz, gamma, 1e-12)
    np.testing.assert_allclose(out[0, 0], -gamma * 30.0, rtol=1e-6)


def test_silu_special_values():
    assert O.silu(0.0) == 0.0
    assert abs(O.silu(40.0) - 40.0) < 1e-5
    assert abs(O.silu(-40.0)) < 1e-15


def test_output_gate_closed_form():
    """attentionMixer's output gate (LocalModel.hpp:2660-2665)"""
    r = _rng(7)
    count, H, D, qs = 5, 3, 8, 20
    out = r.standard_normal((count, H, D)).astype(np.float32)
    q = r.standard_normal((count, H, qs)).astype(np.float32)
    got = O.output_gate(out, q, H, D, qs)
    g = q[:, :, D:2 * D].astype(np.float64)
    np.testing.assert_allclose(got, out * (1 / (1 + np.exp(-g))), rtol=1e-6)
    # only the gate half is read: changing the query half or the tail changes nothing
    q2 = q.copy()
    q2[:, :, :D] = 123.0
    q2[:, :, 2 * D:] = -77.0
    np.testing.assert_array_equal(O.output_gate(out, q2, H, D, qs), got)
    zero = q.copy()
    zero[:, :, D:2 * D] = 0.0
    np.testing.assert_array_equal(O.output_gate(out, zero, H, D, qs), out * np.float32(0.5))


def test_gated_norm_sigmoid_gate_fp64():
    """kimiDeltaMixer's gated norm (LocalModel.hpp:2936-2945): sigmoid, not SiLU"""
    r = _rng(8)
    count, nV, VD = 3, 2, 16
    x = r.standard_normal((count, nV, VD)).astype(np.float32)
    z = r.standard_normal((count, nV, VD)).astype(np.float32) * 3
    gamma = r.uniform(0.5, 1.5, VD).astype(np.float32)
    out = O.gdn_gated_norm(x, z, gamma, 1e-6, gate="sigmoid")
    xd, zd = x.astype(np.float64), z.astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean(-1, keepdims=True) + 1e-6) * gamma / (1 + np.exp(-zd))
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
    assert np.max(np.abs(out - O.gdn_gated_norm(x, z, gamma, 1e-6))) > 1e-2


def _kda_gate_inputs(seed, S=6, H=3, KD=8):
    r = _rng(seed)
    f = (r.standard_normal((S, H, KD)) * 4).astype(np.float32)
    f[0, 0, :3] = [25.0, 21.0, 19.5]         # either side of softplus's x > 20 branch
    b = r.standard_normal((S, H)).astype(np.float32)
    a_log = r.uniform(-1.0, 1.0, H).astype(np.float32)
    dt = r.standard_normal((H, KD)).astype(np.float32)
    dt[0, :3] = 0.0
    return f, b, a_log, dt


def test_kda_gates_softplus_form_fp64():
    """kimiDeltaMixer's default gate (LocalModel.hpp:2900-2901 with
    linSafeGate false): g = -exp(aLog) softplus(f + dtBias)"""
    f, b, a_log, dt = _kda_gate_inputs(9)
    g, beta = O.kda_gates(f, b, a_log, dt, safe_gate=False)
    rate = np.exp(a_log.astype(np.float64))[None, :, None]
    x = f.astype(np.float64) + dt[None].astype(np.float64)
    sp = np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))
    np.testing.assert_allclose(g, -rate * sp, rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(beta, 1 / (1 + np.exp(-b.astype(np.float64))), rtol=1e-6)
    assert np.all(g <= 0)
    assert g[0, 0, 0] == np.float32(-np.float32(np.exp(np.float32(a_log[0]))) * np.float32(25.0))
    # a bias taken per head instead of per channel is a plausible mistake; it must not pass
    bad = -rate * np.log1p(np.exp(np.minimum(f + dt[:, :1][None], 20.0)))
    assert np.max(np.abs(g - bad)) > 1e-2


def test_kda_gates_safe_form_fp64_and_bounds():
    """the bounded gate (LocalModel.hpp:2900, linSafeGate): lowerBound
    sigmoid(exp(aLog) (f + dtBias)), always in [lowerBound, 0]"""
    f, b, a_log, dt = _kda_gate_inputs(10)
    g, _ = O.kda_gates(f, b, a_log, dt, safe_gate=True, lower_bound=-5.0)
    rate = np.exp(a_log.astype(np.float64))[None, :, None]
    x = f.astype(np.float64) + dt[None].astype(np.float64)
    np.testing.assert_allclose(g, -5.0 / (1 + np.exp(-rate * x)), rtol=2e-6, atol=1e-7)
    assert np.all(g >= -5.0) and np.all(g <= 0.0)
    # the rate applied outside the sigmoid is a plausible mistake; it must not pass
    bad = -5.0 * rate / (1 + np.exp(-x))
    assert np.max(np.abs(g - bad)) > 1e-2
