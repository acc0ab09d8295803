"""Pins the oracle's restatement of the projections (apply, LocalModel.hpp:
1052-1078) and the reference's quantised weight encodings (Quant.hpp).

The decode of Q8/Q4 is bit-compared with the reference's own dequantRow
(oracle/_ref, and the golden vectors written from it); the product against
an fp64 closed form."""
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_kernels.npz")


@pytest.mark.parametrize("kind", ["q8", "q4"])
def test_dequant_matches_reference_golden(kind):
    g = np.load(GOLDEN)
    codes, scales = g[f"quant_{kind}_codes"], g[f"quant_{kind}_scales"]
    np.testing.assert_array_equal(O.dequant(codes, scales, kind), g[f"quant_{kind}_dequant"])
    # and the encoding round-trips to within half a step of each block
    src = g["quant_src"]
    step = np.repeat(np.abs(scales), 32, axis=1)
    assert np.all(np.abs(O.dequant(codes, scales, kind) - src) <= step * (0.5 if kind == "q8" else 1.0) + 1e-6)


@pytest.mark.parametrize("kind", ["q8", "q4"])
def test_dequant_matches_reference_build(kind):
    if O.ref() is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    src = O.fill_normal((9, 160), 42, "w")
    codes, scales = O.ref_quantize(src, kind)
    np.testing.assert_array_equal(O.dequant(codes, scales, kind), O.ref_dequant(codes, scales, kind))


def test_q4_nibble_layout_by_hand():
    """byte j of a block: low nibble is code j, high nibble code j + 16, both
    offset by 8; a swapped pairing (j, j+1) would fail"""
    codes = np.array([[(15 - j) << 4 | j for j in range(16)]], np.uint8)
    scales = np.array([[0.5]], np.float32)
    got = O.dequant(codes, scales, "q4")[0]
    want = np.array([(j - 8) * 0.5 for j in range(16)] + [(15 - j - 8) * 0.5 for j in range(16)], np.float32)
    np.testing.assert_array_equal(got, want)


def test_q8_sign_and_scale_index():
    codes = np.arange(-64, 64, dtype=np.int8).reshape(1, 128)
    scales = np.array([[1.0, 2.0, 3.0, 4.0]], np.float32)
    got = O.dequant(codes, scales, "q8")[0]
    want = np.arange(-64, 64, dtype=np.float32) * np.repeat(scales[0], 32)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("kind", ["f32", "bf16", "q8", "q4"])
def test_matmul_fp64_closed_form(kind):
    m, k, n = 3, 96, 7
    a = O.fill_normal((m, k), 43, "a")
    src = O.fill_normal((n, k), 43, "w")
    bias = O.fill_normal((n,), 43, "bias")
    scales = None
    if kind == "f32":
        w, dense = src, src
    elif kind == "bf16":
        w = O.pack_bf16(src).reshape(n, k)
        dense = O.unpack_bf16(w).reshape(n, k)
    else:
        w, scales = (O.ref_quantize(src, kind) if O.ref() is not None else _golden_like(src, kind))
        dense = O.dequant(w, scales, kind)
    got = O.matmul_nt(a, w, kind, scales=scales, bias=bias)
    want = a.astype(np.float64) @ dense.astype(np.float64).T + bias
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)
    # the bias is added once, after the sum
    np.testing.assert_allclose(O.matmul_nt(a, w, kind, scales=scales), got - bias, rtol=1e-6, atol=1e-5)


def _golden_like(src, kind):
    """without the reference build: codes from a fixed rule (the product is
    checked against their own decode, so any valid encoding serves)"""
    n, k = src.shape
    scales = np.full((n, k // 32), 0.25, np.float32)
    if kind == "q8":
        return np.clip(np.round(src / 0.25), -127, 127).astype(np.int8), scales
    q = np.clip(np.round(src / 0.25) + 8, 0, 15).astype(np.uint8).reshape(n, k // 32, 2, 16)
    return (q[:, :, 0, :] | (q[:, :, 1, :] << 4)).reshape(n, k // 2), scales
