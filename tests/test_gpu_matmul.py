"""GPU parity of the projections (gemv_kernel for up to 15 rows of a,
gemm_kernel on MFMA from 16, split_a_kernel and gemm_dma_kernel for bf16
weights with enough 256 x 256 tiles, behind aigpu_matmul_nt* and
aigpu_matmul_device)
against the oracle's restatement of apply
(LocalModel.hpp:1052-1078) over the reference's weight encodings.

Bar: fp32 outputs within 1e-5 of each dot product's absolute size,
|got - want| <= 1e-5 * sum_k |a_k w_k| + 1e-6: the fp32 bar scaled to the
magnitude the sum passes through (the reference's CPU and GPU paths also sum
in different orders)."""
import numpy as np
import pytest

from gpu_util import dev_f32, host, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def weights(n, k, kind, seed):
    src = O.fill_normal((n, k), seed, "w")
    if kind == "f32":
        return src, None, src
    if kind == "bf16":
        bits = O.pack_bf16(src).reshape(n, k)
        return bits, None, O.unpack_bf16(bits).reshape(n, k)
    codes, scales = quantise(src, kind)
    return codes, scales, O.dequant(codes, scales, kind)


def quantise(src, kind):
    """codes with per-block scales, as the reference's layout holds them"""
    n, k = src.shape
    blocks = src.reshape(n, k // 32, 32)
    amax = np.abs(blocks).max(axis=2)
    if kind == "q8":
        scales = (amax / 127.0).astype(np.float32)
        codes = np.clip(np.round(blocks / scales[..., None]), -127, 127).astype(np.int8).reshape(n, k)
        return codes, scales
    scales = (amax / 8.0).astype(np.float32)
    q = np.clip(np.round(blocks / scales[..., None]) + 8, 0, 15).astype(np.uint8)
    return (q[:, :, :16] | (q[:, :, 16:] << 4)).reshape(n, k // 2), scales


def to_device(w):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(w).view(np.uint8).copy())
    return t.cuda()


def bound(a, dense):
    return 1e-5 * (np.abs(a).astype(np.float64) @ np.abs(dense).astype(np.float64).T) + 1e-6


@pytest.mark.parametrize("kind", ["f32", "bf16", "q8", "q4"])
@pytest.mark.parametrize("m", [1, 3, 8, 13, 16, 200])
def test_device_form(gpu, kind, m):
    import torch
    k, n = 1024, 1000
    a = O.fill_normal((m, k), 7 + m, "a")
    w, scales, dense = weights(n, k, kind, 8 + m)
    bias = O.fill_normal((n,), 9, "bias")
    out = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    say("matmul", dict(kind=kind, m=m, k=k, n=n))
    gpu.matmul(dev_f32(a), to_device(w), out, kind, scales=None if scales is None else dev_f32(scales),
               bias=dev_f32(bias))
    want = O.matmul_nt(a, w, kind, scales=scales, bias=bias)
    err = np.abs(host(out) - want)
    assert np.all(err <= bound(a, dense)), f"{kind} m={m}: max err {err.max()}"


@pytest.mark.parametrize("kind", ["bf16", "q8", "q4"])
def test_split_k_for_few_tiles_and_long_k(gpu, kind):
    """3 x 1 tiles against k = 7168: K is split into slices whose partial
    tiles are added in order, then the bias and the residual"""
    import torch
    m, k, n = 300, 7168, 128
    a = O.fill_normal((m, k), 31, "a")
    w, scales, dense = weights(n, k, kind, 32)
    bias = O.fill_normal((n,), 33, "bias")
    base = O.fill_normal((m, n), 34, "residual")
    out = dev_f32(base)
    say("matmul split-k", dict(kind=kind, m=m, k=k, n=n))
    gpu.matmul(dev_f32(a), to_device(w), out, kind, scales=None if scales is None else dev_f32(scales),
               bias=dev_f32(bias), accumulate=True)
    want = O.matmul_nt(a, w, kind, scales=scales, bias=bias) + base
    err = np.abs(host(out) - want)
    assert np.all(err <= bound(a, dense) + 1e-6 * np.abs(base)), f"{kind}: max err {err.max()}"


@pytest.mark.parametrize("kind", ["f32", "bf16", "q8", "q4"])
def test_host_form_and_upload(gpu, kind):
    """the reference's own entry points: host a and c, the weight from aigpu_upload"""
    m, k, n = 2, 512, 333
    a = O.fill_normal((m, k), 21, "a")
    w, scales, dense = weights(n, k, kind, 22)
    wptr = gpu.upload(w)
    sptr = gpu.upload(scales) if scales is not None else None
    try:
        say("matmul host", dict(kind=kind))
        got = gpu.matmul_host(a, wptr, kind, n, sptr)
    finally:
        gpu.release(wptr, np.ascontiguousarray(w).nbytes)
        if sptr:
            gpu.release(sptr, scales.nbytes)
    want = O.matmul_nt(a, w, kind, scales=scales)
    assert np.all(np.abs(got - want) <= bound(a, dense))


def test_accumulate_and_row_stride(gpu):
    """a residual add into a strided output: out[:, :n] += a . w^T"""
    import torch
    m, k, n = 4, 256, 96
    a = O.fill_normal((m, k), 31, "a")
    w, _, dense = weights(n, k, "bf16", 32)
    base = O.fill_normal((m, 128), 33, "base")
    out = dev_f32(base)
    say("matmul accumulate", {})
    gpu.matmul(dev_f32(a), to_device(w), out[:, :n], "bf16", accumulate=True)
    got = host(out)
    want = base.copy()
    want[:, :n] += O.matmul_nt(a, w, "bf16")
    assert np.all(np.abs(got[:, :n] - want[:, :n]) <= bound(a, dense) + 1e-6)
    np.testing.assert_array_equal(got[:, n:], base[:, n:])


@pytest.mark.parametrize("kind,k", [("bf16", 100), ("f32", 98)])
def test_unaligned_rows_take_the_scalar_path(gpu, kind, k):
    import torch
    m, n = 2, 50
    a = O.fill_normal((m, k), 41, "a")
    w, _, dense = weights(n, k, kind, 42)
    out = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    say("matmul scalar", dict(kind=kind, k=k))
    gpu.matmul(dev_f32(a), to_device(w), out, kind)
    assert np.all(np.abs(host(out) - O.matmul_nt(a, w, kind)) <= bound(a, dense))


def test_rejects_quantised_k_not_multiple_of_32(gpu):
    import torch
    a = dev_f32(np.zeros((1, 48), np.float32))
    w = torch.zeros((4, 48), dtype=torch.int8, device="cuda")
    s = dev_f32(np.ones((4, 1), np.float32))
    out = torch.zeros((1, 4), dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError, match="multiple of 32"):
        gpu.matmul(a, w, out, "q8", scales=s)


@pytest.mark.parametrize("kind,k", [("f32", 100), ("bf16", 104), ("q8", 96), ("q4", 160)])
def test_gemm_ragged_tiles(gpu, kind, k):
    """the MFMA GEMM with m, n and k that do not fill its 128 x 128 x 32 tiles"""
    import torch
    m, n = 131, 257
    a = O.fill_normal((m, k), 51, "a")
    w, scales, dense = weights(n, k, kind, 52)
    bias = O.fill_normal((n,), 53, "bias")
    out = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    say("gemm ragged", dict(kind=kind, m=m, k=k, n=n))
    gpu.matmul(dev_f32(a), to_device(w), out, kind, scales=None if scales is None else dev_f32(scales),
               bias=dev_f32(bias))
    want = O.matmul_nt(a, w, kind, scales=scales, bias=bias)
    err = np.abs(host(out) - want)
    assert np.all(err <= bound(a, dense)), f"{kind}: max err {err.max()}"


@pytest.mark.parametrize("k,accumulate", [(32, False), (96, True), (128, False)])
def test_gemm_wide_tiles(gpu, k, accumulate):
    """bf16 weights with enough 256 x 256 tiles for split_a_kernel and
    gemm_dma_kernel (17 x 16 of them here, the last row and column of tiles
    ragged; one, three and four K steps through its three-stage ring), bias,
    and a residual add into a strided output"""
    import torch
    m, n, ld = 4100, 4000, 4008
    a = O.fill_normal((m, k), 61, "a")
    w, _, dense = weights(n, k, "bf16", 62)
    bias = O.fill_normal((n,), 63, "bias")
    base = O.fill_normal((m, ld), 64, "base") if accumulate else np.zeros((m, ld), np.float32)
    out = dev_f32(base)
    say("gemm wide", dict(m=m, k=k, n=n, accumulate=accumulate))
    gpu.matmul(dev_f32(a), to_device(w), out[:, :n], "bf16", bias=dev_f32(bias), accumulate=accumulate)
    got = host(out)
    want = base[:, :n] + O.matmul_nt(a, w, "bf16", bias=bias)
    err = np.abs(got[:, :n] - want)
    assert np.all(err <= bound(a, dense) + 1e-6), f"max err {err.max()}"
    np.testing.assert_array_equal(got[:, n:], base[:, n:])


def test_one_row_against_a_wide_weight_takes_the_gemv(gpu):
    """a decode step's product against a wide weight (an LM head: one row of a,
    65536 weight rows, 256 tiles of 256 x 256) runs on gemv_kernel: the DMA
    GEMM's 256-row tiles would waste 255 of every 256 rows"""
    import torch
    m, k, n = 1, 256, 65536
    a = O.fill_normal((m, k), 65, "a")
    w, _, dense = weights(n, k, "bf16", 66)
    out = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    say("gemv wide", dict(m=m, k=k, n=n))
    gpu.profile_reset()
    gpu.profile(True)
    gpu.matmul(dev_f32(a), to_device(w), out, "bf16")
    torch.cuda.synchronize()
    gpu.profile(False)
    assert gpu.profile_read("gemv_kernel")[1] == 1
    assert gpu.profile_read("gemm_dma_kernel")[1] == 0
    err = np.abs(host(out) - O.matmul_nt(a, w, "bf16"))
    assert np.all(err <= bound(a, dense)), f"max err {err.max()}"
