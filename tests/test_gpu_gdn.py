"""GPU parity of the Gated DeltaNet neighbours of the recurrence against the
oracle's restatement: the fused qkvz de-interleave + causalConvolution + SiLU
(LocalModel.hpp:2678-2708, 2739-2776) and the gated norm (:2833-2841).

fp32 outputs meet the fp32 bound (1e-5). bf16 outputs are the oracle's fp32
values rounded to bf16: they must agree to one bf16 unit in the last place
(the fp32 values may differ by an ulp next to a rounding boundary)."""
import numpy as np
import pytest

from common import assert_f32_parity
from gpu_util import dev_bf16, dev_f32, host, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def bf16_ulps(ref32, got_bf16_as_f32):
    """distance in bf16 ulps between bf16(ref) and the GPU's bf16 values"""
    r = O.pack_bf16(np.asarray(ref32, np.float32)).astype(np.int32)
    g = O.pack_bf16(np.asarray(got_bf16_as_f32, np.float32)).astype(np.int32)   # exact: already bf16
    # sign-magnitude to ordered integers
    r = np.where(r & 0x8000, -(r & 0x7FFF), r)
    g = np.where(g & 0x8000, -(g & 0x7FFF), g)
    return np.abs(r - g)


def fuse(q, k, v, z, b, a):
    """fused projection rows per key head: q, k, the group's v, its z; ba: the
    group's b then its a (the layout LocalModel.hpp:2739-2776 de-interleaves)"""
    count, nK, KD = q.shape
    nV = v.shape[1]
    G = nV // nK
    rows, pairs = [], []
    for kh in range(nK):
        grp = slice(kh * G, (kh + 1) * G)
        rows.append(np.concatenate([q[:, kh], k[:, kh], v[:, grp].reshape(count, -1),
                                    z[:, grp].reshape(count, -1)], axis=1))
        pairs.append(np.concatenate([b[:, grp], a[:, grp]], axis=1))
    return np.ascontiguousarray(np.stack(rows, axis=1)), np.ascontiguousarray(np.stack(pairs, axis=1))


def torch_empty(shape, bf16):
    import torch
    return torch.empty(shape, dtype=torch.bfloat16 if bf16 else torch.float32, device="cuda")


def run_plain(gpu, count, nK, nV, KD, VD, K, seed, out_bf16=False, in_bf16=False, window0=True):
    CW = 2 * nK * KD + nV * VD
    x = O.fill_normal((count, CW), seed, "qkv")
    if in_bf16:
        xb = O.pack_bf16(x)
        x = O.unpack_bf16(xb).reshape(count, CW)
        dx = dev_bf16(xb)
    else:
        dx = dev_f32(x)
    kernel = O.fill_normal((CW, K), seed, "conv") * np.float32(0.5)
    w0 = (O.fill_normal((K - 1, CW), seed, "window") if window0 else np.zeros((K - 1, CW), np.float32))
    dw = dev_f32(w0)
    q, k, v = (torch_empty((count, nK, KD), out_bf16), torch_empty((count, nK, KD), out_bf16),
               torch_empty((count, nV, VD), out_bf16))
    say("gdn conv plain", dict(count=count, CW=CW, K=K, in_bf16=in_bf16, out_bf16=out_bf16))
    gpu.gdn_conv(dx, dev_f32(kernel), dw, q, k, v, nK, nV, KD, VD)
    ref, wref = O.gdn_conv(x, kernel, w0)
    KW = nK * KD
    got = np.concatenate([host(q).reshape(count, -1), host(k).reshape(count, -1), host(v).reshape(count, -1)],
                         axis=1)
    return ref, got, wref, host(dw)


@pytest.mark.parametrize("count", [1, 2, 33, 200])
def test_conv_plain_fp32(gpu, count):
    ref, got, wref, wgot = run_plain(gpu, count, 2, 4, 16, 8, 4, 10 + count)
    assert_f32_parity(ref, got, f"conv count={count}")
    np.testing.assert_array_equal(wgot, wref)


@pytest.mark.parametrize("K", [1, 2, 8])
def test_conv_kernel_sizes(gpu, K):
    ref, got, wref, wgot = run_plain(gpu, 45, 1, 2, 8, 16, K, 40 + K)
    assert_f32_parity(ref, got, f"conv K={K}")
    if K > 1:
        np.testing.assert_array_equal(wgot, wref)


def test_conv_bf16_in_out(gpu):
    ref, got, wref, wgot = run_plain(gpu, 70, 2, 4, 32, 16, 4, 55, out_bf16=True, in_bf16=True)
    assert bf16_ulps(ref, got).max() <= 1
    np.testing.assert_array_equal(wgot, wref)   # bf16 inputs are exact in the fp32 window


def test_conv_window_continuity(gpu):
    """one call equals one call per token with the window carried on the
    device (llm-testing.cpp:853-890 checks the same of the reference)"""
    import torch
    count, nK, nV, KD, VD, K = 9, 1, 2, 8, 8, 4
    CW = 2 * nK * KD + nV * VD
    x = O.fill_normal((count, CW), 7, "qkv")
    kernel = dev_f32(O.fill_normal((CW, K), 7, "conv"))
    w0 = O.fill_normal((K - 1, CW), 7, "window")
    outs = []
    for split in (False, True):
        dw = dev_f32(w0)
        q, k, v = (torch_empty((count, nK, KD), False), torch_empty((count, nK, KD), False),
                   torch_empty((count, nV, VD), False))
        say("gdn conv continuity", dict(split=split))
        if not split:
            gpu.gdn_conv(dev_f32(x), kernel, dw, q, k, v, nK, nV, KD, VD)
        else:
            for t in range(count):
                gpu.gdn_conv(dev_f32(x[t:t + 1]), kernel, dw, q[t:t + 1], k[t:t + 1], v[t:t + 1], nK, nV, KD, VD)
        outs.append((host(q), host(k), host(v), host(dw)))
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)
    torch.cuda.synchronize()


@pytest.mark.parametrize("bf16", [False, True])
def test_conv_fused_layout(gpu, bf16):
    import torch
    count, nK, nV, KD, VD, K = 50, 2, 6, 16, 8, 4
    q = O.fill_normal((count, nK, KD), 3, "q")
    k = O.fill_normal((count, nK, KD), 3, "k")
    v = O.fill_normal((count, nV, VD), 3, "v")
    z = O.fill_normal((count, nV, VD), 3, "z")
    b = O.fill_normal((count, nV), 3, "b")
    a = O.fill_normal((count, nV), 3, "a")
    fused, ba = fuse(q, k, v, z, b, a)
    if bf16:
        fused = O.unpack_bf16(O.pack_bf16(fused)).reshape(fused.shape)
        ba = O.unpack_bf16(O.pack_bf16(ba)).reshape(ba.shape)
        dfused, dba = dev_bf16(O.pack_bf16(fused)), dev_bf16(O.pack_bf16(ba))
    else:
        dfused, dba = dev_f32(fused), dev_f32(ba)
    CW = 2 * nK * KD + nV * VD
    kernel = O.fill_normal((CW, K), 3, "conv") * np.float32(0.5)
    w0 = O.fill_normal((K - 1, CW), 3, "window")
    dw = dev_f32(w0)
    oq, ok, ov = torch_empty((count, nK, KD), bf16), torch_empty((count, nK, KD), bf16), torch_empty((count, nV, VD), bf16)
    oz = torch_empty((count, nV, VD), bf16)
    oa = torch.empty((count, nV), dtype=torch.float32, device="cuda")
    ob = torch.empty((count, nV), dtype=torch.float32, device="cuda")
    say("gdn conv fused", dict(bf16=bf16))
    gpu.gdn_conv(dfused, dev_f32(kernel), dw, oq, ok, ov, nK, nV, KD, VD, ba=dba, z=oz, a=oa, b=ob)
    qkv, zr, br, ar = O.gdn_deinterleave(fused, ba, nK, nV, KD, VD)
    ref, wref = O.gdn_conv(qkv, kernel, w0)
    got = np.concatenate([host(oq).reshape(count, -1), host(ok).reshape(count, -1), host(ov).reshape(count, -1)],
                         axis=1)
    if bf16:
        assert bf16_ulps(ref, got).max() <= 1
    else:
        assert_f32_parity(ref, got, "fused conv")
    np.testing.assert_array_equal(host(oz), zr)
    np.testing.assert_array_equal(host(oa), ar)
    np.testing.assert_array_equal(host(ob), br)
    np.testing.assert_array_equal(host(dw), wref)


@pytest.mark.parametrize("z_bf16,out_bf16,VD", [(False, False, 128), (True, True, 128), (True, False, 128),
                                               (False, False, 48), (True, True, 256), (False, True, 264)])
def test_gated_norm(gpu, z_bf16, out_bf16, VD):
    count, nV = 37, 3
    x = O.fill_normal((count, nV, VD), 21, "x")
    z = O.fill_normal((count, nV, VD), 21, "z") * np.float32(2)
    if z_bf16:
        zb = O.pack_bf16(z)
        z = O.unpack_bf16(zb).reshape(z.shape)
        dz = dev_bf16(zb)
    else:
        dz = dev_f32(z)
    gamma = O.fill_uniform((VD,), 21, "gamma", 0.5, 1.5)
    out = torch_empty((count, nV, VD), out_bf16)
    say("gdn gated norm", dict(z_bf16=z_bf16, out_bf16=out_bf16))
    gpu.gdn_gated_norm(dev_f32(x), dz, dev_f32(gamma), out, eps=1e-6)
    ref = O.gdn_gated_norm(x, z, gamma, 1e-6)
    if out_bf16:
        assert bf16_ulps(ref, host(out)).max() <= 1
    else:
        assert_f32_parity(ref, host(out), "gated norm")


@pytest.mark.parametrize("z_bf16,out_bf16", [(False, False), (True, True)])
def test_gated_norm_sigmoid_gate(gpu, z_bf16, out_bf16):
    """kimiDeltaMixer's form of the gated norm: times sigmoid(z) (LocalModel.hpp:2936-2945)"""
    count, nV, VD = 29, 4, 128
    x = O.fill_normal((count, nV, VD), 23, "x")
    z = O.fill_normal((count, nV, VD), 23, "z") * np.float32(2)
    if z_bf16:
        zb = O.pack_bf16(z)
        z = O.unpack_bf16(zb).reshape(z.shape)
        dz = dev_bf16(zb)
    else:
        dz = dev_f32(z)
    gamma = O.fill_uniform((VD,), 23, "gamma", 0.5, 1.5)
    out = torch_empty((count, nV, VD), out_bf16)
    say("gated norm sigmoid", dict(z_bf16=z_bf16, out_bf16=out_bf16))
    gpu.gdn_gated_norm(dev_f32(x), dz, dev_f32(gamma), out, eps=1e-6, gate="sigmoid")
    ref = O.gdn_gated_norm(x, z, gamma, 1e-6, gate="sigmoid")
    if out_bf16:
        assert bf16_ulps(ref, host(out)).max() <= 1
    else:
        assert_f32_parity(ref, host(out), "gated norm sigmoid")


def test_rejects_bad_shapes(gpu):
    import aigpu
    x = dev_f32(np.zeros((4, 2 * 6 + 6), np.float32))
    q = torch_empty((4, 1, 6), False)
    with pytest.raises(aigpu.AiGpuError, match="multiples of 8"):
        gpu.gdn_conv(x, dev_f32(np.zeros((18, 4), np.float32)), dev_f32(np.zeros((3, 18), np.float32)),
                     q, q, torch_empty((4, 1, 6), False), 1, 1, 6, 6)
