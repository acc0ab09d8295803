"""GPU parity of multi-head latent attention (latent.hip behind
aigpu_latent_attention) against the oracle's restatement of
latentAttentionMixer's attention (LocalModel.hpp:3118-3158).

Bar: fp32 outputs within 1e-5 of max(1, max |out|) (the fold, the scores and
the context are summed in the device's own order)."""
import numpy as np
import pytest

from gpu_util import dev_bf16, dev_f32, dev_u32, host, say
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def run(gpu, count, start, heads, dn, dv, C, seed, bf16_w=False, selection=None):
    import torch
    r = np.random.default_rng(seed)
    q = r.standard_normal((count, heads, dn)).astype(np.float32)
    latent = r.standard_normal((start + count, C)).astype(np.float32)
    wkv = (r.standard_normal((heads * (dn + dv), C)) / np.sqrt(C)).astype(np.float32)
    if bf16_w:
        bits = O.pack_bf16(wkv).reshape(wkv.shape)
        wkv = O.unpack_bf16(bits).reshape(wkv.shape)
        dw = dev_bf16(bits)
    else:
        dw = dev_f32(wkv)
    scale = float(1.0 / np.sqrt(dn + 64))
    out = torch.zeros((count, heads, dv), dtype=torch.float32, device="cuda")
    sel = {}
    if selection is not None:
        st, ct, ks = O.selection_csr(selection, count)
        sel = dict(sel_start=dev_u32(st), sel_count=dev_u32(ct), sel_keys=dev_u32(ks))
    say("latent attention", dict(count=count, start=start, heads=heads, dn=dn, dv=dv, C=C, bf16=bf16_w,
                                 sparse=selection is not None))
    gpu.latent_attention(dev_f32(q), dev_f32(latent), dw, out, start, scale, **sel)
    want = O.latent_attention(q, latent, wkv, start, heads, dn, dv, scale, selection=selection)
    got = host(out)
    err = np.abs(got - want).max()
    assert err <= 1e-5 * max(1.0, np.abs(want).max()), f"max err {err}"


def test_decode_splits_keys(gpu):
    """one token against 300 cached latents: the keys split over workgroups"""
    run(gpu, 1, 300, 20, 64, 48, 512, 1)


def test_prefill_single_split(gpu):
    run(gpu, 300, 5, 16, 128, 128, 256, 2)


def test_small_prefill_bf16_weights(gpu):
    run(gpu, 7, 90, 4, 32, 16, 64, 3, bf16_w=True)


def test_sparse_selection(gpu):
    count, start = 6, 150
    r = np.random.default_rng(4)
    selection = []
    for t in range(count):
        if t % 3 == 1:
            selection.append(None)   # dense
        else:
            n = 40 + 17 * t
            selection.append(np.sort(r.choice(start + t + 1, size=n, replace=False)).tolist())
    run(gpu, count, start, 20, 64, 32, 128, 5, selection=selection)


def test_empty_selection_gives_zero_context(gpu):
    """tokens whose selection is empty (indexTail off, before the first full
    pool) attend to nothing: their output is 0, on one split and when the
    keys of a decode token are split over workgroups"""
    count, start = 5, 40
    selection = [[], [1, 3], [], None, list(range(0, 40, 3))]
    run(gpu, count, start, 20, 64, 32, 128, 6, selection=selection)
    run(gpu, 1, 300, 20, 64, 48, 512, 7, selection=[[]])


def test_rejects_bad_rank(gpu):
    import torch
    q = torch.zeros((1, 2, 8), device="cuda")
    lat = torch.zeros((1, 20), device="cuda")
    w = torch.zeros((2 * 16, 20), device="cuda")
    out = torch.zeros((1, 2, 8), device="cuda")
    with pytest.raises(RuntimeError, match="kvLoraRank"):
        gpu.latent_attention(q, lat, w, out, 0, 1.0)
