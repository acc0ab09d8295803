"""GPU parity of the resident single-token decoder (aigpu_dense_*, dense.hip)
against the oracle's composition of LocalModel::forward for count = 1
(LocalModel.hpp:3705-3799), built from the pinned restatements of
rmsNormRow, apply, the q/k norm and RoPE, kernels::attention and swiglu.

Bar: every logit within 1e-5 of max(1, max |logit|), and the cache read back
within 1e-5 of max(1, max |k|): the fp32 bar on the scale of the outputs (the
device sums in its own order, as the reference's CPU and GPU paths do)."""
import numpy as np
import pytest

from gpu_util import say
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def quantise(src, kind):
    n, k = src.shape
    blocks = src.reshape(n, k // 32, 32)
    amax = np.abs(blocks).max(axis=2)
    if kind == "q8":
        scales = (amax / 127.0).astype(np.float32)
        return np.clip(np.round(blocks / scales[..., None]), -127, 127).astype(np.int8).reshape(n, k), scales
    scales = (amax / 8.0).astype(np.float32)
    q = np.clip(np.round(blocks / scales[..., None]) + 8, 0, 15).astype(np.uint8)
    return (q[:, :, :16] | (q[:, :, 16:] << 4)).reshape(n, k // 2), scales


class Model:
    """random weights of one encoding, uploaded, with the oracle's view"""

    def __init__(self, gpu, cfg, kind, seed, qk_norm=True, biases=False, windows=(0, 0)):
        self.gpu, self.cfg, self.ptrs = gpu, cfg, []
        H, nH, nKV, D, I, V = (cfg[k] for k in ("hidden", "heads", "kv_heads", "head_dim", "intermediate", "vocab"))
        rng = np.random.default_rng(seed)

        def weight(n, k, name, bias=False):
            src = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
            b = (rng.standard_normal(n) * 0.1).astype(np.float32) if bias else None
            if kind == "f32":
                stored, scales = src, None
            elif kind == "bf16":
                stored, scales = O.pack_bf16(src).reshape(n, k), None
            else:
                stored, scales = quantise(src, kind)
            ptr = gpu.upload(stored)
            self.ptrs.append((ptr, stored.nbytes))
            sptr = None
            if scales is not None:
                sptr = gpu.upload(scales)
                self.ptrs.append((sptr, scales.nbytes))
            dev = {"ptr": ptr, "kind": kind, "scales_ptr": sptr, "in": k, "out": n, "bias": b}
            return dev, (stored, kind, scales, b)

        def gamma(n):
            return rng.uniform(0.5, 1.5, n).astype(np.float32)

        self.dev_layers, self.ref_layers = [], []
        for li, win in enumerate(windows):
            d, r = {}, {}
            for name, n, k, b in (("q", nH * D, H, biases), ("k", nKV * D, H, biases), ("v", nKV * D, H, biases),
                                  ("o", H, nH * D, False), ("gate", I, H, False), ("up", I, H, False),
                                  ("down", H, I, False)):
                d[name], r[name] = weight(n, k, name, b)
            for name, n in (("input_norm", H), ("post_norm", H)):
                d[name] = r[name] = gamma(n)
            d["q_norm"] = r["q_norm"] = gamma(D) if qk_norm else None
            d["k_norm"] = r["k_norm"] = gamma(D) if qk_norm else None
            d["window"] = r["window"] = win
            self.dev_layers.append(d)
            self.ref_layers.append(r)
        self.dev_head, self.ref_head = weight(V, H, "head")
        self.final_norm = gamma(H)

    def release(self):
        for ptr, n in self.ptrs:
            self.gpu.release(ptr, n)


def run(gpu, kind, length=5, steps=5, qk_norm=True, biases=False, windows=(0, 0), rot=64, capacity=40, seed=1,
        shape=None):
    cfg = dict(hidden=256, heads=4, kv_heads=2, head_dim=64, intermediate=512, vocab=777, capacity=capacity,
               rotary_dims=rot, eps=1e-6, theta=1e6)
    cfg.update(shape or {})
    m = Model(gpu, cfg, kind, seed, qk_norm=qk_norm, biases=biases, windows=windows)
    rng = np.random.default_rng(seed + 100)
    kvw = cfg["kv_heads"] * cfg["head_dim"]
    keys = [np.zeros((capacity, kvw), np.float32) for _ in windows]
    values = [np.zeros((capacity, kvw), np.float32) for _ in windows]
    for k, v in zip(keys, values):
        k[:length] = rng.standard_normal((length, kvw)).astype(np.float32)
        v[:length] = rng.standard_normal((length, kvw)).astype(np.float32)
    freqs = O.rotary_frequencies(rot, cfg["theta"])
    say("dense decoder", dict(kind=kind, length=length, steps=steps, qk_norm=qk_norm, biases=biases,
                              windows=windows, rot=rot, shape=shape))
    dec = gpu.DenseDecoder(cfg, m.dev_layers, m.dev_head, m.final_norm, keys, values, length)
    rcfg = dict(cfg, freqs=freqs)
    try:
        for t in range(steps):
            pos = length + t
            emb = rng.standard_normal(cfg["hidden"]).astype(np.float32)
            got = dec.decode(emb, pos)
            want = O.dense_decode(rcfg, m.ref_layers, m.ref_head, m.final_norm, emb, keys, values, pos)
            err = np.abs(got - want).max()
            assert err <= 1e-5 * max(1.0, np.abs(want).max()), f"{kind} pos {pos}: logits err {err}"
        gk, gv = dec.read_cache(length + steps)
        for li in range(len(windows)):
            for g, w in ((gk[li], keys[li]), (gv[li], values[li])):
                err = np.abs(g - w[:length + steps]).max()
                assert err <= 1e-5 * max(1.0, np.abs(w).max()), f"layer {li} cache err {err}"
    finally:
        dec.close()
        m.release()


@pytest.mark.parametrize("kind", ["f32", "bf16", "q8", "q4"])
def test_qwen3_layers(gpu, kind):
    run(gpu, kind)


def test_llama_layers_with_biases_window_and_partial_rotary(gpu):
    run(gpu, "bf16", qk_norm=False, biases=True, windows=(3, 0), rot=32)


def test_long_history_crosses_attention_splits(gpu):
    """a cache dealt over several attention workgroups (19 ranges of 32)"""
    run(gpu, "bf16", length=600, steps=2, capacity=620)


def test_very_long_history_fills_every_split(gpu):
    """64 ranges of 130 positions (one pass of up to 160 each), and a window
    of 3000 in 64 ranges of 47"""
    run(gpu, "bf16", length=8300, steps=2, capacity=8310, windows=(0, 3000))


@pytest.mark.parametrize("length,heads", [
    (10300, 4),   # 64 ranges of 161: two passes of up to 160 positions
    (8300, 16),   # eight query heads per kv head, 32 rows per wave: two passes for 130
])
def test_ranges_take_several_passes(gpu, length, heads):
    run(gpu, "bf16", length=length, steps=2, capacity=length + 10, shape=dict(heads=heads, kv_heads=2))


@pytest.mark.parametrize("kind", ["bf16", "q4"])
def test_long_odd_head(gpu, kind):
    """a vocabulary of 70001 rows (8751 workgroups, the last wave's second row
    repeating the last one)"""
    run(gpu, kind, steps=2, shape=dict(vocab=70001))


@pytest.mark.parametrize("heads,kv_heads,head_dim", [
    (4, 4, 64),     # one query head per kv head
    (6, 2, 96),     # three, and a head dim that leaves key pieces and value lanes idle
    (8, 2, 128),    # four
    (8, 1, 128),    # eight
    (4, 2, 256),    # four dims per value lane
    (8, 1, 256),    # both at their largest
])
def test_group_sizes_and_head_dims(gpu, heads, kv_heads, head_dim):
    run(gpu, "bf16", length=300, steps=3, capacity=310, rot=head_dim // 2,
        shape=dict(heads=heads, kv_heads=kv_heads, head_dim=head_dim))


def test_empty_cache_and_position_checks(gpu):
    cfg = dict(hidden=256, heads=4, kv_heads=2, head_dim=64, intermediate=512, vocab=777, capacity=8,
               rotary_dims=64, eps=1e-6, theta=1e6)
    m = Model(gpu, cfg, "bf16", 5)
    kvw = 128
    keys = [np.zeros((8, kvw), np.float32) for _ in range(2)]
    values = [np.zeros((8, kvw), np.float32) for _ in range(2)]
    dec = gpu.DenseDecoder(cfg, m.dev_layers, m.dev_head, m.final_norm, keys, values, 0)
    try:
        emb = np.ones(256, np.float32)
        with pytest.raises(RuntimeError, match="position"):
            dec.decode(emb, 3)
        want = O.dense_decode(dict(cfg, freqs=O.rotary_frequencies(64, 1e6)), m.ref_layers, m.ref_head,
                              m.final_norm, emb, keys, values, 0)
        got = dec.decode(emb, 0)
        assert np.abs(got - want).max() <= 1e-5 * max(1.0, np.abs(want).max())
    finally:
        dec.close()
        m.release()


def test_rejects_bad_config(gpu):
    import aigpu
    c = aigpu.AiGpuDenseConfig(hidden=0)
    L = aigpu.lib()
    assert not L.aigpu_dense_create(c, None, None, None, 0)
    assert "configuration" in aigpu.last_error()


def test_graph_replay_matches_launches_one_by_one(gpu, monkeypatch):
    """the step replayed as a captured HIP graph (the default) gives the same
    logits, bit for bit, as the same kernels launched one by one
    (AIGPU_DENSE_GRAPH=0), step after step across a change of the attention
    grid at position 256 (a second capture), with other GPU work and
    synchronisations between the replays; the caches agree too"""
    import torch
    cfg = dict(hidden=256, heads=4, kv_heads=2, head_dim=64, intermediate=512, vocab=777, capacity=270,
               rotary_dims=64, eps=1e-6, theta=1e6)
    m = Model(gpu, cfg, "bf16", 9)
    rng = np.random.default_rng(77)
    length, steps = 250, 10
    keys = [rng.standard_normal((270, 128)).astype(np.float32) for _ in range(2)]
    values = [rng.standard_normal((270, 128)).astype(np.float32) for _ in range(2)]
    embs = [rng.standard_normal(256).astype(np.float32) for _ in range(steps)]
    say("dense graph replay", dict(length=length, steps=steps))
    graph = gpu.DenseDecoder(cfg, m.dev_layers, m.dev_head, m.final_norm, keys, values, length)
    eager = gpu.DenseDecoder(cfg, m.dev_layers, m.dev_head, m.final_norm, keys, values, length)
    try:
        noise = torch.ones(1 << 20, device="cuda")
        for t in range(steps):
            monkeypatch.delenv("AIGPU_DENSE_GRAPH", raising=False)
            got = graph.decode(embs[t], length + t)
            noise.mul_(1.0001).sum().item()   # eager work and a synchronisation between replays
            monkeypatch.setenv("AIGPU_DENSE_GRAPH", "0")
            want = eager.decode(embs[t], length + t)
            assert np.array_equal(got, want), f"step {t}: graph and launches differ"
        gk, gv = graph.read_cache(length + steps)
        ek, ev = eager.read_cache(length + steps)
        for a, b in zip(gk + gv, ek + ev):
            assert np.array_equal(a, b)
    finally:
        monkeypatch.delenv("AIGPU_DENSE_GRAPH", raising=False)
        graph.close()
        eager.close()
        m.release()
