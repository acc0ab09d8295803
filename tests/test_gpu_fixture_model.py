"""The resident decoder (aigpu_dense_*) against the reference's independent
FP64 NumPy model (tools/make_gpu_fixture.py, through
tests/golden/fixture_model.npz): the bf16 checkpoint's weights uploaded as
they are, all 21 tokens decoded one at a time from an empty cache, every
step's logits held to the reference's own bar for this fixture, maxAbs/rms
< 1e-4 (src/gpu-testing.cpp:791-827). Variants: qwen3 q/k norms, llama3 and
linear RoPE scaling, sliding windows of 7 and 8, qwen2 q/k/v biases."""
import numpy as np
import pytest

import fixture_model as F
from gpu_util import say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", F.variants())
def test_resident_decoder_matches_the_fp64_model(gpu, name):
    m = F.load(name)
    cfg = dict(m["cfg"])
    n = len(m["embeddings"])
    cfg["capacity"] = n
    ptrs = []

    def dev(w):
        stored, kind, scales, bias = w
        ptr = gpu.upload(stored)
        ptrs.append((ptr, stored.nbytes))
        return {"ptr": ptr, "kind": kind, "scales_ptr": None, "in": stored.shape[1], "out": stored.shape[0],
                "bias": bias}

    layers = []
    for L in m["layers"]:
        d = {k: dev(L[k]) for k in ("q", "k", "v", "o", "gate", "up", "down")}
        d.update(input_norm=L["input_norm"], post_norm=L["post_norm"], q_norm=L["q_norm"], k_norm=L["k_norm"],
                 window=L["window"])
        layers.append(d)
    kvw = cfg["kv_heads"] * cfg["head_dim"]
    empty = [np.zeros((n, kvw), np.float32) for _ in layers]
    say("fixture model resident decode", dict(variant=name, tokens=n))
    dec = gpu.DenseDecoder(cfg, layers, dev(m["head"]), m["final_norm"], empty, empty, 0, freqs=cfg["freqs"])
    try:
        worst = 0.0
        for pos in range(n):
            got = dec.decode(m["embeddings"][pos], pos)
            worst = max(worst, F.error(m["logits"][pos], got))
        assert worst < F.LIMIT, f"{name}: maxAbs/rms {worst:.3e}"
    finally:
        dec.close()
        for ptr, nbytes in ptrs:
            gpu.release(ptr, nbytes)
