"""The oracle's dense_decode (the layer loop of LocalModel::forward for one
token, LocalModel.hpp:3705-3799, composed from the pinned primitives) against
the reference's independent FP64 NumPy model (tools/make_gpu_fixture.py),
token by token from an empty cache, for every fixture variant: qwen3 with
q/k norms, llama3 and linear RoPE scaling, sliding windows of 7 and 8, and
qwen2's q/k/v biases. The bar is the reference's own: maxAbs/rms < 1e-4
(src/gpu-testing.cpp:822)."""
import numpy as np
import pytest

import fixture_model as F
from oracle import oracle as O


@pytest.mark.parametrize("name", F.variants())
def test_dense_decode_reproduces_the_fp64_model(name):
    m = F.load(name)
    cfg = m["cfg"]
    n = len(m["embeddings"])
    kvw = cfg["kv_heads"] * cfg["head_dim"]
    keys = [np.zeros((n, kvw), np.float32) for _ in m["layers"]]
    values = [np.zeros((n, kvw), np.float32) for _ in m["layers"]]
    worst = 0.0
    for pos in range(n):
        got = O.dense_decode(cfg, m["layers"], m["head"], m["final_norm"], m["embeddings"][pos], keys, values, pos)
        worst = max(worst, F.error(m["logits"][pos], got))
    assert worst < F.LIMIT, f"{name}: maxAbs/rms {worst:.3e}"


def test_a_composition_mistake_fails_the_fixture():
    """silu(up) * gate in place of silu(gate) * up (or a dropped residual)
    moves the logits far past the bar: the fixture pins the composition"""
    m = F.load("qwen3")
    cfg = m["cfg"]
    layers = [dict(L, gate=L["up"], up=L["gate"]) for L in m["layers"]]
    kvw = cfg["kv_heads"] * cfg["head_dim"]
    keys = [np.zeros((4, kvw), np.float32) for _ in layers]
    values = [np.zeros((4, kvw), np.float32) for _ in layers]
    worst = 0.0
    for pos in range(4):
        got = O.dense_decode(cfg, layers, m["head"], m["final_norm"], m["embeddings"][pos], keys, values, pos)
        worst = max(worst, F.error(m["logits"][pos], got))
    assert worst > 100 * F.LIMIT
