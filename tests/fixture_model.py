"""The reference's FP64 NumPy model oracle (tests/golden/fixture_model.npz,
written by tests/golden/make_fixture_model.py from the reference's
tools/make_gpu_fixture.py) as model descriptions for the oracle's
dense_decode and for the resident decoder.

The model is what the reference's loader builds from the fixture's
config.json (LocalConfig::loadFrom, LocalModel.hpp:795-830): qwen3 carries
per-head q/k RMSNorm weights, qwen2 q/k/v biases, llama neither; rotary
frequencies in fp32 with linear or llama3 scaling; the sliding window on
every layer (max_window_layers = 0). The error measure is the reference's
(src/gpu-testing.cpp:85-95): max |reference - x| over the rms of the
reference logits, held below 1e-4."""
import json
import os

import numpy as np

from oracle import oracle as O

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixture_model.npz")
ROPE_KIND = {"default": 0, "linear": 1, "llama3": 2}
LIMIT = 1e-4


def _npz():
    return np.load(PATH)


def variants():
    return sorted(json.loads(bytes(_npz()["configs_json"]).decode()))


def widen(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def error(reference, other):
    """gpu-testing.cpp compare(): maxAbs over the rms of the reference"""
    reference = np.asarray(reference, np.float64)
    rms = np.sqrt(np.mean(reference ** 2))
    d = np.abs(reference - np.asarray(other, np.float64)).max()
    return d / rms if rms > 0 else d


def load(name):
    z = _npz()
    cfg = json.loads(bytes(z["configs_json"]).decode())[name]
    w = {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(f"weights_{cfg['weights']}/")}
    H, nH, nKV = cfg["hidden_size"], cfg["num_attention_heads"], cfg["num_key_value_heads"]
    D = cfg["head_dim"]
    scaling = cfg.get("rope_scaling") or {}
    kind = ROPE_KIND[scaling.get("rope_type", "default")]
    freqs = O.rotary_frequencies(D, cfg["rope_theta"], kind, scaling.get("factor", 1.0),
                                 scaling.get("low_freq_factor", 1.0), scaling.get("high_freq_factor", 4.0),
                                 scaling.get("original_max_position_embeddings", 0.0))
    window = cfg.get("sliding_window", 0) if cfg.get("use_sliding_window") else 0
    layers = []
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        layer = {"window": int(window)}
        for short, full in (("q", "self_attn.q_proj"), ("k", "self_attn.k_proj"), ("v", "self_attn.v_proj"),
                            ("o", "self_attn.o_proj"), ("gate", "mlp.gate_proj"), ("up", "mlp.up_proj"),
                            ("down", "mlp.down_proj")):
            bias = w.get(p + full + ".bias") if cfg["model_type"] == "qwen2" else None
            layer[short] = (w[p + full + ".weight"], "bf16", None, None if bias is None else widen(bias))
        layer["input_norm"] = widen(w[p + "input_layernorm.weight"])
        layer["post_norm"] = widen(w[p + "post_attention_layernorm.weight"])
        # per-head q/k norms are a qwen3 trait of the architecture, whatever
        # tensors the weight set holds (qwen3 and llama share one)
        qk_norm = cfg["model_type"] == "qwen3"
        layer["q_norm"] = widen(w[p + "self_attn.q_norm.weight"]) if qk_norm else None
        layer["k_norm"] = widen(w[p + "self_attn.k_norm.weight"]) if qk_norm else None
        layers.append(layer)
    vocab = int(z["vocab_kept"])
    model = dict(
        cfg=dict(hidden=H, heads=nH, kv_heads=nKV, head_dim=D, intermediate=cfg["intermediate_size"], vocab=vocab,
                 rotary_dims=D, eps=cfg["rms_norm_eps"], theta=cfg["rope_theta"], freqs=freqs),
        layers=layers,
        head=(w["lm_head"], "bf16", None, None),
        final_norm=widen(w["model.norm.weight"]),
        embeddings=widen(w["embed_rows"]),
        logits=z[f"{name}/logits"],
    )
    return model
