"""Writes tests/golden/fixture_model.npz: the reference's independent FP64
NumPy model oracle for small random bf16 checkpoints.

The reference generates these in tools/make_gpu_fixture.py (:88-156), a
NumPy-only script: a 2-layer model (hidden 64, 4 query / 2 kv heads of 16,
SwiGLU 128, vocab 4096) with bf16 weights drawn from a seeded generator,
and a full causal FP64 pass over token ids 1..21 whose logits its GPU test
holds the CPU and GPU paths to (src/gpu-testing.cpp:791-827, maxAbs/rms
< 1e-4). This script runs that generator in the build container (where the
reference checkout exists) for five variants and keeps only numbers:

  - per weight set (qwen3 and llama draw identical weights; qwen2 draws its
    biases in between), the bf16 bit patterns of every layer weight, the
    embedding rows of the 21 ids, and the first VOCAB rows of lm_head;
  - per variant, the FP64 oracle's logits of those VOCAB rows for each of
    the 21 positions (the logits of a model whose head keeps only those
    rows), and the variant's config.

Run:  python tests/golden/make_fixture_model.py
"""
import json
import os
import struct
import subprocess
import sys
import tempfile

import numpy as np

REF_TOOL = "/root/reference/tools/make_gpu_fixture.py"
HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "fixture_model.npz")
VOCAB = 1024   # head rows kept: a quarter of the fixture's vocabulary

# name -> generator arguments
VARIANTS = {
    "qwen3": [],
    "qwen3_llama3": ["--rope", "llama3"],
    "qwen3_window8": ["--window", "8"],
    "qwen2_llama3_window7": ["--model-type", "qwen2", "--rope", "llama3", "--window", "7"],
    "llama_linear": ["--model-type", "llama", "--rope", "linear"],
}


def read_safetensors(path):
    """header JSON + raw little-endian tensors; returns name -> uint16 array (bf16 bits)"""
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(n))
        data = f.read()
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        assert meta["dtype"] == "BF16", (name, meta["dtype"])
        a, b = meta["data_offsets"]
        out[name] = np.frombuffer(data[a:b], dtype="<u2").reshape(meta["shape"]).copy()
    return out


def main():
    if not os.path.exists(REF_TOOL):
        sys.exit(f"{REF_TOOL} not found: the fixture is generated in the build container only")
    arrays = {"vocab_kept": np.array(VOCAB)}
    weight_sets = {}
    configs = {}
    for name, extra in VARIANTS.items():
        with tempfile.TemporaryDirectory() as tmp:
            subprocess.run([sys.executable, REF_TOOL, tmp] + extra, check=True, capture_output=True)
            cfg = json.load(open(os.path.join(tmp, "config.json")))
            meta = json.load(open(os.path.join(tmp, "oracle.json")))
            tensors = read_safetensors(os.path.join(tmp, "model.safetensors"))
            vocab = int(meta["vocab"])
            ids = np.array(meta["ids"], np.int64)
            logits = np.fromfile(os.path.join(tmp, "oracle-logits.bin"), dtype="<f4").reshape(len(ids), vocab)
        wset = "qwen2" if cfg["model_type"] == "qwen2" else "qwen3"
        kept = {}
        for tname, t in tensors.items():
            if tname == "model.embed_tokens.weight":
                kept["embed_rows"] = t[ids]
            elif tname == "lm_head.weight":
                kept["lm_head"] = t[:VOCAB]
            else:
                kept[tname] = t
        if wset in weight_sets:
            # the same generator stream: the arrays must agree exactly
            for k, v in kept.items():
                if k in weight_sets[wset]:
                    assert np.array_equal(weight_sets[wset][k], v), (name, k)
            weight_sets[wset].update(kept)
        else:
            weight_sets[wset] = kept
        arrays[f"{name}/logits"] = logits[:, :VOCAB].astype(np.float32)
        arrays[f"{name}/logits_rms_full"] = np.array(np.sqrt(np.mean(logits.astype(np.float64) ** 2)))
        configs[name] = dict(weights=wset, ids=ids.tolist(), **{k: cfg[k] for k in cfg})
    for wset, kept in weight_sets.items():
        for k, v in kept.items():
            arrays[f"weights_{wset}/{k}"] = v
    arrays["configs_json"] = np.frombuffer(json.dumps(configs, sort_keys=True).encode(), dtype=np.uint8)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT}: {os.path.getsize(OUT):,} bytes, variants {list(VARIANTS)}")


if __name__ == "__main__":
    main()
