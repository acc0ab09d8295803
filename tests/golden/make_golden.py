"""make_golden.py - writes tests/golden/reference_kernels.npz from the
reference's own CPU kernels, compiled from its headers into oracle/_ref
(oracle/Makefile, oracle/ref_shim.cpp). Run in the build container, where
the reference checkout exists:

    make -C oracle && python tests/golden/make_golden.py

Contents (inputs and the reference's outputs):
  rng_*           math::random::Random streams (Random.hpp:15-89)
  llm_*           the attention inputs of llm-testing.cpp:106-110 and
                  kernels::attention's outputs for windows 0, 1, 7, 200,
                  threaded and serial (Kernels.hpp:132-168)
  gqa_*           a seeded GQA case with cached history (start > 0)
  delta_*         kernels::deltaStep sequences, scalar and per-key decay
                  (Kernels.hpp:105-128)
  quant_*         ai::quant::quantize's Q8 and Q4 codes and scales of a
                  seeded matrix, and dequantRow of them (Quant.hpp:420-558)
"""
import ctypes as C
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as O  # noqa: E402


def main():
    R = O.ref()
    if R is None:
        raise SystemExit("oracle/_ref not built (needs the reference checkout): make -C oracle")
    R.ref_configure_pool(4)
    out = {}

    raw = np.zeros(64, np.uint64)
    R.ref_random(12345, 0, 64, 0, 0, raw.ctypes.data_as(C.c_void_p))
    out["rng_raw_seed12345"] = raw
    nrm = np.zeros(64, np.float64)
    R.ref_random(7, 2, 64, 0, 0, nrm.ctypes.data_as(C.c_void_p))
    out["rng_normal_seed7"] = nrm
    ints = np.zeros(32, np.int64)
    R.ref_random(3, 3, 32, 1024, 32768, ints.ctypes.data_as(C.c_void_p))
    out["rng_randint_1024_32768_seed3"] = ints
    uni = np.zeros(16, np.float64)
    R.ref_random(11, 4, 16, 0.5, 1.5, uni.ctypes.data_as(C.c_void_p))
    out["rng_uniform_05_15_seed11"] = uni

    # llm-testing.cpp:106-110 inputs (float sin/cos of float arguments)
    T, S, H, KV, D, ST = 19, 11, 4, 2, 48, 96
    q = np.array([np.sin(np.float32(i) * np.float32(0.13)) for i in range(T * H * ST)], np.float32)
    n = (S + T) * KV * D
    k = np.array([np.cos(np.float32(i) * np.float32(0.17)) for i in range(n)], np.float32)
    v = np.array([np.sin(np.float32(i) * np.float32(0.23)) for i in range(n)], np.float32)
    out["llm_q"], out["llm_k"], out["llm_v"] = q, k, v
    for w in (0, 1, 7, 200):
        threaded = np.zeros(T * H * D, np.float32)
        serial = np.zeros(T * H * D, np.float32)
        R.ref_attention(q, k, v, threaded, T, S, H, KV, D, ST, w, 1)
        R.ref_attention(q, k, v, serial, T, S, H, KV, D, ST, w, 0)
        out[f"llm_out_w{w}"] = threaded
        out[f"llm_out_serial_w{w}"] = serial

    # seeded GQA case: 5 new tokens after 7 cached, 8 heads over 2 kv heads
    cnt, start, h, kv, d = 5, 7, 8, 2, 64
    gq = O.fill_normal((cnt, h, d), 21, "q")
    gk = O.fill_normal((start + cnt, kv, d), 21, "k")
    gv = O.fill_normal((start + cnt, kv, d), 21, "v")
    go = np.zeros(cnt * h * d, np.float32)
    R.ref_attention(gq.reshape(-1), gk.reshape(-1), gv.reshape(-1), go, cnt, start, h, kv, d, d, 0, 0)
    out["gqa_q"], out["gqa_k"], out["gqa_v"], out["gqa_out"] = gq, gk, gv, go.reshape(cnt, h, d)

    # deltaStep sequences
    for K, V, per_key in ((32, 64, 0), (32, 64, 1), (128, 128, 0)):
        steps = 5
        state = O.fill_normal((K, V), 31, f"state{K}x{V}") * np.float32(0.01)
        keys = O.fill_normal((steps, K), 31, f"key{K}") / np.float32(np.sqrt(K))
        queries = O.fill_normal((steps, K), 31, f"query{K}") / np.float32(K)
        values = O.fill_normal((steps, V), 31, f"value{V}")
        decays = O.fill_uniform((steps, K), 31, f"decay{K}", 0.8, 0.95)
        betas = O.fill_uniform((steps,), 31, "beta", 0.1, 0.9)
        tag = f"delta_{K}x{V}_{'channel' if per_key else 'scalar'}"
        out[tag + "_state0"] = state.copy()
        out[tag + "_keys"], out[tag + "_queries"], out[tag + "_values"] = keys, queries, values
        out[tag + "_decays"], out[tag + "_betas"] = decays, betas
        st = state.copy().reshape(-1)
        outs = np.zeros((steps, V), np.float32)
        pred = np.zeros(V, np.float32)
        delta = np.zeros(V, np.float32)
        for t in range(steps):
            o = np.zeros(V, np.float32)
            R.ref_delta_step(st, keys[t].copy(), queries[t].copy(), values[t].copy(),
                             decays[t].copy(), per_key, float(betas[t]), K, V, o, pred, delta)
            outs[t] = o
        out[tag + "_outs"] = outs
        out[tag + "_state"] = st.reshape(K, V)

    # ai::quant::quantize and dequantRow (Quant.hpp:420-558) on a seeded matrix
    src = O.fill_normal((6, 96), 41, "quant_src")
    src[2, 5] = -4.0   # a block whose signed extreme is negative (Q4's scale sign)
    out["quant_src"] = src
    for kind in ("q8", "q4"):
        codes, scales = O.ref_quantize(src, kind)
        out[f"quant_{kind}_codes"], out[f"quant_{kind}_scales"] = codes, scales
        out[f"quant_{kind}_dequant"] = O.ref_dequant(codes, scales, kind)

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_kernels.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
