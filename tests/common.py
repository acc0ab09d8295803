"""Shared pieces of the parity tests: error metrics with the north-star
tolerances, and the seeded inputs of each configuration built with the
restated reference RNG recipe (oracle.fill_*: Random(seed ^ fnv1a(name) +
chunk*golden) per 2^14-element chunk, LocalModel.hpp:1555-1573)."""
import numpy as np

from oracle import oracle as O

# north-star tolerances
BF16_MAX_ABS = 2e-3
BF16_REL_L2 = 1e-3
F32_MAX_ABS = 1e-5


def errors(ref, got):
    """max-abs, rel-L2 and the reference's maxAbs/rms (gpu-testing.cpp:85-95)."""
    ref = np.asarray(ref, np.float64).reshape(-1)
    got = np.asarray(got, np.float64).reshape(-1)
    d = got - ref
    max_abs = float(np.abs(d).max()) if d.size else 0.0
    norm = float(np.linalg.norm(ref))
    rel = float(np.linalg.norm(d) / norm) if norm > 0 else float(np.linalg.norm(d))
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    return {"max_abs": max_abs, "rel_l2": rel, "ref_error": max_abs / rms if rms > 0 else max_abs}


def assert_bf16_parity(ref, got, what=""):
    e = errors(ref, got)
    assert np.isfinite(np.asarray(got)).all(), f"{what}: non-finite output"
    assert e["max_abs"] <= BF16_MAX_ABS and e["rel_l2"] <= BF16_REL_L2, f"{what}: {e}"
    return e


def assert_f32_parity(ref, got, what="", tol=F32_MAX_ABS):
    e = errors(ref, got)
    assert np.isfinite(np.asarray(got)).all(), f"{what}: non-finite output"
    assert e["max_abs"] <= tol, f"{what}: {e}"
    return e


def bf16_normal(shape, seed, name):
    """N(0,1) drawn in fp32 then rounded to bf16 (RNE); returns (bits, widened)."""
    x = O.fill_normal(shape, seed, name)
    bits = O.pack_bf16(x)
    return bits, O.unpack_bf16(bits).reshape(shape)


def gammas(dim, seed, name):
    return O.fill_uniform((dim,), seed, name, 0.5, 1.5)


def attention_fp64(q, k, v, T, S, H, KV, D, stride, window):
    """textbook softmax(q.K/sqrt(D)) V in fp64 (llm-testing.cpp:114-130)."""
    out = np.zeros((T, H, D))
    q = q.astype(np.float64)
    k = k.astype(np.float64).reshape(-1, KV, D)
    v = v.astype(np.float64).reshape(-1, KV, D)
    for t in range(T):
        end = S + t
        begin = end + 1 - window if window and end + 1 > window else 0
        for h in range(H):
            kv = h // (H // KV)
            qv = q[(t * H + h) * stride:(t * H + h) * stride + D]
            s = k[begin:end + 1, kv] @ qv / np.sqrt(D)
            p = np.exp(s - s.max())
            out[t, h] = p @ v[begin:end + 1, kv] / p.sum()
    return out
