"""oracle.py - numpy front end over the CPU restatement (liboracle_*.so) and,
where it was built, the reference's own kernels (_ref/libref_*.so).

TEST INFRASTRUCTURE ONLY. Imported by tests/, bench.py's cpu_baseline leg and
__graft_entry__.smoke() as the checker; the product path never imports it.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_sz = C.c_size_t


def _has_avx512():
    try:
        with open("/proc/cpuinfo") as f:
            flags = f.read()
        return all(x in flags for x in ("avx512f", "avx512bw", "avx512vl", "avx512dq"))
    except OSError:
        return False


def _pick(stem, folder):
    for level in (("v4", "v3") if _has_avx512() else ("v3",)):
        path = os.path.join(folder, f"{stem}_{level}.so")
        if os.path.exists(path):
            return path
    return None


def build():
    """Compiles the oracle (and _ref where the reference checkout exists)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        path = _pick("liboracle", HERE)
        if path is None:
            raise RuntimeError("oracle not built: run make -C oracle")
        L = C.CDLL(path)
        L.or_rng_seed.argtypes = [C.c_void_p, C.c_uint64]
        L.or_rng_next.restype = C.c_uint64
        L.or_rng_next.argtypes = [C.c_void_p]
        L.or_rng_normal.restype = C.c_double
        L.or_rng_normal.argtypes = [C.c_void_p, C.c_double, C.c_double]
        L.or_rng_uniform.restype = C.c_double
        L.or_rng_uniform.argtypes = [C.c_void_p, C.c_double, C.c_double]
        L.or_rng_int.restype = C.c_int64
        L.or_rng_int.argtypes = [C.c_void_p, C.c_int64, C.c_int64]
        L.or_rng_u01.restype = C.c_double
        L.or_rng_u01.argtypes = [C.c_void_p]
        L.or_fnv1a.restype = C.c_uint64
        L.or_fnv1a.argtypes = [C.c_char_p]
        L.or_fill_normal.argtypes = [_f32p, _sz, C.c_uint64, C.c_char_p, C.c_double, C.c_double, C.c_int]
        L.or_fill_uniform.argtypes = [_f32p, _sz, C.c_uint64, C.c_char_p, C.c_double, C.c_double, C.c_int]
        L.or_round_to_bf16.argtypes = [_f32p, _sz]
        L.or_pack_bf16.argtypes = [_f32p, _u16p, _sz]
        L.or_dot.restype = C.c_float
        L.or_dot.argtypes = [_f32p, _f32p, _sz]
        L.or_attention.argtypes = [_f32p, _f32p, _f32p, _f32p] + [_sz] * 7 + [C.c_int]
        L.or_attention_strided.argtypes = ([_f32p, _f32p, _f32p, _f32p] + [_sz] * 9 +
                                           [C.c_void_p, _sz, C.c_int])
        L.or_rms_norm_row.argtypes = [_f32p, _f32p, _f32p, _sz, C.c_float, C.c_float]
        L.or_rotary_frequencies.restype = C.c_int
        L.or_rotary_frequencies.argtypes = [_f32p, _sz, C.c_float, C.c_int, C.c_float,
                                            C.c_float, C.c_float, C.c_float]
        L.or_qk_norm_rope.argtypes = ([_f32p, _f32p] + [_sz] * 6 + [C.c_void_p, C.c_void_p,
                                      C.c_float, C.c_float, C.c_void_p, _sz])
        L.or_sigmoid.restype = C.c_float
        L.or_sigmoid.argtypes = [C.c_float]
        L.or_softplus.restype = C.c_float
        L.or_softplus.argtypes = [C.c_float]
        L.or_l2normalise.argtypes = [_f32p, _sz, C.c_float]
        L.or_delta_step.argtypes = ([_f32p, _f32p, _f32p, _f32p, _f32p, C.c_int, C.c_float,
                                     _sz, _sz, _f32p, _f32p, _f32p])
        L.or_gdn_gates.argtypes = [_f32p] * 6 + [_sz, _sz]
        L.or_gated_delta_rule.argtypes = [_f32p] * 7 + [_sz] * 5 + [C.c_int, C.c_int]
        L.or_silu.restype = C.c_float
        L.or_silu.argtypes = [C.c_float]
        L.or_gdn_conv.argtypes = [_f32p, _sz, _sz, _sz, _f32p, _f32p, _f32p]
        L.or_gdn_deinterleave.argtypes = [_f32p, _f32p] + [_sz] * 5 + [_f32p] * 4
        L.or_gdn_gated_norm.argtypes = [_f32p, _f32p, _f32p, C.c_float, _f32p, _sz, _sz, _sz, C.c_int]
        L.or_kda_gates.argtypes = [_f32p] * 4 + [C.c_int, C.c_float, _f32p, _f32p, _sz, _sz, _sz]
        L.or_output_gate.argtypes = [_f32p, _f32p, _sz, _sz, _sz, _sz]
        L.or_kda_rule.argtypes = [_f32p] * 7 + [_sz] * 5 + [C.c_int, C.c_int]
        L.or_dequant.argtypes = [C.c_void_p, _f32p, _sz, _sz, C.c_int, _f32p]
        L.or_matmul_nt.argtypes = [_f32p, C.c_void_p, C.c_void_p, C.c_void_p, _f32p, _sz, _sz, _sz, C.c_int]
        L.or_latent_attention.argtypes = [_f32p, _f32p, _f32p, C.c_void_p, C.c_void_p, C.c_void_p, _f32p,
                                          _sz, _sz, _sz, _sz, _sz, _sz, C.c_float]
        L.or_index_update.argtypes = [_f32p, _f32p, C.c_void_p, _f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz]
        L.or_select_keys.argtypes = [_f32p, _f32p, _f32p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                     _sz, _sz, _sz, _sz, _sz, _sz, C.c_int]
        L.or_threads.restype = C.c_int
        L.or_threads.argtypes = [C.c_int]
        _lib = L
    return _lib


def ref():
    """The reference's own kernels (oracle/_ref), or None when not built."""
    global _ref
    if _ref is None:
        path = _pick("libref", os.path.join(HERE, "_ref"))
        if path is None:
            return None
        R = C.CDLL(path)
        R.ref_configure_pool.restype = C.c_int
        R.ref_configure_pool.argtypes = [C.c_int]
        R.ref_attention.argtypes = [_f32p] * 4 + [C.c_uint64] * 7 + [C.c_int]
        R.ref_delta_step.argtypes = ([_f32p] * 5 + [C.c_int, C.c_float, C.c_uint64, C.c_uint64] +
                                     [_f32p] * 3)
        R.ref_dot.restype = C.c_float
        R.ref_matmul_nt_bf16.argtypes = [_f32p, C.c_void_p, _f32p] + [C.c_uint64] * 3 + [C.c_int]
        R.ref_dot.argtypes = [_f32p, _f32p, C.c_uint64]
        R.ref_random.argtypes = [C.c_uint64, C.c_int, C.c_uint64, C.c_double, C.c_double, C.c_void_p]
        R.ref_gated_delta_rule.argtypes = [_f32p] * 7 + [C.c_uint64] * 5 + [C.c_int]
        R.ref_kda_rule.argtypes = [_f32p] * 7 + [C.c_uint64] * 5 + [C.c_int]
        R.ref_quantize.restype = C.c_int
        R.ref_quantize.argtypes = [_f32p, C.c_uint64, C.c_uint64, C.c_int, C.c_void_p, _f32p]
        R.ref_dequant_rows.argtypes = [C.c_void_p, _f32p, C.c_uint64, C.c_uint64, C.c_int, _f32p]
        _ref = R
    return _ref


def ref_gated_delta_rule(q, k, v, g, beta, state=None, normalize=True):
    """The mixer's token loop around the reference's own deltaStep
    (oracle/ref_shim.cpp); None when oracle/_ref is not built."""
    R = ref()
    if R is None:
        return None
    S, Hk, KD = q.shape
    _, Hv, VD = v.shape
    st = (np.zeros((Hv, KD, VD), np.float32) if state is None
          else np.ascontiguousarray(state, np.float32).copy())
    out = np.zeros((S, Hv, VD), np.float32)
    R.ref_gated_delta_rule(np.ascontiguousarray(q, np.float32).reshape(-1),
                           np.ascontiguousarray(k, np.float32).reshape(-1),
                           np.ascontiguousarray(v, np.float32).reshape(-1),
                           np.ascontiguousarray(g, np.float32).reshape(-1),
                           np.ascontiguousarray(beta, np.float32).reshape(-1),
                           st.reshape(-1), out.reshape(-1), S, Hk, Hv, KD, VD, int(bool(normalize)))
    return out, st


def threads(requested=0, cap=16):
    n = lib().or_threads(int(requested))
    return max(1, min(n, cap)) if requested <= 0 else n


# ---------------------------------------------------------------- generator
class Rng:
    """math::random::Random restated (Random.hpp:15-89)."""

    def __init__(self, seed):
        self._buf = C.create_string_buffer(48)
        lib().or_rng_seed(self._buf, C.c_uint64(seed & 0xFFFFFFFFFFFFFFFF))

    def next(self):
        return lib().or_rng_next(self._buf)

    def u01(self):
        return lib().or_rng_u01(self._buf)

    def normal(self, mean=0.0, sd=1.0):
        return lib().or_rng_normal(self._buf, mean, sd)

    def uniform(self, lo, hi):
        return lib().or_rng_uniform(self._buf, lo, hi)

    def randint(self, lo, hi):
        return lib().or_rng_int(self._buf, lo, hi)


def fill_normal(shape, seed, name, mean=0.0, sd=1.0, nthreads=0):
    out = np.empty(int(np.prod(shape)), np.float32)
    lib().or_fill_normal(out, out.size, C.c_uint64(seed), name.encode(), mean, sd,
                         threads(nthreads))
    return out.reshape(shape)


def fill_uniform(shape, seed, name, lo, hi, nthreads=0):
    out = np.empty(int(np.prod(shape)), np.float32)
    lib().or_fill_uniform(out, out.size, C.c_uint64(seed), name.encode(), lo, hi,
                          threads(nthreads))
    return out.reshape(shape)


def round_bf16(x):
    y = np.ascontiguousarray(x, np.float32).copy()
    lib().or_round_to_bf16(y.reshape(-1), y.size)
    return y


def pack_bf16(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_pack_bf16(x.reshape(-1), out.reshape(-1), x.size)
    return out


def unpack_bf16(b):
    b = np.ascontiguousarray(b, np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- attention
def attention(q, keys, values, count, start, heads, kv_heads, dim, q_stride, window=0,
              nthreads=1):
    """kernels::attention restated; position-major keys/values [pos][kv][dim]."""
    q = np.ascontiguousarray(q, np.float32)
    keys = np.ascontiguousarray(keys, np.float32)
    values = np.ascontiguousarray(values, np.float32)
    out = np.zeros(count * heads * dim, np.float32)
    lib().or_attention(q.reshape(-1), keys.reshape(-1), values.reshape(-1), out, count, start,
                       heads, kv_heads, dim, q_stride, window,
                       threads(nthreads) if nthreads != 1 else 1)
    return out.reshape(count, heads, dim)


def attention_strided(q, keys, values, count, start, heads, kv_heads, dim, q_stride,
                      pos_stride, head_stride, window=0, rows=None, nthreads=1):
    q = np.ascontiguousarray(q, np.float32)
    keys = np.ascontiguousarray(keys, np.float32)
    values = np.ascontiguousarray(values, np.float32)
    n = count if rows is None else len(rows)
    out = np.zeros(n * heads * dim, np.float32)
    rows_arr = None if rows is None else np.ascontiguousarray(rows, np.uint32)
    lib().or_attention_strided(q.reshape(-1), keys.reshape(-1), values.reshape(-1), out, count,
                               start, heads, kv_heads, dim, q_stride, pos_stride, head_stride,
                               window,
                               None if rows_arr is None else rows_arr.ctypes.data_as(C.c_void_p),
                               0 if rows_arr is None else len(rows_arr),
                               threads(nthreads) if nthreads != 1 else 1)
    return out.reshape(n, heads, dim)


def rotary_frequencies(rotary_dims, theta, kind=0, factor=1.0, low=1.0, high=4.0,
                       original=0.0):
    out = np.zeros(rotary_dims // 2, np.float32)
    ok = lib().or_rotary_frequencies(out, rotary_dims, theta, kind, factor, low, high, original)
    if not ok:
        raise ValueError("invalid rotary position parameters")
    return out


def qk_norm_rope(q, k, count, start, heads, kv_heads, dim, q_stride, q_gamma, k_gamma, eps,
                 freqs, rotary_dims, weight_offset=0.0):
    """attentionMixer norm + RoPE restated; returns new (q, k) arrays."""
    q = np.ascontiguousarray(q, np.float32).copy()
    k = np.ascontiguousarray(k, np.float32).copy()
    qg = None if q_gamma is None else np.ascontiguousarray(q_gamma, np.float32)
    kg = None if k_gamma is None else np.ascontiguousarray(k_gamma, np.float32)
    fr = None if freqs is None else np.ascontiguousarray(freqs, np.float32)
    lib().or_qk_norm_rope(q.reshape(-1), k.reshape(-1), count, start, heads, kv_heads, dim,
                          q_stride, None if qg is None else qg.ctypes.data_as(C.c_void_p),
                          None if kg is None else kg.ctypes.data_as(C.c_void_p), eps,
                          weight_offset,
                          None if fr is None else fr.ctypes.data_as(C.c_void_p), rotary_dims)
    return q, k


# ------------------------------------------------------------- delta rule
def delta_step(state, key, query, value, decay, per_key, beta):
    """kernels::deltaStep restated; updates `state` in place, returns out."""
    K, V = state.shape
    out = np.zeros(V, np.float32)
    pred = np.zeros(V, np.float32)
    delta = np.zeros(V, np.float32)
    lib().or_delta_step(state.reshape(-1), np.ascontiguousarray(key, np.float32),
                        np.ascontiguousarray(query, np.float32),
                        np.ascontiguousarray(value, np.float32),
                        np.ascontiguousarray(decay, np.float32), int(per_key), beta, K, V, out,
                        pred, delta)
    return out


def gdn_gates(a, b, a_log, dt_bias):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    g = np.zeros_like(a)
    beta = np.zeros_like(a)
    count, nv = a.shape
    lib().or_gdn_gates(a.reshape(-1), b.reshape(-1), np.ascontiguousarray(a_log, np.float32),
                       np.ascontiguousarray(dt_bias, np.float32), g.reshape(-1),
                       beta.reshape(-1), count, nv)
    return g, beta


def gated_delta_rule(q, k, v, g, beta, state=None, normalize=True, nthreads=1):
    """gatedDeltaNetMixer recurrence restated. q,k [S][Hk][KD], v [S][Hv][VD],
    g, beta [S][Hv]. Returns (out [S][Hv][VD], final state [Hv][KD][VD])."""
    S, Hk, KD = q.shape
    _, Hv, VD = v.shape
    st = (np.zeros((Hv, KD, VD), np.float32) if state is None
          else np.ascontiguousarray(state, np.float32).copy())
    out = np.zeros((S, Hv, VD), np.float32)
    lib().or_gated_delta_rule(np.ascontiguousarray(q, np.float32).reshape(-1),
                              np.ascontiguousarray(k, np.float32).reshape(-1),
                              np.ascontiguousarray(v, np.float32).reshape(-1),
                              np.ascontiguousarray(g, np.float32).reshape(-1),
                              np.ascontiguousarray(beta, np.float32).reshape(-1),
                              st.reshape(-1), out.reshape(-1), S, Hk, Hv, KD, VD,
                              int(bool(normalize)),
                              threads(nthreads) if nthreads != 1 else 1)
    return out, st


# ---------------------------------------------------------------- GDN neighbours
def silu(x):
    return lib().or_silu(float(x))


def gdn_conv(x, kernel, window):
    """causalConvolution (LocalModel.hpp:2678-2708) restated: x [count][CW],
    kernel [CW][K], window [K-1][CW]; returns (out, new window)."""
    x = np.ascontiguousarray(x, np.float32)
    kernel = np.ascontiguousarray(kernel, np.float32)
    win = np.ascontiguousarray(window, np.float32).copy()
    count, CW = x.shape
    K = kernel.shape[1]
    out = np.empty((count, CW), np.float32)
    lib().or_gdn_conv(x.reshape(-1), count, CW, K, kernel.reshape(-1), win.reshape(-1), out.reshape(-1))
    return out, win


def gdn_deinterleave(fused, ba, nK, nV, KD, VD):
    """the linFusedQKVZ de-interleave (LocalModel.hpp:2739-2776) restated;
    returns (qkv [count][CW], z [count][nV][VD], b, a [count][nV])."""
    fused = np.ascontiguousarray(fused, np.float32)
    ba = np.ascontiguousarray(ba, np.float32)
    count = fused.shape[0]
    CW = 2 * nK * KD + nV * VD
    qkv = np.empty((count, CW), np.float32)
    z = np.empty((count, nV, VD), np.float32)
    b = np.empty((count, nV), np.float32)
    a = np.empty((count, nV), np.float32)
    lib().or_gdn_deinterleave(fused.reshape(-1), ba.reshape(-1), count, nK, nV, KD, VD, qkv.reshape(-1),
                              z.reshape(-1), b.reshape(-1), a.reshape(-1))
    return qkv, z, b, a


def gdn_gated_norm(x, z, gamma, eps=1e-6, gate="silu"):
    """rmsNormRow then x SiLU(z) per (token, value head) (LocalModel.hpp:2833-2841);
    gate="sigmoid": x sigmoid(z), kimiDeltaMixer's form (:2936-2945)."""
    x = np.ascontiguousarray(x, np.float32)
    z = np.ascontiguousarray(z, np.float32)
    gamma = np.ascontiguousarray(gamma, np.float32)
    count, nV, VD = x.shape
    out = np.empty_like(x)
    lib().or_gdn_gated_norm(x.reshape(-1), z.reshape(-1), gamma, eps, out.reshape(-1), count, nV, VD,
                            1 if gate == "sigmoid" else 0)
    return out


def output_gate(out, q, heads, dim, q_stride):
    """attentionMixer's output gate (LocalModel.hpp:2660-2665) restated: returns
    out [count][heads][dim] times sigmoid of each q row's second half."""
    o = np.ascontiguousarray(out, np.float32).copy()
    q = np.ascontiguousarray(q, np.float32)
    lib().or_output_gate(o.reshape(-1), q.reshape(-1), o.shape[0], heads, dim, q_stride)
    return o


def _kda_args(q, k, v, g, beta, state):
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    S, Hk, KD = q.shape
    _, Hv, VD = v.shape
    st = (np.zeros((Hv, KD, VD), np.float32) if state is None
          else np.ascontiguousarray(state, np.float32).copy())
    g = np.ascontiguousarray(g, np.float32).reshape(S, Hv, KD)
    beta = np.ascontiguousarray(beta, np.float32).reshape(S, Hv)
    return q, k, v, g, beta, st, S, Hk, Hv, KD, VD


def kda_gates(f, b, a_log, dt_bias, safe_gate, lower_bound=-5.0):
    """kimiDeltaMixer's gates (LocalModel.hpp:2894-2905) as log decays:
    f [S][Hv][KD], b [S][Hv], a_log [Hv], dt_bias [Hv][KD] -> (g, beta)."""
    f = np.ascontiguousarray(f, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    S, Hv, KD = f.shape
    g = np.zeros_like(f)
    beta = np.zeros((S, Hv), np.float32)
    lib().or_kda_gates(f.reshape(-1), b.reshape(-1), np.ascontiguousarray(a_log, np.float32),
                       np.ascontiguousarray(dt_bias, np.float32).reshape(-1), int(bool(safe_gate)),
                       float(lower_bound), g.reshape(-1), beta.reshape(-1), S, Hv, KD)
    return g, beta


def kda_rule(q, k, v, g, beta, state=None, normalize=True, nthreads=1):
    """kimiDeltaMixer's recurrence restated: per-key-channel log decay g
    [S][Hv][KD]; returns (out [S][Hv][VD], final state)."""
    q, k, v, g, beta, st, S, Hk, Hv, KD, VD = _kda_args(q, k, v, g, beta, state)
    out = np.zeros((S, Hv, VD), np.float32)
    lib().or_kda_rule(q.reshape(-1), k.reshape(-1), v.reshape(-1), g.reshape(-1), beta.reshape(-1),
                      st.reshape(-1), out.reshape(-1), S, Hk, Hv, KD, VD, int(bool(normalize)),
                      threads(nthreads) if nthreads != 1 else 1)
    return out, st


def ref_kda_rule(q, k, v, g, beta, state=None, normalize=True):
    """the reference's deltaStep (perKeyDecay) driven token by token (oracle/_ref)"""
    R = ref()
    if R is None:
        raise RuntimeError("oracle/_ref is not built")
    q, k, v, g, beta, st, S, Hk, Hv, KD, VD = _kda_args(q, k, v, g, beta, state)
    out = np.zeros((S, Hv, VD), np.float32)
    R.ref_kda_rule(q.reshape(-1), k.reshape(-1), v.reshape(-1), g.reshape(-1), beta.reshape(-1),
                   st.reshape(-1), out.reshape(-1), S, Hk, Hv, KD, VD, int(bool(normalize)))
    return out, st


# ---------------------------------------------------------------- projections
WEIGHT_TYPES = {"f32": 0, "bf16": 1, "q8": 2, "q4": 3}


def dequant(codes, scales, kind):
    """dequantRange (Quant.hpp:528-549) restated: codes [n][k] int8 (q8) or
    [n][k/2] uint8 (q4), scales [n][k/32] -> [n][k] fp32"""
    codes = np.ascontiguousarray(codes)
    scales = np.ascontiguousarray(scales, np.float32)
    n = codes.shape[0]
    k = codes.shape[1] * (2 if kind == "q4" else 1)
    out = np.zeros((n, k), np.float32)
    lib().or_dequant(codes.ctypes.data, scales.reshape(-1), n, k, WEIGHT_TYPES[kind], out.reshape(-1))
    return out


def matmul_nt(a, w, kind, scales=None, bias=None):
    """apply (LocalModel.hpp:1052-1078) restated: a [m][k] fp32; w the weight
    as stored ([n][k] fp32, bf16 bits as uint16, q8 int8 codes, or q4 uint8
    [n][k/2]); the exact sum rounded to fp32, plus the bias."""
    a = np.ascontiguousarray(a, np.float32)
    w = np.ascontiguousarray(w)
    m, k = a.shape
    n = w.shape[0]
    out = np.zeros((m, n), np.float32)
    sc = None if scales is None else np.ascontiguousarray(scales, np.float32)
    bi = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().or_matmul_nt(a.reshape(-1), w.ctypes.data, None if sc is None else sc.ctypes.data,
                       None if bi is None else bi.ctypes.data, out.reshape(-1), m, k, n, WEIGHT_TYPES[kind])
    return out


def ref_quantize(src, kind):
    """the reference's own ai::quant::quantize (oracle/_ref): (codes, scales)"""
    R = ref()
    if R is None:
        raise RuntimeError("oracle/_ref is not built")
    src = np.ascontiguousarray(src, np.float32)
    n, k = src.shape
    codes = np.zeros((n, k // 2), np.uint8) if kind == "q4" else np.zeros((n, k), np.int8)
    scales = np.zeros((n, k // 32), np.float32)
    if not R.ref_quantize(src.reshape(-1), n, k, 1 if kind == "q4" else 0, codes.ctypes.data, scales.reshape(-1)):
        raise ValueError("the reference declines to quantise this shape")
    return codes, scales


def ref_dequant(codes, scales, kind):
    R = ref()
    if R is None:
        raise RuntimeError("oracle/_ref is not built")
    codes = np.ascontiguousarray(codes)
    scales = np.ascontiguousarray(scales, np.float32)
    n = codes.shape[0]
    k = codes.shape[1] * (2 if kind == "q4" else 1)
    out = np.zeros((n, k), np.float32)
    R.ref_dequant_rows(codes.ctypes.data, scales.reshape(-1), n, k, 1 if kind == "q4" else 0, out.reshape(-1))
    return out


# ------------------------------------------------------ resident dense decoder
def rms_norm_row(x, gamma, eps, offset=0.0):
    """rmsNormRow (LocalModel.hpp:1341-1348) restated by or_rms_norm_row"""
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    lib().or_rms_norm_row(x, np.ascontiguousarray(gamma, np.float32), out, x.size, eps, offset)
    return out


def attention_mixer(h, layer, keys, values, start, cfg, q_stride=None, gate=False):
    """attentionMixer restated for `count` = h.shape[0] new rows at positions
    start.. (LocalModel.hpp:2577-2667): the q/k/v projections (apply,
    :2604-2606), per-head q/k RMSNorm and RoPE (:2608-2648), the append of k
    and v into the position-major fp32 cache (:2650-2655), kernels::attention
    over positions [0, start + count) with the layer's window (:2657-2659),
    the optional output gate (:2660-2665) and the o projection (:2667).

    h [count][hidden] (the normed hidden states); layer: weights q, k, v, o as
    (stored, kind, scales, bias), q_norm, k_norm (None for none), window;
    keys / values [capacity][kv_heads * head_dim] fp32, written in place at
    [start, start + count). cfg: heads, kv_heads, head_dim, rotary_dims, eps,
    freqs. q_stride is head_dim, or 2 head_dim with the gate. Returns
    (o-projection output [count][hidden], the normed and rotated q
    [count][heads][q_stride], the appended k rows [count][kv_heads][head_dim])."""
    nH, nKV, D = cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    qs = q_stride or D
    h = np.ascontiguousarray(h, np.float32)
    count = h.shape[0]

    def proj(inp, w):
        arr, kind, scales, bias = w
        return matmul_nt(inp, arr, kind, scales=scales, bias=bias)

    q = proj(h, layer["q"])
    k = proj(h, layer["k"])
    v = proj(h, layer["v"])
    qn, kn = qk_norm_rope(q, k, count, start, nH, nKV, D, qs, layer["q_norm"], layer["k_norm"], cfg["eps"],
                          cfg["freqs"], cfg["rotary_dims"])
    keys[start:start + count] = kn.reshape(count, -1)
    values[start:start + count] = v.reshape(count, -1)
    attn = attention(qn.reshape(-1), keys[:start + count], values[:start + count], count, start, nH, nKV, D, qs,
                     layer.get("window", 0))
    if gate:
        attn = output_gate(attn, q, nH, D, qs)
    out = proj(attn.reshape(count, nH * D), layer["o"])
    return out, qn.reshape(count, nH, qs), kn.reshape(count, nKV, D)


def dense_decode(cfg, layers, head, final_norm, embedding, keys, values, position):
    """One token through a dense RMSNorm / RoPE / SwiGLU model, as
    LocalModel::forward runs it for count = 1 (LocalModel.hpp:3705-3799):
    per layer the input norm, attentionMixer (q/k/v projections, per-head
    q/k RMSNorm, RoPE, cache append, kernels::attention, the output
    projection; :2575-2670), the residual add, the post-attention norm, the
    SwiGLU MLP (swiglu = silu(gate) * up, :3282-3288, :3760-3770) and the
    second residual add; then the final norm and the head (:3793-3799).

    cfg: dict hidden, heads, kv_heads, head_dim, rotary_dims, eps, freqs.
    layers: dicts with weights q, k, v, o, gate, up, down, each a tuple
    (stored array, kind, scales, bias), norms input_norm, post_norm, q_norm,
    k_norm (None for none) and window. keys / values: per layer
    [capacity][kv_heads * head_dim] fp32, written at `position`. Returns the
    logits. The composition is pinned by the reference's independent FP64
    model (tools/make_gpu_fixture.py; tests/test_oracle_fixture_model.py)."""
    H = cfg["hidden"]
    eps = cfg["eps"]
    x = np.ascontiguousarray(embedding, np.float32).reshape(1, H).copy()

    def proj(inp, w):
        arr, kind, scales, bias = w
        return matmul_nt(inp, arr, kind, scales=scales, bias=bias)

    for li, L in enumerate(layers):
        h = rms_norm_row(x[0], L["input_norm"], eps).reshape(1, H)
        x = x + attention_mixer(h, L, keys[li], values[li], position, cfg)[0]
        h = rms_norm_row(x[0], L["post_norm"], eps).reshape(1, H)
        g = proj(h, L["gate"])
        u = proj(h, L["up"])
        g = np.array([silu(float(a)) for a in g.reshape(-1)], np.float32).reshape(g.shape) * u
        x = x + proj(g, L["down"])
    last = rms_norm_row(x[0], final_norm, eps).reshape(1, H)
    return proj(last, head).reshape(-1)


# ------------------------------------------------------ multi-head latent attention
def selection_csr(selection, count):
    """per-token key lists (None = dense) as (start, count, keys) arrays with
    count UINT32_MAX marking a dense token"""
    starts, counts, keys = [], [], []
    for t in range(count):
        sel = None if selection is None or t >= len(selection) else selection[t]
        starts.append(len(keys))
        if sel is None:
            counts.append(0xFFFFFFFF)
        else:
            counts.append(len(sel))
            keys.extend(int(k) for k in sel)
    return (np.array(starts, np.uint32), np.array(counts, np.uint32),
            np.array(keys if keys else [0], np.uint32))


def latent_attention(q, latent, wkv, start_pos, heads, nope_dim, v_dim, scale, selection=None):
    """latentAttentionMixer's attention restated (LocalModel.hpp:3118-3158):
    q [count][heads][nope_dim], latent [positions][C], wkv [heads*(nope+v)][C];
    selection: None, or per token None (dense) / a sorted key list"""
    q = np.ascontiguousarray(q, np.float32)
    latent = np.ascontiguousarray(latent, np.float32)
    wkv = np.ascontiguousarray(wkv, np.float32)
    count = q.shape[0]
    C = latent.shape[1]
    out = np.zeros((count, heads, v_dim), np.float32)
    st, ct, ks = selection_csr(selection, count)
    lib().or_latent_attention(q.reshape(-1), latent.reshape(-1), wkv.reshape(-1), st.ctypes.data, ct.ctypes.data,
                              ks.ctypes.data, out.reshape(-1), count, start_pos, heads, nope_dim, v_dim, C,
                              float(scale))
    return out


# ------------------------------------------------------------- sparse-attention indexer
def index_update(k, k_norm, k_norm_bias, ape, keys, gates, pools, start_pos, pool):
    """selectKeys's cache update restated (LocalModel.hpp:2982-3011): the count
    = k.shape[0] new index keys layer-normed into keys[start_pos:], and the
    pools they complete folded into pools; keys and pools are updated in place."""
    k = np.ascontiguousarray(k, np.float32)
    count, di = k.shape
    bias = None if k_norm_bias is None else np.ascontiguousarray(k_norm_bias, np.float32)
    assert keys.dtype == np.float32 and pools.dtype == np.float32 and keys.flags.c_contiguous
    lib().or_index_update(k.reshape(-1), np.ascontiguousarray(k_norm, np.float32),
                          None if bias is None else bias.ctypes.data, np.ascontiguousarray(ape, np.float32),
                          keys.reshape(-1), np.ascontiguousarray(gates, np.float32).reshape(-1), pools.reshape(-1),
                          count, start_pos, di, pool)


def select_keys(q, w, pools, start_pos, heads, dim, pool, top_k, tail=True):
    """selectKeys's choice restated (LocalModel.hpp:3013-3067): q [count][heads*dim],
    w [count][heads]; returns (per-token key lists, None for a token that sees
    every key; the [count][(start_pos + count) // pool] score table)"""
    q = np.ascontiguousarray(q, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    count = q.shape[0]
    budget = top_k // pool
    stride = budget * pool + pool
    st = np.zeros(count, np.uint32)
    ct = np.zeros(count, np.uint32)
    ks = np.zeros(max(1, count * stride), np.uint32)
    max_pools = (start_pos + count) // pool
    sc = np.zeros(max(1, count * max_pools), np.float32)
    lib().or_select_keys(q.reshape(-1), w.reshape(-1), np.ascontiguousarray(pools, np.float32).reshape(-1),
                         st.ctypes.data, ct.ctypes.data, ks.ctypes.data, sc.ctypes.data, count, start_pos, heads,
                         dim, pool, top_k, 1 if tail else 0)
    sel = [None if ct[t] == 0xFFFFFFFF else ks[st[t]:st[t] + ct[t]].copy() for t in range(count)]
    return sel, sc[:count * max_pools].reshape(count, max_pools)
