"""aigpu - Python binding of the MI355X attention backend's C ABI
(include/aigpu_attention.h), loaded from the in-tree libaigpu.so.

The binding is thin on purpose: every call goes through an extern "C" entry
point; PyTorch only provides device memory and the stream. Loading fails
loudly when the HIP library is missing - there is no CPU fallback here.

Host forms (numpy in, numpy out) mirror the reference's CPU call sites:
    attention(...)          kernels::attention (Kernels.hpp:132-134)
Device forms (torch tensors on the GPU):
    attention_device(...)   fp32 attention over any KV layout
    prefill(...)            attentionMixer norm -> RoPE -> append -> attention
    decode(...)             batched ragged decode with norm/RoPE on load
    gated_delta_rule(...)   gatedDeltaNetMixer recurrence (chunked scan)
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "libaigpu.so")
STUB = os.path.join(HERE, "libaigpu_stub.so")

F32, BF16 = 0, 1

_vp, _u32, _u64, _f32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_float


class AiGpuCounters(C.Structure):
    _fields_ = [("launches", _u64), ("hostToDeviceBytes", _u64), ("deviceToHostBytes", _u64),
                ("kernelSeconds", C.c_double), ("transferSeconds", C.c_double)]


class AiGpuAttention(C.Structure):
    _fields_ = [("q", _vp), ("keys", _vp), ("values", _vp), ("out", _vp),
                ("qType", _u32), ("kvType", _u32),
                ("count", _u64), ("start", _u64), ("heads", _u64), ("kvHeads", _u64),
                ("dim", _u64), ("qStride", _u64), ("window", _u64),
                ("posStride", _u64), ("headStride", _u64), ("stream", _vp)]


class AiGpuPrefill(C.Structure):
    _fields_ = [("q", _vp), ("k", _vp), ("v", _vp), ("out", _vp),
                ("keyCache", _vp), ("valueCache", _vp),
                ("qNorm", _vp), ("kNorm", _vp), ("rotaryFrequencies", _vp),
                ("epsilon", _f32), ("normOffset", _f32), ("rotaryDims", _u32), ("inType", _u32),
                ("outputGate", _u32), ("reserved", _u32),
                ("count", _u64), ("start", _u64), ("heads", _u64), ("kvHeads", _u64),
                ("dim", _u64), ("qStride", _u64), ("window", _u64), ("capacity", _u64),
                ("stream", _vp)]


class AiGpuDecode(C.Structure):
    _fields_ = [("q", _vp), ("k", _vp), ("v", _vp), ("out", _vp),
                ("keyCache", _vp), ("valueCache", _vp), ("positions", _vp),
                ("qNorm", _vp), ("kNorm", _vp), ("rotaryFrequencies", _vp),
                ("epsilon", _f32), ("normOffset", _f32), ("rotaryDims", _u32), ("inType", _u32),
                ("maxPosition", _u32), ("outputGate", _u32),
                ("batch", _u64), ("heads", _u64), ("kvHeads", _u64), ("dim", _u64),
                ("qStride", _u64), ("window", _u64), ("capacity", _u64), ("batchStride", _u64),
                ("stream", _vp)]


class AiGpuDeltaRule(C.Structure):
    _fields_ = [("q", _vp), ("k", _vp), ("v", _vp), ("g", _vp), ("beta", _vp),
                ("a", _vp), ("b", _vp), ("aLog", _vp), ("dtBias", _vp),
                ("state", _vp), ("out", _vp),
                ("inType", _u32), ("normalize", _u32), ("chunk", _u32), ("reserved", _u32),
                ("count", _u64), ("keyHeads", _u64), ("valueHeads", _u64), ("keyDim", _u64),
                ("valueDim", _u64), ("stream", _vp)]


class AiGpuKda(C.Structure):
    _fields_ = [("q", _vp), ("k", _vp), ("v", _vp), ("g", _vp), ("beta", _vp),
                ("f", _vp), ("b", _vp), ("aLog", _vp), ("dtBias", _vp), ("lowerBound", _f32), ("safeGate", _u32),
                ("state", _vp), ("out", _vp), ("inType", _u32), ("normalize", _u32),
                ("count", _u64), ("keyHeads", _u64), ("valueHeads", _u64), ("keyDim", _u64),
                ("valueDim", _u64), ("stream", _vp)]


class AiGpuMatmul(C.Structure):
    _fields_ = [("a", _vp), ("b", _vp), ("scales", _vp), ("bias", _vp), ("c", _vp), ("type", _u32),
                ("accumulate", _u32), ("m", _u64), ("k", _u64), ("n", _u64), ("ldc", _u64), ("stream", _vp)]


class AiGpuGdnConv(C.Structure):
    _fields_ = [("in_", _vp), ("ba", _vp), ("kernel", _vp), ("window", _vp), ("q", _vp), ("k", _vp),
                ("v", _vp), ("z", _vp), ("a", _vp), ("b", _vp),
                ("inType", _u32), ("outType", _u32), ("fused", _u32), ("reserved", _u32),
                ("count", _u64), ("keyHeads", _u64), ("valueHeads", _u64), ("keyDim", _u64),
                ("valueDim", _u64), ("kernelSize", _u64), ("stream", _vp)]


class AiGpuGdnGatedNorm(C.Structure):
    _fields_ = [("x", _vp), ("z", _vp), ("gamma", _vp), ("out", _vp), ("epsilon", C.c_float),
                ("zType", _u32), ("outType", _u32), ("gateKind", _u32),
                ("count", _u64), ("valueHeads", _u64), ("valueDim", _u64), ("stream", _vp)]


# every symbol include/aigpu_attention.h declares, with its signature
SIGNATURES = {
    "aigpu_available": (C.c_int, []),
    "aigpu_device_name": (C.c_char_p, []),
    "aigpu_last_error": (C.c_char_p, []),
    "aigpu_total_memory": (_u64, []),
    "aigpu_free_memory": (_u64, []),
    "aigpu_allocated_bytes": (_u64, []),
    "aigpu_upload": (_vp, [_vp, _u64]),
    "aigpu_release": (None, [_vp, _u64]),
    "aigpu_download": (C.c_int, [_vp, _vp, _u64]),
    "aigpu_synchronize": (None, []),
    "aigpu_counters": (None, [C.POINTER(AiGpuCounters)]),
    "aigpu_reset_counters": (None, []),
    "aigpu_allocate": (_vp, [_u64]),
    "aigpu_write": (C.c_int, [_vp, _u64, _vp, _u64]),
    "aigpu_attention": (C.c_int, [_vp, _vp, _vp, _vp] + [_u64] * 7),
    "aigpu_attention_device": (C.c_int, [C.POINTER(AiGpuAttention)]),
    "aigpu_prefill_attention": (C.c_int, [C.POINTER(AiGpuPrefill)]),
    "aigpu_prefill_attention_host": (C.c_int, [C.POINTER(AiGpuPrefill)]),
    "aigpu_copy_device": (C.c_int, [_vp, _vp, _u64, _vp]),
    "aigpu_range_ticket": (_u64, []),
    "aigpu_range_status": (C.c_int, [C.POINTER(_u64)]),
    "aigpu_decode_attention": (C.c_int, [C.POINTER(AiGpuDecode)]),
    "aigpu_decode_attention_host": (C.c_int, [C.POINTER(AiGpuDecode)]),
    "aigpu_decode_attention_static": (C.c_int, [C.POINTER(AiGpuDecode)]),
    "aigpu_gdn_conv": (C.c_int, [C.POINTER(AiGpuGdnConv)]),
    "aigpu_kda_rule": (C.c_int, [C.POINTER(AiGpuKda)]),
    "aigpu_matmul_nt": (None, [_vp, _vp, _vp, _u64, _u64, _u64]),
    "aigpu_matmul_nt_bf16": (None, [_vp, _vp, _vp, _u64, _u64, _u64]),
    "aigpu_matmul_nt_q8": (None, [_vp, _vp, _vp, _vp, _u64, _u64, _u64]),
    "aigpu_matmul_nt_q4": (None, [_vp, _vp, _vp, _vp, _u64, _u64, _u64]),
    "aigpu_matmul_device": (C.c_int, [C.POINTER(AiGpuMatmul)]),
    "aigpu_gdn_gated_norm": (C.c_int, [C.POINTER(AiGpuGdnGatedNorm)]),
    "aigpu_gated_delta_rule": (C.c_int, [C.POINTER(AiGpuDeltaRule)]),
    "aigpu_gated_delta_rule_host": (C.c_int, [C.POINTER(AiGpuDeltaRule)]),
    "aigpu_profile": (None, [C.c_int]),
    "aigpu_profile_read": (C.c_int, [C.c_char_p, C.POINTER(C.c_double), C.POINTER(_u64)]),
    "aigpu_profile_reset": (None, []),
}


def load_library(path):
    """Loads a backend (.so) and declares every ABI symbol on it.

    PyTorch ships its own libamdhip64.so.7 under the same soname as ROCm's;
    whichever is loaded first serves the whole process. torch is imported
    first (when installed) so that both sides always share torch's runtime."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            raise ImportError(f"HIP backend not built: {LIBRARY} is missing "
                              "(run python math-utils_amd/build.py)")
        _lib = load_library(LIBRARY)
    return _lib


class AiGpuError(RuntimeError):
    pass


def _check(ok):
    if not ok:
        raise AiGpuError(last_error())


def available():
    return bool(lib().aigpu_available())


def device_name():
    return lib().aigpu_device_name().decode()


def last_error():
    return lib().aigpu_last_error().decode()


def require():
    """Raises unless a gfx950 device is usable: the product has no CPU path."""
    if not available():
        raise AiGpuError("no usable gfx950 device: " + last_error())


def counters():
    c = AiGpuCounters()
    lib().aigpu_counters(C.byref(c))
    return {k: getattr(c, k) for k, _ in AiGpuCounters._fields_}


def profile(enable=True):
    lib().aigpu_profile(1 if enable else 0)


def profile_reset():
    lib().aigpu_profile_reset()


def profile_read(kernel=None):
    """(total milliseconds, launches) of kernels whose name contains `kernel`."""
    ms, n = C.c_double(), _u64()
    lib().aigpu_profile_read(None if kernel is None else kernel.encode(), C.byref(ms), C.byref(n))
    return ms.value, n.value


# ------------------------------------------------------------------ helpers
def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is not None:
        return C.c_void_p(stream)
    import torch
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dtype_tag(t):
    import torch
    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.bfloat16:
        return BF16
    raise TypeError(f"unsupported dtype {t.dtype}: float32 or bfloat16")


def _need(t, name, device=True):
    import torch
    if t is None:
        return
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if device and not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


# ---------------------------------------------------------------- 1. host
def attention(q, keys, values, count, start, heads, kv_heads, dim, q_stride, window=0):
    """Drop-in for kernels::attention: numpy fp32 in the reference's layouts,
    returns out [count][heads][dim]."""
    q = np.ascontiguousarray(q, np.float32)
    keys = np.ascontiguousarray(keys, np.float32)
    values = np.ascontiguousarray(values, np.float32)
    out = np.empty((count, heads, dim), np.float32)
    _check(lib().aigpu_attention(q.ctypes.data, keys.ctypes.data, values.ctypes.data,
                                 out.ctypes.data, count, start, heads, kv_heads, dim, q_stride,
                                 window))
    return out


# -------------------------------------------------------------- 2. device
def attention_device(q, keys, values, out, count, start, heads, kv_heads, dim, q_stride,
                     pos_stride, head_stride, window=0, stream=None):
    for t, n in ((q, "q"), (keys, "keys"), (values, "values"), (out, "out")):
        _need(t, n)
    a = AiGpuAttention(q=_ptr(q), keys=_ptr(keys), values=_ptr(values), out=_ptr(out),
                       qType=_dtype_tag(q), kvType=_dtype_tag(keys), count=count, start=start,
                       heads=heads, kvHeads=kv_heads, dim=dim, qStride=q_stride, window=window,
                       posStride=pos_stride, headStride=head_stride, stream=_stream(stream))
    _check(lib().aigpu_attention_device(C.byref(a)))
    return out


def copy_device(dst, src, nbytes=None, stream=None):
    """aigpu_copy_device: nbytes (default: all of src) from GPU tensor src to
    GPU tensor dst with the streaming copy kernel; asynchronous"""
    for t, n in ((dst, "dst"), (src, "src")):
        _need(t, n)
    nbytes = src.numel() * src.element_size() if nbytes is None else nbytes
    if nbytes > dst.numel() * dst.element_size():
        raise ValueError("dst is smaller than the copy")
    _check(lib().aigpu_copy_device(_ptr(dst), _ptr(src), nbytes, _stream(stream)))
    return dst


def range_ticket():
    """the ticket of the latest prefill call (aigpu_range_ticket)"""
    return int(lib().aigpu_range_ticket())


def check_range():
    """waits for the device (aigpu_range_status); raises AiGpuError, with the
    earliest offending call's ticket as .ticket, when a prefill call since the
    last check met a value outside fp16's range"""
    t = _u64(0)
    if not lib().aigpu_range_status(C.byref(t)):
        err = AiGpuError(last_error())
        err.ticket = t.value
        raise err


def prefill(q, k, v, out, key_cache, value_cache, start, heads, kv_heads, dim, q_stride=None,
            q_norm=None, k_norm=None, eps=1e-6, norm_offset=0.0, freqs=None, rotary_dims=0,
            window=0, capacity=None, output_gate=False, stream=None, check=False):
    """Device form of attentionMixer for `count` tokens at positions start..;
    output_gate applies sigmoid of each q row's second half (q_stride >= 2 dim).
    Asynchronous: check=True waits and raises for an fp16 range error
    (check_range)."""
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (out, "out"), (key_cache, "key_cache"),
                 (value_cache, "value_cache"), (q_norm, "q_norm"), (k_norm, "k_norm"),
                 (freqs, "freqs")):
        _need(t, n)
    count = q.shape[0]
    cap = capacity if capacity is not None else key_cache.shape[-2]
    a = AiGpuPrefill(q=_ptr(q), k=_ptr(k), v=_ptr(v), out=_ptr(out), keyCache=_ptr(key_cache),
                     valueCache=_ptr(value_cache), qNorm=_ptr(q_norm), kNorm=_ptr(k_norm),
                     rotaryFrequencies=_ptr(freqs), epsilon=eps, normOffset=norm_offset,
                     rotaryDims=rotary_dims if freqs is not None else 0, inType=_dtype_tag(q),
                     outputGate=1 if output_gate else 0, count=count, start=start, heads=heads, kvHeads=kv_heads, dim=dim,
                     qStride=q_stride or dim, window=window, capacity=cap,
                     stream=_stream(stream))
    _check(lib().aigpu_prefill_attention(C.byref(a)))
    if check:
        check_range()
    return out


def prefill_host(q, k, v, key_cache, value_cache, start, heads, kv_heads, dim, q_stride=None,
                 q_norm=None, k_norm=None, eps=1e-6, norm_offset=0.0, freqs=None, rotary_dims=0,
                 window=0, capacity=None, output_gate=False):
    """Host form (aigpu_prefill_attention_host): q, k, v numpy fp32 arrays
    ([count][heads][q_stride], [count][kv_heads][dim]), the norms and
    frequencies numpy fp32 or None, the caches GPU tensors; returns out
    [count][heads][dim] as numpy. Synchronous: an fp16 range error raises."""
    for t, n in ((key_cache, "key_cache"), (value_cache, "value_cache")):
        _need(t, n)
    arrs = [np.ascontiguousarray(x, np.float32) if x is not None else None
            for x in (q, k, v, q_norm, k_norm, freqs)]
    q, k, v, q_norm, k_norm, freqs = arrs
    count = q.shape[0]
    out = np.zeros((count, heads, dim), np.float32)
    cap = capacity if capacity is not None else key_cache.shape[-2]

    def hp(x):
        return None if x is None else x.ctypes.data

    a = AiGpuPrefill(q=hp(q), k=hp(k), v=hp(v), out=out.ctypes.data, keyCache=_ptr(key_cache),
                     valueCache=_ptr(value_cache), qNorm=hp(q_norm), kNorm=hp(k_norm),
                     rotaryFrequencies=hp(freqs), epsilon=eps, normOffset=norm_offset,
                     rotaryDims=rotary_dims if freqs is not None else 0, inType=F32,
                     outputGate=1 if output_gate else 0, count=count, start=start, heads=heads,
                     kvHeads=kv_heads, dim=dim, qStride=q_stride or dim, window=window, capacity=cap)
    _check(lib().aigpu_prefill_attention_host(C.byref(a)))
    return out


def decode(q, k, v, out, key_cache, value_cache, positions, max_position, heads, kv_heads, dim,
           q_stride=None, q_norm=None, k_norm=None, eps=1e-6, norm_offset=0.0, freqs=None,
           rotary_dims=0, window=0, capacity=None, batch_stride=0, output_gate=False, stream=None):
    """Device form of the batched decode; positions is a uint32/int32 GPU tensor."""
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (out, "out"), (key_cache, "key_cache"),
                 (value_cache, "value_cache"), (positions, "positions"), (q_norm, "q_norm"),
                 (k_norm, "k_norm"), (freqs, "freqs")):
        _need(t, n)
    batch = q.shape[0]
    cap = capacity if capacity is not None else key_cache.shape[-2]
    a = AiGpuDecode(q=_ptr(q), k=_ptr(k), v=_ptr(v), out=_ptr(out), keyCache=_ptr(key_cache),
                    valueCache=_ptr(value_cache), positions=_ptr(positions), qNorm=_ptr(q_norm),
                    kNorm=_ptr(k_norm), rotaryFrequencies=_ptr(freqs), epsilon=eps,
                    normOffset=norm_offset, rotaryDims=rotary_dims if freqs is not None else 0,
                    inType=_dtype_tag(q), maxPosition=max_position, outputGate=1 if output_gate else 0,
                    batch=batch, heads=heads,
                    kvHeads=kv_heads, dim=dim, qStride=q_stride or dim, window=window,
                    capacity=cap, batchStride=batch_stride, stream=_stream(stream))
    _check(lib().aigpu_decode_attention(C.byref(a)))
    return out


def decode_host(q, k, v, key_cache, value_cache, positions, heads, kv_heads, dim, q_stride=None, q_norm=None,
                k_norm=None, eps=1e-6, norm_offset=0.0, freqs=None, rotary_dims=0, window=0, capacity=None,
                batch_stride=0, output_gate=False):
    """Host form (aigpu_decode_attention_host): q [batch][heads][qStride], k,
    v [batch][kvHeads][dim] as numpy fp32 arrays or bf16 bit patterns
    (uint16), positions numpy uint32, norms and frequencies numpy fp32; the
    caches stay device tensors. Returns out [batch][heads][dim] fp32."""
    import numpy as np

    def host(x, dtype=np.float32):
        return None if x is None else np.ascontiguousarray(x, dtype=dtype)

    def addr(x):
        return None if x is None else C.c_void_p(x.ctypes.data)

    for t, n in ((key_cache, "key_cache"), (value_cache, "value_cache")):
        _need(t, n)
    bf16 = np.asarray(q).dtype == np.uint16
    in_type = np.uint16 if bf16 else np.float32
    q, k, v = host(q, in_type), host(k, in_type), host(v, in_type)
    positions = host(positions, np.uint32)
    q_norm, k_norm, freqs = host(q_norm), host(k_norm), host(freqs)
    batch = q.shape[0]
    out = np.empty((batch, heads, dim), np.float32)
    cap = capacity if capacity is not None else key_cache.shape[-2]
    a = AiGpuDecode(q=addr(q), k=addr(k), v=addr(v), out=addr(out), keyCache=_ptr(key_cache),
                    valueCache=_ptr(value_cache), positions=addr(positions), qNorm=addr(q_norm), kNorm=addr(k_norm),
                    rotaryFrequencies=addr(freqs), epsilon=eps, normOffset=norm_offset,
                    rotaryDims=rotary_dims if freqs is not None else 0, inType=BF16 if bf16 else F32,
                    maxPosition=int(positions.max()), outputGate=1 if output_gate else 0, batch=batch, heads=heads,
                    kvHeads=kv_heads, dim=dim, qStride=q_stride or dim, window=window, capacity=cap,
                    batchStride=batch_stride, stream=None)
    _check(lib().aigpu_decode_attention_host(C.byref(a)))
    return out


def gated_delta_rule(q, k, v, state, out, g=None, beta=None, a=None, b=None, a_log=None,
                     dt_bias=None, normalize=True, stream=None):
    """Device form of the gatedDeltaNetMixer recurrence; state updated in place."""
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (state, "state"), (out, "out"), (g, "g"),
                 (beta, "beta"), (a, "a"), (b, "b"), (a_log, "a_log"), (dt_bias, "dt_bias")):
        _need(t, n)
    count, key_heads, key_dim = q.shape
    _, value_heads, value_dim = v.shape
    args = AiGpuDeltaRule(q=_ptr(q), k=_ptr(k), v=_ptr(v), g=_ptr(g), beta=_ptr(beta),
                          a=_ptr(a), b=_ptr(b), aLog=_ptr(a_log), dtBias=_ptr(dt_bias),
                          state=_ptr(state), out=_ptr(out), inType=_dtype_tag(q),
                          normalize=1 if normalize else 0, chunk=64, count=count,
                          keyHeads=key_heads, valueHeads=value_heads, keyDim=key_dim,
                          valueDim=value_dim, stream=_stream(stream))
    _check(lib().aigpu_gated_delta_rule(C.byref(args)))
    return out


def gated_delta_rule_host(q, k, v, state, g=None, beta=None, a=None, b=None, a_log=None, dt_bias=None,
                          normalize=True):
    """Host form (aigpu_gated_delta_rule_host, the entry the reference's C++
    mixer binds): q, k [count][keyHeads][keyDim] and v [count][valueHeads]
    [valueDim] as numpy fp32 arrays or bf16 bit patterns (uint16); gates fp32;
    state fp32 [valueHeads][keyDim][valueDim], updated in place. Returns out
    [count][valueHeads][valueDim] fp32."""
    import numpy as np

    def host(x, dtype=np.float32):
        return None if x is None else np.ascontiguousarray(x, dtype=dtype)

    def addr(x):
        return None if x is None else C.c_void_p(x.ctypes.data)

    bf16 = np.asarray(q).dtype == np.uint16
    in_type = np.uint16 if bf16 else np.float32
    q, k, v = host(q, in_type), host(k, in_type), host(v, in_type)
    g, beta, a, b, a_log, dt_bias = (host(x) for x in (g, beta, a, b, a_log, dt_bias))
    if state.dtype != np.float32 or not state.flags["C_CONTIGUOUS"]:
        raise TypeError("state must be a C-contiguous float32 array (updated in place)")
    count, key_heads, key_dim = q.shape
    _, value_heads, value_dim = v.shape
    out = np.empty((count, value_heads, value_dim), np.float32)
    args = AiGpuDeltaRule(q=addr(q), k=addr(k), v=addr(v), g=addr(g), beta=addr(beta), a=addr(a), b=addr(b),
                          aLog=addr(a_log), dtBias=addr(dt_bias), state=addr(state), out=addr(out),
                          inType=BF16 if bf16 else F32, normalize=1 if normalize else 0, chunk=64, count=count,
                          keyHeads=key_heads, valueHeads=value_heads, keyDim=key_dim, valueDim=value_dim,
                          stream=None)
    _check(lib().aigpu_gated_delta_rule_host(C.byref(args)))
    return out


def gdn_conv(x, kernel, window, q, k, v, key_heads, value_heads, key_dim, value_dim, ba=None, z=None,
             a=None, b=None, stream=None):
    """Device form of gatedDeltaNetMixer's de-interleave + causalConvolution:
    x [count][CW] (plain) or [count][key_heads][2 KD + 2 G VD] with ba (fused);
    writes q, k, v (and z, a, b when fused); window [K-1][CW] fp32 updated."""
    fused = ba is not None
    for t, n in ((x, "x"), (kernel, "kernel"), (window, "window"), (q, "q"), (k, "k"), (v, "v"),
                 (ba, "ba"), (z, "z"), (a, "a"), (b, "b")):
        _need(t, n)
    args = AiGpuGdnConv(in_=_ptr(x), ba=_ptr(ba), kernel=_ptr(kernel), window=_ptr(window), q=_ptr(q),
                        k=_ptr(k), v=_ptr(v), z=_ptr(z), a=_ptr(a), b=_ptr(b), inType=_dtype_tag(x),
                        outType=_dtype_tag(q), fused=1 if fused else 0, count=x.shape[0],
                        keyHeads=key_heads, valueHeads=value_heads, keyDim=key_dim, valueDim=value_dim,
                        kernelSize=kernel.shape[1], stream=_stream(stream))
    _check(lib().aigpu_gdn_conv(C.byref(args)))
    return q, k, v


def gdn_gated_norm(x, z, gamma, out, eps=1e-6, gate="silu", stream=None):
    """Device form of the gated norm after the recurrence: x, z, out
    [count][value_heads][value_dim]; gate "silu" (Gated DeltaNet) or
    "sigmoid" (Kimi Delta Attention)."""
    if gate not in ("silu", "sigmoid"):
        raise ValueError("gate must be 'silu' or 'sigmoid'")
    for t, n in ((x, "x"), (z, "z"), (gamma, "gamma"), (out, "out")):
        _need(t, n)
    count, value_heads, value_dim = x.shape
    args = AiGpuGdnGatedNorm(x=_ptr(x), z=_ptr(z), gamma=_ptr(gamma), out=_ptr(out), epsilon=eps,
                             zType=_dtype_tag(z), outType=_dtype_tag(out),
                             gateKind=1 if gate == "sigmoid" else 0, count=count,
                             valueHeads=value_heads, valueDim=value_dim, stream=_stream(stream))
    _check(lib().aigpu_gdn_gated_norm(C.byref(args)))
    return out


def kda_rule(q, k, v, g, beta, state, out, normalize=True, f=None, b=None, a_log=None, dt_bias=None,
             safe_gate=False, lower_bound=-5.0, stream=None):
    """Device form of Kimi Delta Attention's recurrence: g is the log decay per
    key channel [count][value_heads][key_dim] (or g, beta None and the raw
    gates f, b, a_log, dt_bias given); state updated in place."""
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (g, "g"), (beta, "beta"), (f, "f"), (b, "b"), (a_log, "a_log"),
                 (dt_bias, "dt_bias"), (state, "state"), (out, "out")):
        _need(t, n)
    count, key_heads, key_dim = q.shape
    _, value_heads, value_dim = v.shape
    args = AiGpuKda(q=_ptr(q), k=_ptr(k), v=_ptr(v), g=_ptr(g), beta=_ptr(beta), f=_ptr(f), b=_ptr(b),
                    aLog=_ptr(a_log), dtBias=_ptr(dt_bias), lowerBound=lower_bound,
                    safeGate=1 if safe_gate else 0, state=_ptr(state),
                    out=_ptr(out), inType=_dtype_tag(q), normalize=1 if normalize else 0, count=count,
                    keyHeads=key_heads, valueHeads=value_heads, keyDim=key_dim, valueDim=value_dim,
                    stream=_stream(stream))
    _check(lib().aigpu_kda_rule(C.byref(args)))
    return out


WEIGHT_TYPES = {"f32": 0, "bf16": 1, "q8": 2, "q4": 3}


def matmul(a, b, out, kind, scales=None, bias=None, accumulate=False, stream=None):
    """Device form of the projection: out[m][n] (+)= a[m][k] . w[n][k]^T (+ bias).
    a, out fp32 torch tensors; b the weight bytes as a torch tensor (fp32,
    bf16, int8 codes, or uint8 packed 4-bit); kind one of WEIGHT_TYPES."""
    for t, n in ((a, "a"), (b, "b"), (scales, "scales"), (bias, "bias")):
        _need(t, n)
    if not out.is_cuda or out.dim() != 2 or out.stride(1) != 1:
        raise ValueError("out must be a GPU tensor with unit column stride")
    m, k = a.shape
    n = out.shape[1]
    args = AiGpuMatmul(a=_ptr(a), b=_ptr(b), scales=_ptr(scales), bias=_ptr(bias), c=_ptr(out),
                       type=WEIGHT_TYPES[kind], accumulate=1 if accumulate else 0, m=m, k=k, n=n,
                       ldc=out.stride(0), stream=_stream(stream))
    _check(lib().aigpu_matmul_device(C.byref(args)))
    return out


def matmul_host(a, b_device, kind, n, scales_device=None):
    """The reference's host-staged aigpu_matmul_nt*: a numpy fp32 [m][k]; the
    weight (and scales) as device pointers (ints) from upload(); returns c."""
    import numpy as np
    a = np.ascontiguousarray(a, np.float32)
    m, k = a.shape
    c = np.zeros((m, n), np.float32)
    L = lib()
    if kind == "f32":
        L.aigpu_matmul_nt(a.ctypes.data, b_device, c.ctypes.data, m, k, n)
    elif kind == "bf16":
        L.aigpu_matmul_nt_bf16(a.ctypes.data, b_device, c.ctypes.data, m, k, n)
    elif kind == "q8":
        L.aigpu_matmul_nt_q8(a.ctypes.data, b_device, scales_device, c.ctypes.data, m, k, n)
    else:
        L.aigpu_matmul_nt_q4(a.ctypes.data, b_device, scales_device, c.ctypes.data, m, k, n)
    err = L.aigpu_last_error()
    if err:   # the host forms return nothing; a failure leaves its reason here
        raise RuntimeError(err.decode() if isinstance(err, bytes) else str(err))
    return c


def upload(array):
    """aigpu_upload of a numpy array's bytes; returns the device pointer (int)"""
    import numpy as np
    a = np.ascontiguousarray(array)
    ptr = lib().aigpu_upload(a.ctypes.data, a.nbytes)
    if not ptr:
        _check(0)
    return ptr


def release(ptr, nbytes):
    lib().aigpu_release(ptr, nbytes)


# ---------------------------------------------------------------- 8. resident decoder
class AiGpuDenseWeight(C.Structure):
    _fields_ = [("codes", _vp), ("scales", _vp), ("type", _u32), ("inDim", _u32), ("outDim", _u32), ("bias", _vp)]


class AiGpuDenseLayer(C.Structure):
    _fields_ = [("q", AiGpuDenseWeight), ("k", AiGpuDenseWeight), ("v", AiGpuDenseWeight),
                ("o", AiGpuDenseWeight), ("gate", AiGpuDenseWeight), ("up", AiGpuDenseWeight),
                ("down", AiGpuDenseWeight), ("inputNorm", _vp), ("postNorm", _vp), ("qNorm", _vp),
                ("kNorm", _vp), ("window", _u32)]


class AiGpuDenseConfig(C.Structure):
    _fields_ = [("hidden", _u32), ("layers", _u32), ("heads", _u32), ("kvHeads", _u32), ("headDim", _u32),
                ("intermediate", _u32), ("capacity", _u32), ("rotaryDims", _u32), ("vocab", _u32),
                ("epsilon", _f32), ("theta", _f32), ("finalNorm", _vp), ("head", AiGpuDenseWeight),
                ("rotaryFrequencies", _vp)]


SIGNATURES.update({
    "aigpu_dense_supported": (C.c_int, []),
    "aigpu_dense_create": (_vp, [C.POINTER(AiGpuDenseConfig), C.POINTER(AiGpuDenseLayer), _vp, _vp, _u32]),
    "aigpu_dense_release": (None, [_vp]),
    "aigpu_dense_decode": (None, [_vp, _vp, _vp, _u32]),
    "aigpu_dense_read_cache": (None, [_vp, _vp, _vp, _u32]),
})


class DenseDecoder:
    """The resident decoder through the reference's own entry points.

    weights: dicts with "ptr" (device pointer of the stored weight, e.g. from
    upload()), "kind", "scales_ptr" (Q8/Q4), "in", "out", "bias" (numpy or
    None). layers: dicts q, k, v, o, gate, up, down (weights), input_norm,
    post_norm, q_norm, k_norm (numpy or None), window. keys / values: per
    layer numpy fp32 [capacity][kv_heads * head_dim], the first `length`
    positions valid."""

    def __init__(self, cfg, layers, head, final_norm, keys, values, length, freqs=None):
        import numpy as np
        keep = []
        L = lib()

        def arr(x):
            if x is None:
                return None
            a = np.ascontiguousarray(x, np.float32)
            keep.append(a)
            return a.ctypes.data

        def w(d):
            return AiGpuDenseWeight(codes=d["ptr"], scales=d.get("scales_ptr"), type=WEIGHT_TYPES[d["kind"]],
                                    inDim=d["in"], outDim=d["out"], bias=arr(d.get("bias")))

        self.cfg = cfg
        self.nlayers = len(layers)
        larr = (AiGpuDenseLayer * len(layers))()
        for i, l in enumerate(layers):
            larr[i] = AiGpuDenseLayer(q=w(l["q"]), k=w(l["k"]), v=w(l["v"]), o=w(l["o"]), gate=w(l["gate"]),
                                      up=w(l["up"]), down=w(l["down"]), inputNorm=arr(l["input_norm"]),
                                      postNorm=arr(l["post_norm"]), qNorm=arr(l.get("q_norm")),
                                      kNorm=arr(l.get("k_norm")), window=l.get("window", 0))
        c = AiGpuDenseConfig(hidden=cfg["hidden"], layers=len(layers), heads=cfg["heads"], kvHeads=cfg["kv_heads"],
                             headDim=cfg["head_dim"], intermediate=cfg["intermediate"], capacity=cfg["capacity"],
                             rotaryDims=cfg["rotary_dims"], vocab=cfg["vocab"], epsilon=cfg["eps"],
                             theta=cfg["theta"], finalNorm=arr(final_norm), head=w(head),
                             rotaryFrequencies=arr(freqs))
        kp = (_vp * len(layers))(*[arr(k) for k in keys])
        vp = (_vp * len(layers))(*[arr(v) for v in values])
        self.handle = L.aigpu_dense_create(C.byref(c), larr, C.cast(kp, _vp), C.cast(vp, _vp), length)
        del keep
        if not self.handle:
            _check(0)

    def decode(self, embedding, position):
        import numpy as np
        e = np.ascontiguousarray(embedding, np.float32)
        logits = np.zeros(self.cfg["vocab"], np.float32)
        L = lib()
        L.aigpu_dense_decode(self.handle, e.ctypes.data, logits.ctypes.data, position)
        err = L.aigpu_last_error()
        if err:
            raise RuntimeError(err.decode())
        return logits

    def read_cache(self, length):
        import numpy as np
        kvw = self.cfg["kv_heads"] * self.cfg["head_dim"]
        keys = [np.zeros((length, kvw), np.float32) for _ in range(self.nlayers)]
        values = [np.zeros((length, kvw), np.float32) for _ in range(self.nlayers)]
        kp = (_vp * self.nlayers)(*[k.ctypes.data for k in keys])
        vp = (_vp * self.nlayers)(*[v.ctypes.data for v in values])
        L = lib()
        L.aigpu_dense_read_cache(self.handle, C.cast(kp, _vp), C.cast(vp, _vp), length)
        err = L.aigpu_last_error()
        if err:
            raise RuntimeError(err.decode())
        return keys, values

    def close(self):
        if self.handle:
            lib().aigpu_dense_release(self.handle)
            self.handle = None



# ---------------------------------------------------------------- 5c. latent attention
class AiGpuLatentAttention(C.Structure):
    _fields_ = [("q", _vp), ("latent", _vp), ("kvB", _vp), ("kvBType", _u32), ("reserved", _u32),
                ("selStart", _vp), ("selCount", _vp), ("selKeys", _vp), ("out", _vp), ("scale", _f32),
                ("count", _u64), ("startPos", _u64), ("heads", _u64), ("nopeDim", _u64), ("vDim", _u64),
                ("kvLoraRank", _u64), ("stream", _vp)]


SIGNATURES["aigpu_latent_attention"] = (C.c_int, [C.POINTER(AiGpuLatentAttention)])


def latent_attention(q, latent, kv_b, out, start_pos, scale, sel_start=None, sel_count=None, sel_keys=None,
                     stream=None):
    """Device form of latentAttentionMixer's attention: q [count][heads][nope],
    latent [positions][rank], kv_b [heads*(nope+v)][rank] (fp32 or bf16), out
    [count][heads][v]; the optional selection as int32 tensors (count
    0xFFFFFFFF marks a dense token)."""
    for t, n in ((q, "q"), (latent, "latent"), (kv_b, "kv_b"), (out, "out"), (sel_start, "sel_start"),
                 (sel_count, "sel_count"), (sel_keys, "sel_keys")):
        _need(t, n)
    count, heads, nope = q.shape
    vdim = out.shape[2]
    args = AiGpuLatentAttention(q=_ptr(q), latent=_ptr(latent), kvB=_ptr(kv_b), kvBType=_dtype_tag(kv_b),
                                selStart=_ptr(sel_start), selCount=_ptr(sel_count), selKeys=_ptr(sel_keys),
                                out=_ptr(out), scale=scale, count=count, startPos=start_pos, heads=heads,
                                nopeDim=nope, vDim=vdim, kvLoraRank=latent.shape[1], stream=_stream(stream))
    _check(lib().aigpu_latent_attention(C.byref(args)))
    return out


class AiGpuPrefillMixer(C.Structure):
    _fields_ = [("x", _vp), ("q", AiGpuDenseWeight), ("k", AiGpuDenseWeight), ("v", AiGpuDenseWeight),
                ("o", AiGpuDenseWeight), ("out", _vp), ("keyCache", _vp), ("valueCache", _vp), ("qNorm", _vp),
                ("kNorm", _vp), ("rotaryFrequencies", _vp), ("epsilon", _f32), ("normOffset", _f32),
                ("rotaryDims", _u32), ("outputGate", _u32), ("accumulate", _u32), ("reserved", _u32),
                ("count", _u64), ("start", _u64), ("hidden", _u64), ("heads", _u64), ("kvHeads", _u64),
                ("dim", _u64), ("window", _u64), ("capacity", _u64), ("stream", _vp)]


SIGNATURES["aigpu_prefill_mixer"] = (C.c_int, [C.POINTER(AiGpuPrefillMixer)])


def prefill_mixer(x, weights, out, key_cache, value_cache, start, heads, kv_heads, dim, q_norm=None,
                  k_norm=None, eps=1e-6, norm_offset=0.0, freqs=None, rotary_dims=0, window=0, capacity=None,
                  output_gate=False, accumulate=False, stream=None, check=False):
    """attentionMixer for the x.shape[0] tokens at positions start..: x [count][hidden]
    fp32; weights maps "q", "k", "v", "o" to dicts with "w" (the stored weight
    as a GPU tensor: fp32, bf16, int8 codes or packed 4-bit), "kind" (a
    WEIGHT_TYPES key), "out" (rows) and optional "scales" / "bias" GPU tensors;
    out [count][hidden] fp32 (+= with accumulate); the head-major bf16 caches
    gain positions start .. start + count - 1. Asynchronous: check=True waits
    and raises for an fp16 range error (check_range)."""
    for t, n in ((x, "x"), (out, "out"), (key_cache, "key_cache"), (value_cache, "value_cache"),
                 (q_norm, "q_norm"), (k_norm, "k_norm"), (freqs, "freqs")):
        _need(t, n)
    count, hidden = x.shape

    def w(d):
        for t, n in ((d["w"], "w"), (d.get("scales"), "scales"), (d.get("bias"), "bias")):
            _need(t, n)
        return AiGpuDenseWeight(codes=_ptr(d["w"]), scales=_ptr(d.get("scales")), type=WEIGHT_TYPES[d["kind"]],
                                inDim=d.get("in", hidden), outDim=d["out"], bias=_ptr(d.get("bias")))

    cap = capacity if capacity is not None else key_cache.shape[-2]
    args = AiGpuPrefillMixer(x=_ptr(x), q=w(weights["q"]), k=w(weights["k"]), v=w(weights["v"]),
                             o=w(weights["o"]), out=_ptr(out), keyCache=_ptr(key_cache),
                             valueCache=_ptr(value_cache), qNorm=_ptr(q_norm), kNorm=_ptr(k_norm),
                             rotaryFrequencies=_ptr(freqs), epsilon=eps, normOffset=norm_offset,
                             rotaryDims=rotary_dims if freqs is not None else 0,
                             outputGate=1 if output_gate else 0, accumulate=1 if accumulate else 0,
                             count=count, start=start, hidden=hidden, heads=heads, kvHeads=kv_heads, dim=dim,
                             window=window, capacity=cap, stream=_stream(stream))
    _check(lib().aigpu_prefill_mixer(C.byref(args)))
    if check:
        check_range()
    return out


class AiGpuSelectKeys(C.Structure):
    _fields_ = [("h", _vp), ("qResid", _vp), ("idxK", AiGpuDenseWeight), ("idxGate", AiGpuDenseWeight),
                ("idxQB", AiGpuDenseWeight), ("idxWeights", AiGpuDenseWeight), ("kNorm", _vp), ("kNormBias", _vp),
                ("ape", _vp), ("indexKeys", _vp), ("indexGates", _vp), ("poolKeys", _vp), ("selStart", _vp),
                ("selCount", _vp), ("selKeys", _vp), ("scores", _vp), ("indexTail", _u32), ("reserved", _u32),
                ("count", _u64), ("startPos", _u64), ("hidden", _u64), ("qRank", _u64), ("heads", _u64),
                ("dim", _u64), ("topK", _u64), ("pool", _u64), ("capacity", _u64), ("stream", _vp)]


SIGNATURES["aigpu_select_keys"] = (C.c_int, [C.POINTER(AiGpuSelectKeys)])


def select_keys(h, q_resid, weights, k_norm, k_norm_bias, ape, index_keys, index_gates, pool_keys, sel_start,
                sel_count, sel_keys, start_pos, heads, dim, top_k, pool, tail=True, scores=None, stream=None):
    """selectKeys on the device for the h.shape[0] tokens at start_pos: weights
    maps "k", "gate", "q", "w" (idxK, idxGate, idxQB, idxWeights) to dicts as
    prefill_mixer takes; the index key / gate / pool caches are updated in
    place; sel_start / sel_count / sel_keys (int32 GPU tensors) receive the
    selection aigpu_latent_attention takes."""
    for t, n in ((h, "h"), (q_resid, "q_resid"), (k_norm, "k_norm"), (k_norm_bias, "k_norm_bias"), (ape, "ape"),
                 (index_keys, "index_keys"), (index_gates, "index_gates"), (pool_keys, "pool_keys"),
                 (sel_start, "sel_start"), (sel_count, "sel_count"), (sel_keys, "sel_keys"), (scores, "scores")):
        _need(t, n)
    count, hidden = h.shape

    def w(d, k_in):
        for t, n in ((d["w"], "w"), (d.get("scales"), "scales"), (d.get("bias"), "bias")):
            _need(t, n)
        return AiGpuDenseWeight(codes=_ptr(d["w"]), scales=_ptr(d.get("scales")), type=WEIGHT_TYPES[d["kind"]],
                                inDim=d.get("in", k_in), outDim=d["out"], bias=_ptr(d.get("bias")))

    args = AiGpuSelectKeys(h=_ptr(h), qResid=_ptr(q_resid), idxK=w(weights["k"], hidden),
                           idxGate=w(weights["gate"], hidden), idxQB=w(weights["q"], q_resid.shape[1]),
                           idxWeights=w(weights["w"], hidden), kNorm=_ptr(k_norm), kNormBias=_ptr(k_norm_bias),
                           ape=_ptr(ape), indexKeys=_ptr(index_keys), indexGates=_ptr(index_gates),
                           poolKeys=_ptr(pool_keys), selStart=_ptr(sel_start), selCount=_ptr(sel_count),
                           selKeys=_ptr(sel_keys), scores=_ptr(scores), indexTail=1 if tail else 0, count=count,
                           startPos=start_pos, hidden=hidden, qRank=q_resid.shape[1], heads=heads, dim=dim,
                           topK=top_k, pool=pool, capacity=index_keys.shape[0], stream=_stream(stream))
    _check(lib().aigpu_select_keys(C.byref(args)))
