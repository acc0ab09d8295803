#pragma once

/*
    aigpu_device.hpp - inline C++ wrappers over the attention entry points of
    aigpu_attention.h, in the style of the reference's ai::gpu wrappers
    (include/ai/gpu/Device.hpp:85-160): plain arguments in, a bool out, every
    symbol emitted by the caller's compiler, nothing but C crossing the
    boundary. Device memory is passed as the opaque handle the reference's
    Buffer::ptr() returns (Device.hpp:62-83).

    It can be included before or after the reference's Device.hpp /
    DeviceABI.h: aigpu_attention.h takes the types the two share from
    DeviceABI.h whenever that header is reachable.
*/

#include <cstddef>
#include <cstdint>

#include "aigpu_attention.h"

namespace ai {
namespace gpu {

/* kernels::attention (Kernels.hpp:132-134) on the device: the same arguments,
   fp32, the reference's position-major host K/V [pos][kvHeads][dim] */
inline bool attention(const float* q, const float* keys, const float* values, float* out,
                      size_t count, size_t start, size_t heads, size_t kvHeads,
                      size_t dim, size_t qStride, size_t window = 0) {
    return aigpu_attention(q, keys, values, out, count, start, heads, kvHeads, dim,
                           qStride, window) != 0;
}

/* attentionMixer's norm -> RoPE -> append -> attention for `count` new tokens
   (LocalModel.hpp:2608-2659). q, k, v, out, the norms and the frequencies are
   host fp32; the caches are device handles holding head-major bf16
   [kvHeads][capacity][dim] */
inline bool prefillAttention(const float* q, const float* k, const float* v, float* out,
                             void* keyCache, void* valueCache,
                             const float* qNorm, const float* kNorm, const float* freqs,
                             float eps, float normOffset, size_t rotaryDims,
                             size_t count, size_t start, size_t heads, size_t kvHeads,
                             size_t dim, size_t qStride, size_t window, size_t capacity) {
    AiGpuPrefill a{};
    a.q = q; a.k = k; a.v = v; a.out = out;
    a.keyCache = keyCache; a.valueCache = valueCache;
    a.qNorm = qNorm; a.kNorm = kNorm; a.rotaryFrequencies = freqs;
    a.epsilon = eps; a.normOffset = normOffset; a.rotaryDims = uint32_t(rotaryDims);
    a.inType = AIGPU_F32;
    a.count = count; a.start = start; a.heads = heads; a.kvHeads = kvHeads; a.dim = dim;
    a.qStride = qStride; a.window = window; a.capacity = capacity;
    return aigpu_prefill_attention_host(&a) != 0;
}

/* the same sequence for one decode token (attentionMixer with count = 1) at
   position `position`, which is also the cache's current length */
inline bool decodeAttention(const float* q, const float* k, const float* v, float* out,
                            void* keyCache, void* valueCache,
                            const float* qNorm, const float* kNorm, const float* freqs,
                            float eps, float normOffset, size_t rotaryDims, uint32_t position,
                            size_t heads, size_t kvHeads, size_t dim, size_t qStride,
                            size_t window, size_t capacity) {
    AiGpuDecode a{};
    a.q = q; a.k = k; a.v = v; a.out = out;
    a.keyCache = keyCache; a.valueCache = valueCache;
    a.positions = &position; a.maxPosition = position;
    a.qNorm = qNorm; a.kNorm = kNorm; a.rotaryFrequencies = freqs;
    a.epsilon = eps; a.normOffset = normOffset; a.rotaryDims = uint32_t(rotaryDims);
    a.inType = AIGPU_F32;
    a.batch = 1; a.heads = heads; a.kvHeads = kvHeads; a.dim = dim; a.qStride = qStride;
    a.window = window; a.capacity = capacity;
    return aigpu_decode_attention_host(&a) != 0;
}

/* the token loop of gatedDeltaNetMixer (LocalModel.hpp:2802-2830) over
   `count` tokens at once: q,k [count][kHeads][KD], v [count][vHeads][VD],
   raw gates a,b [count][vHeads]; state [vHeads][KD][VD] updated in place */
inline bool gatedDeltaRule(const float* q, const float* k, const float* v,
                           const float* a, const float* b, const float* aLog, const float* dtBias,
                           float* state, float* out, size_t count, size_t kHeads, size_t vHeads,
                           size_t KD, size_t VD) {
    AiGpuDeltaRule r{};
    r.q = q; r.k = k; r.v = v; r.a = a; r.b = b; r.aLog = aLog; r.dtBias = dtBias;
    r.state = state; r.out = out; r.inType = AIGPU_F32; r.normalize = 1; r.chunk = 64;
    r.count = count; r.keyHeads = kHeads; r.valueHeads = vHeads; r.keyDim = KD; r.valueDim = VD;
    return aigpu_gated_delta_rule_host(&r) != 0;
}

} // namespace gpu
} // namespace ai
