// dense.hip - the resident single-token decoder behind aigpu_dense_*
// (DeviceABI.h:114-157): a dense RMSNorm / RoPE / SwiGLU model (Qwen3,
// Llama) kept on the device between tokens, so one decode step moves only the
// embedding in and the logits out. The reference's HIP backend stubs these
// entry points (Kernels.hip:636-641); LocalModel::residentDecode
// (LocalModel.hpp:3598-3645) is the caller, and the step is LocalModel::
// forward's layer loop for count = 1 (:3705-3799).
//
// Per layer, on one stream:
//   dense_norm_kernel      x -> RMSNorm(x) * inputNorm
//   gemv_kernel x3         q, k, v (+ bias)
//   dense_qk_kernel        per head: q/k RMSNorm, RoPE at the position, and
//                          the k, v rows appended to the fp32 cache
//   dense_attn_kernel      split-K attention: one workgroup per (256
//                          positions, kv head) for all of that kv head's query
//                          heads, so each cached row is read once
//   dense_merge_kernel     the splits' softmax partials combined per head
//   gemv_kernel            x += o . attn
//   dense_norm_kernel      RMSNorm(x) * postNorm
//   gemv_kernel x2, dense_swiglu_kernel, gemv_kernel   x += down . (silu(gate) * up)
// then the final norm and the head. The position is read from device memory
// by every kernel that needs it, so the sequence does not depend on host
// values that change between tokens.
//
// The cache is the reference's own layout, fp32 [capacity][kvHeads * headDim]
// per layer (what aigpu_dense_create copies in and aigpu_dense_read_cache
// copies out).
#include <chrono>
#include <cmath>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "context.hpp"
#include "device.hpp"
#include "kernels.hpp"

namespace aigpu {

namespace {

constexpr int SPLIT = 256;     // positions per attention workgroup
constexpr int MAX_DIM = 256;   // head dim
constexpr int MAX_GROUP = 16;  // query heads per kv head

struct DenseArgs {
    const uint32_t* pos;   // device: the position being decoded
    uint32_t heads, kvHeads, dim, rot, maxSplits, window;
    float eps;
};

/* RMSNorm of one row (rmsNormRow, LocalModel.hpp:1341-1348): out = x *
   1/sqrt(mean(x^2) + eps) * gamma. One workgroup. */
__global__ __launch_bounds__(1024) void dense_norm_kernel(const float* x, const float* gamma, float* out, uint32_t n,
                                                          float eps) {
    __shared__ float part[16];
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) ss = fmaf(x[i], x[i], ss);
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (uint32_t w = 0; w < blockDim.x / 64; ++w) tot += part[w];
    const float inv = 1.0f / sqrtf(tot / float(n) + eps);
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) out[i] = x[i] * inv * gamma[i];
}

/* one wave per head: blocks [0, heads) the query heads (normalised and
   rotated in place), blocks [heads, heads + kvHeads) the key heads
   (normalised, rotated and appended with their value rows) */
__global__ __launch_bounds__(64) void dense_qk_kernel(DenseArgs a, float* q, const float* k, const float* v,
                                                      const float* qNorm, const float* kNorm, const float* freqs,
                                                      float* keys, float* values) {
    __shared__ float row[MAX_DIM];
    const int lane = threadIdx.x;
    const uint32_t b = blockIdx.x, D = a.dim, pos = *a.pos;
    const bool isQ = b < a.heads;
    const uint32_t hh = isQ ? b : b - a.heads;
    const float* src = isQ ? q + size_t(hh) * D : k + size_t(hh) * D;
    for (uint32_t d = lane; d < D; d += WAVE) row[d] = src[d];
    wave_sync();
    norm_rope_row(row, int(D), isQ ? qNorm : kNorm, a.eps, 0.0f, freqs, int(a.rot), pos, lane);
    const size_t kvW = size_t(a.kvHeads) * D;
    if (isQ) {
        for (uint32_t d = lane; d < D; d += WAVE) q[size_t(hh) * D + d] = row[d];
    } else {
        for (uint32_t d = lane; d < D; d += WAVE) {
            keys[size_t(pos) * kvW + size_t(hh) * D + d] = row[d];
            values[size_t(pos) * kvW + size_t(hh) * D + d] = v[size_t(hh) * D + d];
        }
    }
}

/* keys [first(pos), pos] in splits of SPLIT: workgroup (split s, kv head)
   scores its positions for the G query heads of the kv head (lane = position
   in each wave's 64), then accumulates P.V with the lanes on dimensions.
   Each wave leaves a partial record per query head: max, sum, acc[D]. */
__global__ __launch_bounds__(256) void dense_attn_kernel(DenseArgs a, const float* q, const float* keys,
                                                         const float* values, float* partial) {
    __shared__ float qs[MAX_GROUP * MAX_DIM];
    __shared__ float pr[4][MAX_GROUP][WAVE];
    __shared__ float wm[4][MAX_GROUP], wl[4][MAX_GROUP];

    const uint32_t pos = *a.pos;
    const uint32_t first = a.window && pos + 1 > a.window ? pos + 1 - a.window : 0;
    const uint32_t len = pos + 1 - first, splits = (len + SPLIT - 1) / SPLIT;
    const uint32_t s = blockIdx.x, kvh = blockIdx.y;
    if (s >= splits) return;   // whole workgroup leaves before any barrier
    const uint32_t G = a.heads / a.kvHeads, D = a.dim;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const size_t kvW = size_t(a.kvHeads) * D;
    const float scale = 1.0f / sqrtf(float(D));

    for (uint32_t i = tid; i < G * D; i += 256) qs[i] = q[size_t(kvh) * G * D + i];
    __syncthreads();

    const uint32_t j = first + s * SPLIT + 64 * w + lane;
    const bool live = j <= pos && 64 * w + lane < SPLIT;
    float sc[MAX_GROUP];
#pragma unroll
    for (int g = 0; g < MAX_GROUP; ++g) sc[g] = 0.0f;
    if (live) {
        const float* kr = keys + size_t(j) * kvW + size_t(kvh) * D;
        for (uint32_t d = 0; d < D; d += 4) {
            const floatx4 kv4 = *reinterpret_cast<const floatx4*>(kr + d);
#pragma unroll
            for (int g = 0; g < MAX_GROUP; ++g) {
                if (g < int(G)) {
                    const floatx4 q4 = *reinterpret_cast<const floatx4*>(&qs[g * D + d]);
                    sc[g] = fmaf(q4[0], kv4[0], fmaf(q4[1], kv4[1], fmaf(q4[2], kv4[2], fmaf(q4[3], kv4[3], sc[g]))));
                }
            }
        }
    }
    // per wave softmax partials
    constexpr int DPL = MAX_DIM / WAVE;   // dims per lane
    float acc[MAX_GROUP][DPL];
#pragma unroll
    for (int g = 0; g < MAX_GROUP; ++g) {
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[g][e] = 0.0f;
        if (g < int(G)) {
            const float sv = live ? sc[g] * scale : -INFINITY;
            const float m = wave_max(sv);
            const float p = live ? expf(sv - m) : 0.0f;
            const float l = wave_sum(p);
            pr[w][g][lane] = p;
            if (lane == 0) {
                wm[w][g] = m;
                wl[w][g] = l;
            }
        }
    }
    wave_sync();
    const uint32_t jw = first + s * SPLIT + 64 * w;   // this wave's first position
    const uint32_t nw = jw <= pos ? (pos + 1 - jw < 64u ? pos + 1 - jw : 64u) : 0u;
    for (uint32_t jj = 0; jj < nw; ++jj) {
        const float* vr = values + size_t(jw + jj) * kvW + size_t(kvh) * D;
        float vv[DPL];
#pragma unroll
        for (int e = 0; e < DPL; ++e) vv[e] = (lane + 64 * e) < int(D) ? vr[lane + 64 * e] : 0.0f;
#pragma unroll
        for (int g = 0; g < MAX_GROUP; ++g) {
            if (g < int(G)) {
                const float p = pr[w][g][jj];
#pragma unroll
                for (int e = 0; e < DPL; ++e) acc[g][e] = fmaf(p, vv[e], acc[g][e]);
            }
        }
    }
    const size_t rec = size_t(D) + 2;
    for (uint32_t g = 0; g < G; ++g) {
        float* out = partial + ((size_t(kvh) * G + g) * a.maxSplits * 4 + size_t(s) * 4 + w) * rec;
        if (lane == 0) {
            out[0] = wm[w][g];
            out[1] = wl[w][g];
        }
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
            const uint32_t d = lane + 64 * e;
            if (d < D) out[2 + d] = acc[g][e];
        }
    }
}

/* combines the partial records of every (split, wave) of one query head */
__global__ __launch_bounds__(64) void dense_merge_kernel(DenseArgs a, const float* partial, float* attn) {
    const uint32_t h = blockIdx.x, lane = threadIdx.x, D = a.dim;
    const uint32_t pos = *a.pos;
    const uint32_t first = a.window && pos + 1 > a.window ? pos + 1 - a.window : 0;
    const uint32_t len = pos + 1 - first, splits = (len + SPLIT - 1) / SPLIT;
    const size_t rec = size_t(D) + 2;
    const float* base = partial + size_t(h) * a.maxSplits * 4 * rec;
    const uint32_t parts = splits * 4;
    float M = -INFINITY;
    for (uint32_t i = 0; i < parts; ++i) M = fmaxf(M, base[i * rec]);
    float L = 0.0f;
    constexpr int DPL = MAX_DIM / WAVE;
    float acc[DPL] = {};
    for (uint32_t i = 0; i < parts; ++i) {
        const float m = base[i * rec];
        if (m == -INFINITY) continue;
        const float f = expf(m - M);
        L = fmaf(base[i * rec + 1], f, L);
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
            const uint32_t d = lane + 64 * e;
            if (d < D) acc[e] = fmaf(base[i * rec + 2 + d], f, acc[e]);
        }
    }
    const float inv = 1.0f / L;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
        const uint32_t d = lane + 64 * e;
        if (d < D) attn[size_t(h) * D + d] = acc[e] * inv;
    }
}

/* gate = silu(gate) * up (swiglu with no limit, LocalModel.hpp:3282-3288;
   siluOf :1369) */
__global__ __launch_bounds__(256) void dense_swiglu_kernel(float* gate, const float* up, uint32_t n) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) {
        const float g = gate[i];
        gate[i] = g / (1.0f + expf(-g)) * up[i];
    }
}

struct DevWeight {
    const void* codes = nullptr;
    const float* scales = nullptr;
    float* bias = nullptr;   // device copy, or null
    int type = 0;
    uint32_t in = 0, out = 0;
};

struct DevLayer {
    DevWeight q, k, v, o, gate, up, down;
    float *inputNorm = nullptr, *postNorm = nullptr, *qNorm = nullptr, *kNorm = nullptr;
    float *keys = nullptr, *values = nullptr;   // [capacity][kvHeads * headDim]
    uint32_t window = 0;
};

struct DenseModel {
    AiGpuDenseConfig cfg{};
    uint32_t length = 0, maxSplits = 0;
    std::vector<DevLayer> layers;
    DevWeight head;
    float *finalNorm = nullptr, *freqs = nullptr;
    float *x = nullptr, *normed = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr;
    float *gate = nullptr, *up = nullptr, *logits = nullptr, *partial = nullptr;
    uint32_t* pos = nullptr;
    std::vector<void*> owned;
    uint64_t bytes = 0;

    ~DenseModel() {
        for (void* ptr : owned) (void)hipFree(ptr);
        Context::instance().allocated -= bytes;
    }

    /* a device allocation of `count` floats, the first `copy` from `host`,
       the rest zero */
    float* floats(uint64_t count, const float* host = nullptr, uint64_t copy = 0) {
        void* ptr = nullptr;
        const size_t b = size_t(count ? count : 1) * 4;
        if (hipMalloc(&ptr, b) != hipSuccess) {
            (void)hipGetLastError();
            throw std::runtime_error("out of VRAM for the resident decoder");
        }
        owned.push_back(ptr);
        bytes += b;
        Context::instance().allocated += b;
        if (hipMemset(ptr, 0, b) != hipSuccess) throw std::runtime_error("hipMemset failed");
        if (host && copy && hipMemcpy(ptr, host, size_t(copy) * 4, hipMemcpyHostToDevice) != hipSuccess)
            throw std::runtime_error("hipMemcpy to the resident decoder failed");
        return static_cast<float*>(ptr);
    }

    DevWeight weight(const AiGpuDenseWeight& w, uint64_t in, uint64_t out, const char* what) {
        if (w.inDim != in || w.outDim != out)
            throw std::invalid_argument(std::string("resident ") + what + " dimensions do not match config");
        if (!w.codes || w.type > 3 || (w.type >= 2 && (!w.scales || w.inDim % 32)) || w.inDim % 4)
            throw std::invalid_argument(std::string("resident ") + what + " weight is not usable");
        DevWeight d;
        d.codes = w.codes;
        d.scales = static_cast<const float*>(w.scales);
        d.type = int(w.type);
        d.in = w.inDim;
        d.out = w.outDim;
        if (w.bias) d.bias = floats(w.outDim, w.bias, w.outDim);
        return d;
    }
};

bool gemv(const DevWeight& w, const float* a, float* out, bool accumulate, hipStream_t stream) {
    GemvParams p{};
    p.a = a;
    p.w = w.codes;
    p.scales = w.scales;
    p.bias = w.bias;
    p.out = out;
    p.type = w.type;
    p.accumulate = accumulate ? 1 : 0;
    p.m = 1;
    p.k = w.in;
    p.n = w.out;
    p.ldo = w.out;
    return launch_gemv(p, stream);
}

bool norm(const float* x, const float* gamma, float* out, uint32_t n, float eps, hipStream_t stream) {
    return Context::instance().launch("dense_norm_kernel", stream, [&] {
        hipLaunchKernelGGL(dense_norm_kernel, dim3(1), dim3(1024), 0, stream, x, gamma, out, n, eps);
    });
}

/* the launches of one decode step; `splits` attention workgroups per kv head */
bool run_step(DenseModel& d, uint32_t splits, hipStream_t stream) {
    Context& ctx = Context::instance();
    const AiGpuDenseConfig& c = d.cfg;
    DenseArgs a{d.pos, c.heads, c.kvHeads, c.headDim, c.rotaryDims, d.maxSplits, 0, c.epsilon};
    for (const DevLayer& L : d.layers) {
        a.window = L.window;
        if (!norm(d.x, L.inputNorm, d.normed, c.hidden, c.epsilon, stream)) return false;
        if (!gemv(L.q, d.normed, d.q, false, stream) || !gemv(L.k, d.normed, d.k, false, stream) ||
            !gemv(L.v, d.normed, d.v, false, stream))
            return false;
        if (!ctx.launch("dense_qk_kernel", stream, [&] {
                hipLaunchKernelGGL(dense_qk_kernel, dim3(c.heads + c.kvHeads), dim3(64), 0, stream, a, d.q, d.k, d.v,
                                   L.qNorm, L.kNorm, d.freqs, L.keys, L.values);
            }))
            return false;
        if (!ctx.launch("dense_attn_kernel", stream, [&] {
                hipLaunchKernelGGL(dense_attn_kernel, dim3(splits, c.kvHeads), dim3(256), 0, stream, a, d.q, L.keys,
                                   L.values, d.partial);
            }))
            return false;
        if (!ctx.launch("dense_merge_kernel", stream, [&] {
                hipLaunchKernelGGL(dense_merge_kernel, dim3(c.heads), dim3(64), 0, stream, a, d.partial, d.attn);
            }))
            return false;
        if (!gemv(L.o, d.attn, d.x, true, stream)) return false;
        if (!norm(d.x, L.postNorm, d.normed, c.hidden, c.epsilon, stream)) return false;
        if (!gemv(L.gate, d.normed, d.gate, false, stream) || !gemv(L.up, d.normed, d.up, false, stream)) return false;
        if (!ctx.launch("dense_swiglu_kernel", stream, [&] {
                hipLaunchKernelGGL(dense_swiglu_kernel, dim3((c.intermediate + 255) / 256), dim3(256), 0, stream, d.gate,
                                   d.up, c.intermediate);
            }))
            return false;
        if (!gemv(L.down, d.gate, d.x, true, stream)) return false;
    }
    if (!norm(d.x, d.finalNorm, d.normed, c.hidden, c.epsilon, stream)) return false;
    return gemv(d.head, d.normed, d.logits, false, stream);
}

} // namespace
} // namespace aigpu

using aigpu::Context;
using aigpu::DenseModel;

extern "C" {

/* DeviceABI.h:144: this backend always has the resident decoder */
AIGPU_ABI int aigpu_dense_supported(void) { return Context::instance().ok ? 1 : 0; }

/* DeviceABI.h:145-147: the model's weights stay where the caller uploaded
   them; norms, biases, rotary frequencies and the first `length` cached
   positions are copied in */
AIGPU_ABI void* aigpu_dense_create(const AiGpuDenseConfig* c, const AiGpuDenseLayer* layers,
                                   const float* const* keys, const float* const* values, uint32_t length) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return nullptr;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    try {
        if (!c || !layers || !keys || !values || !c->hidden || !c->layers || !c->heads || !c->kvHeads ||
            c->heads % c->kvHeads || !c->headDim || c->headDim % 4 || c->headDim > uint32_t(aigpu::MAX_DIM) ||
            c->heads / c->kvHeads > uint32_t(aigpu::MAX_GROUP) || !c->rotaryDims || c->rotaryDims % 2 ||
            c->rotaryDims > c->headDim || !c->intermediate || !c->capacity || !c->vocab || length > c->capacity ||
            !c->finalNorm)
            throw std::invalid_argument("invalid resident decoder configuration");
        auto d = std::make_unique<DenseModel>();
        d->cfg = *c;
        d->length = length;
        std::vector<float> freqs;
        for (uint32_t j = 0; j < c->rotaryDims / 2; ++j) {
            // attentionMixer's frequency (LocalModel.hpp:2627-2628), in float
            const float f = c->rotaryFrequencies ? c->rotaryFrequencies[j]
                                                 : 1.0f / std::pow(c->theta, float(2 * j) / float(c->rotaryDims));
            if (!std::isfinite(f) || f <= 0) throw std::invalid_argument("invalid rotary frequency");
            freqs.push_back(f);
        }
        d->freqs = d->floats(freqs.size(), freqs.data(), freqs.size());
        const uint64_t H = c->hidden, qw = uint64_t(c->heads) * c->headDim, kw = uint64_t(c->kvHeads) * c->headDim;
        d->head = d->weight(c->head, H, c->vocab, "output projection");
        d->finalNorm = d->floats(H, c->finalNorm, H);
        d->x = d->floats(H);
        d->normed = d->floats(H);
        d->q = d->floats(qw);
        d->k = d->floats(kw);
        d->v = d->floats(kw);
        d->attn = d->floats(qw);
        d->gate = d->floats(c->intermediate);
        d->up = d->floats(c->intermediate);
        d->logits = d->floats(c->vocab);
        d->maxSplits = (c->capacity + aigpu::SPLIT - 1) / aigpu::SPLIT;
        d->partial = d->floats(uint64_t(c->heads) * d->maxSplits * 4 * (c->headDim + 2));
        d->pos = reinterpret_cast<uint32_t*>(d->floats(1));
        for (uint32_t i = 0; i < c->layers; ++i) {
            const AiGpuDenseLayer& l = layers[i];
            if (!l.inputNorm || !l.postNorm || !keys[i] || !values[i])
                throw std::invalid_argument("missing resident decoder norms or cache");
            aigpu::DevLayer L;
            L.q = d->weight(l.q, H, qw, "q");
            L.k = d->weight(l.k, H, kw, "k");
            L.v = d->weight(l.v, H, kw, "v");
            L.o = d->weight(l.o, qw, H, "o");
            L.gate = d->weight(l.gate, H, c->intermediate, "gate");
            L.up = d->weight(l.up, H, c->intermediate, "up");
            L.down = d->weight(l.down, c->intermediate, H, "down");
            L.inputNorm = d->floats(H, l.inputNorm, H);
            L.postNorm = d->floats(H, l.postNorm, H);
            if (l.qNorm) L.qNorm = d->floats(c->headDim, l.qNorm, c->headDim);
            if (l.kNorm) L.kNorm = d->floats(c->headDim, l.kNorm, c->headDim);
            L.keys = d->floats(uint64_t(c->capacity) * kw, keys[i], uint64_t(length) * kw);
            L.values = d->floats(uint64_t(c->capacity) * kw, values[i], uint64_t(length) * kw);
            L.window = l.window;
            d->layers.push_back(L);
        }
        ctx.stats.hostToDeviceBytes += uint64_t(length) * kw * 8 * c->layers;
        ctx.error.clear();
        return d.release();
    } catch (const std::exception& e) {
        ctx.error = e.what();
        return nullptr;
    }
}

/* DeviceABI.h:148 */
AIGPU_ABI void aigpu_dense_release(void* handle) {
    if (!handle) return;
    Context& ctx = Context::instance();
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    (void)hipDeviceSynchronize();
    delete static_cast<DenseModel*>(handle);
}

/* DeviceABI.h:149-150: one token at `position` (which must be the cached
   length): the embedding in, every layer, the logits out */
AIGPU_ABI void aigpu_dense_decode(void* handle, const float* embedding, float* logits, uint32_t position) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    if (!handle || !embedding || !logits) {
        ctx.error = "invalid resident decode arguments";
        return;
    }
    DenseModel& d = *static_cast<DenseModel*>(handle);
    const AiGpuDenseConfig& c = d.cfg;
    if (position >= c.capacity || position != d.length) {
        ctx.error = "resident decode position does not match KV cache";
        return;
    }
    const hipStream_t stream = nullptr;
    const auto mark = std::chrono::steady_clock::now();
    if (hipMemcpyAsync(d.x, embedding, size_t(c.hidden) * 4, hipMemcpyHostToDevice, stream) != hipSuccess ||
        hipMemcpyAsync(d.pos, &position, 4, hipMemcpyHostToDevice, stream) != hipSuccess) {
        (void)hipGetLastError();
        ctx.error = "resident decode upload failed";
        return;
    }
    // the attention grid covers the positions this step reads
    uint32_t splits = 1;
    for (const aigpu::DevLayer& L : d.layers) {
        const uint32_t first = L.window && position + 1 > L.window ? position + 1 - L.window : 0;
        const uint32_t s = (position + 1 - first + aigpu::SPLIT - 1) / aigpu::SPLIT;
        if (s > splits) splits = s;
    }
    if (!aigpu::run_step(d, splits, stream)) return;
    if (hipMemcpyAsync(logits, d.logits, size_t(c.vocab) * 4, hipMemcpyDeviceToHost, stream) != hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess) {
        ctx.error = std::string("resident decode failed: ") + hipGetErrorString(hipGetLastError());
        return;
    }
    ctx.stats.kernelSeconds += std::chrono::duration<double>(std::chrono::steady_clock::now() - mark).count();
    ctx.stats.hostToDeviceBytes += (uint64_t(c.hidden) + 1) * 4;
    ctx.stats.deviceToHostBytes += uint64_t(c.vocab) * 4;
    ++d.length;
    ctx.error.clear();
}

/* DeviceABI.h:151-152: the first `length` cached positions of every layer,
   back into the caller's fp32 arrays */
AIGPU_ABI void aigpu_dense_read_cache(void* handle, float* const* keys, float* const* values, uint32_t length) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    if (!handle || !keys || !values) {
        ctx.error = "invalid resident cache download";
        return;
    }
    DenseModel& d = *static_cast<DenseModel*>(handle);
    if (length != d.length) {
        ctx.error = "resident cache length mismatch";
        return;
    }
    const size_t bytes = size_t(length) * d.cfg.kvHeads * d.cfg.headDim * 4;
    for (size_t i = 0; i < d.layers.size(); ++i) {
        if (!keys[i] || !values[i]) {
            ctx.error = "null resident cache download target";
            return;
        }
        if (hipMemcpy(keys[i], d.layers[i].keys, bytes, hipMemcpyDeviceToHost) != hipSuccess ||
            hipMemcpy(values[i], d.layers[i].values, bytes, hipMemcpyDeviceToHost) != hipSuccess) {
            (void)hipGetLastError();
            ctx.error = "resident cache download failed";
            return;
        }
    }
    ctx.stats.deviceToHostBytes += uint64_t(bytes) * 2 * d.layers.size();
    ctx.error.clear();
}

} // extern "C"
