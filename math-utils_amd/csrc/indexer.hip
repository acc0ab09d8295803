// indexer.hip - the sparse-attention indexer (selectKeys, LocalModel.hpp:
// 2971-3068) in GLM-5.3's pooled form, on the device. Per call of `count`
// tokens at startPos:
//   projections        k = idxK h, gates = idxGate h (into the gate cache),
//                      and, when some token is sparse, q = idxQB qResid and
//                      w = idxWeights h (launch_gemv)
//   index_norm_kernel  layerNormRow (:1355-1367, eps 1e-6) of each k into
//                      the key cache (:2988-2990)
//   index_pool_kernel  every pool a token of the call completes: per channel
//                      the softmax over its members of gate + ape, applied
//                      to their keys (:2994-3009)
//   index_score_kernel per sparse token and pool wholly at or before it:
//                      sum over heads of w headScale relu(q . pool dimScale)
//                      (:3038-3047)
//   index_select_kernel per token: the topK / P best pools by radix select
//                      on the scores' order-preserving bits, expanded to
//                      keys in order, plus the unfinished pool (:3049-3066)
// The selection is the CSR form aigpu_latent_attention takes: token t's keys
// at selKeys + t * (topK / P * P + P), selCount[t] of them, UINT32_MAX for a
// token that sees every key (:3036).
#include "context.hpp"
#include "device.hpp"
#include "kernels.hpp"

namespace aigpu {

namespace {

constexpr int IX_MAX_DIM = 256;     // index head dim
constexpr int IX_MAX_HEADS = 64;    // index heads
constexpr int IX_Q_FLOATS = 8192;   // a token's q in LDS: heads * dim

struct IndexArgs {
    uint32_t count, startPos, Di, nI, P, budget, stride, maxPools, tail;
    float headScale, dimScale;
};

__device__ __forceinline__ bool sees_everything(const IndexArgs& a, uint32_t complete) {
    return complete <= a.budget && a.tail;
}

/* layerNormRow: one wave per token, dim / 64 values per lane */
__global__ __launch_bounds__(64) void index_norm_kernel(IndexArgs a, const float* k, const float* w, const float* b,
                                                        float* keys) {
    const uint32_t t = blockIdx.x, lane = threadIdx.x, Di = a.Di;
    const float* x = k + size_t(t) * Di;
    float v[IX_MAX_DIM / WAVE];
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < IX_MAX_DIM / WAVE; ++e) {
        const uint32_t d = lane + WAVE * e;
        v[e] = d < Di ? x[d] : 0.0f;
        s += v[e];
    }
    const float mean = wave_sum(s) / float(Di);
    float q = 0.0f;
#pragma unroll
    for (int e = 0; e < IX_MAX_DIM / WAVE; ++e) {
        const uint32_t d = lane + WAVE * e;
        const float dv = d < Di ? v[e] - mean : 0.0f;
        q = fmaf(dv, dv, q);
    }
    const float inv = 1.0f / sqrtf(wave_sum(q) / float(Di) + 1e-6f);
    float* out = keys + size_t(a.startPos + t) * Di;
#pragma unroll
    for (int e = 0; e < IX_MAX_DIM / WAVE; ++e) {
        const uint32_t d = lane + WAVE * e;
        if (d < Di) out[d] = (v[e] - mean) * inv * w[d] + (b ? b[d] : 0.0f);
    }
}

/* pool firstPool + blockIdx.x: thread d folds channel d of its P members */
__global__ __launch_bounds__(256) void index_pool_kernel(IndexArgs a, const float* keys, const float* gates,
                                                         const float* ape, float* pools, uint32_t firstPool) {
    const uint32_t p = firstPool + blockIdx.x, d = threadIdx.x, Di = a.Di, P = a.P;
    if (d >= Di) return;
    const size_t first = size_t(p) * P;
    float best = -1e30f;
    for (uint32_t i = 0; i < P; ++i) best = fmaxf(best, gates[(first + i) * Di + d] + ape[size_t(i) * Di + d]);
    float sum = 0.0f;
    for (uint32_t i = 0; i < P; ++i) sum += expf(gates[(first + i) * Di + d] + ape[size_t(i) * Di + d] - best);
    float acc = 0.0f;
    for (uint32_t i = 0; i < P; ++i) {
        const float wgt = expf(gates[(first + i) * Di + d] + ape[size_t(i) * Di + d] - best);
        acc += wgt / sum * keys[(first + i) * Di + d];
    }
    pools[size_t(p) * Di + d] = acc;
}

/* token blockIdx.x; blocks of 32 pools blockIdx.y, blockIdx.y + gridDim.y,
   ..., pool 32 block + lane % 32. The 256 threads are
   32 pools x 8 head groups: wave w holds groups 2w (lanes 0-31) and 2w + 1
   (lanes 32-63), each of ceil(nI / 8) heads, so a decode step still fills
   the chip. The token's q rows and head weights sit in LDS (read as
   broadcasts); each thread streams its pool row in 16-byte pieces. Each
   group's relu-weighted sum (in head order) is combined across the eight
   groups in order. */
constexpr int IX_POOLS = 32, IX_GROUPS = 8, IX_HPT = IX_MAX_HEADS / IX_GROUPS;

__global__ __launch_bounds__(256) void index_score_kernel(IndexArgs a, const float* q, const float* w,
                                                          const float* pools, float* scores) {
    __shared__ __align__(16) float qs[IX_Q_FLOATS];
    __shared__ float ws[IX_MAX_HEADS];
    __shared__ float part[IX_GROUPS][IX_POOLS];
    const uint32_t t = blockIdx.x, pos = a.startPos + t, complete = (pos + 1) / a.P;
    if (sees_everything(a, complete) || blockIdx.y * IX_POOLS >= complete) return;   // uniform, before any barrier
    const uint32_t nI = a.nI, Di = a.Di, tid = threadIdx.x;
    for (uint32_t i = tid; i < nI * Di / 4; i += 256)
        reinterpret_cast<floatx4*>(qs)[i] = reinterpret_cast<const floatx4*>(q + size_t(t) * nI * Di)[i];
    if (tid < nI) ws[tid] = w[size_t(t) * nI + tid];
    __syncthreads();
    const uint32_t pl = tid % IX_POOLS, g = tid / IX_POOLS;
    const uint32_t hpg = (nI + IX_GROUPS - 1) / IX_GROUPS, h0 = g * hpg;
    // pool blocks blockIdx.y, + gridDim.y, ...: one load of q serves them all
    for (uint32_t p0 = blockIdx.y * IX_POOLS; p0 < complete; p0 += gridDim.y * IX_POOLS) {   // uniform
        const uint32_t p = p0 + pl;
        float total = 0.0f;
        if (p < complete) {
            float acc[IX_HPT];
#pragma unroll
            for (int h = 0; h < IX_HPT; ++h) acc[h] = 0.0f;
            const floatx4* pr = reinterpret_cast<const floatx4*>(pools + size_t(p) * Di);
            for (uint32_t d4 = 0; d4 < Di / 4; ++d4) {
                const floatx4 pv = pr[d4];
#pragma unroll
                for (int h = 0; h < IX_HPT; ++h) {
                    if (h < int(hpg) && h0 + h < nI) {
                        const floatx4 qv = reinterpret_cast<const floatx4*>(qs + (h0 + h) * Di)[d4];
                        acc[h] = fmaf(qv[0], pv[0], fmaf(qv[1], pv[1], fmaf(qv[2], pv[2], fmaf(qv[3], pv[3], acc[h]))));
                    }
                }
            }
#pragma unroll
            for (int h = 0; h < IX_HPT; ++h) {
                if (h < int(hpg) && h0 + h < nI) {
                    const float logit = acc[h] * a.dimScale;
                    total += ws[h0 + h] * a.headScale * (logit > 0.0f ? logit : 0.0f);
                }
            }
        }
        part[g][pl] = total;
        __syncthreads();
        if (tid < IX_POOLS && p < complete) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < IX_GROUPS; ++i) s += part[i][tid];
            scores[size_t(t) * a.maxPools + p] = s;
        }
        __syncthreads();   // part is rewritten by the next block
    }
}

/* larger scores give larger keys; -0 counts as +0 */
__device__ __forceinline__ uint32_t order_key(float x) {
    const uint32_t u = __float_as_uint(x + 0.0f);
    return (u >> 31) ? ~u : (u | 0x80000000u);
}

/* exclusive prefix sum of v over the workgroup's 256 threads in order */
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* waveSums) {
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    uint32_t incl = v;
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
        const uint32_t y = __shfl_up(incl, o, WAVE);
        if (int(lane) >= o) incl += y;
    }
    if (lane == WAVE - 1) waveSums[w] = incl;
    __syncthreads();
    uint32_t before = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (i < int(w)) before += waveSums[i];
    __syncthreads();   // waveSums is rewritten by the next scan
    return before + incl - v;
}

constexpr int IX_REG = 32;   // pools per thread held in registers (up to 8192 per token)

/* f(i, key) over this thread's pools b0 + i < b1, in order: from registers
   (REG, i a compile-time index after unrolling) or streamed from the scores */
template <bool REG, typename F>
__device__ __forceinline__ void each_pool(const uint32_t (&u)[IX_REG], const float* sc, uint32_t b0, uint32_t b1, F f) {
    if constexpr (REG) {
#pragma unroll
        for (int i = 0; i < IX_REG; ++i)
            if (b0 + uint32_t(i) < b1) f(uint32_t(i), u[i]);
    } else {
        for (uint32_t i = 0; b0 + i < b1; ++i) f(i, order_key(sc[b0 + i]));
    }
}

/* one workgroup per token; thread tid owns the contiguous pools
   [tid R, tid R + R), R = ceil(complete / 256), so pool order is thread
   order and the emission needs only two workgroup scans */
template <bool REG>
__global__ __launch_bounds__(256) void index_select_kernel(IndexArgs a, const float* scores, uint32_t* selStart,
                                                           uint32_t* selCount, uint32_t* selKeys) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t found[2];
    __shared__ uint32_t waveSums[4];
    const uint32_t t = blockIdx.x, pos = a.startPos + t, complete = (pos + 1) / a.P, tid = threadIdx.x;
    if (tid == 0) selStart[t] = t * a.stride;
    if (sees_everything(a, complete)) {
        if (tid == 0) selCount[t] = 0xFFFFFFFFu;
        return;
    }
    const uint32_t keep = complete < a.budget ? complete : a.budget;
    const float* sc = scores + size_t(t) * a.maxPools;
    const uint32_t R = (complete + 255) / 256, b0 = tid * R < complete ? tid * R : complete;
    const uint32_t b1 = b0 + R < complete ? b0 + R : complete;
    uint32_t u[IX_REG];
    if constexpr (REG) {
#pragma unroll
        for (int i = 0; i < IX_REG; ++i) u[i] = b0 + uint32_t(i) < b1 ? order_key(sc[b0 + i]) : 0u;
    }

    // the keep-th largest key, eight bits at a time from the top; `remaining`
    // ends as the number of keys equal to it that are taken
    uint32_t prefix = 0, prefixMask = 0, remaining = keep;
    const bool all = keep == complete;   // every complete pool is taken
    if (!all && keep > 0) {
        for (int shift = 24; shift >= 0; shift -= 8) {
            hist[tid] = 0;
            __syncthreads();
            each_pool<REG>(u, sc, b0, b1, [&](uint32_t, uint32_t key) {
                if ((key & prefixMask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
            });
            __syncthreads();
            if (tid < WAVE) {   // the digit: counts from the top, 4 bins per lane
                uint32_t c[4], s = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    c[i] = hist[255 - (4 * tid + i)];
                    s += c[i];
                }
                uint32_t incl = s;
#pragma unroll
                for (int o = 1; o < WAVE; o <<= 1) {
                    const uint32_t y = __shfl_up(incl, o, WAVE);
                    if (int(tid) >= o) incl += y;
                }
                uint32_t cum = incl - s;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (cum < remaining && cum + c[i] >= remaining) {
                        found[0] = 255 - (4 * tid + i);
                        found[1] = remaining - cum;
                    }
                    cum += c[i];
                }
            }
            __syncthreads();
            prefix |= found[0] << shift;
            prefixMask |= 255u << shift;
            remaining = found[1];
            __syncthreads();   // found and hist are rewritten by the next pass
        }
    }

    // the chosen pools in index order: above the threshold, or equal to it
    // and among the first `remaining` such
    uint32_t eqLocal = 0, gtLocal = 0;
    if (!all)
        each_pool<REG>(u, sc, b0, b1, [&](uint32_t, uint32_t key) {
            eqLocal += key == prefix ? 1u : 0u;
            gtLocal += key > prefix ? 1u : 0u;
        });
    const uint32_t eqBefore = block_exclusive_scan(eqLocal, waveSums);
    const uint32_t takeEq = all || eqBefore >= remaining ? 0u : (remaining - eqBefore < eqLocal ? remaining - eqBefore : eqLocal);
    const uint32_t chosenLocal = all ? b1 - b0 : gtLocal + takeEq;
    uint32_t n = block_exclusive_scan(chosenLocal, waveSums);
    uint32_t* out = selKeys + size_t(t) * a.stride;
    uint32_t eqSeen = 0;
    each_pool<REG>(u, sc, b0, b1, [&](uint32_t i, uint32_t key) {
        bool chosen = all || key > prefix;
        if (!all && key == prefix) chosen = eqSeen++ < takeEq;
        if (chosen) {
            for (uint32_t j = 0; j < a.P; ++j) out[n * a.P + j] = (b0 + i) * a.P + j;
            ++n;
        }
    });
    uint32_t total = keep * a.P;
    if (a.tail) {
        for (uint32_t j = complete * a.P + tid; j <= pos; j += 256) out[total + (j - complete * a.P)] = j;
        total += pos + 1 - complete * a.P;
    }
    if (tid == 0) selCount[t] = total;
}

GemvParams projection(const MixerWeight& w, const float* a, float* out, uint32_t m, uint32_t ldo) {
    GemvParams g{};
    g.a = a;
    g.w = w.codes;
    g.scales = w.scales;
    g.bias = w.bias;
    g.out = out;
    g.type = w.type;
    g.m = m;
    g.k = w.in;
    g.n = w.out;
    g.ldo = ldo;
    return g;
}

} // namespace

bool launch_select_keys(const IndexerParams& p, hipStream_t stream) {
    Context& ctx = Context::instance();
    const uint64_t Di = p.dim, nI = p.heads, P = p.pool;
    if (!p.h || !p.qResid || !p.kNorm || !p.ape || !p.keys || !p.gates || !p.pools || !p.selStart ||
        !p.selCount || !p.selKeys || !p.wk.codes || !p.wgate.codes || !p.wq.codes || !p.ww.codes)
        return ctx.fail("select keys: null tensor");
    if (Di == 0 || Di % 4 || Di > IX_MAX_DIM) return ctx.fail("select keys: index head dim must be a multiple of 4 up to 256");
    if (nI == 0 || nI > IX_MAX_HEADS || nI * Di > IX_Q_FLOATS)
        return ctx.fail("select keys: at most 64 index heads and heads * dim <= 8192");
    if (P == 0 || p.topK < P) return ctx.fail("select keys: need 1 <= pool <= topK");
    if (p.wk.in != p.hidden || p.wk.out != Di || p.wgate.in != p.hidden || p.wgate.out != Di ||
        p.wq.in != p.qRank || p.wq.out != nI * Di || p.ww.in != p.hidden || p.ww.out != nI)
        return ctx.fail("select keys: weight shapes do not match hidden, qRank, heads, dim");
    if (p.count == 0) return true;
    const uint64_t end = p.startPos + p.count;
    if (end > p.capacity) return ctx.fail("select keys: cache capacity below startPos + count");
    const uint64_t budget = p.topK / P, stride = budget * P + P, maxPools = end / P;
    if (p.count * stride >= (1ull << 32) || p.count * (maxPools + 1) >= (1ull << 40) || end >= (1ull << 31) ||
        (maxPools + IX_POOLS - 1) / IX_POOLS > 65535)
        return ctx.fail("select keys: too many tokens or keys");
    if ((reinterpret_cast<uintptr_t>(p.pools) | reinterpret_cast<uintptr_t>(p.keys)) % 16)
        return ctx.fail("select keys: the key and pool caches must be 16-byte aligned");

    bool anySparse = false;   // :3014-3018, from the shapes alone
    for (uint64_t t = 0; t < p.count && !anySparse; ++t)
        if ((p.startPos + t + 1) / P > budget || !p.tail) anySparse = true;

    const size_t kBytes = p.count * Di * 4, qBytes = anySparse ? p.count * nI * Di * 4 : 0;
    const size_t wBytes = anySparse ? p.count * nI * 4 : 0;
    const size_t sBytes = anySparse && !p.scores ? p.count * maxPools * 4 : 0;
    auto align = [](size_t b) { return (b + 255) & ~size_t(255); };
    char* work = static_cast<char*>(ctx.grow(SLOT_INDEXER, align(kBytes) + align(qBytes) + align(wBytes) + sBytes));
    if (!work) return false;
    float* k = reinterpret_cast<float*>(work);
    float* q = reinterpret_cast<float*>(work + align(kBytes));
    float* w = reinterpret_cast<float*>(work + align(kBytes) + align(qBytes));
    float* scores = p.scores ? p.scores : reinterpret_cast<float*>(work + align(kBytes) + align(qBytes) + align(wBytes));

    const uint32_t m = uint32_t(p.count);
    if (!launch_gemv(projection(p.wk, p.h, k, m, uint32_t(Di)), stream)) return false;
    if (!launch_gemv(projection(p.wgate, p.h, p.gates + p.startPos * Di, m, uint32_t(Di)), stream)) return false;

    IndexArgs a{};
    a.count = m;
    a.startPos = uint32_t(p.startPos);
    a.Di = uint32_t(Di);
    a.nI = uint32_t(nI);
    a.P = uint32_t(P);
    a.budget = uint32_t(budget);
    a.stride = uint32_t(stride);
    a.maxPools = uint32_t(maxPools);
    a.tail = p.tail ? 1u : 0u;
    a.headScale = 1.0f / sqrtf(float(nI));
    a.dimScale = 1.0f / sqrtf(float(Di));
    if (!ctx.launch("index_norm_kernel", stream, [&] {
            hipLaunchKernelGGL(index_norm_kernel, dim3(m), dim3(WAVE), 0, stream, a, k, p.kNorm, p.kNormBias, p.keys);
        }))
        return false;
    const uint64_t firstPool = p.startPos / P, endPool = end / P;   // pools whose last member is in the call
    if (endPool > firstPool &&
        !ctx.launch("index_pool_kernel", stream, [&] {
            hipLaunchKernelGGL(index_pool_kernel, dim3(unsigned(endPool - firstPool)), dim3(256), 0, stream, a, p.keys,
                               p.gates, p.ape, p.pools, uint32_t(firstPool));
        }))
        return false;
    if (anySparse) {
        if (!launch_gemv(projection(p.wq, p.qResid, q, m, uint32_t(nI * Di)), stream)) return false;
        if (!launch_gemv(projection(p.ww, p.h, w, m, uint32_t(nI)), stream)) return false;
        if (maxPools > 0 &&
            !ctx.launch("index_score_kernel", stream, [&] {
                // about 2048 workgroups: a decode step splits its pools 256 ways,
                // a long prefill gives each token one workgroup and one load of q
                const uint64_t blocks = (maxPools + IX_POOLS - 1) / IX_POOLS;
                const uint64_t want = m >= 2048 ? 1 : (2048 + m - 1) / m;
                const unsigned gy = unsigned(blocks < want ? blocks : want);
                hipLaunchKernelGGL(index_score_kernel, dim3(m, gy), dim3(256), 0, stream, a, q, w, p.pools, scores);
            }))
            return false;
    }
    return ctx.launch("index_select_kernel", stream, [&] {
        if ((maxPools + 255) / 256 <= uint64_t(IX_REG))
            hipLaunchKernelGGL((index_select_kernel<true>), dim3(m), dim3(256), 0, stream, a, scores, p.selStart,
                               p.selCount, p.selKeys);
        else
            hipLaunchKernelGGL((index_select_kernel<false>), dim3(m), dim3(256), 0, stream, a, scores, p.selStart,
                               p.selCount, p.selKeys);
    });
}

} // namespace aigpu
