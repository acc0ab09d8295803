// latent.hip - multi-head latent attention (latentAttentionMixer,
// LocalModel.hpp:3086-3163; DeepSeek's MLA as GLM-5.3 uses it, without
// positional encoding). Every token's key and value are one kvLoraRank-wide
// latent c; head h's key would be Wk_h c and its value Wv_h c, Wk_h and Wv_h
// its rows of kv_b_proj. Both are linear, so
//   q . (Wk_h c) = (Wk_h^T q) . c         sum_j p_j Wv_h c_j = Wv_h (sum_j p_j c_j)
// and nothing is ever expanded:
//   latent_fold_kernel    folded[t][h] = Wk_h^T q[t][h]
//   latent_attn_kernel    softmax(folded . c_j * scale) over the token's keys
//                         (all positions up to it, or the indexer's sorted
//                         selection), context = sum p_j c_j; every cached
//                         latent is read once per group of 16 heads
//   latent_merge_kernel   (decode-sized calls) the key splits combined
//   latent_unfold_kernel  out[t][h] = Wv_h context[t][h]
// fp32 throughout, as the reference computes it; kv_b_proj may be fp32 or
// bf16 (widened).
#include "context.hpp"
#include "device.hpp"
#include "kernels.hpp"

namespace aigpu {

namespace {

constexpr int HG = 16;          // heads per attention workgroup
constexpr int KPB = 64;         // keys per block (eight lanes per pair of keys)
constexpr int MAX_RANK = 512;   // kvLoraRank
constexpr int MAX_NOPE = 256;
constexpr int TT = 8;           // tokens per fold / unfold workgroup

struct LatentArgs {
    LatentParams p;
    float* folded;    // [count][heads][C]
    float* context;   // [count][heads][C]
    float* partial;   // [count][heads][splits][C + 2]
    uint32_t splits;
};

template <bool BF16>
__device__ __forceinline__ float wkv_at(const void* w, size_t i) {
    if constexpr (BF16) return bf16_bits_to_float(static_cast<const uint16_t*>(w)[i]);
    return static_cast<const float*>(w)[i];
}

/* folded[t][h][c] = sum_d q[t][h][d] Wk_h[d][c] (:3124-3129): workgroup
   (head, 64 columns, TT tokens); the four waves take a quarter of d each (the
   lanes on columns, coalesced rows of Wk) and add their sums in LDS */
template <bool BF16>
__global__ __launch_bounds__(256) void latent_fold_kernel(LatentArgs a) {
    __shared__ float qs[TT][MAX_NOPE];
    __shared__ float part[4][TT][WAVE];
    const LatentParams& p = a.p;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t h = blockIdx.x, c = blockIdx.y * WAVE + lane;
    const uint64_t t0 = uint64_t(blockIdx.z) * TT;
    const uint32_t Dn = uint32_t(p.nope), C = uint32_t(p.rank);
    for (uint32_t i = threadIdx.x; i < TT * Dn; i += 256) {
        const uint32_t t = i / Dn, d = i % Dn;
        qs[t][d] = t0 + t < p.count ? p.q[((t0 + t) * p.heads + h) * Dn + d] : 0.0f;
    }
    __syncthreads();
    const size_t wk = size_t(h) * (p.nope + p.vdim) * C;
    float acc[TT] = {};
    if (c < C) {
#pragma unroll 8
        for (uint32_t d = w; d < Dn; d += 4) {
            const float wv = wkv_at<BF16>(p.wkv, wk + size_t(d) * C + c);
#pragma unroll
            for (int t = 0; t < TT; ++t) acc[t] = fmaf(qs[t][d], wv, acc[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) part[w][t][lane] = acc[t];
    __syncthreads();
    if (w == 0 && c < C) {
#pragma unroll
        for (int t = 0; t < TT; ++t)
            if (t0 + t < p.count)
                a.folded[((t0 + t) * p.heads + h) * C + c] = part[0][t][lane] + part[1][t][lane] + part[2][t][lane] + part[3][t][lane];
    }
}

/* workgroup (token, 16 heads, key split): online softmax over blocks of KPB
   keys; eight lanes share a pair of keys' rows in the scores, the lanes own
   columns in the context */
__global__ __launch_bounds__(256) void latent_attn_kernel(LatentArgs a) {
    __shared__ float F[HG * MAX_RANK];
    __shared__ __align__(16) float pr[HG][KPB];
    __shared__ uint32_t keyAt[KPB];
    __shared__ float wred[4][HG];

    const LatentParams& p = a.p;
    const uint64_t t = blockIdx.x;
    const uint32_t h0 = blockIdx.y * HG, s = blockIdx.z;
    const uint32_t C = uint32_t(p.rank);
    const uint32_t nh = uint32_t(p.heads - h0 < HG ? p.heads - h0 : HG);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint64_t pos = p.startPos + t;
    const bool dense = !p.selCount || p.selCount[t] == 0xFFFFFFFFu;
    const uint64_t n = dense ? pos + 1 : p.selCount[t];
    const uint32_t* sel = dense ? nullptr : p.selKeys + p.selStart[t];
    const uint64_t blocks = (n + KPB - 1) / KPB;
    const uint64_t per = (blocks + a.splits - 1) / a.splits;
    const uint64_t bBegin = uint64_t(s) * per, bEnd = bBegin + per < blocks ? bBegin + per : blocks;

    {
        // 16 rows of C floats as float4, every load in flight (C % 16 == 0)
        const uint32_t q4 = C / 4;
        floatx4 fv[HG * MAX_RANK / 4 / 256];
#pragma unroll
        for (int e = 0; e < HG * MAX_RANK / 4 / 256; ++e) {
            const uint32_t i = tid + 256 * e, hh = i / q4, c = 4 * (i % q4);
            fv[e] = (i < HG * q4 && hh < nh)
                        ? *reinterpret_cast<const floatx4*>(&a.folded[(t * p.heads + h0 + hh) * C + c])
                        : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int e = 0; e < HG * MAX_RANK / 4 / 256; ++e) {
            const uint32_t i = tid + 256 * e, hh = i / q4, c = 4 * (i % q4);
            if (i < HG * q4) *reinterpret_cast<floatx4*>(&F[hh * MAX_RANK + c]) = fv[e];
        }
    }
    __syncthreads();

    constexpr int CPT = MAX_RANK / 256;   // context columns per thread
    float m[HG], l[HG], acc[HG][CPT];
#pragma unroll
    for (int hh = 0; hh < HG; ++hh) {
        m[hh] = -INFINITY;
        l[hh] = 0.0f;
#pragma unroll
        for (int e = 0; e < CPT; ++e) acc[hh][e] = 0.0f;
    }
    // scores: thread (kq, part) takes keys kq and kq + 32 of the block, and
    // in each 256-column chunk the interleaved 16-byte pieces 32 j + 4 part:
    // the eight parts of a key read 128 contiguous bytes, and each piece of
    // F read from LDS serves both keys
    const uint32_t kq = uint32_t(tid) >> 3, part = uint32_t(tid) & 7;
    for (uint64_t b = bBegin; b < bEnd; ++b) {
        const uint64_t i0 = b * KPB + kq, i1 = i0 + KPB / 2;
        const bool live0 = i0 < n, live1 = i1 < n;
        const uint32_t key0 = live0 ? (dense ? uint32_t(i0) : sel[i0]) : 0u;
        const uint32_t key1 = live1 ? (dense ? uint32_t(i1) : sel[i1]) : 0u;
        if (part == 0) {
            keyAt[kq] = key0;
            keyAt[kq + KPB / 2] = key1;
        }
        float s0[HG], s1[HG];
#pragma unroll
        for (int hh = 0; hh < HG; ++hh) s0[hh] = s1[hh] = 0.0f;
        {
            // rows past n read row `key` 0 (finite) and are masked below
            const float* r0 = p.latent + size_t(key0) * C + 4 * part;
            const float* r1 = p.latent + size_t(key1) * C + 4 * part;
            for (uint32_t c0 = 0; c0 < C; c0 += 256) {
                floatx4 k0v[8], k1v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const bool in = c0 + 32 * e < C;
                    k0v[e] = in ? *reinterpret_cast<const floatx4*>(r0 + c0 + 32 * e) : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
                    k1v[e] = in ? *reinterpret_cast<const floatx4*>(r1 + c0 + 32 * e) : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
                }
#pragma unroll
                for (int hh = 0; hh < HG; ++hh) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        if (c0 + 32 * e < C) {
                            const floatx4 f4 = *reinterpret_cast<const floatx4*>(&F[hh * MAX_RANK + c0 + 32 * e + 4 * part]);
                            s0[hh] = fmaf(f4[0], k0v[e][0], fmaf(f4[1], k0v[e][1], fmaf(f4[2], k0v[e][2], fmaf(f4[3], k0v[e][3], s0[hh]))));
                            s1[hh] = fmaf(f4[0], k1v[e][0], fmaf(f4[1], k1v[e][1], fmaf(f4[2], k1v[e][2], fmaf(f4[3], k1v[e][3], s1[hh]))));
                        }
                    }
                }
            }
        }
        // the keys' eight parts, then the block's max per head
#pragma unroll
        for (int hh = 0; hh < HG; ++hh) {
#pragma unroll
            for (int o = 1; o < 8; o <<= 1) {
                s0[hh] += __shfl_xor(s0[hh], o, WAVE);
                s1[hh] += __shfl_xor(s1[hh], o, WAVE);
            }
            s0[hh] = live0 ? s0[hh] * p.scale : -INFINITY;
            s1[hh] = live1 ? s1[hh] * p.scale : -INFINITY;
            const float bm = wave_max(fmaxf(s0[hh], s1[hh]));
            if (lane == 0) wred[w][hh] = bm;
        }
        __syncthreads();
        float f[HG];
#pragma unroll
        for (int hh = 0; hh < HG; ++hh) {
            const float bm = fmaxf(fmaxf(wred[0][hh], wred[1][hh]), fmaxf(wred[2][hh], wred[3][hh]));
            const float mn = fmaxf(m[hh], bm);
            f[hh] = expf(m[hh] - mn);   // 0 on the first block
            m[hh] = mn;
            if (part == 0) {
                pr[hh][kq] = live0 ? expf(s0[hh] - mn) : 0.0f;
                pr[hh][kq + KPB / 2] = live1 ? expf(s1[hh] - mn) : 0.0f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int hh = 0; hh < HG; ++hh) {
            l[hh] = l[hh] * f[hh] + wave_sum(pr[hh][lane]);   // KPB == WAVE: lane = key
#pragma unroll
            for (int e = 0; e < CPT; ++e) acc[hh][e] *= f[hh];
        }
        // context: the block's keys against the thread's columns
        const uint32_t nb = uint32_t(n - b * KPB < uint64_t(KPB) ? n - b * KPB : uint64_t(KPB));
        for (uint32_t k0 = 0; k0 < nb; k0 += 16) {
            float lv[16][CPT];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const uint32_t kk = k0 + u < nb ? k0 + u : k0;
                const float* lr = p.latent + size_t(keyAt[kk]) * C;
#pragma unroll
                for (int e = 0; e < CPT; ++e) lv[u][e] = tid + 256 * e < int(C) ? lr[tid + 256 * e] : 0.0f;
            }
            // keys past nb have probability 0 against a finite row
#pragma unroll
            for (int v = 0; v < 4; ++v) {
#pragma unroll
                for (int hh = 0; hh < HG; ++hh) {
                    const floatx4 p4 = *reinterpret_cast<const floatx4*>(&pr[hh][k0 + 4 * v]);
#pragma unroll
                    for (int u = 0; u < 4; ++u)
#pragma unroll
                        for (int e = 0; e < CPT; ++e) acc[hh][e] = fmaf(p4[u], lv[4 * v + u][e], acc[hh][e]);
                }
            }
        }
        __syncthreads();   // pr and keyAt are rewritten by the next block
    }

    if (a.splits == 1) {
#pragma unroll
        for (int hh = 0; hh < HG; ++hh) {
            if (uint32_t(hh) >= nh) break;
            // an empty selection (no key at or before the token) leaves the
            // context at zero, as the mixer's job does (l = 0, acc = 0)
            const float inv = l[hh] > 0.0f ? 1.0f / l[hh] : 0.0f;
#pragma unroll
            for (int e = 0; e < CPT; ++e)
                if (tid + 256 * e < int(C)) a.context[(t * p.heads + h0 + hh) * C + tid + 256 * e] = acc[hh][e] * inv;
        }
    } else {
        const size_t rec = size_t(C) + 2;
#pragma unroll
        for (int hh = 0; hh < HG; ++hh) {
            if (uint32_t(hh) >= nh) break;
            float* out = a.partial + ((t * p.heads + h0 + hh) * a.splits + s) * rec;
            if (tid == 0) {
                out[0] = m[hh];
                out[1] = l[hh];
            }
#pragma unroll
            for (int e = 0; e < CPT; ++e)
                if (tid + 256 * e < int(C)) out[2 + tid + 256 * e] = acc[hh][e];
        }
    }
}

/* the splits' records of one (token, head) combined into its context: each
   wave reduces the (at most 64) maxima and sums with a lane per split, then
   the threads sum the accumulators column by column */
__global__ __launch_bounds__(256) void latent_merge_kernel(LatentArgs a) {
    const LatentParams& p = a.p;
    const uint64_t t = blockIdx.x;
    const uint32_t h = blockIdx.y, C = uint32_t(p.rank);
    const int lane = threadIdx.x & 63;
    const size_t rec = size_t(C) + 2;
    const float* base = a.partial + (t * p.heads + h) * a.splits * rec;
    const float mi = lane < int(a.splits) ? base[lane * rec] : -INFINITY;
    const float M = wave_max(mi);
    const float fi = (lane < int(a.splits) && mi != -INFINITY) ? expf(mi - M) : 0.0f;
    const float L = wave_sum(lane < int(a.splits) ? base[lane * rec + 1] * fi : 0.0f);
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;   // every split empty: a zero context
    for (uint32_t c = threadIdx.x; c < C; c += 256) {
        float acc = 0.0f;
#pragma unroll 8
        for (uint32_t i = 0; i < a.splits; ++i) {
            const float m = base[i * rec];
            acc = fmaf(base[i * rec + 2 + c], m == -INFINITY ? 0.0f : expf(m - M), acc);
        }
        a.context[(t * p.heads + h) * C + c] = acc * inv;
    }
}

/* out[t][h][v] = Wv_h[v] . context[t][h] (:3153-3154): workgroup (head,
   TT tokens), each wave a quarter of the v rows, the lanes along the rank
   (16-byte loads of the row), the TT contexts in LDS, a wave reduction per
   (row, token) */
template <bool BF16>
__global__ __launch_bounds__(256) void latent_unfold_kernel(LatentArgs a) {
    __shared__ float cs[TT * MAX_RANK];
    const LatentParams& p = a.p;
    const uint32_t h = blockIdx.x;
    const uint64_t t0 = uint64_t(blockIdx.y) * TT;
    const uint32_t C = uint32_t(p.rank), Dv = uint32_t(p.vdim);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    for (uint32_t i = threadIdx.x; i < TT * C / 4; i += 256) {
        const uint32_t t = i / (C / 4), c = 4 * (i % (C / 4));
        *reinterpret_cast<floatx4*>(&cs[t * MAX_RANK + c]) =
            t0 + t < p.count ? *reinterpret_cast<const floatx4*>(&a.context[((t0 + t) * p.heads + h) * C + c])
                             : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    __syncthreads();
    const size_t wv0 = (size_t(h) * (p.nope + p.vdim) + p.nope) * C;
    const int tn = int(p.count - t0 < uint64_t(TT) ? p.count - t0 : uint64_t(TT));
    for (uint32_t v = w; v < Dv; v += 4) {
        float acc[TT] = {};
        for (uint32_t c = 4 * lane; c < C; c += 4 * WAVE) {
            float wr[4];
            if constexpr (BF16) {
                const u32x2 b = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(p.wkv) + wv0 + size_t(v) * C + c);
                wr[0] = __uint_as_float(b[0] << 16);
                wr[1] = __uint_as_float(b[0] & 0xFFFF0000u);
                wr[2] = __uint_as_float(b[1] << 16);
                wr[3] = __uint_as_float(b[1] & 0xFFFF0000u);
            } else {
                const floatx4 f = *reinterpret_cast<const floatx4*>(static_cast<const float*>(p.wkv) + wv0 + size_t(v) * C + c);
#pragma unroll
                for (int e = 0; e < 4; ++e) wr[e] = f[e];
            }
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) {
                if (tt >= tn) break;   // uniform
                const floatx4 x = *reinterpret_cast<const floatx4*>(&cs[tt * MAX_RANK + c]);
                acc[tt] = fmaf(wr[0], x[0], fmaf(wr[1], x[1], fmaf(wr[2], x[2], fmaf(wr[3], x[3], acc[tt]))));
            }
        }
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
            if (tt >= tn) break;   // uniform
            const float sum = wave_sum(acc[tt]);
            if (lane == 0) p.out[((t0 + tt) * p.heads + h) * Dv + v] = sum;
        }
    }
}

} // namespace

bool launch_latent_attention(const LatentParams& p, hipStream_t stream) {
    Context& ctx = Context::instance();
    if (!p.q || !p.latent || !p.wkv || !p.out) return ctx.fail("latent attention: null tensor");
    if (p.selCount && (!p.selStart || !p.selKeys)) return ctx.fail("latent attention: a selection needs start and keys");
    if (p.wType > 1) return ctx.fail("latent attention: kv_b_proj must be fp32 or bf16");
    if (p.rank == 0 || p.rank > uint64_t(MAX_RANK) || p.rank % 16)
        return ctx.fail("latent attention: kvLoraRank must be a multiple of 16 up to 512");
    if (p.nope == 0 || p.nope > uint64_t(MAX_NOPE)) return ctx.fail("latent attention: qk_nope_head_dim must be 1 to 256");
    if (p.vdim == 0 || p.vdim > 256) return ctx.fail("latent attention: v_head_dim must be 1 to 256");
    if (p.heads == 0) return ctx.fail("latent attention: no heads");
    if (reinterpret_cast<uintptr_t>(p.latent) % 16) return ctx.fail("latent attention: latents must be 16-byte aligned");
    if (p.count == 0) return true;
    if (p.count > 0x7FFFFFFFull || p.heads > 65535u) return ctx.fail("latent attention: too many tokens or heads");
    LatentArgs a{};
    a.p = p;
    const uint32_t groups = uint32_t((p.heads + HG - 1) / HG);
    // decode-sized calls split the keys so that about 256 workgroups run
    const uint64_t maxKeys = p.startPos + p.count;
    const uint64_t maxBlocks = (maxKeys + KPB - 1) / KPB;
    uint64_t want = (256 + p.count * groups - 1) / (p.count * groups);
    if (want > maxBlocks) want = maxBlocks;
    if (want < 1) want = 1;
    if (want > 64) want = 64;
    const uint64_t per = (maxBlocks + want - 1) / want;
    a.splits = uint32_t((maxBlocks + per - 1) / per);   // every split of the longest token has blocks
    const size_t cells = size_t(p.count) * p.heads * p.rank;
    const size_t bytes = (2 * cells + (a.splits > 1 ? size_t(p.count) * p.heads * a.splits * (p.rank + 2) : 0)) * 4;
    float* work = static_cast<float*>(ctx.grow(SLOT_LATENT, bytes));
    if (!work) return false;
    a.folded = work;
    a.context = work + cells;
    a.partial = work + 2 * cells;
    const bool bf16 = p.wType == 1;
    const dim3 fgrid(unsigned(p.heads), unsigned((p.rank + WAVE - 1) / WAVE), unsigned((p.count + TT - 1) / TT));
    if (fgrid.z > 65535u) return ctx.fail("latent attention: too many tokens for one call");
    if (!ctx.launch("latent_fold_kernel", stream, [&] {
            if (bf16) hipLaunchKernelGGL(latent_fold_kernel<true>, fgrid, dim3(256), 0, stream, a);
            else hipLaunchKernelGGL(latent_fold_kernel<false>, fgrid, dim3(256), 0, stream, a);
        }))
        return false;
    if (!ctx.launch("latent_attn_kernel", stream, [&] {
            hipLaunchKernelGGL(latent_attn_kernel, dim3(unsigned(p.count), groups, a.splits), dim3(256), 0, stream, a);
        }))
        return false;
    if (a.splits > 1 && !ctx.launch("latent_merge_kernel", stream, [&] {
            hipLaunchKernelGGL(latent_merge_kernel, dim3(unsigned(p.count), unsigned(p.heads)), dim3(256), 0, stream, a);
        }))
        return false;
    const dim3 ugrid(unsigned(p.heads), unsigned((p.count + TT - 1) / TT));
    return ctx.launch("latent_unfold_kernel", stream, [&] {
        if (bf16) hipLaunchKernelGGL(latent_unfold_kernel<true>, ugrid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL(latent_unfold_kernel<false>, ugrid, dim3(256), 0, stream, a);
    });
}

} // namespace aigpu
