// dense.hip - the resident single-token decoder behind aigpu_dense_*
// (DeviceABI.h:119-152): a dense RMSNorm / RoPE / SwiGLU model (Qwen3,
// Llama) kept on the device between tokens, so one decode step moves only the
// embedding in and the logits out. The reference's HIP backend stubs these
// entry points (Kernels.hip:636-641); LocalModel::residentDecode
// (LocalModel.hpp:3598-3645) is the caller, and the step is LocalModel::
// forward's layer loop for count = 1 (:3705-3799).
//
// Per layer, six launches on one stream:
//   dense_gemv_kernel   q, k, v (+ bias) of RMSNorm(x) * inputNorm, the
//                       normalised row built once per workgroup in LDS
//   dense_attn_kernel   per (span of positions, kv head): q/k RMSNorm and
//                       RoPE at the position, the k, v rows appended to the
//                       cache, split-K attention for all of the kv head's
//                       query heads
//   dense_merge_kernel  the splits combined per kv head
//   dense_gemv_kernel   x += o . attn
//   dense_gemv_kernel   gate, up of RMSNorm(x) * postNorm
//   dense_gemv_kernel   x += down . (silu(gate) * up)
// then the head of RMSNorm(x) * finalNorm. The position is read from device
// memory by the kernels that need it, so the sequence does not depend on
// host values that change between tokens.
//
// The cache is the reference's own layout, fp32 [capacity][kvHeads * headDim]
// per layer (what aigpu_dense_create copies in and aigpu_dense_read_cache
// copies out).
#include <chrono>
#include <cstdlib>
#include <cmath>
#include <cstring>
#include <initializer_list>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "context.hpp"
#include "device.hpp"
#include "gemv.hpp"
#include "kernels.hpp"

namespace aigpu {

namespace {

constexpr int PW_MAX = 40;     // positions per wave and pass of the attention
constexpr int MAX_DIM = 256;   // head dim
constexpr int MAX_GROUP = 8;   // query heads per kv head

struct DenseArgs {
    const uint32_t* pos;   // device: the position being decoded
    uint32_t heads, kvHeads, dim, rot, maxSplits, window, capacity;
    float eps;
};

/* ---- projections with the step before them fused into the input ----
   PRE 0: a = x;  PRE 1: a = RMSNorm(x) * gamma (rmsNormRow,
   LocalModel.hpp:1341-1348), the workgroup computing the norm once;
   PRE 2: a = silu(x) * x2 (swiglu, :3282-3288).
   Up to three weights of one encoding share the launch (q, k, v; gate, up):
   rows [start_s, start_s + n_s) belong to segment s. */
constexpr int DG_ROWS = 2;   // weight rows per wave, at most

struct DenseSeg {
    const char* w;
    const float* scales;
    const float* bias;
    float* out;
    uint32_t n, start;
};

struct DenseGemvArgs {
    DenseSeg seg[3];
    int nseg, accumulate;
    uint32_t rows, k;
    const float* x;
    const float* x2;
    const float* gamma;
    float eps;
};

constexpr int DG_LDS_K = 12288;   // activation floats staged in LDS (at most 48 KB, sized to k)
constexpr int DG_BATCH = 8;       // weight pieces per lane and row loaded together

/* The workgroup first requests each wave's first DG_BATCH weight pieces,
   then builds the activation (PRE applied) once in LDS, then the waves dot
   their rows against it; k up to DG_LDS_K. */
template <int TYPE, int PRE, int ROWS>   // ROWS weight rows per wave: 2, or 1 for short weights
__global__ __launch_bounds__(256) void dense_gemv_kernel(DenseGemvArgs p) {
    static_assert(ROWS == 1 || ROWS == DG_ROWS, "one or two rows per wave");
    constexpr int E = piece_elems<TYPE>();
    extern __shared__ __align__(16) float xa[];   // k floats
    __shared__ float part[4];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint32_t row0 = (blockIdx.x * 4 + w) * ROWS;
    const bool active = row0 < p.rows;
    int sg = 0;
    if (p.nseg > 1 && row0 >= p.seg[1].start) sg = 1;
    if (p.nseg > 2 && row0 >= p.seg[2].start) sg = 2;
    const DenseSeg S = p.seg[sg];
    const uint32_t r0 = active ? row0 - S.start : 0;   // ROWS rows never straddle segments (every n is even)
    const size_t rowBytes = size_t(p.k) * row_bytes_per_k_x2<TYPE>() / 2;
    const uint32_t pieces = p.k / E, blocks = p.k / 32;
    const uint32_t rr1 = r0 + 1 < S.n ? r0 + 1 : r0;   // a row count that is odd repeats the last row

    // the first batch of weight pieces, before anything waits (nontemporal:
    // each weight byte is read once per token)
    u32x4 wv[DG_BATCH][ROWS];
#pragma unroll
    for (int b = 0; b < DG_BATCH; ++b) {
        const uint32_t c = lane + WAVE * b;
        if (active && c < pieces) {
            wv[b][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(S.w + r0 * rowBytes + size_t(c) * 16));
            if constexpr (ROWS == 2)
                wv[b][1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(S.w + rr1 * rowBytes + size_t(c) * 16));
        }
    }

    // the activation, once per workgroup
    float inv = 1.0f;
    if constexpr (PRE == 1) {
        float ss = 0.0f;
        for (uint32_t i = tid; i < p.k / 4; i += 256) {
            const floatx4 v = reinterpret_cast<const floatx4*>(p.x)[i];
            ss = fmaf(v[0], v[0], fmaf(v[1], v[1], fmaf(v[2], v[2], fmaf(v[3], v[3], ss))));
        }
        ss = wave_sum(ss);
        if (lane == 0) part[w] = ss;
        __syncthreads();
        inv = 1.0f / sqrtf((part[0] + part[1] + part[2] + part[3]) / float(p.k) + p.eps);
    }
    for (uint32_t i = tid; i < p.k / 4; i += 256) {
        const floatx4 v = reinterpret_cast<const floatx4*>(p.x)[i];
        floatx4 o;
        if constexpr (PRE == 1) {
            const floatx4 gm = reinterpret_cast<const floatx4*>(p.gamma)[i];
#pragma unroll
            for (int t = 0; t < 4; ++t) o[t] = v[t] * inv * gm[t];
        } else if constexpr (PRE == 2) {
            const floatx4 u = reinterpret_cast<const floatx4*>(p.x2)[i];
#pragma unroll
            for (int t = 0; t < 4; ++t) o[t] = v[t] / (1.0f + expf(-v[t])) * u[t];
        } else {
            o = v;
        }
        reinterpret_cast<floatx4*>(xa)[i] = o;
    }
    __syncthreads();
    if (!active) return;

    float acc[ROWS] = {};
    const float* s0 = TYPE >= 2 ? S.scales + size_t(r0) * blocks : nullptr;
    const float* s1 = TYPE >= 2 ? S.scales + size_t(rr1) * blocks : nullptr;
    for (uint32_t c0 = 0; c0 < pieces; c0 += WAVE * DG_BATCH) {
        if (c0 > 0) {
#pragma unroll
            for (int b = 0; b < DG_BATCH; ++b) {
                const uint32_t c = c0 + lane + WAVE * b;
                if (c < pieces) {
                    wv[b][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(S.w + r0 * rowBytes + size_t(c) * 16));
                    if constexpr (ROWS == 2)
                        wv[b][1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(S.w + rr1 * rowBytes + size_t(c) * 16));
                }
            }
        }
#pragma unroll
        for (int b = 0; b < DG_BATCH; ++b) {
            const uint32_t c = c0 + lane + WAVE * b;
            if (c < pieces) {
                const float* x = xa + size_t(c) * E;
#pragma unroll
                for (int r = 0; r < ROWS; ++r) {
                    const float d = piece_dot<TYPE>(wv[b][r], x);
                    if constexpr (TYPE == 2) acc[r] = fmaf(d, (r ? s1 : s0)[c >> 1], acc[r]);
                    else if constexpr (TYPE == 3) acc[r] = fmaf(d, (r ? s1 : s0)[c], acc[r]);
                    else acc[r] += d;
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r) acc[r] = wave_sum(acc[r]);
    if (lane < ROWS) {
        const uint32_t n = r0 + lane;
        if (n < S.n) {
            const float v = lane == 0 ? acc[0] : acc[ROWS - 1];
            float* o = S.out + n;
            *o = (p.accumulate ? *o : 0.0f) + v + (S.bias ? S.bias[n] : 0.0f);
        }
    }
}

/* ---- attention ----
   Keys [first(pos), pos] in `splits` contiguous ranges of P positions per kv
   head (the last one shorter), one workgroup each: at most 256 workgroups
   (one per CU: 264 for 33 ranges of 128 put two on eight CUs, whose waves
   then set the kernel's length) and at least 32 positions per range. A
   workgroup takes its range in passes of at most 4 x PW_MAX positions,
   with an online softmax across them. Workgroup (split s, kv head):
   - norms and rotates the G query heads of the kv head itself (attentionMixer,
     LocalModel.hpp:2606-2648) and, in the split holding `pos`, the new key,
     appending it and the value row to the cache;
   - per pass, each wave takes a quarter of the positions (up to PW_MAX)
     with a softmax state of its own (no barrier inside the pass loop): every key and value load of
     the wave is issued before anything waits, the keys eight lanes to a row
     so that one load instruction covers 8 rows x 128 contiguous bytes;
     scores, probabilities and P.V stay in the wave's registers;
   - combines the four waves into one record per query head: max, sum, pad,
     acc[D] (D + 4 floats, so acc is 16-byte aligned). */
constexpr int MAX_SPLITS = 64;
constexpr int REC_PAD = 4;   // max, sum, two unused floats before acc
constexpr int BUFFER_FLAGS = 0x00020000;   // buffer descriptor word 3: 32-bit data format, raw (stride 0) access

constexpr uint32_t MIN_RANGE = 32;   // positions per split, at least

/* the attention's ranges at `pos`: positions [first, pos], `splits` of them
   per kv head, P positions each (the last one what is left, at least one:
   splits (splits - 1) < pos + 1 - first for every splits this picks) */
__host__ __device__ __forceinline__ void attn_span(uint32_t pos, uint32_t window, uint32_t kvHeads, uint32_t& first,
                                                   uint32_t& splits, uint32_t& P) {
    first = window && pos + 1 > window ? pos + 1 - window : 0;
    const uint32_t range = pos + 1 - first;
    uint32_t target = 256 / kvHeads;
    target = target < 1 ? 1 : (target > uint32_t(MAX_SPLITS) ? uint32_t(MAX_SPLITS) : target);
    const uint32_t most = (range + MIN_RANGE - 1) / MIN_RANGE;
    splits = most < target ? most : target;
    P = (range + splits - 1) / splits;
}

/* the sum over each group of 8 lanes (lanes 8i .. 8i + 7), in every lane of
   the group: quad_perm xor 1, quad_perm xor 2, then row_half_mirror, which
   pairs each lane of a quad with one of the other quad */
__device__ __forceinline__ float sum8(float x) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xf, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xf, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xf, 0xf, false));
    return x;
}

/* over lanes l, l ^ 8, l ^ 16, ..., l ^ 56 (the eight groups' lane l % 8):
   row_ror 8 swaps the halves of each 16-lane row, then two cross-row steps */
__device__ __forceinline__ float max_across8(float x) {
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false)));
    x = fmaxf(x, __shfl_xor(x, 16, WAVE));
    return fmaxf(x, __shfl_xor(x, 32, WAVE));
}
__device__ __forceinline__ float sum_across8(float x) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false));
    x += __shfl_xor(x, 16, WAVE);
    return x + __shfl_xor(x, 32, WAVE);
}

template <int DPL, int GMAX>   // value dimensions per lane: 2 (D <= 128) or 4 (D <= 256); G <= GMAX
__global__ __launch_bounds__(256) void dense_attn_kernel(DenseArgs a, const float* qRaw, const float* kRaw,
                                                         const float* vRaw, const float* qNorm, const float* kNorm,
                                                         const float* freqs, float* keys, float* values,
                                                         float* partial) {
    constexpr int KE = 2 * DPL;   // 16-byte key pieces per lane and row (32 floats apart)
    // rows per wave and pass, at most: 40, or 32 where the query heads' state
    // would not fit the registers (a range past 128 positions then takes two
    // passes)
    constexpr int PW = DPL * GMAX <= 8 ? PW_MAX : 32;
    constexpr int RG = PW / 8;    // groups of 8 rows
    static_assert(PW == RG * 8 && PW <= PW_MAX, "a wave's rows are RG groups of 8");
    constexpr int QPT = GMAX * MAX_DIM / 256;   // query floats per thread, at most
    __shared__ __align__(16) float qs[GMAX * MAX_DIM];
    __shared__ __align__(16) float kn[MAX_DIM];
    __shared__ __align__(16) float vn[MAX_DIM];
    __shared__ __align__(16) float pb[4][PW];   // a wave's probabilities, broadcast to its lanes
    __shared__ float wm[4][GMAX], wl[4][GMAX];
    __shared__ __align__(16) float wacc[4][GMAX * MAX_DIM];

    const uint32_t pos = *a.pos;
    uint32_t first, splits, P;
    attn_span(pos, a.window, a.kvHeads, first, splits, P);
    const uint32_t s = blockIdx.x, kvh = blockIdx.y;
    if (s >= splits) return;   // whole workgroup leaves before any barrier
    const uint32_t G = a.heads / a.kvHeads, D = a.dim;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform, so row offsets stay scalar
    const size_t kvW = size_t(a.kvHeads) * D;
    const float scale = 1.0f / sqrtf(float(D));
    const bool holdsPos = s + 1 == splits;
    const uint32_t sub = lane & 7, rl = lane >> 3;   // key layout: row rl of a group, floats 4 sub + 32 e
    const bool vlive = uint32_t(DPL * lane) < D;     // value layout: floats DPL lane .. + DPL - 1
    // the layer's cache through buffer descriptors: a lane offset in a VGPR,
    // the row in a scalar offset (byte offsets fit 32 bits: checked at
    // creation); cache policy 2, nontemporal: each row is read once per step
    const uint32_t cacheBytes = uint32_t((a.capacity * kvW + MAX_DIM) * sizeof(float));
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(keys, 0, cacheBytes, BUFFER_FLAGS);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(values, 0, cacheBytes, BUFFER_FLAGS);
    const uint32_t rowBytes = uint32_t(kvW * sizeof(float));
    // pieces past D read on into the next head or row (the cache carries
    // MAX_DIM floats of padding, so the last row's stay inside it) and are zeroed
    bool kLive[KE];
#pragma unroll
    for (int e = 0; e < KE; ++e) kLive[e] = 4 * sub + 32 * e < D;
    const uint32_t kOff = uint32_t((kvh * D + 4 * sub) * sizeof(float));
    const uint32_t vOff = uint32_t((kvh * D + (vlive ? DPL * lane : 0)) * sizeof(float));

    // the raw query rows and new key/value rows first, so that their use
    // below does not wait for the cache loads issued after them
    float qr[QPT], knr = 0.0f, vnr = 0.0f;
#pragma unroll
    for (int t = 0; t < QPT; ++t) {
        const uint32_t i = uint32_t(tid) + 256 * t;
        qr[t] = i < G * D ? qRaw[size_t(kvh) * G * D + i] : 0.0f;
    }
    if (holdsPos && uint32_t(tid) < D) {
        knr = kRaw[size_t(kvh) * D + tid];
        vnr = vRaw[size_t(kvh) * D + tid];
    }

    float mrun[GMAX], lrun[GMAX], acc[GMAX][DPL];
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
        mrun[g] = -INFINITY;
        lrun[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[g][e] = 0.0f;
    }
    // this split's positions [j0s, j0s + rows), in passes of R (a quarter to each wave)
    const uint32_t j0s = first + s * P;
    const uint32_t rows = pos + 1 - j0s < P ? pos + 1 - j0s : P;
    const uint32_t passes = (rows + 4 * PW - 1) / (4 * PW);
    const uint32_t R = (rows + passes - 1) / passes;
    const uint32_t pw = (R + 3) / 4;   // rows per wave, <= PW
#pragma unroll 1
    for (uint32_t c = 0; c < passes; ++c) {
        const uint32_t j0 = j0s + c * R;
        const uint32_t n = rows - c * R < R ? rows - c * R : R;      // positions in this pass
        const uint32_t jp = pos - j0 < n ? pos - j0 : 0xFFFFFFFFu;   // the new position, if in this pass
        const uint32_t r0 = uint32_t(w) * pw;                        // the wave's rows r0 .. r0 + pw - 1
        auto live = [&](uint32_t u) { return u < pw && r0 + u < n; };

        // every key and value load of the wave's rows; rows not live read row 0
        // of the pass (finite: the cache is zeroed at creation) and are masked
        floatx4 k4[RG][KE];
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) {
            const uint32_t u = 8 * rg + rl;
            const uint32_t off = (j0 + (live(u) ? r0 + u : 0)) * rowBytes + kOff;
#pragma unroll
            for (int e = 0; e < KE; ++e)
                k4[rg][e] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(krs, off + 128 * e, 0, 2));
        }
        float vv[PW][DPL];
        // value rows from the wave's first row on, in a lane offset; row u in the
        // scalar offset. Rows past the wave's pw are not read (zeros); the
        // last wave's rows past n are read as they are (later positions' rows,
        // zero rows never written, or past the descriptor's end, where the
        // load returns 0: finite, and their probabilities are 0)
        const uint32_t vRow0 = vOff + (j0 + r0) * rowBytes;
#pragma unroll
        for (int u = 0; u < PW; ++u) {
            if (uint32_t(u) >= pw) {   // uniform
#pragma unroll
                for (int e = 0; e < DPL; ++e) vv[u][e] = 0.0f;
            } else if constexpr (DPL == 2) {
                const float2 t = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(vrs, vRow0, u * rowBytes, 2));
                vv[u][0] = t.x;
                vv[u][1] = t.y;
            } else {
                const floatx4 t = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(vrs, vRow0, u * rowBytes, 2));
#pragma unroll
                for (int e = 0; e < DPL; ++e) vv[u][e] = t[e];
            }
        }

        if (c == 0) {   // uniform: the query rows normed and rotated while the loads are in flight
#pragma unroll
            for (int t = 0; t < QPT; ++t) {
                const uint32_t i = uint32_t(tid) + 256 * t;
                if (i < G * D) qs[i] = qr[t];
            }
            if (holdsPos && uint32_t(tid) < D) {
                kn[tid] = knr;
                vn[tid] = vnr;
            }
            lds_barrier();
            for (uint32_t g = w; g < G; g += 4)
                norm_rope_row(&qs[g * D], int(D), qNorm, a.eps, 0.0f, freqs, int(a.rot), pos, lane);
            if (holdsPos && w == int(G % 4)) {
                norm_rope_row(kn, int(D), kNorm, a.eps, 0.0f, freqs, int(a.rot), pos, lane);
                for (uint32_t d = lane; d < D; d += WAVE) {
                    keys[size_t(pos) * kvW + size_t(kvh) * D + d] = kn[d];
                    values[size_t(pos) * kvW + size_t(kvh) * D + d] = vn[d];
                }
            }
            lds_barrier();
        }
        if (jp - r0 < pw) {   // uniform: the new position is one of this wave's rows; from LDS
            const uint32_t ju = jp - r0;
#pragma unroll
            for (int rg = 0; rg < RG; ++rg)
                if (8 * rg + rl == ju) {
#pragma unroll
                    for (int e = 0; e < KE; ++e)
                        if (kLive[e]) k4[rg][e] = *reinterpret_cast<const floatx4*>(&kn[4 * sub + 32 * e]);
                }
#pragma unroll
            for (int u = 0; u < PW; ++u)
                if (u == int(ju)) {
#pragma unroll
                    for (int e = 0; e < DPL; ++e) vv[u][e] = vn[vlive ? DPL * lane + e : e];
                }
        }
#pragma unroll
        for (int rg = 0; rg < RG; ++rg)
#pragma unroll
            for (int e = 0; e < KE; ++e)
                if (!kLive[e]) k4[rg][e] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
            if (g >= int(G)) break;   // uniform
            // scores: the 8 lanes of a row sum their pieces
            float sc[RG];
#pragma unroll
            for (int rg = 0; rg < RG; ++rg) sc[rg] = 0.0f;
#pragma unroll
            for (int e = 0; e < KE; ++e) {
                // past D: the next query head's or unwritten LDS (in qs's bounds), zeroed
                floatx4 q4 = *reinterpret_cast<const floatx4*>(&qs[g * D + 4 * sub + 32 * e]);
                if (!kLive[e]) q4 = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int rg = 0; rg < RG; ++rg)
                    sc[rg] = fmaf(q4[0], k4[rg][e][0],
                                  fmaf(q4[1], k4[rg][e][1], fmaf(q4[2], k4[rg][e][2], fmaf(q4[3], k4[rg][e][3], sc[rg]))));
            }
            float m = -INFINITY;
#pragma unroll
            for (int rg = 0; rg < RG; ++rg) {
                sc[rg] = live(uint32_t(8 * rg + rl)) ? sum8(sc[rg]) * scale : -INFINITY;
                m = fmaxf(m, sc[rg]);
            }
            m = max_across8(m);
            // the wave's running max; -inf until the wave has seen a position
            const float mn = fmaxf(mrun[g], m);
            const float f = mrun[g] == -INFINITY ? 0.0f : expf(mrun[g] - mn);
            float l = 0.0f;
#pragma unroll
            for (int rg = 0; rg < RG; ++rg) {
                sc[rg] = sc[rg] == -INFINITY ? 0.0f : expf(sc[rg] - mn);
                l += sc[rg];
            }
            l = sum_across8(l);
            mrun[g] = mn;
            lrun[g] = lrun[g] * f + l;
#pragma unroll
            for (int e = 0; e < DPL; ++e) acc[g][e] *= f;
            // P.V: the probabilities through LDS, read back as broadcasts
            if (sub == 0) {
#pragma unroll
                for (int rg = 0; rg < RG; ++rg) pb[w][8 * rg + rl] = sc[rg];
            }
            wave_sync();
#pragma unroll
            for (int u4 = 0; u4 < PW / 4; ++u4) {
                const floatx4 p4 = *reinterpret_cast<const floatx4*>(&pb[w][4 * u4]);
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int e = 0; e < DPL; ++e) acc[g][e] = fmaf(p4[t], vv[4 * u4 + t][e], acc[g][e]);
            }
            wave_sync();   // pb is rewritten by the next query head
        }
    }

    // the split's record per query head: the four waves combined
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
        if (g >= int(G)) break;   // uniform
        if (lane == 0) {
            wm[w][g] = mrun[g];
            wl[w][g] = lrun[g];
        }
        if (vlive) {
#pragma unroll
            for (int e = 0; e < DPL; ++e) wacc[w][g * D + DPL * lane + e] = acc[g][e];
        }
    }
    __syncthreads();
    const size_t rec = size_t(D) + REC_PAD;
    for (uint32_t i = tid; i < G * D; i += 256) {
        const uint32_t g = i / D, d = i - g * D;
        // wave 0 always holds position j0s (pw >= 1), so M is finite
        const float M = fmaxf(fmaxf(wm[0][g], wm[1][g]), fmaxf(wm[2][g], wm[3][g]));
        float v = 0.0f;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) v = fmaf(wacc[ww][i], expf(wm[ww][g] - M), v);
        float* out = partial + ((size_t(kvh) * G + g) * a.maxSplits + s) * rec;
        out[REC_PAD + d] = v;
        if (d == 0) {
            float L = 0.0f;
#pragma unroll
            for (int ww = 0; ww < 4; ++ww) L = fmaf(wl[ww][g], expf(wm[ww][g] - M), L);
            out[0] = M;
            out[1] = L;
        }
    }
}


/* the splits' records of one query head combined (a launch of its own: a
   workgroup-to-workgroup handoff inside the attention kernel needs a
   device-scope fence, which on this part writes back the L2). Workgroup
   (query head in the group, kv head); every load issued at once. */
__global__ __launch_bounds__(256) void dense_merge_kernel(DenseArgs a, const float* partial, float* attn) {
    constexpr int MAXT = MAX_SPLITS / 4;   // splits per thread when D = 256
    __shared__ floatx4 red[256];
    const uint32_t pos = *a.pos;
    uint32_t first, splits, P;
    attn_span(pos, a.window, a.kvHeads, first, splits, P);
    const uint32_t g = blockIdx.x, kvh = blockIdx.y, G = a.heads / a.kvHeads, D = a.dim;
    const int tid = threadIdx.x, lane = tid & 63;
    const size_t rec = size_t(D) + REC_PAD;
    const uint32_t quads = D / 4, RL = 256 / quads;   // D % 4 == 0, D <= 256: RL >= 4
    const uint32_t dq = tid % quads, r = tid / quads;
    const float* base = partial + (size_t(kvh) * G + g) * a.maxSplits * rec;
    const bool mine = uint32_t(lane) < splits;
    const float mi = mine ? base[size_t(lane) * rec] : -INFINITY;
    const float li = mine ? base[size_t(lane) * rec + 1] : 0.0f;
    floatx4 v[MAXT];
#pragma unroll
    for (int t = 0; t < MAXT; ++t) {
        const uint32_t i = r + RL * t;
        v[t] = r < RL && i < splits ? *reinterpret_cast<const floatx4*>(base + i * rec + REC_PAD + 4 * dq)
                                    : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    const float M = wave_max(mi);
    const float L = wave_sum(li * expf(mi - M));
    floatx4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < MAXT; ++t) {
        const uint32_t i = r + RL * t;
        const float fi = __shfl(mi, int(i < splits ? i : 0), WAVE);
        if (r < RL && i < splits) {
            const float e = expf(fi - M);
#pragma unroll
            for (int k = 0; k < 4; ++k) sum[k] = fmaf(v[t][k], e, sum[k]);
        }
    }
    red[tid] = sum;
    __syncthreads();
    if (tid < int(quads)) {
        floatx4 t = red[tid];
        for (uint32_t rr = 1; rr < RL; ++rr) {
            const floatx4 u = red[rr * quads + tid];
#pragma unroll
            for (int k = 0; k < 4; ++k) t[k] += u[k];
        }
        const float inv = 1.0f / L;
        *reinterpret_cast<floatx4*>(attn + (size_t(kvh) * G + g) * D + 4 * tid) =
            floatx4{t[0] * inv, t[1] * inv, t[2] * inv, t[3] * inv};
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

/* one captured decode step: the step's kernels for a given attention grid,
   replayed as a HIP graph (the kernels read the position from device memory,
   so one capture serves every position with the same grid) */
struct StepGraph {
    uint32_t splits = 0;
    hipGraphExec_t exec = nullptr;
    uint64_t launches = 0;   // kernels per replay
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
    // the decoder's own stream (blocking: ordered after the legacy default
    // stream, where callers upload weights) and its captured steps
    hipStream_t stream = nullptr;
    std::vector<StepGraph> graphs;

    ~DenseModel() {
        for (StepGraph& g : graphs)
            if (g.exec) (void)hipGraphExecDestroy(g.exec);
        if (stream) (void)hipStreamDestroy(stream);
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
        if (!w.codes || w.type > 3 || (w.type >= 2 && (!w.scales || w.inDim % 32)) || w.inDim % 4 ||
            (w.type == 1 && w.inDim % 8) || (reinterpret_cast<uintptr_t>(w.codes) % 16) ||
            w.inDim > uint32_t(DG_LDS_K))
            throw std::invalid_argument(std::string("resident ") + what +
                                        " weight is not usable (bf16 rows need inDim % 8, quantised inDim % 32, "
                                        "inDim at most 12288, and the codes 16-byte aligned)");
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

struct Seg {
    const DevWeight* w;
    float* out;
};

template <int TYPE, int PRE>
void launch_dense_gemv(const DenseGemvArgs& p, hipStream_t stream) {
    // one row per wave where two would leave CUs without a workgroup
    const uint32_t grid2 = (p.rows + 4 * DG_ROWS - 1) / (4 * DG_ROWS);
    if (grid2 < 256) {
        hipLaunchKernelGGL((dense_gemv_kernel<TYPE, PRE, 1>), dim3((p.rows + 3) / 4), dim3(256), size_t(p.k) * sizeof(float),
                           stream, p);
    } else {
        hipLaunchKernelGGL((dense_gemv_kernel<TYPE, PRE, DG_ROWS>), dim3(grid2), dim3(256), size_t(p.k) * sizeof(float),
                           stream, p);
    }
}

/* one launch for weights of one encoding whose row counts are even (rows
   of a wave never straddle two of them); otherwise one launch per weight */
bool dense_gemv(std::initializer_list<Seg> segs, const float* x, const float* x2, const float* gamma, float eps,
                int pre, bool accumulate, hipStream_t stream) {
    const Seg* sv = segs.begin();
    const size_t ns = segs.size();
    bool together = ns <= 3;
    for (size_t i = 0; i < ns; ++i)
        if (sv[i].w->type != sv[0].w->type || sv[i].w->in != sv[0].w->in || (ns > 1 && sv[i].w->out % 2)) together = false;
    if (!together) {
        for (size_t i = 0; i < ns; ++i)
            if (!dense_gemv({sv[i]}, x, x2, gamma, eps, pre, accumulate, stream)) return false;
        return true;
    }
    DenseGemvArgs p{};
    uint32_t start = 0;
    for (size_t i = 0; i < ns; ++i) {
        p.seg[i] = {static_cast<const char*>(sv[i].w->codes), sv[i].w->scales, sv[i].w->bias, sv[i].out, sv[i].w->out, start};
        start += sv[i].w->out;
    }
    p.nseg = int(ns);
    p.rows = start;
    p.k = sv[0].w->in;
    p.accumulate = accumulate ? 1 : 0;
    p.x = x;
    p.x2 = x2;
    p.gamma = gamma;
    p.eps = eps;
    const int type = sv[0].w->type;
    return Context::instance().launch("dense_gemv_kernel", stream, [&] {
#define AIGPU_DG(T)                                                                                          \
    if (type == T) {                                                                                         \
        if (pre == 0) launch_dense_gemv<T, 0>(p, stream);                                                    \
        else if (pre == 1) launch_dense_gemv<T, 1>(p, stream);                                               \
        else launch_dense_gemv<T, 2>(p, stream);                                                             \
    }
        AIGPU_DG(0) AIGPU_DG(1) AIGPU_DG(2) AIGPU_DG(3)
#undef AIGPU_DG
    });
}

/* the workgroups per kv head of the attention of a step at `pos` */
uint32_t host_splits(uint32_t pos, uint32_t window, uint32_t kvHeads) {
    uint32_t first, splits, P;
    attn_span(pos, window, kvHeads, first, splits, P);
    return splits;
}

/* the launches of one decode step; `splits` attention workgroups per kv head
   (the most any layer needs; the others leave at once) */
bool run_step(DenseModel& d, uint32_t splits, hipStream_t stream) {
    Context& ctx = Context::instance();
    const AiGpuDenseConfig& c = d.cfg;
    DenseArgs a{d.pos, c.heads, c.kvHeads, c.headDim, c.rotaryDims, d.maxSplits, 0, c.capacity, c.epsilon};
    for (const DevLayer& L : d.layers) {
        a.window = L.window;
        if (!dense_gemv({{&L.q, d.q}, {&L.k, d.k}, {&L.v, d.v}}, d.x, nullptr, L.inputNorm, c.epsilon, 1, false, stream))
            return false;
        if (!ctx.launch("dense_attn_kernel", stream, [&] {
                const dim3 grid(splits, c.kvHeads);
                const uint32_t G = c.heads / c.kvHeads;
#define AIGPU_DA(DPL, GM)                                                                                   \
    hipLaunchKernelGGL((dense_attn_kernel<DPL, GM>), grid, dim3(256), 0, stream, a, d.q, d.k, d.v, L.qNorm, \
                       L.kNorm, d.freqs, L.keys, L.values, d.partial)
                if (c.headDim <= 128) {
                    if (G <= 2) AIGPU_DA(2, 2);
                    else if (G <= 4) AIGPU_DA(2, 4);
                    else AIGPU_DA(2, 8);
                } else {
                    if (G <= 2) AIGPU_DA(4, 2);
                    else if (G <= 4) AIGPU_DA(4, 4);
                    else AIGPU_DA(4, 8);
                }
#undef AIGPU_DA
            }))
            return false;
        if (!ctx.launch("dense_merge_kernel", stream, [&] {
                hipLaunchKernelGGL(dense_merge_kernel, dim3(c.heads / c.kvHeads, c.kvHeads), dim3(256), 0, stream, a,
                                   d.partial, d.attn);
            }))
            return false;
        if (!dense_gemv({{&L.o, d.x}}, d.attn, nullptr, nullptr, 0.0f, 0, true, stream)) return false;
        if (!dense_gemv({{&L.gate, d.gate}, {&L.up, d.up}}, d.x, nullptr, L.postNorm, c.epsilon, 1, false, stream))
            return false;
        if (!dense_gemv({{&L.down, d.x}}, d.gate, d.up, nullptr, 0.0f, 2, true, stream)) return false;
    }
    return dense_gemv({{&d.head, d.logits}}, d.x, nullptr, d.finalNorm, c.epsilon, 1, false, stream);
}

/* the step for `splits`, as a replayed graph: captured on first use of each
   attention grid (the grid grows by one workgroup per kv head every 32
   positions up to 256 / kvHeads, at most 64, so a sequence captures at most
   64 graphs). Without
   graphs (AIGPU_DENSE_GRAPH=0, or profiling, whose per-launch events a graph
   cannot carry) the kernels are launched one by one. */
bool launch_step(DenseModel& d, uint32_t splits) {
    Context& ctx = Context::instance();
    const char* env = std::getenv("AIGPU_DENSE_GRAPH");
    if (ctx.profiling || (env && std::atoi(env) == 0)) return run_step(d, splits, d.stream);
    StepGraph* g = nullptr;
    for (StepGraph& x : d.graphs)
        if (x.splits == splits) g = &x;
    if (!g) {
        const uint64_t before = ctx.stats.launches;
        if (hipStreamBeginCapture(d.stream, hipStreamCaptureModeThreadLocal) != hipSuccess) {
            (void)hipGetLastError();
            return ctx.fail("resident decode: graph capture could not begin");
        }
        const bool ok = run_step(d, splits, d.stream);
        hipGraph_t graph = nullptr;
        const hipError_t e = hipStreamEndCapture(d.stream, &graph);
        if (!ok || e != hipSuccess || !graph) {
            (void)hipGetLastError();
            if (graph) (void)hipGraphDestroy(graph);
            return ok ? ctx.fail("resident decode: graph capture failed") : false;
        }
        StepGraph fresh;
        fresh.splits = splits;
        fresh.launches = ctx.stats.launches - before;
        const hipError_t ie = hipGraphInstantiate(&fresh.exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (ie != hipSuccess) {
            (void)hipGetLastError();
            return ctx.fail(std::string("resident decode: graph instantiation failed: ") + hipGetErrorString(ie));
        }
        ctx.stats.launches = before;   // counted per replay below
        d.graphs.push_back(fresh);
        g = &d.graphs.back();
    }
    if (hipGraphLaunch(g->exec, d.stream) != hipSuccess) {
        (void)hipGetLastError();
        return ctx.fail("resident decode: graph launch failed");
    }
    ctx.stats.launches += g->launches;
    return true;
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
        // 32-bit buffer offsets over the cache and its one head row of padding
        if ((uint64_t(c->capacity) * c->kvHeads * c->headDim + aigpu::MAX_DIM) * sizeof(float) >= (uint64_t(1) << 32))
            throw std::invalid_argument("resident decoder cache over 4 GiB per layer (capacity * kvHeads * headDim * 4)");
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
        d->maxSplits = aigpu::host_splits(c->capacity - 1, 0, c->kvHeads);
        d->partial = d->floats(uint64_t(c->heads) * d->maxSplits * (c->headDim + aigpu::REC_PAD));
        d->pos = reinterpret_cast<uint32_t*>(d->floats(1));
        if (hipStreamCreate(&d->stream) != hipSuccess) {
            (void)hipGetLastError();
            throw std::runtime_error("resident decoder stream creation failed");
        }
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
            // one head row of padding: the attention's key pieces past headDim
            // read into it (and are zeroed) when headDim is not 128 or 256
            L.keys = d->floats(uint64_t(c->capacity) * kw + aigpu::MAX_DIM, keys[i], uint64_t(length) * kw);
            L.values = d->floats(uint64_t(c->capacity) * kw + aigpu::MAX_DIM, values[i], uint64_t(length) * kw);
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
    const hipStream_t stream = d.stream;
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
        const uint32_t s = aigpu::host_splits(position, L.window, c.kvHeads);
        if (s > splits) splits = s;
    }
    if (!aigpu::launch_step(d, splits)) return;
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
