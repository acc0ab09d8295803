// decode.hip - batched single-token GQA decode for gfx950, HBM-bound.
//
// Two launches:
//   decode_attention_kernel  one persistent launch over a flattened work list of
//                            (sequence, kv head, chunk of CH positions) items;
//                            workgroup i takes items i, i + gridDim.x, ... so
//                            ragged lengths leave no empty workgroups. Each item
//                            first prepares its query rows: QK-RMSNorm and RoPE
//                            at position positions[b] for the G query heads
//                            (attentionMixer, LocalModel.hpp:2608-2648), packed
//                            as the score MFMA's B operand; the item holding
//                            the sequence's last chunk also norms and rotates
//                            the new k, appends the new k and v to the bf16
//                            cache at positions[b] (LocalModel.hpp:2650-2655)
//                            and scores the new token;
//   decode_merge_kernel      combines the (m, l, acc) records of sequences that
//                            span several chunks.
// Per item, 4 waves split the chunk into slabs of 32 positions, software-
// pipelined: a wave's next slab is requested before the current one computes.
//   - scores: v_mfma_f32_16x16x32_bf16 with K rows (16-byte loads straight
//     from HBM, each K byte read once for all G heads) as A and q as B, q split
//     into a bf16 high part (columns 0-7) and the bf16 residual (columns 8-15)
//     so the two halves add back to ~16 significant bits;
//   - P.V: v_mfma_f32_16x16x32_bf16 with P split like q (bf16 high part in
//     rows 0-7, residual in rows 8-15) against V: V rows arrive as whole
//     1 KB-per-instruction nontemporal loads, pass through LDS, and come back
//     through ds_read_b64_tr_b16 as the k-contiguous B operand;
//   - online softmax inside a wave, a cross-wave merge in LDS; a sequence
//     that fits one chunk writes its output directly, otherwise each chunk
//     leaves a (m, l, acc) record, combined by decode_merge_kernel with the
//     split-K algebra of the reference's Metal decoder
//     (src/gpu/Kernels.metal:318-345).
// A kernel boundary, not an in-kernel device-scope fence, publishes the
// records: on gfx950 such a fence writes back and invalidates the XCD's whole
// L2, which costs far more than a launch.
//
// Calls on different streams share the backend's scratch (the records); the
// entry points order a call after the previous one when its stream differs
// (an event handoff), so their kernels never overlap on it.
#include "context.hpp"
#include "device.hpp"
#include "kernels.hpp"


namespace aigpu {

namespace {

constexpr int MAXG = 8;          // query heads per kv head handled by one workgroup
constexpr int SLAB = 32;         // positions per wave step
constexpr int MAXB = 1024;       // sequences per launch (larger batches are split)
constexpr uint32_t GRID = 512;   // persistent workgroups (two per CU)

struct DecodeArgs {
    DecodeParams p;
    float* parts;                // [batch][kvHeads][maxChunks][RS]
    uint32_t chunkLen;           // CH, a multiple of 4 * SLAB
    uint32_t maxChunks;
    float scaleLog2;
};

__host__ __device__ constexpr int record_floats(int D) { return 2 * MAXG + MAXG * D; }

/* the attention output of (sequence b, head h, column d), times sigmoid of the
   gate half of its q row when the output gate is on (LocalModel.hpp:2660-2665) */
__device__ __forceinline__ float gated(const DecodeParams& p, uint32_t b, uint32_t h, uint32_t d, float x) {
    if (!p.outputGate) return x;
    const float gt = load_elem(p.q, (size_t(b) * p.heads + h) * p.qStride + p.dim + d, p.inType);
    return x * (1.0f / (1.0f + expf(-gt)));
}

__device__ __forceinline__ uint32_t first_position(const DecodeParams& p, uint32_t L) {
    return (p.window && uint64_t(L) + 1 > p.window) ? uint32_t(uint64_t(L) + 1 - p.window) : 0u;
}

typedef __bf16 bf16x4 __attribute__((__vector_size__(4 * sizeof(__bf16))));

/* x from lane (lane ^ 8) of the same 16-lane row: a DPP row rotate by 8 */
__device__ __forceinline__ float row_rotate8(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false));
}

/* ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i % 4
   of the 8-byte rows addressed by lanes i/4, i/4 + 4, i/4 + 8, i/4 + 12 */
__device__ __forceinline__ bf16x4 read_tr16(const uint16_t* lds) {
    typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(lds));
}

/* V slabs in LDS: rows of D halfs, RPL rows per 1 KB DMA block; the 16-byte
   column block x of row r sits at x ^ v_swizzle(r), so the 8 rows x 32 bytes a
   32-lane transposed read touches hit distinct banks */
__device__ __forceinline__ int v_swizzle(int r, int D) { return D == 128 ? 2 * (r & 7) : 2 * ((r >> 1) & 3); }

template <int D>
__device__ __forceinline__ int v_offset(int r, int x) {
    return r * D + 8 * (x ^ v_swizzle(r, D));
}

/* s_waitcnt vmcnt(N) leaving the other counters alone (gfx9 encoding) */
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

template <int D>
__global__ __launch_bounds__(256, 2) void decode_attention_kernel(DecodeArgs a) {
    constexpr int DB = D / 32;   // 32-deep d blocks of the score MFMA
    constexpr int CT = D / 16;   // 16-column tiles of the P.V product
    constexpr int LPR = D / 8;   // lanes covering one V row with 16-byte loads
    constexpr int RPL = WAVE / LPR;                 // V rows per load instruction
    constexpr int VLOADS = SLAB / RPL;              // V load instructions per slab
    constexpr int VSLAB = SLAB * D;                 // halfs of one V slab in LDS
    constexpr int RS = record_floats(D);
    static_assert(2 * MAXG * D * 4 <= 2 * VSLAB * 2, "per-wave state must fit in the wave's V slabs");
    typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

    const DecodeParams& p = a.p;
    const uint32_t B = uint32_t(p.batch), KVH = uint32_t(p.kvHeads);
    const uint32_t G = uint32_t(p.heads / p.kvHeads);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, c16 = lane & 15;

    __shared__ uint32_t pre[MAXB + 1];
    __shared__ float wm[4][MAXG], wl[4][MAXG];
    __shared__ float rows[MAXG + 1][D];           // normed, rotated q rows (scaled) and the new key
    __shared__ float snew[MAXG], vnew[D];         // the new token's scores and value
    __shared__ __attribute__((aligned(16))) uint16_t vbuf[4 * 2 * VSLAB];   // per-wave V slabs (x2)

    // ---- chunk counts -> prefix over the batch (the work list) ----
    for (uint32_t i = tid; i < B; i += 256) {
        const uint32_t L = p.positions[i];
        pre[i + 1] = L > p.maxPosition ? 0u : (L + 1 - first_position(p, L) + a.chunkLen - 1) / a.chunkLen;
    }
    if (tid == 0) pre[0] = 0;
    __syncthreads();
    if (w == 0) {
        uint32_t carry = 0;
        for (uint32_t base = 0; base < B; base += 64) {
            const uint32_t i = base + lane;
            uint32_t x = i < B ? pre[i + 1] : 0u;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t y = __shfl_up(x, off, WAVE);
                if (lane >= off) x += y;
            }
            x += carry;
            if (i < B) pre[i + 1] = x;
            carry = __shfl(x, 63, WAVE);
        }
    }
    __syncthreads();
    // items in (sequence, kv head, chunk) order, chunk fastest; workgroup i
    // takes a contiguous run of them, so consecutive items mostly share a
    // (sequence, kv head) and its prepared queries
    const uint32_t items = pre[B] * KVH;
    const uint32_t perWg = items / gridDim.x, extra = items % gridDim.x;
    const uint32_t itBegin = blockIdx.x * perWg + (blockIdx.x < extra ? blockIdx.x : extra);
    const uint32_t itEnd = itBegin + perWg + (blockIdx.x < extra ? 1u : 0u);
    uint16_t* vw = vbuf + w * (2 * VSLAB);
    uint32_t preparedPair = 0xFFFFFFFFu;
    bf16x8 qb[DB];   // the prepared (sequence, kv head)'s queries as the score B operand

    for (uint32_t item = itBegin; item < itEnd; ++item) {
        const uint32_t j = item / KVH;   // pre[b] <= j < pre[b + 1] for item's sequence b
        uint32_t lo_b = 0, hi_b = B;
        while (hi_b - lo_b > 1) {
            const uint32_t mid = (lo_b + hi_b) / 2;
            if (pre[mid] <= j) lo_b = mid;
            else hi_b = mid;
        }
        const uint32_t b = lo_b, nChunks = pre[b + 1] - pre[b];
        const uint32_t local = item - KVH * pre[b];
        const uint32_t kvh = local / nChunks, chunk = local % nChunks;
        const bool samePair = b * KVH + kvh == preparedPair;
        preparedPair = b * KVH + kvh;
        const uint32_t L = p.positions[b];
        const uint32_t first = first_position(p, L);
        const uint32_t lo = first + chunk * a.chunkLen;
        const uint32_t hi = (lo + a.chunkLen < L + 1) ? lo + a.chunkLen : L + 1;
        const bool hasNew = hi == L + 1;
        const uint32_t cachedHi = hi < L ? hi : L;   // cached positions are [lo, cachedHi)
        const uint32_t lastRow = cachedHi ? cachedHi - 1 : 0;
        const size_t cacheBase = size_t(b) * p.batchStride + size_t(kvh) * p.capacity * D;
        const uint16_t* kc = p.keyCache + cacheBase;
        const uint16_t* vc = p.valueCache + cacheBase;

        // a slab's loads: K rows into registers as MFMA A operands (row =
        // lane % 16); V rows straight into LDS slab `half` by DMA, 1 KB per
        // instruction, each lane's 16-byte column block XOR-swizzled by its
        // row so the transposed reads below are bank-conflict free
        auto issue = [&](uint32_t p0, u32x4 (&kr)[2][DB], int half) {
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                uint32_t row = p0 + 16 * rb + c16;
                if (row > lastRow) row = lastRow;
#pragma unroll
                for (int db = 0; db < DB; ++db)
                    kr[rb][db] = *reinterpret_cast<const u32x4*>(kc + size_t(row) * D + 32 * db + 8 * g);
            }
            uint16_t* vs = vw + half * VSLAB;
#pragma unroll
            for (int jj = 0; jj < VLOADS; ++jj) {
                const int r = jj * RPL + lane / LPR;                 // row within the slab
                const int cb = (lane % LPR) ^ v_swizzle(r, D);          // 16-byte column block
                uint32_t row = p0 + r;
                if (row > lastRow) row = lastRow;
                // cache policy 2: nontemporal (each V byte is read once)
                __builtin_amdgcn_global_load_lds(vc + size_t(row) * D + 8 * cb,
                                                 (__attribute__((address_space(3))) void*)(vs + jj * RPL * D),
                                                 16, 0, 2);
            }
        };

        __syncthreads();   // LDS of the previous item is free

        // ---- this item's query rows, QK-RMSNorm and RoPE at position L
        //      (attentionMixer, LocalModel.hpp:2608-2648), scaled by
        //      log2(e)/sqrt(D); the item with the new token also prepares the
        //      new key (row G) and appends it and the new value to the cache
        //      (LocalModel.hpp:2650-2655). The rows are requested before the
        //      first slab, so they arrive first and their preparation runs
        //      while the slab is in flight ----
        constexpr int EPL = D / WAVE;   // elements per lane of one row
        const uint32_t firstRow = samePair ? G : 0u;   // rows < G are still prepared
        const uint32_t nRows = G + (hasNew ? 1u : 0u);
        float xin[3][EPL], vin[EPL];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const uint32_t r = w + 4 * i;
            if (r >= firstRow && r < nRows) {
                const bool isKey = r == G;
                const size_t src = isKey ? (size_t(b) * p.kvHeads + kvh) * D
                                         : (size_t(b) * p.heads + size_t(kvh) * G + r) * p.qStride;
#pragma unroll
                for (int e = 0; e < EPL; ++e) xin[i][e] = load_elem(isKey ? p.k : p.q, src + lane + WAVE * e, p.inType);
                if (isKey) {
#pragma unroll
                    for (int e = 0; e < EPL; ++e) vin[e] = load_elem(p.v, src + lane + WAVE * e, p.inType);
                }
            }
        }

        // the first two slabs go out before the preparation too, so the
        // pipeline is full while it runs
        u32x4 krA[2][DB], krB[2][DB];
        uint32_t pA = lo + SLAB * w;
        if (pA < cachedHi) issue(pA, krA, 0);
        if (pA + 4 * SLAB < cachedHi) issue(pA + 4 * SLAB, krB, 1);
        __builtin_amdgcn_sched_barrier(0);

#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const uint32_t r = w + 4 * i;
            if (r >= firstRow && r < nRows) {
#pragma unroll
                for (int e = 0; e < EPL; ++e) rows[r][lane + WAVE * e] = xin[i][e];
            }
        }
        wave_sync();
        // the rotation at position L, lane j < rotaryDims / 2 holding pair
        // (j, j + rotaryDims / 2): shared by every row of the item
        const int half = p.freqs ? p.rotaryDims / 2 : 0;
        float rc = 1.0f, rs = 0.0f;
        if (lane < half && firstRow < nRows) sincosf(float(L) * p.freqs[lane], &rs, &rc);
        const uint32_t rowStart = w >= firstRow ? w : w + 4 * ((firstRow - w + 3) / 4);
#pragma unroll 1
        for (uint32_t r = rowStart; r < nRows; r += 4) {
            const bool isKey = r == G;
            float* x = rows[r];
            const float* gamma = isKey ? p.kNorm : p.qNorm;
            if (gamma) {   // rmsNormRow (LocalModel.hpp:1341-1348)
                float ss = 0.0f;
#pragma unroll
                for (int e = 0; e < EPL; ++e) ss += x[lane + WAVE * e] * x[lane + WAVE * e];
                const float inv = 1.0f / sqrtf(wave_sum(ss) / float(D) + p.eps);
#pragma unroll
                for (int e = 0; e < EPL; ++e)
                    x[lane + WAVE * e] = x[lane + WAVE * e] * inv * (gamma[lane + WAVE * e] + p.normOffset);
                wave_sync();
            }
            if (lane < half) {   // rotate-half pairs (LocalModel.hpp:2624-2641)
                const float u = x[lane], v = x[lane + half];
                x[lane] = u * rc - v * rs;
                x[lane + half] = v * rc + u * rs;
            }
            wave_sync();
            if (isKey) {
                uint16_t* kdst = p.keyCache + cacheBase + size_t(L) * D;
                uint16_t* vdst = p.valueCache + cacheBase + size_t(L) * D;
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    const int d = lane + WAVE * e;
                    kdst[d] = float_to_bf16_bits(x[d]);
                    vdst[d] = float_to_bf16_bits(vin[e]);
                    vnew[d] = vin[e];
                }
            } else {
#pragma unroll
                for (int e = 0; e < EPL; ++e) x[lane + WAVE * e] *= a.scaleLog2;
            }
            wave_sync();
        }
        __syncthreads();
        if (hasNew) {   // the new token's scores, one head per wave
            for (uint32_t h = w; h < G; h += 4) {
                float part = 0.0f;
#pragma unroll
                for (int e = 0; e < EPL; ++e) part += rows[h][lane + WAVE * e] * rows[G][lane + WAVE * e];
                part = wave_sum(part);
                if (lane == 0) snew[h] = part;
            }
        }
        // q as the B operand: column j < 8 is head j's bf16 high part, column
        // 8 + j its residual; lane group g holds d = 32 db + 8 g + 0..7
        if (!samePair) {
            const uint32_t h = c16 & 7;
            const bool residual = c16 >= 8;
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                u16x8 bits;
#pragma unroll
                for (int s8 = 0; s8 < 8; ++s8) {
                    const float x = h < G ? rows[h][32 * db + 8 * g + s8] : 0.0f;
                    const uint16_t top = float_to_bf16_bits(x);
                    bits[s8] = residual ? float_to_bf16_bits(x - bf16_bits_to_float(top)) : top;
                }
                qb[db] = __builtin_bit_cast(bf16x8, bits);
            }
        }

        float m = -INFINITY, lsum = 0.0f;   // per lane: head c16 & 7
        floatx4 acc[CT];                    // rows 0-7: P_hi.V, rows 8-15: P_lo.V
#pragma unroll
        for (int t = 0; t < CT; ++t) acc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

        // one slab: scores, online softmax, P.V; `half` picks the LDS V buffer
        auto compute = [&](uint32_t p0, const u32x4 (&kr)[2][DB], int half, bool nextInFlight) {
            const uint16_t* vs = vw + half * VSLAB;
            floatx4 sc[2];
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                sc[rb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int db = 0; db < DB; ++db)
                    sc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[rb][db]),
                                                                     qb[db], sc[rb], 0, 0, 0);
            }
            float sv[2][4];
            float mx = -INFINITY;
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float x = sc[rb][i];
                    x += row_rotate8(x);   // high part + residual (columns j and j^8)
                    const uint32_t pos = p0 + 16 * rb + 4 * g + i;
                    x = pos < cachedHi ? x : -INFINITY;
                    sv[rb][i] = x;
                    mx = fmaxf(mx, x);
                }
            mx = fmaxf(mx, __shfl_xor(mx, 16, WAVE));
            mx = fmaxf(mx, __shfl_xor(mx, 32, WAVE));
            const float mn = fmaxf(m, mx);
            const float base = mn == -INFINITY ? 0.0f : mn;
            const float alpha = exp2f(m - base);
            float ps = 0.0f;
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    sv[rb][i] = exp2f(sv[rb][i] - base);
                    ps += sv[rb][i];
                }
            lsum = lsum * alpha + ps;
            m = mn;

            // accumulator rows 4g + r hold head (4g + r) & 7: rescale them
            float ar[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, (4 * g + r) & 7, WAVE);
#pragma unroll
            for (int t = 0; t < CT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[t][r] *= ar[r];

            // P as the A operand: row j < 8 is head j's bf16 high part, row 8 + j
            // its residual; the k slots of lane group g are positions
            // 4g + (s & 3) + 16 (s >> 2), exactly the scores this lane holds
            u16x8 bits;
#pragma unroll
            for (int s8 = 0; s8 < 8; ++s8) {
                const float pv = sv[s8 >> 2][s8 & 3];
                const uint16_t top = float_to_bf16_bits(pv);
                bits[s8] = c16 >= 8 ? float_to_bf16_bits(pv - bf16_bits_to_float(top)) : top;
            }
            const bf16x8 pa = __builtin_bit_cast(bf16x8, bits);

            // the slab's V DMA has landed: only the next slab's loads may be pending
            if (nextInFlight) wait_vmcnt<2 * DB + VLOADS>();
            else wait_vmcnt<0>();
            wave_sync();
#pragma unroll
            for (int t = 0; t < CT; ++t) {
                // transposed reads: lane c16 of group g gets column 16t + c16 at
                // positions 4g + 0..3, then 16 + 4g + 0..3
                const int r0 = 4 * g + (c16 >> 2), r1 = r0 + 16;
                const int x = 2 * t + ((c16 >> 1) & 1), sub = 4 * (c16 & 1);
                const bf16x4 lo4 = read_tr16(vs + v_offset<D>(r0, x) + sub);
                const bf16x4 hi4 = read_tr16(vs + v_offset<D>(r1, x) + sub);
                const bf16x8 vb = __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, vb, acc[t], 0, 0, 0);
            }
        };

        // ---- slabs, software-pipelined: the next slab's loads are in flight
        //      while the current one computes (two register/LDS buffers) ----
        bool bIssued = true;   // the first slab B went out with slab A
        while (pA < cachedHi) {
            const uint32_t pB = pA + 4 * SLAB;
            if (pB < cachedHi && !bIssued) issue(pB, krB, 1);
            bIssued = false;
            __builtin_amdgcn_sched_barrier(0);
            compute(pA, krA, 0, pB < cachedHi);
            if (pB >= cachedHi) break;
            const uint32_t pC = pB + 4 * SLAB;
            wave_sync();   // slab A's LDS reads are done before its buffer refills
            if (pC < cachedHi) issue(pC, krA, 0);
            __builtin_amdgcn_sched_barrier(0);
            compute(pB, krB, 1, pC < cachedHi);
            wave_sync();
            pA = pC;
        }

        // ---- per-wave state to LDS (each wave inside its own V slabs) ----
        lsum += __shfl_xor(lsum, 16, WAVE);
        lsum += __shfl_xor(lsum, 32, WAVE);
        if (g == 0 && c16 < MAXG) {
            wm[w][c16] = m;
            wl[w][c16] = lsum;
        }
        wave_sync();   // the last slab's LDS reads are done before the slabs are reused
        float* waccw = reinterpret_cast<float*>(vw);   // [16][D]: rows h and 8 + h add up
#pragma unroll
        for (int t = 0; t < CT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) waccw[(4 * g + r) * D + 16 * t + c16] = acc[t][r];
        __syncthreads();

        // ---- the waves (and the new token) merged: this chunk's (M, l, acc);
        //      a one-chunk sequence is finished here ----
        float* rec = a.parts + ((size_t(b) * KVH + kvh) * a.maxChunks + chunk) * RS;
        float* outRow = p.out + (size_t(b) * p.heads + size_t(kvh) * G) * D;
        for (uint32_t idx = tid; idx < G * D; idx += 256) {
            const uint32_t h = idx / D, d = idx % D;
            const float sn = hasNew ? snew[h] : -INFINITY;
            float M = fmaxf(fmaxf(wm[0][h], wm[1][h]), fmaxf(wm[2][h], wm[3][h]));
            M = fmaxf(M, sn);
            float lt = 0.0f, at = 0.0f;
#pragma unroll
            for (int ww = 0; ww < 4; ++ww) {
                const float f = wm[ww][h] == -INFINITY ? 0.0f : exp2f(wm[ww][h] - M);
                const float* wa = reinterpret_cast<const float*>(vbuf + ww * (2 * VSLAB));
                lt += wl[ww][h] * f;
                at += (wa[h * D + d] + wa[(8 + h) * D + d]) * f;
            }
            if (hasNew) {
                const float f = exp2f(sn - M);
                lt += f;
                at += f * vnew[d];
            }
            if (nChunks == 1) {
                outRow[h * D + d] = gated(p, b, kvh * G + h, d, at / lt);
            } else {
                rec[2 * MAXG + h * D + d] = at;
                if (d == 0) {
                    rec[h] = M;
                    rec[MAXG + h] = lt;
                }
            }
        }
    }

    // sequences whose position exceeds the launch's maxPosition are marked NaN
    for (uint32_t i = blockIdx.x; i < B; i += gridDim.x) {
        if (p.positions[i] <= p.maxPosition) continue;
        for (uint32_t idx = tid; idx < p.heads * D; idx += 256)
            p.out[size_t(i) * p.heads * D + idx] = __builtin_nanf("");
    }
}

/* combines the chunk records of every (sequence, query head) whose sequence
   spans more than one chunk (the split-K algebra of Kernels.metal:318-345);
   one workgroup of D threads per (sequence, kv head, head of the group),
   thread d owning output column d. A tile of chunks is read at once (the
   chunk's m and l are the same address across the workgroup, the
   accumulators contiguous across it), all its loads independent, so a tile
   costs one memory round trip; the running sums are rescaled to each tile's
   new maximum. */
template <int D>
__global__ __launch_bounds__(D) void decode_merge_kernel(DecodeArgs a) {
    constexpr int RS = record_floats(D);
    constexpr int TILE = 16;
    const DecodeParams& p = a.p;
    const uint32_t KVH = uint32_t(p.kvHeads), G = uint32_t(p.heads / p.kvHeads);
    const uint32_t pair = blockIdx.x / G, h = blockIdx.x % G;
    const uint32_t b = pair / KVH, kvh = pair % KVH;
    const uint32_t L = p.positions[b];
    if (L > p.maxPosition) return;
    const uint32_t nChunks = (L + 1 - first_position(p, L) + a.chunkLen - 1) / a.chunkLen;
    if (nChunks < 2) return;   // written by the attention kernel itself
    const float* recs = a.parts + size_t(pair) * a.maxChunks * RS;
    const uint32_t d = threadIdx.x;
    float M = -INFINITY, lt = 0.0f, at = 0.0f;
    for (uint32_t c0 = 0; c0 < nChunks; c0 += TILE) {
        float mc[TILE], lc[TILE], ac[TILE];
#pragma unroll
        for (int c = 0; c < TILE; ++c) {
            const bool in = c0 + c < nChunks;
            const float* r = recs + size_t(in ? c0 + c : c0) * RS;
            mc[c] = in ? r[h] : -INFINITY;
            lc[c] = r[MAXG + h];
            ac[c] = r[2 * MAXG + h * D + d];
        }
        float mt = M;
#pragma unroll
        for (int c = 0; c < TILE; ++c) mt = fmaxf(mt, mc[c]);
        const float scale = M == -INFINITY ? 0.0f : exp2f(M - mt);
        lt *= scale;
        at *= scale;
#pragma unroll
        for (int c = 0; c < TILE; ++c) {
            const float f = mc[c] == -INFINITY ? 0.0f : exp2f(mc[c] - mt);
            lt += lc[c] * f;
            at += ac[c] * f;
        }
        M = mt;
    }
    p.out[(size_t(b) * p.heads + size_t(kvh) * G + h) * D + d] = gated(p, b, kvh * G + h, d, at / lt);
}

/*
    The fixed scratch of aigpu_decode_attention_static: the split-K records
    (the queries are prepared inside the attention kernel and need no
    scratch), in device memory that exists from module load
    until the process ends, so that the entry point allocates nothing. Each
    GPU holds its own copy at its own address; host code never passes the
    array's name (a host-side stand-in) to a kernel, only the address
    hipGetSymbolAddress returns for the current device.
*/
constexpr size_t DECODE_STATIC_SCRATCH = size_t(32) << 20;
__device__ __align__(256) unsigned char scratch[DECODE_STATIC_SCRATCH];

constexpr int MAX_DEVICES = 64;
void* staticScratch[MAX_DEVICES] = {};

} // namespace

bool decode_static_scratch(void** base, size_t* bytes) {
    Context& ctx = Context::instance();
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
        (void)hipGetLastError();
        return ctx.fail("decode (no allocation): no current device");
    }
    if (!staticScratch[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            (void)hipGetLastError();
            return ctx.fail(std::string("decode (no allocation): hipGetSymbolAddress of the fixed scratch failed: ") +
                            hipGetErrorString(e));
        }
        staticScratch[dev] = ptr;
    }
    *base = staticScratch[dev];
    *bytes = DECODE_STATIC_SCRATCH;
    return true;
}

bool launch_decode(const DecodeParams& p, hipStream_t stream, const FixedScratch* fixed) {
    Context& ctx = Context::instance();
    if (p.dim != 64 && p.dim != 128) return ctx.fail("decode: dim must be 64 or 128");
    if (p.kvHeads == 0 || p.heads % p.kvHeads) return ctx.fail("decode: heads must be a multiple of kvHeads");
    if (p.heads / p.kvHeads > MAXG) return ctx.fail("decode: at most 8 query heads per kv head");
    if (p.qStride < p.dim) return ctx.fail("decode: qStride < dim");
    if (p.outputGate && p.qStride < 2 * p.dim) return ctx.fail("decode: the output gate needs qStride >= 2 dim");
    if (p.freqs && (p.rotaryDims == 0 || p.rotaryDims > int(p.dim) || (p.rotaryDims & 1)))
        return ctx.fail("decode: rotaryDims must be even and within dim");
    if (p.inType != 0 && p.inType != 1) return ctx.fail("decode: unknown input type");
    if (!p.q || !p.k || !p.v || !p.out || !p.keyCache || !p.valueCache || !p.positions)
        return ctx.fail("decode: null tensor");
    if (p.batch == 0) return true;
    if (uint64_t(p.maxPosition) + 1 > p.capacity)
        return ctx.fail("decode: maxPosition + 1 exceeds the cache capacity");
    if (p.kvHeads > 65535) return ctx.fail("decode: kvHeads too large");

    // chunk length: the longest of 2048/1024/512/256 positions that still
    // gives every resident workgroup (2 per CU, GRID in all) two items; below
    // that, 128 positions (one slab per wave) when 256 would leave CUs idle
    auto chunk_for = [&](uint64_t bs) {
        auto items = [&](uint32_t len) { return bs * p.kvHeads * ((uint64_t(p.maxPosition) + len) / len); };
        uint32_t len = 2048;
        while (len > 256 && items(len) < 2ull * GRID) len /= 2;
        if (items(len) < GRID / 2 && items(4 * SLAB) > items(len)) len = 4 * SLAB;
        return len;
    };
    const size_t rs = size_t(record_floats(int(p.dim)));
    uint64_t slice = p.batch < MAXB ? p.batch : MAXB;
    uint32_t chunkLen = chunk_for(slice);
    uint32_t maxChunks = (p.maxPosition + 1 + chunkLen - 1) / chunkLen;
    auto parts_bytes = [&] { return (slice * p.kvHeads * maxChunks * rs * sizeof(float) + 255) & ~size_t(255); };
    float* parts = nullptr;
    if (fixed) {
        // the records of a slice of sequences must fit the fixed scratch:
        // halve the slice until they do
        while (slice > 1 && parts_bytes() > fixed->bytes) {
            slice = (slice + 1) / 2;
            chunkLen = chunk_for(slice);
            maxChunks = (p.maxPosition + 1 + chunkLen - 1) / chunkLen;
        }
        if (parts_bytes() > fixed->bytes)
            return ctx.fail("decode (no allocation): one sequence's split-K records need " +
                            std::to_string(parts_bytes()) + " bytes, above the fixed scratch of " +
                            std::to_string(fixed->bytes));
        parts = static_cast<float*>(fixed->base);
    } else {
        parts = static_cast<float*>(ctx.grow(SLOT_DECODE_PARTS, parts_bytes()));
        if (!parts) return false;
    }

    const uint64_t batchStride = p.batchStride ? p.batchStride : p.kvHeads * p.capacity * p.dim;
    for (uint64_t b0 = 0; b0 < p.batch; b0 += slice) {
        DecodeArgs a{};
        a.p = p;
        a.p.batch = (p.batch - b0 < slice) ? p.batch - b0 : slice;
        a.p.batchStride = batchStride;
        const size_t es = p.inType == 1 ? 2 : 4;
        a.p.q = static_cast<const char*>(p.q) + b0 * p.heads * p.qStride * es;
        a.p.k = static_cast<const char*>(p.k) + b0 * p.kvHeads * p.dim * es;
        a.p.v = static_cast<const char*>(p.v) + b0 * p.kvHeads * p.dim * es;
        a.p.out = p.out + b0 * p.heads * p.dim;
        a.p.keyCache = p.keyCache + b0 * batchStride;
        a.p.valueCache = p.valueCache + b0 * batchStride;
        a.p.positions = p.positions + b0;
        a.parts = parts;
        a.chunkLen = chunkLen;
        a.maxChunks = maxChunks;
        a.scaleLog2 = LOG2E / sqrtf(float(p.dim));
        const uint64_t upper = a.p.batch * p.kvHeads * maxChunks;
        const unsigned grid = unsigned(upper < GRID ? upper : GRID);
        const unsigned mgrid = unsigned(a.p.batch * p.heads);   // one merge workgroup per query head
        const bool ok = p.dim == 128
            ? ctx.launch("decode_attention_kernel", stream, [&] {
                  hipLaunchKernelGGL(decode_attention_kernel<128>, dim3(grid), dim3(256), 0, stream, a);
              }) && (maxChunks < 2 || ctx.launch("decode_merge_kernel", stream, [&] {
                  hipLaunchKernelGGL(decode_merge_kernel<128>, dim3(mgrid), dim3(128), 0, stream, a);
              }))
            : ctx.launch("decode_attention_kernel", stream, [&] {
                  hipLaunchKernelGGL(decode_attention_kernel<64>, dim3(grid), dim3(256), 0, stream, a);
              }) && (maxChunks < 2 || ctx.launch("decode_merge_kernel", stream, [&] {
                  hipLaunchKernelGGL(decode_merge_kernel<64>, dim3(mgrid), dim3(64), 0, stream, a);
              }));
        if (!ok) return false;
    }
    return true;
}

} // namespace aigpu
