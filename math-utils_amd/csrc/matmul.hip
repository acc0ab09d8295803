// matmul.hip - out[m][n] = a[m][k] . w[n][k] (+ bias[n]) (+ out), the
// projection every mixer and MLP applies (LocalModel.hpp:1044-1078 apply,
// behind gpu::matmulNT*), for the reference's four weight encodings:
//   F32    [n][k] fp32
//   BF16   [n][k] bf16 (widened by a 16-bit shift, Kernels.hip widenBF16)
//   Q8     [n][k] int8 codes, one fp32 scale per 32 codes (Quant.hpp:528-538)
//   Q4     [n][k/2] bytes, one fp32 scale per 32 codes; byte j of a block
//          holds code j in its low nibble and code j+16 in its high nibble,
//          each offset by 8 (Quant.hpp:540-549)
//
// gemv_kernel serves up to 8 rows of a (decode, small batches): it is bound
// by the weight bytes, so every lane streams 16-byte pieces of a weight row
// (4, 8, 16 or 32 weights), one wave owns GEMV_ROWS weight rows and keeps an
// fp32 accumulator per (weight row, a row), and a shuffle tree reduces the
// lanes. Up to GEMM_MIN_M - 1 rows of a run as blocks of 8 along grid.y;
// more rows take gemm_kernel on MFMA, and bf16 weights with enough rows for
// 256 x 256 tiles split_a_kernel and gemm_dma_kernel.
#include <type_traits>
#include "context.hpp"
#include "device.hpp"
#include "gemv.hpp"
#include "kernels.hpp"

namespace aigpu {

namespace {

constexpr int GEMV_ROWS = 2;   // weight rows per wave
constexpr int GEMV_MAX_M = 8;  // rows of a per launch block
constexpr uint32_t GEMM_MIN_M = 16;   // from here on the MFMA GEMM

template <int TYPE, int M>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams p) {
    constexpr int E = piece_elems<TYPE>();
    const int lane = threadIdx.x & 63;
    const uint32_t row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * GEMV_ROWS;
    if (row0 >= p.n) return;   // whole wave leaves; no block barriers below
    const uint32_t m0 = blockIdx.y * M;
    const uint32_t pieces = p.k / E;
    const size_t rowBytes = size_t(p.k) * row_bytes_per_k_x2<TYPE>() / 2;
    const uint32_t blocks = p.k / 32;

    const char* wrow[GEMV_ROWS];
    const float* srow[GEMV_ROWS];
#pragma unroll
    for (int r = 0; r < GEMV_ROWS; ++r) {
        const uint32_t rr = row0 + r < p.n ? row0 + r : p.n - 1;
        wrow[r] = static_cast<const char*>(p.w) + rr * rowBytes;
        srow[r] = TYPE >= 2 ? p.scales + size_t(rr) * blocks : nullptr;
    }
    float acc[GEMV_ROWS][M];
#pragma unroll
    for (int r = 0; r < GEMV_ROWS; ++r)
#pragma unroll
        for (int i = 0; i < M; ++i) acc[r][i] = 0.0f;

#pragma unroll 2
    for (uint32_t c = lane; c < pieces; c += WAVE) {
        u32x4 wv[GEMV_ROWS];
#pragma unroll
        for (int r = 0; r < GEMV_ROWS; ++r) wv[r] = *reinterpret_cast<const u32x4*>(wrow[r] + size_t(c) * 16);
        float sc[GEMV_ROWS];
#pragma unroll
        for (int r = 0; r < GEMV_ROWS; ++r) sc[r] = TYPE == 2 ? srow[r][c >> 1] : (TYPE == 3 ? srow[r][c] : 1.0f);
#pragma unroll
        for (int i = 0; i < M; ++i) {
            if (m0 + i < p.m) {
                const float* x = p.a + size_t(m0 + i) * p.k + size_t(c) * E;
#pragma unroll
                for (int r = 0; r < GEMV_ROWS; ++r) {
                    const float d = piece_dot<TYPE>(wv[r], x);
                    acc[r][i] = TYPE >= 2 ? fmaf(d, sc[r], acc[r][i]) : acc[r][i] + d;
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < GEMV_ROWS; ++r)
#pragma unroll
        for (int i = 0; i < M; ++i) acc[r][i] = wave_sum(acc[r][i]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < GEMV_ROWS; ++r) {
            const uint32_t n = row0 + r;
            if (n >= p.n) continue;
            const float b = p.bias ? p.bias[n] : 0.0f;
#pragma unroll
            for (int i = 0; i < M; ++i) {
                if (m0 + i >= p.m) continue;
                float* o = p.out + size_t(m0 + i) * p.ldo + n;
                *o = (p.accumulate ? *o : 0.0f) + acc[r][i] + b;
            }
        }
    }
}

/*
    gemm_kernel: many rows of a (prefill), on v_mfma_f32_16x16x32_bf16.
    A stays fp32 at the boundary; each value is split into a bf16 high part
    and the bf16 residual, and hi.B + lo.B keeps about 16 bits of it. BF16
    weights and the Q8/Q4 codes are exact in bf16; fp32 weights are split
    the same way (a third product, hi_a.lo_w). For Q8/Q4 one 32-wide K step
    is one scale block, so each step's products go through a scratch
    accumulator and are added in times the column's block scale.
    Tile 128 x 128 x 32 over four waves of 64 x 64 (4 x 4 MFMA tiles); the
    next K step is loaded into registers while the current one computes.
    LDS rows are padded to 40 bf16 (80 bytes), so the 16 lanes of each 16-byte
    operand read land on distinct banks.
*/
constexpr int GM_BM = 128, GM_BN = 128, GM_BK = 32, GM_AS = GM_BK + 8;
constexpr int GM_OP = GM_BM * GM_AS;   // bf16 elements of one operand buffer
constexpr int GM_ES = GM_BN + 4;       // row stride (floats) of the epilogue's half tile

/* KV: the k / v epilogue of a prefill (launch_gemm_kv) instead of the plain
   store. It takes the tile through LDS in two halves of 64 rows; four threads
   per row, each 32 consecutive columns, which lie in one head (dim 64 or 128,
   tiles start on multiples of 128). */
template <int TYPE, bool KV>
__global__ __launch_bounds__(256) void gemm_kernel(GemvParams p, KvEpilogue ep, uint32_t kSlice) {
    constexpr bool SPLIT_W = TYPE == 0, QUANT = TYPE >= 2;
    constexpr int OPS = (SPLIT_W ? 4 : 3) * GM_OP;   // Ah, Al, Bh (, Bl)
    constexpr int EPI = KV ? 64 * GM_ES * 2 : 0;      // the half tile in fp32, counted in bf16
    __shared__ __align__(16) __bf16 smem[OPS > EPI ? OPS : EPI];
    __bf16* const Ah = smem;
    __bf16* const Al = smem + GM_OP;
    __bf16* const Bh = smem + 2 * GM_OP;
    __bf16* const Bl = smem + 3 * GM_OP;   // SPLIT_W only
    __shared__ float Sc[QUANT ? GM_BN : 1];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, wm = w >> 1, wn = w & 1;
    const uint32_t m0 = blockIdx.y * GM_BM, n0 = blockIdx.x * GM_BN;
    const uint32_t K = p.k, M = p.m, N = p.n;
    const int srow = tid >> 1, shalf = tid & 1;   // staging: row and 16-element half of the K step

    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    floatx4 ra[4];                   // a: 16 floats
    u32x4 rw[SPLIT_W ? 4 : 2];       // w: 16 fp32 / 16 bf16 / 16 Q8 codes / a Q4 block
    float rs = 0.0f;
    auto load = [&](uint32_t k0) {
        const uint32_t gm = m0 + srow, kk = k0 + 16 * shalf;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            ra[e] = (gm < M && kk + 4 * e < K) ? *reinterpret_cast<const floatx4*>(p.a + size_t(gm) * K + kk + 4 * e)
                                               : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        const uint32_t gn = n0 + srow;
        if constexpr (TYPE == 0) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                rw[e] = (gn < N && kk + 4 * e < K)
                            ? *reinterpret_cast<const u32x4*>(static_cast<const float*>(p.w) + size_t(gn) * K + kk + 4 * e)
                            : u32x4{0u, 0u, 0u, 0u};
        } else if constexpr (TYPE == 1) {
#pragma unroll
            for (int e = 0; e < 2; ++e)
                rw[e] = (gn < N && kk + 8 * e < K)
                            ? *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p.w) + size_t(gn) * K + kk + 8 * e)
                            : u32x4{0u, 0u, 0u, 0u};
        } else if constexpr (TYPE == 2) {
            rw[0] = gn < N ? *reinterpret_cast<const u32x4*>(static_cast<const int8_t*>(p.w) + size_t(gn) * K + kk)
                           : u32x4{0u, 0u, 0u, 0u};
        } else {
            // a Q4 block is 16 bytes: threads 0..127 take one row's block each
            const uint32_t qn = n0 + uint32_t(tid & 127);
            rw[0] = (tid < 128 && qn < N)
                        ? *reinterpret_cast<const u32x4*>(static_cast<const uint8_t*>(p.w) + size_t(qn) * (K / 2) + k0 / 2)
                        : u32x4{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
        }
        if constexpr (QUANT) rs = (tid < 128 && n0 + tid < N) ? p.scales[size_t(n0 + tid) * (K / 32) + k0 / 32] : 0.0f;
    };
    auto split_store = [&](__bf16* hi, __bf16* lo, const float (&x)[16]) {
        bf16x8 h0, h1, l0, l1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            h0[e] = __bf16(x[e]);
            h1[e] = __bf16(x[8 + e]);
            l0[e] = __bf16(x[e] - float(h0[e]));
            l1[e] = __bf16(x[8 + e] - float(h1[e]));
        }
        *reinterpret_cast<bf16x8*>(hi) = h0;
        *reinterpret_cast<bf16x8*>(hi + 8) = h1;
        *reinterpret_cast<bf16x8*>(lo) = l0;
        *reinterpret_cast<bf16x8*>(lo + 8) = l1;
    };
    auto store = [&]() {
        float x[16];
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int c = 0; c < 4; ++c) x[4 * e + c] = ra[e][c];
        split_store(&Ah[srow * GM_AS + 16 * shalf], &Al[srow * GM_AS + 16 * shalf], x);
        if constexpr (TYPE == 0) {
            float y[16];
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int c = 0; c < 4; ++c) y[4 * e + c] = __uint_as_float(rw[e][c]);
            split_store(&Bh[srow * GM_AS + 16 * shalf], &Bl[srow * GM_AS + 16 * shalf], y);
        } else if constexpr (TYPE == 1) {
            *reinterpret_cast<u32x4*>(&Bh[srow * GM_AS + 16 * shalf]) = rw[0];
            *reinterpret_cast<u32x4*>(&Bh[srow * GM_AS + 16 * shalf + 8]) = rw[1];
        } else if constexpr (TYPE == 2) {
            bf16x8 b0, b1;
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float c = float(int32_t(rw[0][e] << (24 - 8 * j)) >> 24);
                    if (e < 2) b0[4 * e + j] = __bf16(c);
                    else b1[4 * (e - 2) + j] = __bf16(c);
                }
            *reinterpret_cast<bf16x8*>(&Bh[srow * GM_AS + 16 * shalf]) = b0;
            *reinterpret_cast<bf16x8*>(&Bh[srow * GM_AS + 16 * shalf + 8]) = b1;
        } else {
            if (tid < 128) {
                __bf16* row = &Bh[tid * GM_AS];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    bf16x8 lo4, hi4;   // codes 4e..4e+3 and 16+4e..16+4e+3, two bytes at a time
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t byte = (rw[0][e] >> (8 * j)) & 0xFFu;
                        lo4[j] = __bf16(float(int(byte & 0xFu) - 8));
                        hi4[j] = __bf16(float(int(byte >> 4) - 8));
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        row[4 * e + j] = lo4[j];
                        row[16 + 4 * e + j] = hi4[j];
                    }
                }
            }
        }
        if constexpr (QUANT)
            if (tid < 128) Sc[tid] = rs;
    };

    // split K: slice blockIdx.z of kSlice (a multiple of GM_BK) columns
    const uint32_t kBegin = blockIdx.z * kSlice, kEnd = kBegin + kSlice < K ? kBegin + kSlice : K;
    load(kBegin);
    for (uint32_t k0 = kBegin; k0 < kEnd; k0 += GM_BK) {
        __syncthreads();   // the previous step's operand reads are done
        store();
        __syncthreads();
        if (k0 + GM_BK < kEnd) load(k0 + GM_BK);
        bf16x8 ah[4], al[4], bh[4], bl[4];
        const int fr = lane & 15, fk = 8 * (lane >> 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ah[i] = *reinterpret_cast<const bf16x8*>(&Ah[(64 * wm + 16 * i + fr) * GM_AS + fk]);
            al[i] = *reinterpret_cast<const bf16x8*>(&Al[(64 * wm + 16 * i + fr) * GM_AS + fk]);
            bh[i] = *reinterpret_cast<const bf16x8*>(&Bh[(64 * wn + 16 * i + fr) * GM_AS + fk]);
            if constexpr (SPLIT_W) bl[i] = *reinterpret_cast<const bf16x8*>(&Bl[(64 * wn + 16 * i + fr) * GM_AS + fk]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (QUANT) {
                    floatx4 t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], bh[j], floatx4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[i], bh[j], t, 0, 0, 0);
                    const float sc = Sc[64 * wn + 16 * j + fr];
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf(sc, t[r], acc[i][j][r]);
                } else {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], bh[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[i], bh[j], acc[i][j], 0, 0, 0);
                    if constexpr (SPLIT_W) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], bl[j], acc[i][j], 0, 0, 0);
                }
            }
    }
    // the accumulator layout: lane holds rows 4 (lane / 16) + r of column lane % 16
    if constexpr (!KV) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t n = n0 + 64 * wn + 16 * j + (lane & 15);
                if (n >= N) continue;
                const float b = p.bias ? p.bias[n] : 0.0f;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t m = m0 + 64 * wm + 16 * i + 4 * (lane >> 4) + r;
                    if (m >= M) continue;
                    // a K slice writes its own partial tile (no bias, no accumulate)
                    float* o = p.out + size_t(blockIdx.z) * M * p.ldo + size_t(m) * p.ldo + n;
                    *o = (p.accumulate ? *o : 0.0f) + acc[i][j][r] + b;
                }
            }
    } else {
        float* tile = reinterpret_cast<float*>(smem);
        const uint32_t D = ep.dim;
        const int row = tid >> 2, c0 = 32 * (tid & 3);   // half-tile row, first column
        const uint32_t n = n0 + uint32_t(c0);                // k or v column: head n / D, dim n % D
        const uint32_t d0 = n % D, head = n / D, hc = uint32_t(c0) - d0;
        const uint32_t half = ep.freqs ? ep.rot / 2 : 0;
        bool bad = false;   // an fp16 conversion out of range
        for (int hf = 0; hf < 2; ++hf) {
            __syncthreads();   // the operand reads, or the previous half's tile reads, are done
            if (wm == hf) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t c = 64 * wn + 16 * j + (lane & 15);
                        const float b = p.bias && n0 + c < N ? p.bias[n0 + c] : 0.0f;
#pragma unroll
                        for (int r = 0; r < 4; ++r) tile[(16 * i + 4 * (lane >> 4) + r) * GM_ES + c] = acc[i][j][r] + b;
                    }
            }
            __syncthreads();
            const float* tr = tile + row * GM_ES;
            float x[32];
#pragma unroll
            for (int e = 0; e < 32; e += 4) {
                const floatx4 t = *reinterpret_cast<const floatx4*>(tr + c0 + e);
                x[e] = t[0];
                x[e + 1] = t[1];
                x[e + 2] = t[2];
                x[e + 3] = t[3];
            }
            // the head's D / 32 threads are lanes 4 t + (0..3) or (0, 1) / (2, 3): the
            // butterflies run in every lane, rows past M or columns past N included
            float inv = 1.0f;
            if (ep.gamma) {   // rmsNormRow (LocalModel.hpp:1341-1348)
                float ss = 0.0f;
#pragma unroll
                for (int e = 0; e < 32; ++e) ss = fmaf(x[e], x[e], ss);
                ss += __shfl_xor(ss, 1, WAVE);
                if (D == 128) ss += __shfl_xor(ss, 2, WAVE);
                inv = 1.0f / sqrtf(ss / float(D) + ep.eps);
            }
            const uint32_t m = m0 + 64 * hf + row;
            if (m < M && n < N) {
                const uint32_t pos = ep.start + m;
                float y[32];
#pragma unroll
                for (int e = 0; e < 32; ++e) y[e] = ep.gamma ? x[e] * inv * (ep.gamma[d0 + e] + ep.offset) : x[e];
                if (half) {   // rotate-half pairs (LocalModel.hpp:2624-2641), the angle float(pos) * freq
                    const float fpos = float(pos);
#pragma unroll
                    for (int e = 0; e < 32; ++e) {
                        const uint32_t d = d0 + e;
                        if (d < 2 * half) {
                            const bool low = d < half;
                            const uint32_t dp = low ? d + half : d - half;
                            const float xp = ep.gamma ? tr[hc + dp] * inv * (ep.gamma[dp] + ep.offset) : tr[hc + dp];
                            float sn, cs;
                            sincosf(fpos * ep.freqs[low ? d : dp], &sn, &cs);
                            y[e] = low ? y[e] * cs - xp * sn : y[e] * cs + xp * sn;
                        }
                    }
                }
                uint16_t* cdst = ep.cache + (size_t(head) * ep.capacity + pos) * D + d0;
                _Float16* wdst = static_cast<_Float16*>(ep.work) + (size_t(head) * ep.T + pos) * D + d0;
#pragma unroll
                for (int e = 0; e < 32; e += 8) {
                    u32x4 wb;
                    half8 wh;
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        wb[t] = uint32_t(float_to_bf16_bits(y[e + 2 * t])) |
                                (uint32_t(float_to_bf16_bits(y[e + 2 * t + 1])) << 16);
#pragma unroll
                    for (int t = 0; t < 8; ++t) wh[t] = to_f16_checked(y[e + t], bad);
                    *reinterpret_cast<u32x4*>(cdst + e) = wb;
                    *reinterpret_cast<half8*>(wdst + e) = wh;
                }
            }
        }
        raise_range_flag(ep.rangeFlag, bad);
    }
}

/*
    gemm_dma_kernel: bf16 weights and enough rows for 256 x 256 tiles, after
    split_a_kernel has split a into bf16 high parts and residuals ([M][K]
    each). Four waves of 128 x 128 (8 x 8 v_mfma_f32_16x16x32_bf16 tiles, the
    256 fp32 accumulators per lane in AGPRs, one workgroup per CU); per
    32-wide K step a wave reads 24 KB of operands from LDS for 128 MFMAs.
    Every operand comes in by DMA (global_load_lds, 1 KB blocks) into a
    three-stage LDS ring of 48 KB stages, step t + 2 issued between step t's
    MFMAs, so nothing passes through registers or the VALU and each step's
    loads have two steps of compute to land; one barrier per step. Within a
    1 KB block (16 rows of 64 bytes) row r keeps its 16-byte chunk c at
    position c ^ s(r % 16), s(x) = ((x / 2) % 4) ^ (x / 8): the 16 rows of an
    operand read fall on distinct banks both as one 256-byte access and as
    two 128-byte halves.
*/
constexpr int GD_BM = 256, GD_BN = 256, GD_BK = 32, GD_STAGES = 3;
constexpr int GD_OPB = GD_BM * GD_BK * 2;   // bytes of one operand's tile per step (16 KB)
constexpr int GD_STAGE = 3 * GD_OPB;         // a hi, a lo, w

__global__ __launch_bounds__(256) void split_a_kernel(const float* a, bf16x8* hi, bf16x8* lo, uint64_t pieces) {
    for (uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x; i < pieces; i += uint64_t(gridDim.x) * 256) {
        const floatx4 x0 = reinterpret_cast<const floatx4*>(a)[2 * i];
        const floatx4 x1 = reinterpret_cast<const floatx4*>(a)[2 * i + 1];
        bf16x8 h, l;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            h[t] = __bf16(x0[t]);
            l[t] = __bf16(x0[t] - float(h[t]));
            h[4 + t] = __bf16(x1[t]);
            l[4 + t] = __bf16(x1[t] - float(h[4 + t]));
        }
        hi[i] = h;
        lo[i] = l;
    }
}

/* s_waitcnt vmcnt(N) alone (N < 64) */
template <int N>
__device__ __forceinline__ void gd_wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

/* w2: columns from nSplit on come from w2's rows (n - nSplit), a multiple of
   256 so that no tile straddles the two; null for one weight */
__global__ __launch_bounds__(256) void gemm_dma_kernel(GemvParams p, const __bf16* ahi, const __bf16* alo,
                                                       const void* w2, uint32_t nSplit) {
    __shared__ __align__(16) uint8_t smem[GD_STAGES * GD_STAGE];
    const int tid = threadIdx.x, lane = tid & 63, wm = (tid >> 6) >> 1, wn = (tid >> 6) & 1;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: DMA targets are scalar
    const uint32_t K = p.k, M = p.m, N = p.n;
    const uint32_t ntN = (N + GD_BN - 1) / GD_BN;
    // consecutive workgroups go to different XCDs: remap them so that each XCD
    // takes a band of whole rows of tiles (its L2 then holds a band of a and
    // every XCD reads w), when the tile count splits evenly over the eight
    uint32_t lg = blockIdx.x;
    if (gridDim.x % 8 == 0) lg = (lg % 8) * (gridDim.x / 8) + lg / 8;
    const uint32_t m0 = (lg / ntN) * GD_BM, n0 = (lg % ntN) * GD_BN;
    const uint32_t ldsBase = lds_address(smem);

    // this wave's twelve DMA blocks of a step: block j is operand j / 4 (a hi,
    // a lo, w), rows 16 (4 w + j % 4) .. + 15 of its tile; lane l takes row
    // + l / 4, LDS chunk l % 4, which holds the row's chunk (l % 4) ^ s(l / 4).
    // Rows past M or N read the last row: they only reach outputs past M or
    // N, which are not stored.
    const bool second = w2 && n0 >= nSplit;
    const uint32_t wn0 = second ? n0 - nSplit : n0, wlim = w2 ? (second ? N - nSplit : nSplit) : N;
    uint32_t doff[12];
#pragma unroll
    for (int j = 0; j < 12; ++j) {
        const uint32_t row = 16u * (4u * uint32_t(w) + (j & 3)) + uint32_t(lane >> 2);
        const uint32_t chunk = uint32_t(lane & 3) ^ uint32_t(((lane >> 3) & 3) ^ (lane >> 5));
        const uint32_t g = (j < 8 ? m0 : wn0) + row, lim = j < 8 ? M : wlim;
        doff[j] = ((g < lim ? g : lim - 1) * K + 8 * chunk) * 2;
    }
    const uint8_t* const bases[3] = {reinterpret_cast<const uint8_t*>(ahi), reinterpret_cast<const uint8_t*>(alo),
                                     static_cast<const uint8_t*>(second ? w2 : p.w)};
    auto dma = [&](uint32_t kt, int j) __attribute__((always_inline)) {
        const uint32_t stage = kt % GD_STAGES;
        dma_block(bases[j >> 2] + size_t(kt) * GD_BK * 2, doff[j],
                  ldsBase + stage * GD_STAGE + (j >> 2) * GD_OPB + (4 * w + (j & 3)) * 1024);
    };

    floatx4 acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    const int fr = lane & 15, sw = 16 * ((lane >> 4) ^ ((fr >> 1) & 3) ^ (fr >> 3));   // swizzled chunk of k 8 (lane / 16) ..
    const uint32_t nk = K / GD_BK;
#pragma unroll
    for (int j = 0; j < 12; ++j) dma(0, j);
    if (nk > 1) {
#pragma unroll
        for (int j = 0; j < 12; ++j) dma(1, j);
    }
    // step kt; MORE: step kt + 2's DMA goes out between its row tiles
    auto step = [&](uint32_t kt, auto MORE) __attribute__((always_inline)) {
        // step kt's blocks have landed (in order: step kt + 1's may still be
        // in flight); after the barrier every wave's have, and every read of
        // the stage step kt + 2 goes into (that of step kt - 1) is done. Not
        // __syncthreads(): its fence would wait for step kt + 1's blocks too.
        if (kt + 1 < nk) gd_wait_vmcnt<12>();
        else gd_wait_vmcnt<0>();
        lds_barrier();
        const uint8_t* st = smem + (kt % GD_STAGES) * GD_STAGE;
        bf16x8 bh[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            bh[j] = *reinterpret_cast<const bf16x8*>(st + 2 * GD_OPB + (128 * wn + 16 * j + fr) * 64 + sw);
        const int ro = (128 * wm + fr) * 64 + sw;
        bf16x8 ah = *reinterpret_cast<const bf16x8*>(st + ro);
        bf16x8 al = *reinterpret_cast<const bf16x8*>(st + GD_OPB + ro);
#pragma unroll
        for (int i = 0; i < 8; ++i) {   // row tile i + 1's a operands are read while tile i computes
            bf16x8 nh = ah, nl = al;
            if (i < 7) {
                nh = *reinterpret_cast<const bf16x8*>(st + ro + (i + 1) * 1024);
                nl = *reinterpret_cast<const bf16x8*>(st + GD_OPB + ro + (i + 1) * 1024);
            }
            if constexpr (decltype(MORE)::value) {   // the 12 blocks over the 8 row tiles: two, one, two, ...
                dma(kt + 2, 3 * (i / 2) + 2 * (i & 1));
                if (!(i & 1)) dma(kt + 2, 3 * (i / 2) + 1);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh[j], acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh[j], acc[i][j], 0, 0, 0);
            }
            ah = nh;
            al = nl;
        }
    };
    uint32_t kt = 0;
    for (; kt + 2 < nk; ++kt) step(kt, std::integral_constant<bool, true>{});
    for (; kt < nk; ++kt) step(kt, std::integral_constant<bool, false>{});
    // the accumulator layout: lane holds rows 4 (lane / 16) + r of column lane % 16
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t n = n0 + 128 * wn + 16 * j + fr;
        if (n >= N) continue;
        const float b = p.bias ? p.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t m = m0 + 128 * wm + 16 * i + 4 * (lane >> 4) + r;
                if (m >= M) continue;
                float* o = p.out + size_t(m) * p.ldo + n;
                *o = (p.accumulate ? *o : 0.0f) + acc[i][j][r] + b;
            }
    }
}

/* The k and v projections' per-token work after one GEMM over both
   (kv[m][0 .. N1) k, [N1 .. 2 N1) v, fp32): the bias, then for k RMSNorm
   (gamma) and rotate-half RoPE (freqs), and each row appended to its bf16
   cache and to the flash kernel's fp16 copy, as gemm_kernel's k / v
   epilogue does (the same operations in the same order per element; the
   norm's sum of squares is reduced in another order). One workgroup per
   token: the token's rotation angles float(pos) * freq go through sincosf
   once into LDS, then the four waves take its 2 * heads rows (k and v of
   each kv head) in turn, a row staged in LDS for the RoPE partner. A lane
   holds D / 64 consecutive elements. With rope set, the angles' cos and sin
   also go to the flash kernel's table (rope_at);
   with padK / padV set, workgroup 0 zeroes pad16 16-byte pieces of each
   (the working copies' pad rows). */
__global__ __launch_bounds__(256) void kv_epilogue_kernel(const float* kv, const float* kBias, const float* vBias,
                                                          KvEpilogue ek, KvEpilogue ev, uint32_t heads, float* rope,
                                                          uint4* padK, uint4* padV, uint32_t pad16) {
    __shared__ float row[4][128];
    __shared__ float sinT[64], cosT[64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t t = blockIdx.x, pos = ek.start + t;
    const uint32_t half = ek.freqs ? ek.rot / 2 : 0;   // rot <= D <= 128
    if (w == 0 && uint32_t(lane) < half) {
        float sn, cs;
        sincosf(float(pos) * ek.freqs[lane], &sn, &cs);
        sinT[lane] = sn;
        cosT[lane] = cs;
        if (rope) {
            rope[rope_at(t, 0, uint32_t(lane), half, gridDim.x)] = cs;
            rope[rope_at(t, 1, uint32_t(lane), half, gridDim.x)] = sn;
        }
    }
    if (padK && t == 0)
        for (uint32_t i = threadIdx.x; i < pad16; i += 256) {
            padK[i] = uint4{0u, 0u, 0u, 0u};
            padV[i] = uint4{0u, 0u, 0u, 0u};
        }
    __syncthreads();
    const uint32_t D = ek.dim, N1 = heads * D, EPL = D / 64;   // D 64 or 128
    const uint32_t d0 = uint32_t(lane) * EPL;
    for (uint32_t r = uint32_t(w); r < 2 * heads; r += 4) {
        const uint32_t which = r & 1, h = r >> 1;
        const KvEpilogue& e = which ? ev : ek;
        const float* bias = which ? vBias : kBias;
        const float* src = kv + (size_t(t) * 2 + which) * N1 + size_t(h) * D + d0;
        float x[2] = {0.0f, 0.0f};
        if (EPL == 2) {
            const float2 v2 = *reinterpret_cast<const float2*>(src);   // kv rows are 8-byte aligned
            x[0] = v2.x;
            x[1] = v2.y;
        } else {
            x[0] = src[0];
        }
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if (bias && uint32_t(i) < EPL) x[i] += bias[size_t(h) * D + d0 + i];
            ss = fmaf(x[i], x[i], ss);
        }
        float inv = 1.0f;
        if (e.gamma) inv = 1.0f / sqrtf(wave_sum(ss) / float(D) + e.eps);
        float y[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            y[i] = e.gamma && uint32_t(i) < EPL ? x[i] * inv * (e.gamma[d0 + i] + e.offset) : x[i];
            if (uint32_t(i) < EPL) row[w][d0 + i] = y[i];
        }
        wave_sync();
        const uint32_t hf = e.freqs ? half : 0;
        bool bad = false;
        uint16_t cb[2];
        _Float16 wb[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t d = d0 + i;
            float v = y[i];
            if (d < 2 * hf) {   // rotate-half pairs (LocalModel.hpp:2624-2641)
                const bool low = d < hf;
                const uint32_t j = low ? d : d - hf, dp = low ? d + hf : d - hf;
                v = low ? y[i] * cosT[j] - row[w][dp] * sinT[j] : y[i] * cosT[j] + row[w][dp] * sinT[j];
            }
            cb[i] = float_to_bf16_bits(v);
            wb[i] = to_f16_checked(v, bad);
        }
        uint16_t* cdst = e.cache + (size_t(h) * e.capacity + pos) * D + d0;
        _Float16* wdst = static_cast<_Float16*>(e.work) + (size_t(h) * e.T + pos) * D + d0;
        if (EPL == 2) {   // 4-byte stores: rows are 16-byte aligned, d0 even
            *reinterpret_cast<uint32_t*>(cdst) = uint32_t(cb[0]) | (uint32_t(cb[1]) << 16);
            _Float16 __attribute__((ext_vector_type(2))) w2 = {wb[0], wb[1]};
            *reinterpret_cast<decltype(w2)*>(wdst) = w2;
        } else {
            cdst[0] = cb[0];
            wdst[0] = wb[0];
        }
        raise_range_flag(e.rangeFlag, bad);
        wave_sync();   // the row's partner reads are done before the next row is staged
    }
}

/* the K slices' partial tiles added in slice order, then the bias and the
   accumulate: out[m][n] (+)= sum_s part[s][m][n] + bias[n] */
__global__ __launch_bounds__(256) void split_reduce_kernel(GemvParams p, const float* part, uint32_t slices) {
    const uint64_t outs = uint64_t(p.m) * p.n;
    for (uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x; i < outs; i += uint64_t(gridDim.x) * 256) {
        float v = 0.0f;
        for (uint32_t sl = 0; sl < slices; ++sl) v += part[uint64_t(sl) * outs + i];
        const uint32_t m = uint32_t(i / p.n), n = uint32_t(i % p.n);
        float* o = p.out + size_t(m) * p.ldo + n;
        *o = (p.accumulate ? *o : 0.0f) + v + (p.bias ? p.bias[n] : 0.0f);
    }
}

/* any k for F32 and BF16 (rows not on 16-byte boundaries): one wave per
   weight row and a row of a, element by element */
template <int TYPE>
__global__ __launch_bounds__(256) void gemv_scalar_kernel(GemvParams p) {
    const int lane = threadIdx.x & 63;
    const uint64_t task = uint64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (task >= uint64_t(p.n) * p.m) return;
    const uint32_t n = uint32_t(task % p.n), i = uint32_t(task / p.n);
    const float* x = p.a + size_t(i) * p.k;
    float s = 0.0f;
    for (uint32_t t = lane; t < p.k; t += WAVE) {
        const float wv = TYPE == 0 ? static_cast<const float*>(p.w)[size_t(n) * p.k + t]
                                   : bf16_bits_to_float(static_cast<const uint16_t*>(p.w)[size_t(n) * p.k + t]);
        s = fmaf(x[t], wv, s);
    }
    s = wave_sum(s);
    if (lane == 0) {
        float* o = p.out + size_t(i) * p.ldo + n;
        *o = (p.accumulate ? *o : 0.0f) + s + (p.bias ? p.bias[n] : 0.0f);
    }
}

/* bf16 weights with at least 256 tiles of 256 x 256 (a and w under 4 GB,
   k a multiple of 32) take split_a_kernel and gemm_dma_kernel */
bool dma_eligible(const GemvParams& p) {
    // at least half a 256-row tile of a: fewer rows (a decode step's GEMV
    // against a wide weight such as an LM head) would waste most of every tile
    if (p.type != 1 || p.m < GD_BM / 2 || p.k % GD_BK || (reinterpret_cast<uintptr_t>(p.w) % 16) ||
        (reinterpret_cast<uintptr_t>(p.a) % 16))
        return false;
    const uint64_t wide = uint64_t((p.m + GD_BM - 1) / GD_BM) * ((p.n + GD_BN - 1) / GD_BN);
    return wide >= 256 && wide <= 0x7FFFFFFFull && uint64_t(p.m) * p.k * 2 < (1ull << 32) &&
           uint64_t(p.n) * p.k * 2 < (1ull << 32);
}

/* a split into its bf16 high parts and residuals (scratch slot SLOT_GEMM_A),
   unless `split` says the slot already holds them, then the DMA GEMM; w2 /
   nSplit as gemm_dma_kernel */
bool launch_dma(Context& ctx, const GemvParams& p, const void* w2, uint32_t nSplit, bool split, hipStream_t stream) {
    const uint64_t wide = uint64_t((p.m + GD_BM - 1) / GD_BM) * ((p.n + GD_BN - 1) / GD_BN);
    const uint64_t aBytes = uint64_t(p.m) * p.k * 2;   // one bf16 image of a
    uint8_t* img = static_cast<uint8_t*>(ctx.grow(SLOT_GEMM_A, 2 * aBytes));
    if (!img) return false;
    bf16x8* hi = reinterpret_cast<bf16x8*>(img);
    bf16x8* lo = reinterpret_cast<bf16x8*>(img + aBytes);
    if (!split) {
        const uint64_t pieces = aBytes / 16;
        const unsigned sg = unsigned((pieces + 255) / 256 < 8192 ? (pieces + 255) / 256 : 8192);
        if (!ctx.launch("split_a_kernel", stream, [&] {
                hipLaunchKernelGGL(split_a_kernel, dim3(sg), dim3(256), 0, stream, p.a, hi, lo, pieces);
            }))
            return false;
    }
    return ctx.launch("gemm_dma_kernel", stream, [&] {
        hipLaunchKernelGGL(gemm_dma_kernel, dim3(unsigned(wide)), dim3(256), 0, stream, p,
                           reinterpret_cast<const __bf16*>(hi), reinterpret_cast<const __bf16*>(lo), w2, nSplit);
    });
}

template <int TYPE>
bool launch_type(Context& ctx, const GemvParams& p, hipStream_t stream) {
    constexpr int E = piece_elems<TYPE>();
    if (p.k % E || (reinterpret_cast<uintptr_t>(p.w) % 16) || (reinterpret_cast<uintptr_t>(p.a) % 16)) {
        if constexpr (TYPE <= 1) {
            const uint64_t tasks = uint64_t(p.n) * p.m;
            if ((tasks + 3) / 4 > 0x7FFFFFFFull) return ctx.fail("matmul: too many outputs");
            return ctx.launch("gemv_scalar_kernel", stream, [&] {
                hipLaunchKernelGGL((gemv_scalar_kernel<TYPE>), dim3(unsigned((tasks + 3) / 4)), dim3(256), 0, stream, p);
            });
        }
        return ctx.fail("matmul: quantised weights need k a multiple of 32 and 16-byte aligned rows");
    }
    if constexpr (TYPE == 1) {
        if (dma_eligible(p)) return launch_dma(ctx, p, nullptr, 0, false, stream);
    }
    if (p.m >= GEMM_MIN_M) {
        const uint32_t tiles = ((p.n + GM_BN - 1) / GM_BN) * ((p.m + GM_BM - 1) / GM_BM);
        // fewer tiles than CUs and a long K: split K into slices of at least
        // 256 (multiples of a 32-wide step, so Q8/Q4 scale blocks stay whole),
        // each writing a partial tile; split_reduce_kernel adds them in order
        uint32_t slices = 1;
        if (tiles < 256 && p.k >= 512) {
            slices = (512 + tiles - 1) / tiles;
            if (slices > p.k / 256) slices = p.k / 256;
            if (slices > 64) slices = 64;
        }
        const uint32_t kSlice = ((p.k + slices - 1) / slices + GM_BK - 1) / GM_BK * GM_BK;
        slices = (p.k + kSlice - 1) / kSlice;
        const dim3 grid(unsigned((p.n + GM_BN - 1) / GM_BN), unsigned((p.m + GM_BM - 1) / GM_BM), slices);
        if (grid.y > 65535u) return ctx.fail("matmul: too many rows of a");
        if (slices == 1)
            return ctx.launch("gemm_kernel", stream, [&] {
                hipLaunchKernelGGL((gemm_kernel<TYPE, false>), grid, dim3(256), 0, stream, p, KvEpilogue{}, kSlice);
            });
        float* part = static_cast<float*>(ctx.grow(SLOT_GEMM_SPLIT, size_t(slices) * p.m * p.n * sizeof(float)));
        if (!part) return false;
        GemvParams q = p;
        q.out = part;
        q.ldo = p.n;
        q.bias = nullptr;
        q.accumulate = 0;
        if (!ctx.launch("gemm_kernel", stream, [&] {
                hipLaunchKernelGGL((gemm_kernel<TYPE, false>), grid, dim3(256), 0, stream, q, KvEpilogue{}, kSlice);
            }))
            return false;
        const uint64_t outs = uint64_t(p.m) * p.n;
        const unsigned rg = unsigned((outs + 255) / 256 < 65536 ? (outs + 255) / 256 : 65536);
        return ctx.launch("split_reduce_kernel", stream, [&] {
            hipLaunchKernelGGL(split_reduce_kernel, dim3(rg), dim3(256), 0, stream, p, part, slices);
        });
    }
    const unsigned gx = unsigned((p.n + 4 * GEMV_ROWS - 1) / (4 * GEMV_ROWS));
    const int M = p.m <= 1 ? 1 : (p.m <= 2 ? 2 : (p.m <= 4 ? 4 : GEMV_MAX_M));
    const unsigned gy = unsigned((p.m + M - 1) / M);
    if (gy > 65535u) return ctx.fail("matmul: too many rows of a");
    return ctx.launch("gemv_kernel", stream, [&] {
        const dim3 grid(gx, gy);
        if (M == 1) hipLaunchKernelGGL((gemv_kernel<TYPE, 1>), grid, dim3(256), 0, stream, p);
        else if (M == 2) hipLaunchKernelGGL((gemv_kernel<TYPE, 2>), grid, dim3(256), 0, stream, p);
        else if (M == 4) hipLaunchKernelGGL((gemv_kernel<TYPE, 4>), grid, dim3(256), 0, stream, p);
        else hipLaunchKernelGGL((gemv_kernel<TYPE, 8>), grid, dim3(256), 0, stream, p);
    });
}

} // namespace

bool launch_gemv(const GemvParams& p, hipStream_t stream) {
    Context& ctx = Context::instance();
    if (p.m == 0 || p.n == 0) return true;
    if (!p.a || !p.w || !p.out) return ctx.fail("matmul: null tensor");
    if (p.k == 0) return ctx.fail("matmul: k must be positive");
    if (p.ldo < p.n) return ctx.fail("matmul: output row stride below n");
    if (p.type >= 2 && !p.scales) return ctx.fail("matmul: quantised weights need scales");
    if (p.type >= 2 && p.k % 32) return ctx.fail("matmul: quantised weights need k a multiple of 32");
    switch (p.type) {
        case 0: return launch_type<0>(ctx, p, stream);
        case 1: return launch_type<1>(ctx, p, stream);
        case 2: return launch_type<2>(ctx, p, stream);
        case 3: return launch_type<3>(ctx, p, stream);
        default: return ctx.fail("matmul: unknown weight type");
    }
}

static bool kv_checks(Context& ctx, const GemvParams& p, const KvEpilogue& e);

bool gemm_splits_a(const GemvParams& p) { return dma_eligible(p); }

uint16_t* gemm_split_image(const GemvParams& p) {
    if (!dma_eligible(p)) return nullptr;
    return static_cast<uint16_t*>(Context::instance().grow(SLOT_GEMM_A, 2 * uint64_t(p.m) * p.k * 2));
}

bool launch_gemv_presplit(const GemvParams& p, hipStream_t stream) {
    Context& ctx = Context::instance();
    if (p.m == 0 || p.n == 0) return true;
    if (!p.w || !p.out || p.ldo < p.n || !dma_eligible(p)) return ctx.fail("matmul: no presplit GEMM for this shape");
    return launch_dma(ctx, p, nullptr, 0, true, stream);
}

bool launch_gemm_kv_pair(const GemvParams& pk, const GemvParams& pv, const KvEpilogue& ek, const KvEpilogue& ev,
                         bool aSplit, bool fold, float* rope, bool* folded, hipStream_t stream) {
    Context& ctx = Context::instance();
    *folded = false;
    // one DMA GEMM over both weights when each is a multiple of 256 columns
    // (no tile straddles them) and the pair has the tiles for it
    GemvParams both = pk;
    both.n = pk.n + pv.n;
    both.ldo = both.n;
    both.bias = nullptr;
    both.accumulate = 0;
    const bool pair = pk.type == 1 && pv.type == 1 && pk.k == pv.k && pk.m == pv.m && pk.a == pv.a && pk.n == pv.n &&
                      pk.n % GD_BN == 0 && (ek.dim == 64 || ek.dim == 128) && ek.dim == ev.dim &&
                      (reinterpret_cast<uintptr_t>(pv.w) % 16) == 0 && dma_eligible(both);
    if (!pair) return launch_gemm_kv(pk, ek, stream) && launch_gemm_kv(pv, ev, stream);
    if (pk.m == 0) return true;
    if (!kv_checks(ctx, pk, ek) || !kv_checks(ctx, pv, ev)) return false;
    float* kv = static_cast<float*>(ctx.grow(SLOT_MIXER_KV, size_t(pk.m) * both.n * sizeof(float)));
    if (!kv) return false;
    both.out = kv;
    if (!launch_dma(ctx, both, pv.w, pk.n, aSplit, stream)) return false;
    const uint32_t heads = pk.n / ek.dim;
    if (pk.m > 0x7FFFFFFFu) return ctx.fail("projection epilogue: too many rows");
    if (fold && rope && !ek.freqs) return ctx.fail("projection epilogue: a cos/sin table needs RoPE");
    // the pad rows start past the last head's T rows (16-byte aligned: dim is 64 or 128)
    const size_t padAt = size_t(heads) * ek.T * ek.dim * 2;
    uint4* padK = fold ? reinterpret_cast<uint4*>(static_cast<uint8_t*>(ek.work) + padAt) : nullptr;
    uint4* padV = fold ? reinterpret_cast<uint4*>(static_cast<uint8_t*>(ev.work) + padAt) : nullptr;
    const uint32_t pad16 = PREFILL_PAD_ROWS * ek.dim * 2 / 16;
    if (!ctx.launch("kv_epilogue_kernel", stream, [&] {
            hipLaunchKernelGGL(kv_epilogue_kernel, dim3(pk.m), dim3(256), 0, stream, kv, pk.bias, pv.bias, ek, ev,
                               heads, fold ? rope : nullptr, padK, padV, pad16);
        }))
        return false;
    *folded = fold;
    return true;
}

/* the shapes and alignments a k or v projection with its epilogue needs */
static bool kv_checks(Context& ctx, const GemvParams& p, const KvEpilogue& e) {
    if (!p.a || !p.w || !e.cache || !e.work) return ctx.fail("projection epilogue: null tensor");
    if (e.dim != 64 && e.dim != 128) return ctx.fail("projection epilogue: dim must be 64 or 128");
    if (p.n == 0 || p.n % e.dim) return ctx.fail("projection epilogue: n must be a multiple of dim");
    if (e.freqs && (e.rot == 0 || e.rot > e.dim || e.rot % 2)) return ctx.fail("projection epilogue: bad rotaryDims");
    if (uint64_t(e.start) + p.m > e.T || e.T > e.capacity) return ctx.fail("projection epilogue: rows past the cache");
    if (p.k == 0) return ctx.fail("matmul: k must be positive");
    if (p.type >= 2 && (!p.scales || p.k % 32)) return ctx.fail("matmul: quantised weights need scales and k % 32");
    const int E = p.type == 0 ? 4 : (p.type == 1 ? 8 : (p.type == 2 ? 16 : 32));
    if (p.k % E || (reinterpret_cast<uintptr_t>(p.w) % 16) || (reinterpret_cast<uintptr_t>(p.a) % 16) ||
        (reinterpret_cast<uintptr_t>(e.cache) % 16) || (reinterpret_cast<uintptr_t>(e.work) % 16))
        return ctx.fail("projection epilogue: rows of a, w and the caches must be 16-byte aligned");
    return true;
}

bool launch_gemm_kv(const GemvParams& p, const KvEpilogue& e, hipStream_t stream) {
    Context& ctx = Context::instance();
    if (p.m == 0) return true;
    if (!kv_checks(ctx, p, e)) return false;
    const dim3 grid(unsigned((p.n + GM_BN - 1) / GM_BN), unsigned((p.m + GM_BM - 1) / GM_BM));
    if (grid.y > 65535u) return ctx.fail("matmul: too many rows of a");
    return ctx.launch("gemm_kv_kernel", stream, [&] {
        switch (p.type) {
            case 0: hipLaunchKernelGGL((gemm_kernel<0, true>), grid, dim3(256), 0, stream, p, e, p.k + GM_BK); break;
            case 1: hipLaunchKernelGGL((gemm_kernel<1, true>), grid, dim3(256), 0, stream, p, e, p.k + GM_BK); break;
            case 2: hipLaunchKernelGGL((gemm_kernel<2, true>), grid, dim3(256), 0, stream, p, e, p.k + GM_BK); break;
            default: hipLaunchKernelGGL((gemm_kernel<3, true>), grid, dim3(256), 0, stream, p, e, p.k + GM_BK); break;
        }
    });
}

} // namespace aigpu
