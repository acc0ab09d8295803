// delta_rule.hip - the gated delta rule of gatedDeltaNetMixer
// (LocalModel.hpp:2802-2830, deltaStep at Kernels.hpp:105-128) as a chunked
// scan for gfx950.
//
// Per value head h, token t (key head h / (valueHeads/keyHeads)):
//   S_t = a_t S_{t-1} + k_t u_t^T,  u_t = beta_t (v_t - a_t S_{t-1}^T k_t),
//   o_t = S_t^T q_t,                a_t = exp(g_t)
// Over a chunk of C = 64 tokens with gamma_t = exp(gc_t) (gc the in-chunk
// cumulative sum of g) this unrolls to
//   (I + A) U = diag(beta) (V - diag(gamma) K S0),
//       A[i][j] = beta_i (k_i.k_j) exp(gc_i - gc_j)      (j < i)
//   O  = diag(gamma) Q S0 + QKm U,  QKm[i][j] = (q_i.k_j) exp(gc_i - gc_j)  (j <= i)
//   S' = gamma_last S0 + sum_j exp(gc_last - gc_j) k_j u_j^T
// Every exponent is a difference gc_i - gc_j <= 0 or gc itself, so nothing
// overflows however strongly the gates decay.
//
// Two launches:
//   delta_solve_kernel  parallel over (head, chunk): l2 norms, KK^T, QK^T,
//                       the decayed masks and T = (I + A)^-1 (blocked: four
//                       16 x 16 diagonal blocks by forward substitution, the
//                       rest by block products); writes T, QKm, gc, beta and
//                       the per-row inverse norms to a workspace
//   delta_scan_kernel   per (head, 16 value columns): walks the chunks in
//                       order carrying S (fp32, in LDS), U = T R, outputs
//                       and the state update on v_mfma_f32_16x16x4f32. It
//                       reads the raw q/k rows and applies the inverse norms
//                       as row scales of the products (k_i = k_raw_i kinv_i
//                       enters every product linearly), and it loads chunk
//                       c + 1 into registers while it computes chunk c.
// State columns evolve independently (Kernels.hpp:113-125 touches column d
// only through delta[d]), which is what lets one head split over 16-column
// workgroups.
#include "context.hpp"
#include "device.hpp"
#include "kernels.hpp"

namespace aigpu {

namespace {

constexpr int CH = 64;                   // chunk length
constexpr int CS = CH + 1;               // LDS row stride of CH x CH matrices
constexpr int NB = 16;                   // value columns per scan workgroup
constexpr int NS = NB + 1;
constexpr int SC = 4 * CH;               // gc, beta, kinv, qinv per chunk
constexpr int WORK = 2 * CH * CH + SC;   // floats per (head, chunk) record

struct DeltaArgs {
    DeltaRuleParams p;
    float* work;       // [valueHeads][nChunks][WORK]: T, QKm, gc, beta, kinv, qinv
    uint32_t nChunks;
    uint32_t vec;      // q, k, v 16-byte aligned: vector loads
};

__device__ __forceinline__ float softplus_of(float x) { return x > 20.0f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float sigmoid_of(float x) { return 1.0f / (1.0f + expf(-x)); }

/* raw bits of 16 bytes of input starting at element i: 8 bf16 or 4 f32;
   one vector load when the tensor is 16-byte aligned */
template <bool F32>
__device__ __forceinline__ u32x4 load_raw16(const void* base, size_t i, bool vec) {
    if (vec) {
        if (F32) return *reinterpret_cast<const u32x4*>(static_cast<const float*>(base) + i);
        return *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + i);
    }
    u32x4 r;
    if (F32) {
        const uint32_t* s = static_cast<const uint32_t*>(base) + i;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = s[e];
    } else {
        const uint16_t* s = static_cast<const uint16_t*>(base) + i;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = uint32_t(s[2 * e]) | (uint32_t(s[2 * e + 1]) << 16);
    }
    return r;
}

/* element e of a 16-byte raw group as fp32 (e < 8 for bf16, e < 4 for f32) */
template <bool F32>
__device__ __forceinline__ float raw_elem(const u32x4& r, int e) {
    if (F32) return __uint_as_float(r[e]);
    const uint32_t w = r[e >> 1];
    return __uint_as_float((e & 1) ? (w & 0xFFFF0000u) : (w << 16));
}

/* the gates of tokens t0 .. t0+63 for value head h: lane = token; g is
   cumulated over the chunk (LocalModel.hpp:2820-2823 for the raw form) */
__device__ __forceinline__ void chunk_gates(const DeltaRuleParams& p, uint64_t t0, uint32_t n, uint32_t h,
                                            int lane, float& gc, float& beta) {
    float gt = 0.0f, bt = 0.0f;
    if (uint32_t(lane) < n) {
        const size_t i = (t0 + lane) * p.valueHeads + h;
        if (p.aLog) {
            gt = -expf(p.aLog[h]) * softplus_of(p.a[i] + p.dtBias[h]);
            bt = sigmoid_of(p.b[i]);
        } else {
            gt = p.g[i];
            bt = p.beta[i];
        }
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(gt, off, WAVE);
        if (lane >= off) gt += y;
    }
    gc = gt;
    beta = bt;
}

template <int KD, bool F32>
__global__ __launch_bounds__(256) void delta_solve_kernel(DeltaArgs a) {
    constexpr int KS = KD + 1;
    constexpr int PE = KD / 4;              // elements of a row per thread
    constexpr int EPL = F32 ? 4 : 8;        // elements per 16-byte load
    __shared__ float ks[CH * KS];
    __shared__ float qs[CH * KS];
    __shared__ float Am[CH * CS];
    __shared__ float Tm[CH * CS];
    __shared__ float Xs[4][16 * 17];
    __shared__ float sc[SC];                // gc, beta, kinv, qinv

    const DeltaRuleParams& p = a.p;
    const uint32_t chunk = blockIdx.x, h = blockIdx.y;
    const uint32_t kh = uint32_t(h / (p.valueHeads / p.keyHeads));
    const uint64_t t0 = uint64_t(chunk) * CH;
    const uint32_t n = uint32_t(p.count - t0 < CH ? p.count - t0 : CH);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c16 = lane & 15;
    float* rec = a.work + (size_t(h) * a.nChunks + chunk) * WORK;

    // rows: thread -> (row tid / 4, quarter tid % 4); l2 norms over the 4
    // threads of a row (LocalModel.hpp:2814-2818, l2normalise at :1380-1386)
    {
        const int r = tid >> 2, qq = tid & 3;
        u32x4 kr[PE / EPL], qr[PE / EPL];
        const size_t src = ((t0 + r) * p.keyHeads + kh) * KD + qq * PE;
#pragma unroll
        for (int i = 0; i < PE / EPL; ++i) {
            kr[i] = uint32_t(r) < n ? load_raw16<F32>(p.k, src + i * EPL, a.vec) : u32x4{0, 0, 0, 0};
            qr[i] = uint32_t(r) < n ? load_raw16<F32>(p.q, src + i * EPL, a.vec) : u32x4{0, 0, 0, 0};
        }
        float kss = 0.0f, qss = 0.0f;
#pragma unroll
        for (int i = 0; i < PE / EPL; ++i)
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const float kx = raw_elem<F32>(kr[i], e), qx = raw_elem<F32>(qr[i], e);
                kss += kx * kx;
                qss += qx * qx;
            }
        kss += __shfl_xor(kss, 1, WAVE);
        kss += __shfl_xor(kss, 2, WAVE);
        qss += __shfl_xor(qss, 1, WAVE);
        qss += __shfl_xor(qss, 2, WAVE);
        float kinv = 1.0f, qinv = 1.0f;
        if (p.normalize) {
            kinv = 1.0f / sqrtf(kss + 1e-6f);
            qinv = (1.0f / sqrtf(qss + 1e-6f)) * (1.0f / sqrtf(float(KD)));
        }
#pragma unroll
        for (int i = 0; i < PE / EPL; ++i)
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                ks[r * KS + qq * PE + i * EPL + e] = raw_elem<F32>(kr[i], e) * kinv;
                qs[r * KS + qq * PE + i * EPL + e] = raw_elem<F32>(qr[i], e) * qinv;
            }
        if (qq == 0) {
            sc[2 * CH + r] = kinv;
            sc[3 * CH + r] = qinv;
        }
    }
    if (w == 0) {
        float gc, bt;
        chunk_gates(p, t0, n, h, lane, gc, bt);
        sc[lane] = gc;
        sc[CH + lane] = bt;
    }
    // T starts as zero above the diagonal blocks
    for (int idx = tid; idx < CH * CH; idx += 256) {
        const int i = idx / CH, j = idx % CH;
        if ((j >> 4) > (i >> 4)) Tm[i * CS + j] = 0.0f;
    }
    __syncthreads();

    // KK^T and QK^T: wave w owns rows 16w..16w+15
    float* qkm = rec + CH * CH;
    for (int ct = 0; ct < 4; ++ct) {
        floatx4 kk = {0.0f, 0.0f, 0.0f, 0.0f}, qk = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
        for (int s = 0; s < KD / 4; ++s) {
            const float kj = ks[(16 * ct + c16) * KS + 4 * s + g];
            kk = __builtin_amdgcn_mfma_f32_16x16x4f32(ks[(16 * w + c16) * KS + 4 * s + g], kj, kk, 0, 0, 0);
            qk = __builtin_amdgcn_mfma_f32_16x16x4f32(qs[(16 * w + c16) * KS + 4 * s + g], kj, qk, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 16 * w + 4 * g + r, j = 16 * ct + c16;
            const float dec = j <= i ? expf(sc[i] - sc[j]) : 0.0f;
            Am[i * CS + j] = j < i ? sc[CH + i] * dec * kk[r] : 0.0f;
            qkm[i * CH + j] = dec * qk[r];
        }
    }
    __syncthreads();

    // T = (I + A)^-1. Diagonal blocks: wave w inverts block w by forward
    // substitution, lane = column within the block.
    {
        const int b0 = 16 * w;
        for (int i = 0; i < 16; ++i) {
            if (lane < 16) {
                float acc = 0.0f;
                for (int mm = lane; mm < i; ++mm) acc = fmaf(Am[(b0 + i) * CS + b0 + mm], Tm[(b0 + mm) * CS + b0 + lane], acc);
                Tm[(b0 + i) * CS + b0 + lane] = lane < i ? -acc : (lane == i ? 1.0f : 0.0f);
            }
            wave_sync();
        }
    }
    // Off-diagonal block (I, J): T_IJ = -T_II sum_{M=J}^{I-1} A_IM T_MJ; the
    // blocks of one block row are independent, one wave each.
    for (int I = 1; I < 4; ++I) {
        __syncthreads();
        if (w < I) {
            const int J = w;
            floatx4 x = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int M = J; M < I; ++M)
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    x = __builtin_amdgcn_mfma_f32_16x16x4f32(Am[(16 * I + c16) * CS + 16 * M + 4 * s + g],
                                                             Tm[(16 * M + 4 * s + g) * CS + 16 * J + c16], x, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) Xs[w][(4 * g + r) * 17 + c16] = x[r];
            wave_sync();
            floatx4 y = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < 4; ++s)
                y = __builtin_amdgcn_mfma_f32_16x16x4f32(Tm[(16 * I + c16) * CS + 16 * I + 4 * s + g],
                                                         Xs[w][(4 * s + g) * 17 + c16], y, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) Tm[(16 * I + 4 * g + r) * CS + 16 * J + c16] = -y[r];
        }
    }
    __syncthreads();

    for (int idx = tid; idx < CH * CH; idx += 256) rec[idx] = Tm[(idx / CH) * CS + idx % CH];
    rec[2 * CH * CH + tid] = sc[tid];
}

template <int KD, bool F32>
__global__ __launch_bounds__(256) void delta_scan_kernel(DeltaArgs a) {
    constexpr int KS = KD + 1;
    constexpr int EPL = F32 ? 4 : 8;                 // elements per 16-byte load
    constexpr int KQL = CH * KD / (256 * EPL);       // 16-byte loads per thread for k (and q)
    __shared__ float ks[CH * KS];                    // raw k rows of the chunk
    __shared__ float qs[CH * KS];                    // raw q rows
    __shared__ float Tm[CH * CS];
    __shared__ float Qm[CH * CS];
    __shared__ float Ss[KD * NS];
    __shared__ float Rs[CH * NS], Vn[CH * NS], vs[CH * NS];
    __shared__ float sc[SC];                         // gc, beta, kinv, qinv
    __shared__ float kdk[CH];                        // kinv_i exp(gc_last - gc_i)

    const DeltaRuleParams& p = a.p;
    // keep a head's column blocks on one XCD: they read the same records
    uint32_t bid = blockIdx.x;
    const uint32_t nb = gridDim.x, nCol = uint32_t(p.valueDim / NB);
    if (nb % 8 == 0) bid = (bid % 8) * (nb / 8) + bid / 8;
    const uint32_t h = bid / nCol, cb = bid % nCol;
    const uint32_t kh = uint32_t(h / (p.valueHeads / p.keyHeads));
    const uint32_t col0 = cb * NB;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c16 = lane & 15;
    const size_t VD = p.valueDim, Hv = p.valueHeads;
    const bool vec = a.vec != 0;

    float* state = p.state + size_t(h) * KD * VD;
    for (int idx = tid; idx < KD * NB; idx += 256) {
        const int i = idx / NB, j = idx % NB;
        Ss[i * NS + j] = state[size_t(i) * VD + col0 + j];
    }

    // registers holding the next chunk's inputs while the current one computes
    u32x4 kst[KQL], qst[KQL];
    floatx4 tst[4], mst[4];
    u32x4 vst;      // 4 value columns of one row (bf16: 8 bytes used)
    float sst;
    auto stage = [&](uint32_t chunk) {
        const uint64_t t0 = uint64_t(chunk) * CH;
        const uint32_t n = uint32_t(p.count - t0 < CH ? p.count - t0 : CH);
#pragma unroll
        for (int i = 0; i < KQL; ++i) {
            const int e = (tid + 256 * i) * EPL, r = e / KD, col = e % KD;
            const size_t src = ((t0 + r) * p.keyHeads + kh) * KD + col;
            kst[i] = uint32_t(r) < n ? load_raw16<F32>(p.k, src, vec) : u32x4{0, 0, 0, 0};
            qst[i] = uint32_t(r) < n ? load_raw16<F32>(p.q, src, vec) : u32x4{0, 0, 0, 0};
        }
        const float* rec = a.work + (size_t(h) * a.nChunks + chunk) * WORK;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            tst[i] = *reinterpret_cast<const floatx4*>(rec + 4 * (tid + 256 * i));
            mst[i] = *reinterpret_cast<const floatx4*>(rec + CH * CH + 4 * (tid + 256 * i));
        }
        sst = rec[2 * CH * CH + tid];
        {
            const int r = tid >> 2, c4 = 4 * (tid & 3);
            vst = u32x4{0, 0, 0, 0};
            if (uint32_t(r) < n) {
                const size_t src = ((t0 + r) * Hv + h) * VD + col0 + c4;
                if (F32) {
                    vst = vec ? *reinterpret_cast<const u32x4*>(static_cast<const float*>(p.v) + src)
                              : u32x4{__float_as_uint(static_cast<const float*>(p.v)[src]),
                                      __float_as_uint(static_cast<const float*>(p.v)[src + 1]),
                                      __float_as_uint(static_cast<const float*>(p.v)[src + 2]),
                                      __float_as_uint(static_cast<const float*>(p.v)[src + 3])};
                } else {
                    const uint16_t* vb = static_cast<const uint16_t*>(p.v) + src;
                    if (vec) {
                        const u32x2 x = *reinterpret_cast<const u32x2*>(vb);
                        vst = u32x4{x[0], x[1], 0, 0};
                    } else {
                        vst = u32x4{uint32_t(vb[0]) | (uint32_t(vb[1]) << 16), uint32_t(vb[2]) | (uint32_t(vb[3]) << 16), 0, 0};
                    }
                }
            }
        }
    };
    auto commit = [&]() {
#pragma unroll
        for (int i = 0; i < KQL; ++i) {
            const int e = (tid + 256 * i) * EPL, r = e / KD, col = e % KD;
#pragma unroll
            for (int x = 0; x < EPL; ++x) {
                ks[r * KS + col + x] = raw_elem<F32>(kst[i], x);
                qs[r * KS + col + x] = raw_elem<F32>(qst[i], x);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                const int idx = 4 * (tid + 256 * i) + x;
                Tm[(idx / CH) * CS + idx % CH] = tst[i][x];
                Qm[(idx / CH) * CS + idx % CH] = mst[i][x];
            }
        sc[tid] = sst;
        const int r = tid >> 2, c4 = 4 * (tid & 3);
#pragma unroll
        for (int x = 0; x < 4; ++x) vs[r * NS + c4 + x] = F32 ? __uint_as_float(vst[x]) : raw_elem<false>(vst, x);
    };

    stage(0);
    commit();
    for (uint32_t chunk = 0; chunk < a.nChunks; ++chunk) {
        const uint64_t t0 = uint64_t(chunk) * CH;
        const uint32_t n = uint32_t(p.count - t0 < CH ? p.count - t0 : CH);
        __syncthreads();   // chunk's inputs and S are in LDS
        if (chunk + 1 < a.nChunks) stage(chunk + 1);
        const float* gcs = sc;
        const float* bs = sc + CH;
        const float* kinv = sc + 2 * CH;
        const float* qinv = sc + 3 * CH;
        const float gLast = gcs[CH - 1];
        if (tid < CH) kdk[tid] = kinv[tid] * expf(gLast - gcs[tid]);

        // R = beta (V - gamma kinv (K_raw S))
        floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
        for (int s = 0; s < KD / 4; ++s)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ks[(16 * w + c16) * KS + 4 * s + g],
                                                       Ss[(4 * s + g) * NS + c16], acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 16 * w + 4 * g + r;
            Rs[i * NS + c16] = bs[i] * (vs[i * NS + c16] - expf(gcs[i]) * (kinv[i] * acc[r]));
        }
        __syncthreads();

        // U = T R
        acc = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < CH / 4; ++s)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(Tm[(16 * w + c16) * CS + 4 * s + g],
                                                       Rs[(4 * s + g) * NS + c16], acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) Vn[(16 * w + 4 * g + r) * NS + c16] = acc[r];
        __syncthreads();

        // O = gamma qinv (Q_raw S) + QKm U
        acc = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
        for (int s = 0; s < KD / 4; ++s)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qs[(16 * w + c16) * KS + 4 * s + g],
                                                       Ss[(4 * s + g) * NS + c16], acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 16 * w + 4 * g + r;
            acc[r] *= expf(gcs[i]) * qinv[i];
        }
#pragma unroll
        for (int s = 0; s < CH / 4; ++s)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(Qm[(16 * w + c16) * CS + 4 * s + g],
                                                       Vn[(4 * s + g) * NS + c16], acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t i = 16 * w + 4 * g + r;
            if (i < n) p.out[((t0 + i) * Hv + h) * VD + col0 + c16] = acc[r];
        }

        // S' = gamma_last S + sum_i k_raw_i (kinv_i exp(gc_last - gc_i)) U_i
        constexpr int MT = KD / 64;   // key-dim tiles per wave
        floatx4 sn[MT];
        const float eLast = expf(gLast);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int mt = w + 4 * t;
#pragma unroll
            for (int r = 0; r < 4; ++r) sn[t][r] = eLast * Ss[(16 * mt + 4 * g + r) * NS + c16];
#pragma unroll
            for (int s = 0; s < CH / 4; ++s)
                sn[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(ks[(4 * s + g) * KS + 16 * mt + c16] * kdk[4 * s + g],
                                                             Vn[(4 * s + g) * NS + c16], sn[t], 0, 0, 0);
        }
        __syncthreads();   // every read of this chunk's LDS is done
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int mt = w + 4 * t;
#pragma unroll
            for (int r = 0; r < 4; ++r) Ss[(16 * mt + 4 * g + r) * NS + c16] = sn[t][r];
        }
        if (chunk + 1 < a.nChunks) commit();
    }
    __syncthreads();
    for (int idx = tid; idx < KD * NB; idx += 256) {
        const int i = idx / NB, j = idx % NB;
        state[size_t(i) * VD + col0 + j] = Ss[i * NS + j];
    }
}

} // namespace

bool launch_delta_rule(const DeltaRuleParams& p, hipStream_t stream) {
    Context& ctx = Context::instance();
    if (p.keyDim != 64 && p.keyDim != 128) return ctx.fail("delta rule: keyDim must be 64 or 128");
    if (p.valueDim == 0 || p.valueDim % NB) return ctx.fail("delta rule: valueDim must be a multiple of 16");
    if (p.keyHeads == 0 || p.valueHeads % p.keyHeads) return ctx.fail("delta rule: valueHeads must be a multiple of keyHeads");
    if (p.chunk != 0 && p.chunk != CH) return ctx.fail("delta rule: chunk must be 64");
    if (p.inType != 0 && p.inType != 1) return ctx.fail("delta rule: unknown input type");
    if (!p.q || !p.k || !p.v || !p.state || !p.out) return ctx.fail("delta rule: null tensor");
    if (p.aLog ? (!p.a || !p.b || !p.dtBias) : (!p.g || !p.beta)) return ctx.fail("delta rule: missing gates");
    if (p.count == 0) return true;

    DeltaArgs a{};
    a.p = p;
    a.nChunks = uint32_t((p.count + CH - 1) / CH);
    if (a.nChunks > 65535u * 1024u) return ctx.fail("delta rule: sequence too long");
    a.work = static_cast<float*>(ctx.grow(SLOT_DELTA_WORK, size_t(p.valueHeads) * a.nChunks * WORK * sizeof(float)));
    if (!a.work) return false;
    auto aligned = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    a.vec = aligned(p.q) && aligned(p.k) && aligned(p.v) ? 1u : 0u;

    const dim3 sgrid(a.nChunks, unsigned(p.valueHeads));
    const unsigned scanBlocks = unsigned(p.valueHeads * (p.valueDim / NB));
#define AIGPU_DELTA(KD, F)                                                                                    \
    if (p.keyDim == KD && (p.inType == 0) == F) {                                                             \
        if (!ctx.launch("delta_solve_kernel", stream, [&] {                                                   \
                hipLaunchKernelGGL((delta_solve_kernel<KD, F>), sgrid, dim3(256), 0, stream, a);             \
            }))                                                                                               \
            return false;                                                                                     \
        return ctx.launch("delta_scan_kernel", stream, [&] {                                                  \
            hipLaunchKernelGGL((delta_scan_kernel<KD, F>), dim3(scanBlocks), dim3(256), 0, stream, a);       \
        });                                                                                                   \
    }
    AIGPU_DELTA(128, false)
    AIGPU_DELTA(128, true)
    AIGPU_DELTA(64, false)
    AIGPU_DELTA(64, true)
#undef AIGPU_DELTA
    return ctx.fail("delta rule: unsupported configuration");
}

} // namespace aigpu
