// kda.hip - Kimi Delta Attention's recurrence (kimiDeltaMixer,
// LocalModel.hpp:2928-2947; deltaStep with perKeyDecay, Kernels.hpp:105-128)
// as a chunked scan for gfx950: the gated delta rule with one decay per KEY
// CHANNEL instead of one per head.
//
// Per value head, token t, with a_t[i] = exp(g_t[i]) the decay of state row i:
//   S_t = diag(a_t) S_{t-1} + k_t u_t^T,  u_t = beta_t (v_t - (diag(a_t) S_{t-1})^T k_t),
//   o_t = S_t^T q_t
// Over a chunk of C = 64 tokens, with gc_t[i] the in-chunk cumulative log
// decay of channel i and Gamma_t = diag(exp(gc_t)):
//   (I + A) U = diag(beta) (V - Kg S0),   Kg_t = k_t * exp(gc_t),
//       A[t][j] = beta_t sum_i k_t[i] k_j[i] exp(gc_t[i] - gc_j[i])   (j < t)
//   O  = Qg S0 + QKm U,   Qg_t = q_t * exp(gc_t),
//       QKm[t][j] = sum_i q_t[i] k_j[i] exp(gc_t[i] - gc_j[i])        (j <= t)
//   S' = diag(exp(gc_last)) S0 + Kt^T U,   Kt_j = k_j * exp(gc_last - gc_j)
// Every exponent is <= 0. The decayed products A and QKm cannot be one
// matrix product (the decay depends on the channel of both rows); between
// 16-token blocks I > J they become one against the first row r of block I,
//   exp(gc_t - gc_j) = exp(gc_t - gc_r) exp(gc_r - gc_j),
// both factors <= 1, and inside a diagonal block they are summed directly.
//
// Two launches:
//   kda_solve_kernel  per (value head, chunk): norms, cumulative decays, A,
//                     QKm, T = (I + A)^-1, and the scaled rows Kg, Qg, Kt
//   kda_scan_kernel   per (value head, 16 value columns): the chunks in order
//                     on v_mfma_f32_16x16x4f32 (fp32 operands, so fp32 inputs
//                     keep fp32 accuracy)
#include "context.hpp"
#include "device.hpp"
#include "kernels.hpp"

namespace aigpu {

namespace {

constexpr int CH = 64;        // chunk length
constexpr int CS = CH + 1;    // LDS row stride of CH x CH matrices
constexpr int NB = 16;        // value columns per scan workgroup
constexpr int NS = NB + 1;

/* floats per (value head, chunk) record: T, QKm, Kg, Qg, Kt, beta, exp(gc_last) */
__host__ __device__ constexpr int kda_record(int KD) { return 2 * CH * CH + 3 * CH * KD + CH + KD; }

struct KdaArgs {
    KdaParams p;
    float* work;
    uint32_t nChunks;
};

template <bool F32>
__device__ __forceinline__ float in_elem(const void* base, size_t i) {
    if constexpr (F32) return static_cast<const float*>(base)[i];
    return bf16_bits_to_float(static_cast<const uint16_t*>(base)[i]);
}

/*
    Per (value head, chunk). Thread roles:
      - norms: 4 threads per row (LocalModel.hpp:1380-1386, q also scaled by
        1/sqrt(KD) as :2935);
      - cumulative decays: one thread per channel down the chunk;
      - decayed products: wave w takes block row I = w of A and QKm; its
        diagonal block by direct sums, the blocks left of it on MFMA against
        block I's first row;
      - T = (I + A)^-1 as in the scalar-decay solve.
*/
template <int KD, bool F32>
__global__ __launch_bounds__(256) void kda_solve_kernel(KdaArgs a) {
    constexpr int KS = KD + 1;
    __shared__ float kn[CH * KS];
    __shared__ float qn[CH * KS];
    __shared__ float gc[CH * KS];
    __shared__ float Am[CH * CS];
    __shared__ float Qm[CH * CS];
    __shared__ float Tm[CH * CS];
    __shared__ float Xs[4][16 * 17];
    __shared__ float bet[CH];

    const KdaParams& p = a.p;
    const uint32_t chunk = blockIdx.x, h = blockIdx.y;
    const uint32_t kh = uint32_t(h / (p.valueHeads / p.keyHeads));
    const uint64_t t0 = uint64_t(chunk) * CH;
    const uint32_t n = uint32_t(p.count - t0 < CH ? p.count - t0 : CH);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c16 = lane & 15;

    // ---- normalised rows; rows past the sequence's end are zero (beta 0) ----
    {
        const int r = tid >> 2, qq = tid & 3;
        constexpr int PE = KD / 4;
        const bool live = uint32_t(r) < n;
        const size_t src = ((t0 + (live ? r : 0)) * p.keyHeads + kh) * KD + qq * PE;
        float kss = 0.0f, qss = 0.0f;
        for (int e = 0; e < PE; ++e) {
            const float kx = live ? in_elem<F32>(p.k, src + e) : 0.0f;
            const float qx = live ? in_elem<F32>(p.q, src + e) : 0.0f;
            kn[r * KS + qq * PE + e] = kx;
            qn[r * KS + qq * PE + e] = qx;
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
        for (int e = 0; e < PE; ++e) {
            kn[r * KS + qq * PE + e] *= kinv;
            qn[r * KS + qq * PE + e] *= qinv;
        }
        if (tid < CH) {
            float bt = 0.0f;
            if (uint32_t(tid) < n) {
                const size_t i = (t0 + tid) * p.valueHeads + h;
                bt = p.beta ? p.beta[i] : sigmoid_of(p.b[i]);
            }
            bet[tid] = bt;
        }
    }
    // ---- cumulative log decay of each channel over the chunk; raw gates
    //      become log decays as LocalModel.hpp:2894-2905 computes them ----
    if (tid < KD) {
        const bool raw = p.g == nullptr;
        const float rate = raw ? expf(p.aLog[h]) : 0.0f;
        const float bias = raw ? p.dtBias[size_t(h) * KD + tid] : 0.0f;
        float acc = 0.0f;
        for (int r = 0; r < CH; ++r) {
            if (uint32_t(r) < n) {
                const size_t i = ((t0 + r) * p.valueHeads + h) * KD + tid;
                float gt;
                if (!raw) {
                    gt = p.g[i];
                } else {
                    const float f = p.f[i] + bias;
                    gt = p.safeGate ? p.lowerBound * sigmoid_of(rate * f) : -rate * softplus_of(f);
                }
                acc += gt;
            }
            gc[r * KS + tid] = acc;
        }
    }
    // T is zero above its diagonal blocks
    for (int idx = tid; idx < CH * CH; idx += 256) {
        const int i = idx / CH, j = idx % CH;
        if ((j >> 4) > (i >> 4)) Tm[i * CS + j] = 0.0f;
    }
    __syncthreads();

    // ---- block row I = w of A and QKm ----
    {
        const int I = w, r0 = 16 * I;
        // diagonal block: lane (c16, g) holds rows 4g + rr, column c16
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int t = r0 + 4 * g + rr, j = r0 + c16;
            float sa = 0.0f, sq = 0.0f;
            for (int i = 0; i < KD; ++i) {
                const float e = expf(fminf(gc[t * KS + i] - gc[j * KS + i], 0.0f));
                const float kj = kn[j * KS + i] * e;
                sa = fmaf(kn[t * KS + i], kj, sa);
                sq = fmaf(qn[t * KS + i], kj, sq);
            }
            Am[t * CS + j] = j < t ? bet[t] * sa : 0.0f;
            Qm[t * CS + j] = j <= t ? sq : 0.0f;
        }
        // blocks J < I against row r0: left factors exp(gc_t - gc_r0) per
        // (row, channel), right factors exp(gc_r0 - gc_j)
        for (int J = 0; J < I; ++J) {
            floatx4 xa = {0.0f, 0.0f, 0.0f, 0.0f}, xq = {0.0f, 0.0f, 0.0f, 0.0f};
            const int t = r0 + c16, j = 16 * J + c16;
#pragma unroll 4
            for (int s = 0; s < KD / 4; ++s) {
                const int i = 4 * s + g;
                const float gr = gc[r0 * KS + i];
                const float lt = expf(gc[t * KS + i] - gr);
                const float rj = kn[j * KS + i] * expf(gr - gc[j * KS + i]);
                xa = __builtin_amdgcn_mfma_f32_16x16x4f32(kn[t * KS + i] * lt, rj, xa, 0, 0, 0);
                xq = __builtin_amdgcn_mfma_f32_16x16x4f32(qn[t * KS + i] * lt, rj, xq, 0, 0, 0);
            }
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int tt = r0 + 4 * g + rr;
                Am[tt * CS + j] = bet[tt] * xa[rr];
                Qm[tt * CS + j] = xq[rr];
            }
        }
        // the rest of the row is zero
        for (int idx = lane; idx < 16 * CH; idx += WAVE) {
            const int tt = r0 + idx / CH, j = idx % CH;
            if (j >= r0 + 16) {
                Am[tt * CS + j] = 0.0f;
                Qm[tt * CS + j] = 0.0f;
            }
        }
    }
    __syncthreads();

    // ---- T = (I + A)^-1: diagonal blocks by forward substitution in
    //      registers, then the block rows below on MFMA ----
    {
        const int b0 = 16 * w, j = lane & 15;
        float t[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float acc = i == j ? 1.0f : 0.0f;
#pragma unroll
            for (int m = 0; m < i; ++m) acc = fmaf(-Am[(b0 + i) * CS + b0 + m], t[m], acc);
            t[i] = acc;
        }
        if (lane < 16) {
#pragma unroll
            for (int i = 0; i < 16; ++i) Tm[(b0 + i) * CS + b0 + j] = t[i];
        }
    }
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

    // ---- the record ----
    float* rec = a.work + (size_t(h) * a.nChunks + chunk) * kda_record(KD);
    float* rT = rec;
    float* rQ = rec + CH * CH;
    float* rKg = rec + 2 * CH * CH;
    float* rQg = rKg + CH * KD;
    float* rKt = rQg + CH * KD;
    float* rB = rKt + CH * KD;
    float* rE = rB + CH;
    for (int idx = tid; idx < CH * CH; idx += 256) {
        rT[idx] = Tm[(idx / CH) * CS + idx % CH];
        rQ[idx] = Qm[(idx / CH) * CS + idx % CH];
    }
    for (int idx = tid; idx < CH * KD; idx += 256) {
        const int r = idx / KD, i = idx % KD;
        const float gi = gc[r * KS + i];
        const float eg = expf(gi);
        rKg[idx] = kn[r * KS + i] * eg;
        rQg[idx] = qn[r * KS + i] * eg;
        rKt[idx] = kn[r * KS + i] * expf(gc[(CH - 1) * KS + i] - gi);
    }
    if (tid < CH) rB[tid] = bet[tid];
    if (tid < KD) rE[tid] = expf(gc[(CH - 1) * KS + tid]);
}

/*
    Per (value head, 16 value columns), chunk by chunk:
      R  = diag(beta) (V - Kg S)      U = T R
      O  = Qg S + QKm U               S' = diag(exp(gc_last)) S + Kt^T U
    S lives in LDS (fp32). Each chunk's record is loaded whole before its
    products; the products are fp32 MFMAs.
*/
template <int KD, bool F32>
__global__ __launch_bounds__(256) void kda_scan_kernel(KdaArgs a) {
    constexpr int KS = KD + 1;
    __shared__ float Kg[CH * KS];
    __shared__ float Qg[CH * KS];
    __shared__ float Kt[CH * KS];
    __shared__ float Tm[CH * CS];
    __shared__ float Qm[CH * CS];
    __shared__ float Ss[KD * NS];
    __shared__ float Rs[CH * NS], Un[CH * NS], vs[CH * NS];
    __shared__ float bet[CH], eL[KD];

    const KdaParams& p = a.p;
    uint32_t bid = blockIdx.x;
    const uint32_t nb = gridDim.x, nCol = uint32_t(p.valueDim / NB);
    if (nb % 8 == 0) bid = (bid % 8) * (nb / 8) + bid / 8;   // a head's column blocks on one XCD
    const uint32_t h = bid / nCol, cb = bid % nCol;
    const uint32_t col0 = cb * NB;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c16 = lane & 15;
    const size_t VD = p.valueDim, Hv = p.valueHeads;

    float* state = p.state + size_t(h) * KD * VD;
    for (int idx = tid; idx < KD * NB; idx += 256) Ss[(idx / NB) * NS + idx % NB] = state[size_t(idx / NB) * VD + col0 + idx % NB];

    for (uint32_t chunk = 0; chunk < a.nChunks; ++chunk) {
        const uint64_t t0 = uint64_t(chunk) * CH;
        const uint32_t n = uint32_t(p.count - t0 < CH ? p.count - t0 : CH);
        const float* rec = a.work + (size_t(h) * a.nChunks + chunk) * kda_record(KD);
        __syncthreads();   // the previous chunk's reads are done
        for (int idx = tid; idx < CH * CH; idx += 256) {
            Tm[(idx / CH) * CS + idx % CH] = rec[idx];
            Qm[(idx / CH) * CS + idx % CH] = rec[CH * CH + idx];
        }
        for (int idx = tid; idx < CH * KD; idx += 256) {
            const int r = idx / KD, i = idx % KD;
            Kg[r * KS + i] = rec[2 * CH * CH + idx];
            Qg[r * KS + i] = rec[2 * CH * CH + CH * KD + idx];
            Kt[r * KS + i] = rec[2 * CH * CH + 2 * CH * KD + idx];
        }
        if (tid < CH) bet[tid] = rec[2 * CH * CH + 3 * CH * KD + tid];
        if (tid < KD) eL[tid] = rec[2 * CH * CH + 3 * CH * KD + CH + tid];
        for (int idx = tid; idx < CH * NB; idx += 256) {
            const int r = idx / NB, c = idx % NB;
            vs[r * NS + c] = uint32_t(r) < n ? in_elem<F32>(p.v, ((t0 + r) * Hv + h) * VD + col0 + c) : 0.0f;
        }
        __syncthreads();

        // R = beta (V - Kg S)
        floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
        for (int s = 0; s < KD / 4; ++s)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(Kg[(16 * w + c16) * KS + 4 * s + g], Ss[(4 * s + g) * NS + c16],
                                                       acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 16 * w + 4 * g + r;
            Rs[i * NS + c16] = bet[i] * (vs[i * NS + c16] - acc[r]);
        }
        __syncthreads();

        // U = T R
        acc = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < CH / 4; ++s)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(Tm[(16 * w + c16) * CS + 4 * s + g], Rs[(4 * s + g) * NS + c16],
                                                       acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) Un[(16 * w + 4 * g + r) * NS + c16] = acc[r];
        __syncthreads();

        // O = Qg S + QKm U
        acc = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
        for (int s = 0; s < KD / 4; ++s)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(Qg[(16 * w + c16) * KS + 4 * s + g], Ss[(4 * s + g) * NS + c16],
                                                       acc, 0, 0, 0);
#pragma unroll
        for (int s = 0; s < CH / 4; ++s)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(Qm[(16 * w + c16) * CS + 4 * s + g], Un[(4 * s + g) * NS + c16],
                                                       acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t i = 16 * w + 4 * g + r;
            if (i < n) p.out[((t0 + i) * Hv + h) * VD + col0 + c16] = acc[r];
        }

        // S' = diag(exp(gc_last)) S + Kt^T U: wave w's key tiles mt = w + 4t
        constexpr int MT = KD / 64;
        floatx4 sn[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int mt = w + 4 * t;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 16 * mt + 4 * g + r;
                sn[t][r] = eL[i] * Ss[i * NS + c16];
            }
#pragma unroll
            for (int s = 0; s < CH / 4; ++s)
                sn[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(Kt[(4 * s + g) * KS + 16 * mt + c16], Un[(4 * s + g) * NS + c16],
                                                             sn[t], 0, 0, 0);
        }
        __syncthreads();   // every read of S is done
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int mt = w + 4 * t;
#pragma unroll
            for (int r = 0; r < 4; ++r) Ss[(16 * mt + 4 * g + r) * NS + c16] = sn[t][r];
        }
    }
    __syncthreads();
    for (int idx = tid; idx < KD * NB; idx += 256) state[size_t(idx / NB) * VD + col0 + idx % NB] = Ss[(idx / NB) * NS + idx % NB];
}

} // namespace

bool launch_kda(const KdaParams& p, hipStream_t stream) {
    Context& ctx = Context::instance();
    if (p.keyDim != 64 && p.keyDim != 128) return ctx.fail("kda: keyDim must be 64 or 128");
    if (p.valueDim == 0 || p.valueDim % NB) return ctx.fail("kda: valueDim must be a multiple of 16");
    if (p.keyHeads == 0 || p.valueHeads % p.keyHeads) return ctx.fail("kda: valueHeads must be a multiple of keyHeads");
    if (p.inType != 0 && p.inType != 1) return ctx.fail("kda: unknown input type");
    if (!p.q || !p.k || !p.v || !p.state || !p.out) return ctx.fail("kda: null tensor");
    if (!p.g != !p.beta) return ctx.fail("kda: give g and beta together, or neither (raw gates)");
    if (!p.g && (!p.f || !p.b || !p.aLog || !p.dtBias))
        return ctx.fail("kda: raw gates need f, b, aLog and dtBias");
    if (!p.g && p.safeGate && !(p.lowerBound <= 0.0f)) return ctx.fail("kda: lowerBound must be <= 0");
    if (p.count == 0) return true;
    KdaArgs a{};
    a.p = p;
    a.nChunks = uint32_t((p.count + CH - 1) / CH);
    if (a.nChunks > 65535u * 1024u) return ctx.fail("kda: sequence too long");
    const size_t rec = size_t(kda_record(int(p.keyDim)));
    a.work = static_cast<float*>(ctx.grow(SLOT_DELTA_WORK, size_t(p.valueHeads) * a.nChunks * rec * sizeof(float)));
    if (!a.work) return false;
    const dim3 sgrid(a.nChunks, unsigned(p.valueHeads));
    const dim3 grid{unsigned(p.valueHeads * (p.valueDim / NB))}, block{256};
#define AIGPU_KDA(KD, F)                                                                                       \
    if (p.keyDim == KD && (p.inType == 0) == F) {                                                              \
        if (!ctx.launch("kda_solve_kernel", stream, [&] {                                                      \
                hipLaunchKernelGGL((kda_solve_kernel<KD, F>), sgrid, dim3(256), 0, stream, a);                 \
            }))                                                                                                \
            return false;                                                                                      \
        return ctx.launch("kda_scan_kernel", stream, [&] {                                                     \
            hipLaunchKernelGGL((kda_scan_kernel<KD, F>), grid, block, 0, stream, a);                           \
        });                                                                                                    \
    }
    AIGPU_KDA(128, true)
    AIGPU_KDA(128, false)
    AIGPU_KDA(64, true)
    AIGPU_KDA(64, false)
#undef AIGPU_KDA
    return ctx.fail("kda: unsupported configuration");
}

} // namespace aigpu
