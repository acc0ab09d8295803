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
//   delta_solve_kernel  parallel over (head, chunk): KK^T, QK^T, the decayed
//                       masks and T = (I + A)^-1 by forward substitution;
//                       writes T, QKm, gc, beta to a workspace
//   delta_scan_kernel   per (head, 16 value columns): walks the chunks in
//                       order carrying S (fp32, in LDS), U = T R, outputs
//                       and the state update on v_mfma_f32_16x16x4f32
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
constexpr int WORK = 2 * CH * CH + 2 * CH;   // floats per (head, chunk) record

struct DeltaArgs {
    DeltaRuleParams p;
    float* work;       // [valueHeads][nChunks][WORK]
    uint32_t nChunks;
};

__device__ __forceinline__ float softplus_of(float x) { return x > 20.0f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float sigmoid_of(float x) { return 1.0f / (1.0f + expf(-x)); }

/* rows t0 .. t0+CH-1 of q and k for key head kh into LDS (row stride KD+1),
   l2normalised and q-scaled as gatedDeltaNetMixer does (LocalModel.hpp:
   2814-2818, l2normalise at :1380-1386); rows past `count` are zero */
template <int KD>
__device__ void load_qk_rows(const DeltaRuleParams& p, uint64_t t0, uint32_t n, uint32_t kh,
                             float* ks, float* qs) {
    constexpr int KS = KD + 1;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const float qScale = 1.0f / sqrtf(float(KD));
    for (int r = w; r < CH; r += 4) {
        float kv[KD / 64 > 0 ? KD / 64 : 1], qv[KD / 64 > 0 ? KD / 64 : 1];
        float kss = 0.0f, qss = 0.0f;
#pragma unroll
        for (int i = 0; i < KD / 64; ++i) {
            const int d = lane + 64 * i;
            float kx = 0.0f, qx = 0.0f;
            if (uint32_t(r) < n) {
                const size_t src = ((t0 + r) * p.keyHeads + kh) * KD + d;
                kx = load_elem(p.k, src, p.inType);
                qx = load_elem(p.q, src, p.inType);
            }
            kv[i] = kx;
            qv[i] = qx;
            kss += kx * kx;
            qss += qx * qx;
        }
        if (p.normalize) {
            kss = wave_sum(kss);
            qss = wave_sum(qss);
            const float kinv = 1.0f / sqrtf(kss + 1e-6f), qinv = 1.0f / sqrtf(qss + 1e-6f);
#pragma unroll
            for (int i = 0; i < KD / 64; ++i) {
                kv[i] *= kinv;
                qv[i] = (qv[i] * qinv) * qScale;
            }
        }
#pragma unroll
        for (int i = 0; i < KD / 64; ++i) {
            ks[r * KS + lane + 64 * i] = kv[i];
            qs[r * KS + lane + 64 * i] = qv[i];
        }
    }
}

template <int KD>
__global__ __launch_bounds__(256) void delta_solve_kernel(DeltaArgs a) {
    constexpr int KS = KD + 1;
    __shared__ float ks[CH * KS];
    __shared__ float qs[CH * KS];
    __shared__ float Am[CH * CS];
    __shared__ float Tm[CH * CS];
    __shared__ float gcs[CH], bs[CH];

    const DeltaRuleParams& p = a.p;
    const uint32_t chunk = blockIdx.x, h = blockIdx.y;
    const uint32_t kh = uint32_t(h / (p.valueHeads / p.keyHeads));
    const uint64_t t0 = uint64_t(chunk) * CH;
    const uint32_t n = uint32_t(p.count - t0 < CH ? p.count - t0 : CH);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c16 = lane & 15;
    float* rec = a.work + (size_t(h) * a.nChunks + chunk) * WORK;

    load_qk_rows<KD>(p, t0, n, kh, ks, qs);
    if (w == 0) {
        float gt = 0.0f, bt = 0.0f;
        if (uint32_t(lane) < n) {
            const size_t i = (t0 + lane) * p.valueHeads + h;
            if (p.aLog) {   // LocalModel.hpp:2820-2823
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
        gcs[lane] = gt;
        bs[lane] = bt;
    }
    __syncthreads();

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
            const float dec = j <= i ? expf(gcs[i] - gcs[j]) : 0.0f;
            Am[i * CS + j] = j < i ? bs[i] * dec * kk[r] : 0.0f;
            qkm[i * CH + j] = dec * qk[r];
        }
    }
    __syncthreads();

    if (w == 0) {   // T = (I + A)^-1, lane = column
        for (int i = 0; i < CH; ++i) {
            float acc = 0.0f;
            for (int mm = 0; mm < i; ++mm) acc = fmaf(Am[i * CS + mm], Tm[mm * CS + lane], acc);
            Tm[i * CS + lane] = lane < i ? -acc : (lane == i ? 1.0f : 0.0f);
            wave_sync();
        }
    }
    __syncthreads();

    for (int idx = tid; idx < CH * CH; idx += 256) rec[idx] = Tm[(idx / CH) * CS + idx % CH];
    if (tid < CH) {
        rec[2 * CH * CH + tid] = gcs[tid];
        rec[2 * CH * CH + CH + tid] = bs[tid];
    }
}

template <int KD>
__global__ __launch_bounds__(256) void delta_scan_kernel(DeltaArgs a) {
    constexpr int KS = KD + 1;
    __shared__ float ks[CH * KS];
    __shared__ float qs[CH * KS];
    __shared__ float Tm[CH * CS];
    __shared__ float Qm[CH * CS];
    __shared__ float Ss[KD * NS];
    __shared__ float Rs[CH * NS], Vn[CH * NS], vs[CH * NS];
    __shared__ float gcs[CH], bs[CH], dk[CH];

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

    float* state = p.state + size_t(h) * KD * VD;
    for (int idx = tid; idx < KD * NB; idx += 256) {
        const int i = idx / NB, j = idx % NB;
        Ss[i * NS + j] = state[size_t(i) * VD + col0 + j];
    }

    for (uint32_t chunk = 0; chunk < a.nChunks; ++chunk) {
        const uint64_t t0 = uint64_t(chunk) * CH;
        const uint32_t n = uint32_t(p.count - t0 < CH ? p.count - t0 : CH);
        const float* rec = a.work + (size_t(h) * a.nChunks + chunk) * WORK;
        __syncthreads();
        load_qk_rows<KD>(p, t0, n, kh, ks, qs);
        for (int idx = tid; idx < CH * NB; idx += 256) {
            const int r = idx / NB, j = idx % NB;
            vs[r * NS + j] = uint32_t(r) < n ? load_elem(p.v, ((t0 + r) * Hv + h) * VD + col0 + j, p.inType) : 0.0f;
        }
        for (int idx = tid; idx < CH * CH; idx += 256) {
            const int i = idx / CH, j = idx % CH;
            Tm[i * CS + j] = rec[idx];
            Qm[i * CS + j] = rec[CH * CH + idx];
        }
        if (tid < CH) {
            gcs[tid] = rec[2 * CH * CH + tid];
            bs[tid] = rec[2 * CH * CH + CH + tid];
        }
        __syncthreads();
        const float gLast = gcs[CH - 1];
        if (tid < CH) dk[tid] = expf(gLast - gcs[tid]);

        // R = beta (V - gamma K S)
        floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
        for (int s = 0; s < KD / 4; ++s)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ks[(16 * w + c16) * KS + 4 * s + g],
                                                       Ss[(4 * s + g) * NS + c16], acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 16 * w + 4 * g + r;
            Rs[i * NS + c16] = bs[i] * (vs[i * NS + c16] - expf(gcs[i]) * acc[r]);
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

        // O = gamma Q S + QKm U
        acc = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
        for (int s = 0; s < KD / 4; ++s)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qs[(16 * w + c16) * KS + 4 * s + g],
                                                       Ss[(4 * s + g) * NS + c16], acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] *= expf(gcs[16 * w + 4 * g + r]);
#pragma unroll
        for (int s = 0; s < CH / 4; ++s)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(Qm[(16 * w + c16) * CS + 4 * s + g],
                                                       Vn[(4 * s + g) * NS + c16], acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t i = 16 * w + 4 * g + r;
            if (i < n) p.out[((t0 + i) * Hv + h) * VD + col0 + c16] = acc[r];
        }

        // S' = gamma_last S + (decayed K)^T U
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
                sn[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(ks[(4 * s + g) * KS + 16 * mt + c16] * dk[4 * s + g],
                                                             Vn[(4 * s + g) * NS + c16], sn[t], 0, 0, 0);
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int mt = w + 4 * t;
#pragma unroll
            for (int r = 0; r < 4; ++r) Ss[(16 * mt + 4 * g + r) * NS + c16] = sn[t][r];
        }
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

    const dim3 sgrid(a.nChunks, unsigned(p.valueHeads));
    const unsigned scanBlocks = unsigned(p.valueHeads * (p.valueDim / NB));
    if (p.keyDim == 128) {
        if (!ctx.launch("delta_solve_kernel", stream, [&] {
                hipLaunchKernelGGL(delta_solve_kernel<128>, sgrid, dim3(256), 0, stream, a);
            }))
            return false;
        return ctx.launch("delta_scan_kernel", stream, [&] {
            hipLaunchKernelGGL(delta_scan_kernel<128>, dim3(scanBlocks), dim3(256), 0, stream, a);
        });
    }
    if (!ctx.launch("delta_solve_kernel", stream, [&] {
            hipLaunchKernelGGL(delta_solve_kernel<64>, sgrid, dim3(256), 0, stream, a);
        }))
        return false;
    return ctx.launch("delta_scan_kernel", stream, [&] {
        hipLaunchKernelGGL(delta_scan_kernel<64>, dim3(scanBlocks), dim3(256), 0, stream, a);
    });
}

} // namespace aigpu
