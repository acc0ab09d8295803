// kda.hip - Kimi Delta Attention's recurrence (kimiDeltaMixer,
// LocalModel.hpp:2928-2947; deltaStep with perKeyDecay, Kernels.hpp:105-128)
// as a chunked scan for gfx950: the gated delta rule with one decay per KEY
// CHANNEL instead of one per head.
//
// Per value head, token t, with a_t[i] = exp(g_t[i]) <= 1 the decay of state
// row i:
//   S_t = diag(a_t) S_{t-1} + k_t u_t^T,  u_t = beta_t (v_t - (diag(a_t) S_{t-1})^T k_t),
//   o_t = S_t^T q_t
// Over a chunk of C = 64 tokens, with gc_t[i] the in-chunk cumulative log
// decay of channel i:
//   (I + A) U = diag(beta) (V - Kg S0),   Kg_t = k_t * exp(gc_t),
//       A[t][j] = beta_t sum_i k_t[i] k_j[i] exp(gc_t[i] - gc_j[i])   (j < t)
//   O  = Qg S0 + QKm U,   Qg_t = q_t * exp(gc_t),
//       QKm[t][j] = sum_i q_t[i] k_j[i] exp(gc_t[i] - gc_j[i])        (j <= t)
//   S' = diag(exp(gc_last)) S0 + Kt^T U,   Kt_j = k_j * exp(gc_last - gc_j)
// With Tb = (I + A)^-1 diag(beta) and P = QKm Tb, everything that does not
// depend on S0 is folded in per chunk, independently of the other chunks:
//   W = Tb Kg,  Qt = Qg - P Kg,  Ut = Tb V,  Ot = P V
//   U = Ut - W S0,   O = Ot + Qt S0,   S' = diag(exp(gc_last)) S0 + Kt^T U
// so the sequential part is two products per chunk.
//
// The decayed products A and QKm are not one matrix product (the decay
// depends on the channel of both rows). Between 16-token blocks I > J they
// become one against the first row r of block I,
//   exp(gc_t - gc_j) = exp(gc_t - gc_r) exp(gc_r - gc_j),  both factors <= 1;
// inside a diagonal block against its middle row m, where one factor can
// exceed 1, as long as the block's decay span keeps both within 2^100
// (always for Kimi's bounded gate, lowerBound >= -5 per token); a block whose
// span is larger is summed directly. Logs are kept in base 2 so that every
// factor is one v_exp_f32.
//
// Two launches:
//   kda_solve_kernel  per (value head, chunk): norms, gates, cumulative
//                     decays, A, QKm, Tb, P, then W, Qt, Kt, Ut, Ot
//   kda_scan_kernel   per (value head, 16 value columns): the chunks in order,
//                     the next chunk's operands loaded into registers while
//                     the current one computes
// Every product is v_mfma_f32_16x16x4f32 (fp32 operands), so fp32 inputs keep
// fp32 accuracy.
#include "context.hpp"
#include "device.hpp"
#include "kernels.hpp"

namespace aigpu {

namespace {

constexpr int CH = 64;       // chunk length
constexpr int CS = CH + 4;   // LDS row stride of CH x CH matrices
constexpr int NB = 16;       // value columns per scan workgroup
constexpr float SPAN_MAX = 100.0f;   // log2 span of a diagonal block factorised through its middle row

/* the per-(value head, chunk) record, in floats, laid out as the scan's
   MFMA operands so that each of its lanes loads 16 bytes per 4 products:
     WF  [CH/16 row block][KD/16 k group][64 lanes][4]   -W = -Tb Kg (negated:
         the scan accumulates onto Ut); lane (c16, g) of row block rb, group q
         holds row 16 rb + c16, k = 16 q + 4 g .. +3
     QF  the same for Qt = Qg - P Kg
     KF  [KD/16 key tile][CH/16 token group][64][4]   Kt^T: lane (c16, g) of
         tile mt, group q holds key 16 mt + c16, tokens 16 q + 4 g .. +3
     eL  [KD]   exp(gc_last)
     UO  [VD/16 column block][2: Ut, Ot][CH/16 row block][64][4]   the MFMA
         accumulator layout: lane (c16, g) holds rows 4 g .. +3, column c16 */
__host__ __device__ constexpr size_t kda_record(int KD, size_t VD) { return 3 * size_t(CH) * KD + KD + 2 * CH * VD; }

struct KdaArgs {
    KdaParams p;
    float* work;
    uint32_t nChunks;
};

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

/* N consecutive input elements (fp32 or bf16) at element index i, as fp32; i
   a multiple of 8 (bf16) or 4 (fp32) and the base 16-byte aligned */
template <bool F32, int N>
__device__ __forceinline__ void load_row(const void* base, size_t i, float (&x)[N]) {
    if constexpr (F32) {
#pragma unroll
        for (int e = 0; e < N / 4; ++e) {
            const floatx4 v = *reinterpret_cast<const floatx4*>(static_cast<const float*>(base) + i + 4 * e);
#pragma unroll
            for (int c = 0; c < 4; ++c) x[4 * e + c] = v[c];
        }
    } else {
#pragma unroll
        for (int e = 0; e < N / 8; ++e) {
            const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + i + 8 * e);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                x[8 * e + 2 * c] = __uint_as_float(w[c] << 16);
                x[8 * e + 2 * c + 1] = __uint_as_float(w[c] & 0xFFFF0000u);
            }
        }
    }
}

/* block (I, J), J <= I, of the ten lower 16 x 16 blocks of a 64 x 64 matrix */
__device__ __forceinline__ void lower_block(int b, int& I, int& J) {
    I = b >= 6 ? 3 : (b >= 3 ? 2 : (b >= 1 ? 1 : 0));
    J = b - I * (I + 1) / 2;
}

/*
    Per (value head, chunk), 256 threads. LDS (KD 128): kn, qn, gc
    [64][KD+4] and Am, Qm, Tm [64][68], about 155 KB.
*/
template <int KD, bool F32>
__global__ __launch_bounds__(256) void kda_solve_kernel(KdaArgs a) {
    constexpr int KS = KD + 4;
    constexpr int PE = KD / 4;   // row elements per thread in the row passes
    constexpr int VPRE = CH * KD / 8 / 256;   // 8-element value pieces per thread per slab
    __shared__ __align__(16) float kn[CH * KS];
    __shared__ __align__(16) float qn[CH * KS];
    __shared__ __align__(16) float gc[CH * KS];   // log2 decays; later the value slabs
    __shared__ __align__(16) float Am[CH * CS];   // A; later P
    __shared__ __align__(16) float Qm[CH * CS];
    __shared__ __align__(16) float Tm[CH * CS];
    __shared__ float Xs[4][16 * 17];
    __shared__ float bet[CH];

    const KdaParams& p = a.p;
    const uint32_t chunk = blockIdx.x, h = blockIdx.y;
    const uint32_t kh = uint32_t(h / (p.valueHeads / p.keyHeads));
    const uint64_t t0 = uint64_t(chunk) * CH;
    const uint32_t n = uint32_t(p.count - t0 < CH ? p.count - t0 : CH);
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c16 = lane & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const size_t VD = p.valueDim, Hv = p.valueHeads;

    // ---- q, k rows normalised (LocalModel.hpp:1380-1386, q also scaled by
    //      1/sqrt(KD) as :2935); log2 decays; beta. Rows past the end are zero.
    {
        const int r = tid >> 2, qq = tid & 3;
        const bool live = uint32_t(r) < n;
        const uint64_t tr = t0 + (live ? r : 0);
        float kx[PE], qx[PE];
        load_row<F32, PE>(p.k, (tr * p.keyHeads + kh) * KD + qq * PE, kx);
        load_row<F32, PE>(p.q, (tr * p.keyHeads + kh) * KD + qq * PE, qx);
        float kss = 0.0f, qss = 0.0f;
#pragma unroll
        for (int e = 0; e < PE; ++e) {
            kss = fmaf(kx[e], kx[e], kss);
            qss = fmaf(qx[e], qx[e], qss);
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
        if (!live) kinv = qinv = 0.0f;
#pragma unroll
        for (int e = 0; e < PE; e += 4) {
            *reinterpret_cast<floatx4*>(&kn[r * KS + qq * PE + e]) =
                floatx4{kx[e] * kinv, kx[e + 1] * kinv, kx[e + 2] * kinv, kx[e + 3] * kinv};
            *reinterpret_cast<floatx4*>(&qn[r * KS + qq * PE + e]) =
                floatx4{qx[e] * qinv, qx[e + 1] * qinv, qx[e + 2] * qinv, qx[e + 3] * qinv};
        }

        // gates as LocalModel.hpp:2894-2905 computes them, or given
        const bool raw = p.g == nullptr;
        float gx[PE];
        load_row<true, PE>(raw ? p.f : p.g, (tr * Hv + h) * KD + qq * PE, gx);
        const float rate = raw ? expf(p.aLog[h]) : 0.0f;
#pragma unroll
        for (int e = 0; e < PE; e += 4) {
            floatx4 o;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                float gt = gx[e + c];
                if (raw) {
                    const float x = gt + p.dtBias[size_t(h) * KD + qq * PE + e + c];
                    gt = p.safeGate ? p.lowerBound * sigmoid_of(rate * x) : -rate * softplus_of(x);
                }
                o[c] = live ? gt * LOG2E : 0.0f;
            }
            *reinterpret_cast<floatx4*>(&gc[r * KS + qq * PE + e]) = o;
        }
        if (tid < CH) {
            float bt = 0.0f;
            if (uint32_t(tid) < n) {
                const size_t i = (t0 + tid) * Hv + h;
                bt = p.beta ? p.beta[i] : sigmoid_of(p.b[i]);
            }
            bet[tid] = bt;
        }
    }
    // the first value slab is requested now and written to LDS when gc is free
    const int sw0 = int(VD < size_t(KD) ? VD : KD);
    float vpre[VPRE][8];
    auto vload = [&](size_t c0, int sw, int it, float (&x)[8]) {
        const int idx = tid + 256 * it;
        const int t = idx / (sw / 8), c = 8 * (idx % (sw / 8));
        if (idx < CH * (sw / 8) && uint32_t(t) < n) {
            load_row<F32, 8>(p.v, ((t0 + t) * Hv + h) * VD + c0 + c, x);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = 0.0f;
        }
    };
    auto vstore = [&](int sw, int it, const float (&x)[8]) {
        const int idx = tid + 256 * it;
        if (idx < CH * (sw / 8)) {
            const int t = idx / (sw / 8), c = 8 * (idx % (sw / 8));
            *reinterpret_cast<floatx4*>(&gc[t * KS + c]) = floatx4{x[0], x[1], x[2], x[3]};
            *reinterpret_cast<floatx4*>(&gc[t * KS + c + 4]) = floatx4{x[4], x[5], x[6], x[7]};
        }
    };
#pragma unroll
    for (int it = 0; it < VPRE; ++it) vload(0, sw0, it, vpre[it]);
    __syncthreads();

    // ---- cumulative log2 decay of each channel down the chunk: the rows in
    //      256 / KD parts, each summed by its own thread, then offset ----
    {
        constexpr int PARTS = 256 / KD, RPP = CH / PARTS;
        const int ch = tid % KD, part = tid / KD;
        float col[RPP];
#pragma unroll
        for (int r = 0; r < RPP; ++r) col[r] = gc[(part * RPP + r) * KS + ch];
#pragma unroll
        for (int r = 1; r < RPP; ++r) col[r] += col[r - 1];
        gc[(part * RPP + RPP - 1) * KS + ch] = col[RPP - 1];
        __syncthreads();
        float off = 0.0f;
        for (int q2 = 0; q2 < part; ++q2) off += gc[((q2 + 1) * RPP - 1) * KS + ch];
        __syncthreads();
#pragma unroll
        for (int r = 0; r < RPP; ++r) gc[(part * RPP + r) * KS + ch] = col[r] + off;
    }
    __syncthreads();

    // ---- the ten lower blocks of A and QKm: wave w takes blocks w, w+4, w+8 ----
    for (int b = w; b < 10; b += 4) {
        int I, J;
        lower_block(b, I, J);
        const int r0 = 16 * I, j0 = 16 * J;
        int ref = r0;
        bool direct = false;
        if (I == J) {   // factorise through the middle row if the span allows it
            ref = r0 + 8;
            float span = 0.0f;
            for (int ch = lane; ch < KD; ch += WAVE) {
                const float gm = gc[ref * KS + ch];
                span = fmaxf(span, fmaxf(gc[r0 * KS + ch] - gm, gm - gc[(r0 + 15) * KS + ch]));
            }
            direct = !(wave_max(span) <= SPAN_MAX);
        }
        if (!direct) {
            // within each group of 16 channels lane (c16, g) supplies channel
            // 16q + 4g + s on the s-th of four MFMAs: 16-byte reads
            floatx4 xa = {0.0f, 0.0f, 0.0f, 0.0f}, xq = {0.0f, 0.0f, 0.0f, 0.0f};
            const int t = r0 + c16, j = j0 + c16;
            auto ld4 = [](const float* ptr) { return *reinterpret_cast<const floatx4*>(ptr); };
#pragma unroll 2
            for (int q = 0; q < KD / 16; ++q) {
                const int i = 16 * q + 4 * g;
                const floatx4 gr = ld4(&gc[ref * KS + i]);
                const floatx4 gt = ld4(&gc[t * KS + i]), kt = ld4(&kn[t * KS + i]), qt = ld4(&qn[t * KS + i]);
                const floatx4 gj = ld4(&gc[j * KS + i]), kj = ld4(&kn[j * KS + i]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float lt = exp2_fast(gt[e] - gr[e]);
                    const float rj = kj[e] * exp2_fast(gr[e] - gj[e]);
                    xa = mfma4(kt[e] * lt, rj, xa);
                    xq = mfma4(qt[e] * lt, rj, xq);
                }
            }
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int tt = r0 + 4 * g + rr;
                Am[tt * CS + j] = (I != J || j < tt) ? bet[tt] * xa[rr] : 0.0f;
                Qm[tt * CS + j] = (I != J || j <= tt) ? xq[rr] : 0.0f;
            }
        } else {   // a diagonal block whose span is too wide to factorise
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int t = r0 + 4 * g + rr, j = r0 + c16;
                float sa = 0.0f, sq = 0.0f;
                for (int i = 0; i < KD; ++i) {
                    const float e = exp2_fast(fminf(gc[t * KS + i] - gc[j * KS + i], 0.0f));
                    const float kj = kn[j * KS + i] * e;
                    sa = fmaf(kn[t * KS + i], kj, sa);
                    sq = fmaf(qn[t * KS + i], kj, sq);
                }
                Am[t * CS + j] = j < t ? bet[t] * sa : 0.0f;
                Qm[t * CS + j] = j <= t ? sq : 0.0f;
            }
        }
    }
    __syncthreads();

    // ---- T = (I + A)^-1 (lower blocks only): diagonal blocks by forward
    //      substitution in registers, then the block rows below on MFMA ----
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
                    x = mfma4(Am[(16 * I + c16) * CS + 16 * M + 4 * s + g], Tm[(16 * M + 4 * s + g) * CS + 16 * J + c16], x);
#pragma unroll
            for (int r = 0; r < 4; ++r) Xs[w][(4 * g + r) * 17 + c16] = x[r];
            wave_sync();
            floatx4 y = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < 4; ++s)
                y = mfma4(Tm[(16 * I + c16) * CS + 16 * I + 4 * s + g], Xs[w][(4 * s + g) * 17 + c16], y);
#pragma unroll
            for (int r = 0; r < 4; ++r) Tm[(16 * I + 4 * g + r) * CS + 16 * J + c16] = -y[r];
        }
    }
    __syncthreads();

    // ---- Tb = T diag(beta), in place ----
    for (int idx = tid; idx < CH * CH; idx += 256) {
        const int t = idx / CH, j = idx % CH;
        if ((j >> 4) <= (t >> 4)) Tm[t * CS + j] *= bet[j];
    }
    __syncthreads();

    // ---- P = QKm Tb into Am: wave w takes block row I = w ----
    {
        const int I = w;
        for (int J = 0; J <= I; ++J) {
            floatx4 x = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int M = J; M <= I; ++M)
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    x = mfma4(Qm[(16 * I + c16) * CS + 16 * M + 4 * s + g], Tm[(16 * M + 4 * s + g) * CS + 16 * J + c16], x);
#pragma unroll
            for (int r = 0; r < 4; ++r) Am[(16 * I + 4 * g + r) * CS + 16 * J + c16] = x[r];
        }
    }

    // ---- the record: Kt and exp(gc_last) straight from kn, gc ----
    float* rec = a.work + (size_t(h) * a.nChunks + chunk) * kda_record(KD, VD);
    float* rW = rec;
    float* rQ = rec + CH * KD;
    float* rK = rec + 2 * CH * KD;
    float* rE = rec + 3 * CH * KD;
    float* rUO = rE + KD;
    for (int idx = tid; idx < CH * KD / 4; idx += 256) {
        const int ln = idx % 64, q = (idx / 64) % (CH / 16), mt = idx / 64 / (CH / 16);
        const int m = 16 * mt + (ln & 15), j0 = 16 * q + 4 * (ln >> 4);
        const float gl = gc[(CH - 1) * KS + m];
        floatx4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = kn[(j0 + e) * KS + m] * exp2_fast(gl - gc[(j0 + e) * KS + m]);
        reinterpret_cast<floatx4*>(rK)[idx] = o;
    }
    if (tid < KD) rE[tid] = exp2_fast(gc[(CH - 1) * KS + tid]);
    __syncthreads();
    // Kg, Qg in place
    for (int idx = tid; idx < CH * KD / 4; idx += 256) {
        const int t = idx / (KD / 4), i = 4 * (idx % (KD / 4));
        const floatx4 gv = *reinterpret_cast<const floatx4*>(&gc[t * KS + i]);
        floatx4 kv = *reinterpret_cast<floatx4*>(&kn[t * KS + i]);
        floatx4 qv = *reinterpret_cast<floatx4*>(&qn[t * KS + i]);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float e = exp2_fast(gv[c]);
            kv[c] *= e;
            qv[c] *= e;
        }
        *reinterpret_cast<floatx4*>(&kn[t * KS + i]) = kv;
        *reinterpret_cast<floatx4*>(&qn[t * KS + i]) = qv;
    }
    __syncthreads();

    // Block row I of Tb and of P has I + 1 nonzero blocks: waves 0, 1 take
    // rows 0 and 3, waves 2, 3 rows 1 and 2, each half of the column tiles.
    const int rowA = (w < 2) ? 0 : 1, rowB = 3 - rowA, par = w & 1;

    // ---- -W = -Tb Kg and Qt = Qg - P Kg, computed transposed (key rows,
    //      token columns) so each lane's accumulator is one scan fragment ----
    for (int pass = 0; pass < 2; ++pass) {
        const int I = pass ? rowB : rowA;
        for (int c = par; c < KD / 16; c += 2) {
            floatx4 xw = {0.0f, 0.0f, 0.0f, 0.0f};
            floatx4 xq = *reinterpret_cast<const floatx4*>(&qn[(16 * I + c16) * KS + 16 * c + 4 * g]);
            for (int M = 0; M <= I; ++M)
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const int k = 16 * M + 4 * s + g;
                    const float ak = kn[k * KS + 16 * c + c16];
                    xw = mfma4(ak, -Tm[(16 * I + c16) * CS + k], xw);
                    xq = mfma4(ak, -Am[(16 * I + c16) * CS + k], xq);
                }
            const int frag = (I * (KD / 16) + c) * 64 + lane;
            reinterpret_cast<floatx4*>(rW)[frag] = xw;
            reinterpret_cast<floatx4*>(rQ)[frag] = xq;
        }
    }
    __syncthreads();   // gc is free: it holds the value slabs from here

    // ---- Ut = Tb V and Ot = P V, KD value columns at a time ----
    for (size_t c0 = 0; c0 < VD; c0 += KD) {
        const int sw = int(VD - c0 < size_t(KD) ? VD - c0 : KD);
        if (c0 == 0) {
#pragma unroll
            for (int it = 0; it < VPRE; ++it) vstore(sw, it, vpre[it]);
        } else {
            for (int it = 0; it < VPRE; ++it) {
                float x[8];
                vload(c0, sw, it, x);
                vstore(sw, it, x);
            }
        }
        __syncthreads();
        for (int pass = 0; pass < 2; ++pass) {
            const int I = pass ? rowB : rowA;
            for (int c = par; c < sw / 16; c += 2) {
                floatx4 xu = {0.0f, 0.0f, 0.0f, 0.0f}, xo = {0.0f, 0.0f, 0.0f, 0.0f};
                for (int M = 0; M <= I; ++M)
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        const int k = 16 * M + 4 * s + g;
                        const float bv = gc[k * KS + 16 * c + c16];
                        xu = mfma4(Tm[(16 * I + c16) * CS + k], bv, xu);
                        xo = mfma4(Am[(16 * I + c16) * CS + k], bv, xo);
                    }
                floatx4* blk = reinterpret_cast<floatx4*>(rUO + (c0 / 16 + c) * (2 * CH * 16));
                blk[I * 64 + lane] = xu;
                blk[(CH / 16 + I) * 64 + lane] = xo;
            }
        }
        __syncthreads();
    }
}

/*
    Per (value head, 16 value columns), chunk by chunk, S (fp32) in LDS,
    eight waves (two per SIMD, so one can issue while the other waits):
      phase A, wave w on rows 16 (w % 4)..+15:
          w < 4:  U = Ut - W S  (into LDS)      w >= 4:  O = Ot + Qt S  (out)
      phase B, wave w on key tile w (KD / 16 tiles):  S' = diag(eL) S + Kt^T U
    Each wave's W / Qt / Kt operands and its Ut / Ot accumulator start come
    straight from the record into registers, one chunk ahead. Only S and U
    are in LDS, both transposed (St[col][k], Ut[col][token]) so that a lane
    reads k = 16q + 4g .. +3 of its column at once: within each group of 16 k,
    lane (c16, g) supplies k = 16q + 4g + s on the s-th of four MFMAs. Row
    strides of KD + 4 and CH + 4 floats (odd in 16-byte units) keep each
    16-lane read phase on distinct banks.
*/
constexpr int SCAN_THREADS = 512;

template <int KD>
__global__ __launch_bounds__(SCAN_THREADS) void kda_scan_kernel(KdaArgs a) {
    constexpr int KS = KD + 4;
    constexpr int QA = KD / 16, QB = CH / 16;
    __shared__ __align__(16) float St[NB * KS];
    __shared__ __align__(16) float Ut[NB * CS];

    const KdaParams& p = a.p;
    uint32_t bid = blockIdx.x;
    const uint32_t nb = gridDim.x, nCol = uint32_t(p.valueDim / NB);
    if (nb % 8 == 0) bid = (bid % 8) * (nb / 8) + bid / 8;   // a head's column blocks on one XCD
    const uint32_t h = bid / nCol, cb = bid % nCol;
    const uint32_t col0 = cb * NB;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c16 = lane & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rb = w & 3;               // phase A row block
    const int role = w >> 2;            // phase A: 0 U, 1 O
    const bool tileWave = w < KD / 16;  // phase B
    const size_t VD = p.valueDim, Hv = p.valueHeads;
    const size_t recSize = kda_record(KD, VD);

    float* state = p.state + size_t(h) * KD * VD;
    for (int idx = tid; idx < KD * NB; idx += SCAN_THREADS) {
        const int k = idx / NB, c = idx % NB;
        St[c * KS + k] = state[size_t(k) * VD + col0 + c];
    }

    // the next chunk's operands, requested at the top of the current one
    floatx4 fa[QA], fb[QB], fu, fe = {0.0f, 0.0f, 0.0f, 0.0f};
    auto fetch = [&](uint32_t chunk) {
        const float* rec = a.work + (size_t(h) * a.nChunks + chunk) * recSize;
        const floatx4* ra = reinterpret_cast<const floatx4*>(rec + role * CH * KD) + rb * QA * 64 + lane;
#pragma unroll
        for (int q = 0; q < QA; ++q) fa[q] = ra[q * 64];
        if (tileWave) {
            const floatx4* rk = reinterpret_cast<const floatx4*>(rec + 2 * CH * KD) + w * QB * 64 + lane;
#pragma unroll
            for (int q = 0; q < QB; ++q) fb[q] = rk[q * 64];
            fe = *reinterpret_cast<const floatx4*>(rec + 3 * CH * KD + 16 * w + 4 * g);
        }
        fu = reinterpret_cast<const floatx4*>(rec + 3 * CH * KD + KD)[((cb * 2 + role) * QB + rb) * 64 + lane];
    };
    auto ld4 = [](const float* ptr) { return *reinterpret_cast<const floatx4*>(ptr); };

    fetch(0);
    __syncthreads();
    for (uint32_t chunk = 0; chunk < a.nChunks; ++chunk) {
        const uint64_t t0 = uint64_t(chunk) * CH;
        const uint32_t n = uint32_t(p.count - t0 < CH ? p.count - t0 : CH);
        floatx4 ca[QA], cbk[QB], x = fu, ce = fe;
#pragma unroll
        for (int q = 0; q < QA; ++q) ca[q] = fa[q];
#pragma unroll
        for (int q = 0; q < QB; ++q) cbk[q] = fb[q];
        if (chunk + 1 < a.nChunks) fetch(chunk + 1);

        // phase A
        const float* srow = &St[c16 * KS + 4 * g];
#pragma unroll
        for (int q = 0; q < QA; ++q) {
            const floatx4 bs = ld4(srow + 16 * q);
#pragma unroll
            for (int s = 0; s < 4; ++s) x = mfma4(ca[q][s], bs[s], x);
        }
        if (role == 0) {
            *reinterpret_cast<floatx4*>(&Ut[c16 * CS + 16 * rb + 4 * g]) = x;
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t i = 16 * rb + 4 * g + r;
                if (i < n) p.out[((t0 + i) * Hv + h) * VD + col0 + c16] = x[r];
            }
        }
        __syncthreads();

        // phase B: each wave reads and then rewrites only its own tile of S
        if (tileWave) {
            const floatx4 s4 = ld4(&St[c16 * KS + 16 * w + 4 * g]);
            floatx4 sn;
#pragma unroll
            for (int r = 0; r < 4; ++r) sn[r] = ce[r] * s4[r];
            const float* urow = &Ut[c16 * CS + 4 * g];
#pragma unroll
            for (int q = 0; q < QB; ++q) {
                const floatx4 bu = ld4(urow + 16 * q);
#pragma unroll
                for (int s = 0; s < 4; ++s) sn = mfma4(cbk[q][s], bu[s], sn);
            }
            *reinterpret_cast<floatx4*>(&St[c16 * KS + 16 * w + 4 * g]) = sn;
        }
        __syncthreads();
    }
    for (int idx = tid; idx < KD * NB; idx += SCAN_THREADS) {
        const int k = idx / NB, c = idx % NB;
        state[size_t(k) * VD + col0 + c] = St[c * KS + k];
    }
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
    auto aligned = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) % 16) == 0; };
    if (!aligned(p.q) || !aligned(p.k) || !aligned(p.v) || !aligned(p.g ? p.g : p.f) ||
        (!p.g && !aligned(p.dtBias)))
        return ctx.fail("kda: q, k, v and g (or f and dtBias) must be 16-byte aligned");
    if (p.count == 0) return true;
    KdaArgs a{};
    a.p = p;
    a.nChunks = uint32_t((p.count + CH - 1) / CH);
    if (a.nChunks > 65535u * 1024u) return ctx.fail("kda: sequence too long");
    if (p.valueHeads > 65535u) return ctx.fail("kda: too many value heads");
    const size_t rec = kda_record(int(p.keyDim), p.valueDim);
    a.work = static_cast<float*>(ctx.grow(SLOT_DELTA_WORK, size_t(p.valueHeads) * a.nChunks * rec * sizeof(float)));
    if (!a.work) return false;
    const dim3 sgrid(a.nChunks, unsigned(p.valueHeads));
    const dim3 grid{unsigned(p.valueHeads * (p.valueDim / NB))}, block{SCAN_THREADS};
#define AIGPU_KDA(KD, F)                                                                                       \
    if (p.keyDim == KD && (p.inType == 0) == F) {                                                              \
        if (!ctx.launch("kda_solve_kernel", stream, [&] {                                                      \
                hipLaunchKernelGGL((kda_solve_kernel<KD, F>), sgrid, dim3(256), 0, stream, a);                 \
            }))                                                                                                \
            return false;                                                                                      \
        return ctx.launch("kda_scan_kernel", stream, [&] {                                                     \
            hipLaunchKernelGGL((kda_scan_kernel<KD>), grid, block, 0, stream, a);                              \
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
