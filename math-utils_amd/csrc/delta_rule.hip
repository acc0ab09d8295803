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
// The single-level form is two launches (the two-level scan for long 128 x
// 128 heads, further down, replaces the second with three):
//   delta_solve_kernel  parallel over (key head, chunk): l2 norms, KK^T, QK^T,
//                       then per value head the decayed masks and
//                       T = (I + A)^-1 (blocked: four 16 x 16 diagonal blocks
//                       by forward substitution, the rest by block products);
//                       writes a record per (value head, chunk): T, QKm and
//                       per-row scalars, fp32 or split into bf16 hi/lo
//   delta_scan_*        per (value head, 16 value columns): walks the chunks
//                       in order carrying S in registers. The DMA scan (bf16
//                       inputs on 16-byte boundaries) takes every chunk input
//                       into LDS by DMA a chunk ahead; the register-staged
//                       scans (unaligned bf16, fp32) load the next chunk into
//                       registers while the current one computes. They read
//                       the raw q/k rows and apply the inverse norms as row
//                       scales of the products (k_i = k_raw_i kinv_i enters
//                       every product linearly).
// State columns evolve independently (Kernels.hpp:113-125 touches column d
// only through delta[d]), which is what lets one head split over 16-column
// workgroups.
#include "context.hpp"
#include "device.hpp"
#include "kernels.hpp"

#include <type_traits>

namespace aigpu {

namespace {

constexpr int CH = 64;                   // chunk length
constexpr int CS = CH + 1;               // LDS row stride of CH x CH matrices
constexpr int NB = 16;                   // value columns per scan workgroup
constexpr int NS = NB + 1;
constexpr int SC = 4 * CH;               // gc, beta, kinv, qinv per chunk
constexpr int WORK = 2 * CH * CH + SC;   // floats per (head, chunk) record, fp32 form
// the split form, laid out as the DMA scan's LDS image: T hi, T lo, QKm hi,
// QKm lo (left unwritten for the two-level scan, which forms QKm itself), then
// 512 floats: beta, gamma kinv, gamma qinv, kinv exp(gc_last - gc),
// exp(gc_last) (64 copies), a = gc log2(e) + log2(qinv), b = gc log2(e) -
// log2(kinv), zeros. T and QKm are lower triangular, so
// rows 0-31 keep only their first 32 columns (the scan's waves 0 and 1 read
// no other k block): a packed bf16 matrix is rows 0-31 x 32 columns (16-byte
// block b of row r at b ^ ((r >> 1 ^ r >> 3) & 3)) followed by rows 32-63 x
// 64 columns (block b at b ^ (r & 7)), 3,072 elements, a quarter less than
// the square. Both swizzles keep any 8 or 16 consecutive rows' reads of one
// block column on distinct banks.
constexpr int PMAT = 32 * 32 + 32 * 64;         // bf16 elements per packed matrix
constexpr int PMAT_BYTES = PMAT * 2;
constexpr int SPLIT_SC = 512;
constexpr int WORK_SPLIT = 4 * PMAT / 2 + SPLIT_SC;   // floats

/* element offset of row r's 16-byte block b in a packed T / QKm matrix */
__host__ __device__ constexpr int pmat_offset(int r, int b) {
    return r < 32 ? r * 32 + 8 * (b ^ (((r >> 1) ^ (r >> 3)) & 3)) : 1024 + (r - 32) * 64 + 8 * (b ^ (r & 7));
}

struct DeltaArgs {
    DeltaRuleParams p;
    float* work;       // [valueHeads][nChunks][record]: fp32 or split form
    uint32_t nChunks;
    uint32_t vec;      // q, k, v 16-byte aligned: vector loads
};


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

/* fp32 -> bf16 high part and bf16 residual (round to nearest even): hi + lo
   carries ~16 significant bits over fp32's whole exponent range */
__device__ __forceinline__ void split_bf16(float x, __bf16& hi, __bf16& lo) {
    hi = __bf16(x);
    lo = __bf16(x - float(hi));
}
/* the same for four values, two to a conversion instruction: the high
   parts are widened back from the packed pair by a shift and a mask */
__device__ __forceinline__ void split_bf16x4(const floatx4& x, bf16x4& hi, bf16x4& lo) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    u32x2 h, l;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        h[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{x[2 * i], x[2 * i + 1]}, b2));
        const f2 r{x[2 * i] - __uint_as_float(h[i] << 16), x[2 * i + 1] - __uint_as_float(h[i] & 0xFFFF0000u)};
        l[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, b2));
    }
    hi = __builtin_bit_cast(bf16x4, h);
    lo = __builtin_bit_cast(bf16x4, l);
}

/* e^x for the solve's decays (x <= 0): the library expf where the record is
   fp32, and the hardware 2^x (1 ulp) of x log2(e) where it is split into
   bf16 parts (~16 significant bits), which cannot carry the difference */
template <bool FAST>
__device__ __forceinline__ float decay_exp(float x) {
    if constexpr (FAST) return __builtin_amdgcn_exp2f(x * LOG2E);
    else return expf(x);
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

/*
    Per (key head, chunk): the raw products K K^T and Q K^T of the chunk's rows
    (exact bf16 products on v_mfma_f32_16x16x32_bf16 for bf16 inputs, fp32
    MFMA for fp32 inputs) scaled by the inverse l2 norms, held in registers;
    then for each of the G value heads that share the key head, its gates,
    the decayed masks A and QKm and T = (I + A)^-1, written to that value
    head's record.
*/
template <int KD, bool F32, bool SPLIT, bool QKM = true>
__global__ __launch_bounds__(256, F32 ? 1 : 3) void delta_solve_kernel(DeltaArgs a) {
    static_assert(!(F32 && SPLIT), "the split form serves bf16 inputs");
    static_assert(QKM || SPLIT, "only the split form leaves QKm to the scan");
    constexpr int PE = KD / 4;              // elements of a row per thread
    constexpr int EPL = F32 ? 4 : 8;        // elements per 16-byte load
    constexpr int KH = F32 ? KD + 1 : KD + 8;   // LDS row stride in elements
    using Raw = std::conditional_t<F32, float, __bf16>;
    // The raw q/k rows are dead once K K^T and Q K^T are in registers, and
    // the masks and T are written only after that: they share one LDS pool,
    // so that the LDS holds four workgroups per CU (bf16 inputs) instead of
    // two; the registers then allow three (four, at 128 VGPRs, spilled and
    // ran no faster)
    constexpr int KQB = (CH * KH * int(sizeof(Raw)) + 15) / 16 * 16;   // bytes of ks (and qs)
    constexpr int AMB = (CH * CS * 4 + 15) / 16 * 16;                  // bytes of Am (and Tm)
    constexpr int POOL = 2 * KQB > 2 * AMB ? 2 * KQB : 2 * AMB;
    __shared__ __attribute__((aligned(16))) unsigned char pool[POOL];
    Raw* ks = reinterpret_cast<Raw*>(pool);          // raw k rows
    Raw* qs = reinterpret_cast<Raw*>(pool + KQB);    // raw q rows
    float* Am = reinterpret_cast<float*>(pool);
    float* Tm = reinterpret_cast<float*>(pool + AMB);
    __shared__ float Xs[4][16 * 17];
    __shared__ float nrm[2 * CH];           // kinv, qinv
    __shared__ float gsc[2 * CH];           // gc, beta of the current value head

    const DeltaRuleParams& p = a.p;
    const uint32_t chunk = blockIdx.x, kh = blockIdx.y;
    const uint32_t G = uint32_t(p.valueHeads / p.keyHeads);
    const uint64_t t0 = uint64_t(chunk) * CH;
    const uint32_t n = uint32_t(p.count - t0 < CH ? p.count - t0 : CH);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, c16 = lane & 15;

    float gcEarly = 0.0f, btEarly = 0.0f;
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
        // the gates of value heads 0-3 of this key head, one wave each, while
        // the rows are in flight (later heads load theirs in the loop)
        if (uint32_t(w) < G) chunk_gates(p, t0, n, kh * G + w, lane, gcEarly, btEarly);
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
        for (int i = 0; i < PE / EPL; ++i) {
            const int col = qq * PE + i * EPL;
            if (F32) {
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    reinterpret_cast<float*>(ks)[r * KH + col + e] = raw_elem<true>(kr[i], e);
                    reinterpret_cast<float*>(qs)[r * KH + col + e] = raw_elem<true>(qr[i], e);
                }
            } else {
                *reinterpret_cast<u32x4*>(&ks[r * KH + col]) = kr[i];
                *reinterpret_cast<u32x4*>(&qs[r * KH + col]) = qr[i];
            }
        }
        if (qq == 0) {
            nrm[r] = kinv;
            nrm[CH + r] = qinv;
        }
    }
    __syncthreads();

    // K K^T and Q K^T of the normalised rows: wave w owns rows 16w..16w+15
    floatx4 kk[4], qk[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
        floatx4 x = {0.0f, 0.0f, 0.0f, 0.0f}, y = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (F32) {
            const float* kf = reinterpret_cast<const float*>(ks);
            const float* qf = reinterpret_cast<const float*>(qs);
#pragma unroll 8
            for (int s = 0; s < KD / 4; ++s) {
                const float kj = kf[(16 * ct + c16) * KH + 4 * s + g];
                x = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[(16 * w + c16) * KH + 4 * s + g], kj, x, 0, 0, 0);
                y = __builtin_amdgcn_mfma_f32_16x16x4f32(qf[(16 * w + c16) * KH + 4 * s + g], kj, y, 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int kb = 0; kb < KD / 32; ++kb) {
                const bf16x8 kj = *reinterpret_cast<const bf16x8*>(&ks[(16 * ct + c16) * KH + 32 * kb + 8 * g]);
                x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    *reinterpret_cast<const bf16x8*>(&ks[(16 * w + c16) * KH + 32 * kb + 8 * g]), kj, x, 0, 0, 0);
                if constexpr (QKM)
                    y = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        *reinterpret_cast<const bf16x8*>(&qs[(16 * w + c16) * KH + 32 * kb + 8 * g]), kj, y, 0, 0, 0);
            }
        }
        const int j = 16 * ct + c16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 16 * w + 4 * g + r;
            kk[ct][r] = x[r] * (nrm[i] * nrm[j]);
            qk[ct][r] = y[r] * (nrm[CH + i] * nrm[j]);
        }
    }
    __syncthreads();   // the q/k rows are dead: Am and Tm take their LDS
    // T is zero above its diagonal blocks for every value head
    for (int idx = tid; idx < CH * CH; idx += 256) {
        const int i = idx / CH, j = idx % CH;
        if ((j >> 4) > (i >> 4)) Tm[i * CS + j] = 0.0f;
    }

    for (uint32_t m = 0; m < G; ++m) {
        const uint32_t h = kh * G + m;
        float* rec = a.work + (size_t(h) * a.nChunks + chunk) * (SPLIT ? WORK_SPLIT : WORK);
        if (m < 4 ? uint32_t(w) == m : w == 0) {
            float gc = gcEarly, bt = btEarly;
            if (m >= 4) chunk_gates(p, t0, n, h, lane, gc, bt);
            gsc[lane] = gc;
            gsc[CH + lane] = bt;
        }
        __syncthreads();

        float* qkm = rec + CH * CH;
        floatx4 qkv[4];   // this value head's QKm, written once T is done (split form)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 16 * w + 4 * g + r, j = 16 * ct + c16;
                const float dec = j <= i ? decay_exp<SPLIT>(gsc[i] - gsc[j]) : 0.0f;
                Am[i * CS + j] = j < i ? gsc[CH + i] * dec * kk[ct][r] : 0.0f;
                if constexpr (SPLIT) {
                    if constexpr (QKM) qkv[ct][r] = dec * qk[ct][r];
                } else {
                    qkm[i * CH + j] = dec * qk[ct][r];
                }
            }
        __syncthreads();

        // T = (I + A)^-1. Diagonal blocks: wave w inverts block w by forward
        // substitution, T[i][j] = [i == j] - sum_{m < i} A[i][m] T[m][j], with
        // column j = lane % 16 of every row in registers and each A row read
        // as a broadcast; terms with m < j are exact zeros (T[m][j] = 0), so
        // the sum is the one over j <= m < i.
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

        if constexpr (!SPLIT) {
            for (int idx = tid; idx < CH * CH; idx += 256) rec[idx] = Tm[(idx / CH) * CS + idx % CH];
            rec[2 * CH * CH + tid] = tid < 2 * CH ? gsc[tid] : nrm[tid - 2 * CH];
        } else {
            // QKm into Am (free now that T is done), then both matrices split
            // into bf16 hi/lo rows, 16 bytes per store, in the scan's LDS image
            // (without QKm, the two-level scan's form: T alone)
            if constexpr (QKM) {
#pragma unroll
                for (int ct = 0; ct < 4; ++ct)
#pragma unroll
                    for (int r = 0; r < 4; ++r) Am[(16 * w + 4 * g + r) * CS + 16 * ct + c16] = qkv[ct][r];
                __syncthreads();
            }
            uint16_t* out16 = reinterpret_cast<uint16_t*>(rec);
#pragma unroll
            for (int it = 0; it < 2; ++it) {
                const int idx = tid + 256 * it, r = idx >> 3, b = idx & 7;
                if (r < 32 && b >= 4) continue;   // above the diagonal blocks: zero, not stored
                const int dst = pmat_offset(r, b);
#pragma unroll
                for (int m = 0; m < (QKM ? 2 : 1); ++m) {
                    const float* src = (m == 0 ? Tm : Am) + r * CS + 8 * b;
                    bf16x4 h0, l0, h1, l1;
                    split_bf16x4(floatx4{src[0], src[1], src[2], src[3]}, h0, l0);
                    split_bf16x4(floatx4{src[4], src[5], src[6], src[7]}, h1, l1);
                    *reinterpret_cast<bf16x8*>(out16 + (2 * m) * PMAT + dst) =
                        __builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7);
                    *reinterpret_cast<bf16x8*>(out16 + (2 * m + 1) * PMAT + dst) =
                        __builtin_shufflevector(l0, l1, 0, 1, 2, 3, 4, 5, 6, 7);
                }
            }
            // per-row scalars of the scan: rows past the sequence's end have
            // beta 0, so they add nothing to U, O or the state
            float* sc = rec + 2 * PMAT;
            const float gLast = gsc[CH - 1];
            for (int idx = tid; idx < SPLIT_SC; idx += 256) {
                const int i = idx & (CH - 1), part = idx >> 6;
                float x = 0.0f;
                if (part == 0) x = gsc[CH + i];
                else if (part == 1) x = decay_exp<true>(gsc[i]) * nrm[i];
                else if (part == 2) x = decay_exp<true>(gsc[i]) * nrm[CH + i];
                else if (part == 3) x = nrm[i] * decay_exp<true>(gLast - gsc[i]);
                else if (part == 4) x = decay_exp<true>(gLast);
                // the factors of QKm for a scan that forms it from the raw
                // products: QKm_ij = (q_i.k_j) 2^(a_i - b_j), j <= i
                else if (part == 5) x = gsc[i] * LOG2E + __builtin_amdgcn_logf(nrm[CH + i]);
                else if (part == 6) x = gsc[i] * LOG2E - __builtin_amdgcn_logf(nrm[i]);
                sc[idx] = x;
            }
        }
        __syncthreads();   // gsc, Am and Tm are rewritten for the next value head
    }
}

/*
    The scan on v_mfma_f32_16x16x4f32 for fp32 inputs, whose parity bound
    (1e-5) a split into 16-bit parts does not meet: the fp16 residual of values
    below 2^-3 is subnormal, and bf16 parts carry 8 bits each.
*/
template <int KD, bool VEC>
__global__ __launch_bounds__(256) void delta_scan_f32_kernel(DeltaArgs a) {
    constexpr bool F32 = true;
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
    constexpr bool vec = VEC;

    float* state = p.state + size_t(h) * KD * VD;
    for (int idx = tid; idx < KD * NB; idx += 256) {
        const int i = idx / NB, j = idx % NB;
        Ss[i * NS + j] = state[size_t(i) * VD + col0 + j];
    }

    // registers holding the next chunk's inputs while the current one computes
    u32x4 kst[KQL], qst[KQL];
    floatx4 tst[4], mst[4];
    u32x4 vst;      // 4 value columns of one row
    float sst;
    uint32_t stagedN = 0;
    // Loads are unconditional (rows past the chunk's end read its last row)
    // and those rows are zeroed at the commit: a load guarded by a condition
    // makes the compiler load into a temporary and copy, and the copy waits
    // for the load, which would serialise the prefetch.
    auto stage = [&](uint32_t chunk) {
        const uint64_t t0 = uint64_t(chunk) * CH;
        const uint32_t n = uint32_t(p.count - t0 < CH ? p.count - t0 : CH);
        stagedN = n;
#pragma unroll
        for (int i = 0; i < KQL; ++i) {
            const int e = (tid + 256 * i) * EPL, r = e / KD, col = e % KD;
            const uint32_t rr = uint32_t(r) < n ? uint32_t(r) : n - 1;
            const size_t src = ((t0 + rr) * p.keyHeads + kh) * KD + col;
            kst[i] = load_raw16<F32>(p.k, src, vec);
            qst[i] = load_raw16<F32>(p.q, src, vec);
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
            const uint32_t rr = uint32_t(r) < n ? uint32_t(r) : n - 1;
            const float* vf = static_cast<const float*>(p.v) + ((t0 + rr) * Hv + h) * VD + col0 + c4;
            if (vec) vst = *reinterpret_cast<const u32x4*>(vf);
            else vst = u32x4{__float_as_uint(vf[0]), __float_as_uint(vf[1]), __float_as_uint(vf[2]), __float_as_uint(vf[3])};
        }
    };
    auto commit = [&]() {
#pragma unroll
        for (int i = 0; i < KQL; ++i) {
            const int e = (tid + 256 * i) * EPL, r = e / KD, col = e % KD;
            const bool ok = uint32_t(r) < stagedN;
#pragma unroll
            for (int x = 0; x < EPL; ++x) {
                ks[r * KS + col + x] = ok ? raw_elem<F32>(kst[i], x) : 0.0f;
                qs[r * KS + col + x] = ok ? raw_elem<F32>(qst[i], x) : 0.0f;
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
        const bool ok = uint32_t(r) < stagedN;
#pragma unroll
        for (int x = 0; x < 4; ++x) vs[r * NS + c4 + x] = ok ? __uint_as_float(vst[x]) : 0.0f;
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
        const floatx4 oacc = acc;   // stored after the commit below

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
        // The output leaves after the commit: stores count in vmcnt with the
        // staged loads, so the commit's wait for those loads would otherwise
        // also wait out the latency of this chunk's stores.
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t i = 16 * w + 4 * g + r;
            if (i < n) p.out[((t0 + i) * Hv + h) * VD + col0 + c16] = oacc[r];
        }
    }
    __syncthreads();
    for (int idx = tid; idx < KD * NB; idx += 256) {
        const int i = idx / NB, j = idx % NB;
        state[size_t(i) * VD + col0 + j] = Ss[i * NS + j];
    }
}

typedef __fp16 fp16x4v __attribute__((__vector_size__(4 * sizeof(__fp16))));


/* ds_read_b64_tr_b16 pair: lane i of each 16-lane group receives column
   `base + i` of rows P0..P0+7 when lane L addresses row P0 + L/4 (and +4),
   columns base + 4 (L % 4) .. +3 */
__device__ __forceinline__ bf16x8 tr_pair(const __bf16* a0, const __bf16* a1) {
    typedef __attribute__((address_space(3))) fp16x4v lds_x4;
    const fp16x4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_x4*)(a0));
    const fp16x4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_x4*)(a1));
    const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
    return __builtin_bit_cast(bf16x8, u32x4{l2[0], l2[1], h2[0], h2[1]});
}

__device__ __forceinline__ floatx4 mfma_bf(const bf16x8& a, const bf16x8& b, const floatx4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

/*
    The scan for bf16 inputs: value head h, value columns col0 .. col0+15,
    chunk by chunk, on v_mfma_f32_16x16x32_bf16. Raw q/k rows are exact in
    bf16; every fp32 operand (S, T, QKm, R, U, W) is split into a bf16 high
    part and the bf16 residual, and each product takes hi*hi + hi*lo + lo*hi
    (or hi*hi + hi*lo against an exact raw row) with fp32 accumulation, ~2^-16
    relative. Per chunk:
      R  = diag(beta) (V - diag(gamma kinv) K_raw S)       rows i, cols c
      U  = T R
      O  = diag(gamma qinv) Q_raw S + QKm U
      S' = e^{gc_last} S + K_raw^T W,  W = diag(kinv e^{gc_last - gc}) U
    S stays in registers as each wave's fp32 accumulators (wave w owns key
    rows 16 (w + 4t) + 0..15) across all chunks; LDS holds its transposed
    split as the next chunk's B operand. Matrices sit in LDS row-major with 16
    bytes of padding per row (A-operand reads of 16 rows x 16 bytes hit
    distinct banks); B operands are stored transposed, so every operand read
    is one 16-byte LDS load; K^T comes from row-major K through transposed
    reads.
*/
template <int KD, bool VEC>
__global__ __launch_bounds__(256) void delta_scan_kernel(DeltaArgs a) {
    constexpr int KQL = CH * KD / (256 * 8);         // 16-byte loads per thread for k (and q)
    constexpr int KH = KD + 8;                       // elements per K/Q row in LDS
    constexpr int CHH = CH + 8;                      // elements per row of CH-wide matrices
    constexpr int MT = KD / 64;                      // 16-row state tiles per wave
    __shared__ __attribute__((aligned(16))) __bf16 Kb[CH * KH];       // raw k rows
    __shared__ __attribute__((aligned(16))) __bf16 Qb[CH * KH];       // raw q rows
    __shared__ __attribute__((aligned(16))) __bf16 Tb[2][CH * CHH];   // T, hi / lo
    __shared__ __attribute__((aligned(16))) __bf16 Mb[2][CH * CHH];   // QKm, hi / lo
    __shared__ __attribute__((aligned(16))) __bf16 St[2][NB * KH];    // S^T [col][key]
    __shared__ __attribute__((aligned(16))) __bf16 Rt[2][NB * CHH];   // R^T [col][token]
    __shared__ __attribute__((aligned(16))) __bf16 Ut[2][NB * CHH];   // U^T
    __shared__ __attribute__((aligned(16))) __bf16 Wt[2][NB * CHH];   // W^T
    __shared__ float vs[CH * NS];
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
    constexpr bool vec = VEC;

    // C-layout tile (rows row0 + 4g + r, column c16) -> transposed split [col][row]
    auto put_t = [&](__bf16* dhi, __bf16* dlo, int stride, int row0, const floatx4& x) {
        bf16x4 hv, lv;
        split_bf16x4(x, hv, lv);
        *reinterpret_cast<bf16x4*>(&dhi[c16 * stride + row0 + 4 * g]) = hv;
        *reinterpret_cast<bf16x4*>(&dlo[c16 * stride + row0 + 4 * g]) = lv;
    };

    // S: wave w's tiles mt = w + 4t hold key rows 16 mt + 4g + r, column c16
    float* state = p.state + size_t(h) * KD * VD;
    floatx4 sacc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            sacc[t][r] = state[size_t(16 * (w + 4 * t) + 4 * g + r) * VD + col0 + c16];
    auto publish_state = [&]() {
#pragma unroll
        for (int t = 0; t < MT; ++t) put_t(St[0], St[1], KH, 16 * (w + 4 * t), sacc[t]);
    };
    publish_state();

    // registers holding the next chunk's inputs while the current one computes
    u32x4 kst[KQL], qst[KQL];
    floatx4 tst[4], mst[4];
    u32x2 vst;
    float sst;
    uint32_t stagedN = 0;
    // Loads are unconditional (rows past the chunk's end read its last row)
    // and those rows are zeroed at the commit: a load guarded by a condition
    // makes the compiler load into a temporary and copy, and the copy waits
    // for the load, which would serialise the prefetch.
    auto stage = [&](uint32_t chunk) {
        const uint64_t t0 = uint64_t(chunk) * CH;
        const uint32_t n = uint32_t(p.count - t0 < CH ? p.count - t0 : CH);
        stagedN = n;
#pragma unroll
        for (int i = 0; i < KQL; ++i) {
            const int e = (tid + 256 * i) * 8, r = e / KD, col = e % KD;
            const uint32_t rr = uint32_t(r) < n ? uint32_t(r) : n - 1;
            const size_t src = ((t0 + rr) * p.keyHeads + kh) * KD + col;
            kst[i] = load_raw16<false>(p.k, src, vec);
            qst[i] = load_raw16<false>(p.q, src, vec);
        }
        const float* rec = a.work + (size_t(h) * a.nChunks + chunk) * WORK;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            tst[i] = *reinterpret_cast<const floatx4*>(rec + 4 * (tid + 256 * i));
            mst[i] = *reinterpret_cast<const floatx4*>(rec + CH * CH + 4 * (tid + 256 * i));
        }
        sst = rec[2 * CH * CH + tid];
        const int r = tid >> 2, c4 = 4 * (tid & 3);
        const uint32_t rr = uint32_t(r) < n ? uint32_t(r) : n - 1;
        const uint16_t* vb = static_cast<const uint16_t*>(p.v) + ((t0 + rr) * Hv + h) * VD + col0 + c4;
        if (vec) vst = *reinterpret_cast<const u32x2*>(vb);
        else vst = u32x2{uint32_t(vb[0]) | (uint32_t(vb[1]) << 16), uint32_t(vb[2]) | (uint32_t(vb[3]) << 16)};
    };
    auto commit = [&]() {
#pragma unroll
        for (int i = 0; i < KQL; ++i) {   // raw bf16 rows go in as they are
            const int e = (tid + 256 * i) * 8, r = e / KD, col = e % KD;
            const bool ok = uint32_t(r) < stagedN;
            *reinterpret_cast<u32x4*>(&Kb[r * KH + col]) = ok ? kst[i] : u32x4{0, 0, 0, 0};
            *reinterpret_cast<u32x4*>(&Qb[r * KH + col]) = ok ? qst[i] : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = 4 * (tid + 256 * i), r = idx / CH, col = idx % CH;
            bf16x4 th, tl, mh, ml;
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                __bf16 hi, lo;
                split_bf16(tst[i][x], hi, lo);
                th[x] = hi;
                tl[x] = lo;
                split_bf16(mst[i][x], hi, lo);
                mh[x] = hi;
                ml[x] = lo;
            }
            *reinterpret_cast<bf16x4*>(&Tb[0][r * CHH + col]) = th;
            *reinterpret_cast<bf16x4*>(&Tb[1][r * CHH + col]) = tl;
            *reinterpret_cast<bf16x4*>(&Mb[0][r * CHH + col]) = mh;
            *reinterpret_cast<bf16x4*>(&Mb[1][r * CHH + col]) = ml;
        }
        sc[tid] = sst;
        const int r = tid >> 2, c4 = 4 * (tid & 3);
        const bool ok = uint32_t(r) < stagedN;
        const u32x4 v4{ok ? vst[0] : 0u, ok ? vst[1] : 0u, 0, 0};
#pragma unroll
        for (int x = 0; x < 4; ++x) vs[r * NS + c4 + x] = raw_elem<false>(v4, x);
    };
    // acc += X[rows 16w .. +15][k] Y[k][cols], k in [0, K): X row-major (one
    // exact part, or hi/lo when X1 is given), Y transposed split [col][k]
    auto gemm = [&](floatx4 acc, const __bf16* X0, const __bf16* X1, int XS, const __bf16* Y0, const __bf16* Y1,
                    int YS, int K) {
#pragma unroll
        for (int kb = 0; kb < K / 32; ++kb) {
            const int xo = (16 * w + c16) * XS + 32 * kb + 8 * g, yo = c16 * YS + 32 * kb + 8 * g;
            const bf16x8 xh = *reinterpret_cast<const bf16x8*>(X0 + xo);
            const bf16x8 yh = *reinterpret_cast<const bf16x8*>(Y0 + yo);
            acc = mfma_bf(xh, yh, acc);
            acc = mfma_bf(xh, *reinterpret_cast<const bf16x8*>(Y1 + yo), acc);
            if (X1) acc = mfma_bf(*reinterpret_cast<const bf16x8*>(X1 + xo), yh, acc);
        }
        return acc;
    };

    stage(0);
    commit();
    for (uint32_t chunk = 0; chunk < a.nChunks; ++chunk) {
        const uint64_t t0 = uint64_t(chunk) * CH;
        const uint32_t n = uint32_t(p.count - t0 < CH ? p.count - t0 : CH);
        __syncthreads();   // the chunk's inputs and S^T are in LDS
        if (chunk + 1 < a.nChunks) stage(chunk + 1);
        const float* gcs = sc;
        const float* bs = sc + CH;
        const float* kinv = sc + 2 * CH;
        const float* qinv = sc + 3 * CH;
        const float gLast = gcs[CH - 1];
        if (tid < CH) kdk[tid] = kinv[tid] * expf(gLast - gcs[tid]);

        // R = beta (V - gamma kinv (K_raw S))
        floatx4 acc = gemm(floatx4{0.0f, 0.0f, 0.0f, 0.0f}, Kb, nullptr, KH, St[0], St[1], KH, KD);
        {
            floatx4 rv;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 16 * w + 4 * g + r;
                rv[r] = bs[i] * (vs[i * NS + c16] - expf(gcs[i]) * (kinv[i] * acc[r]));
            }
            put_t(Rt[0], Rt[1], CHH, 16 * w, rv);
        }
        __syncthreads();

        // U = T R, and W = diag(kdk) U for the state update
        const floatx4 u = gemm(floatx4{0.0f, 0.0f, 0.0f, 0.0f}, Tb[0], Tb[1], CHH, Rt[0], Rt[1], CHH, CH);
        put_t(Ut[0], Ut[1], CHH, 16 * w, u);
        {
            floatx4 wv;
#pragma unroll
            for (int r = 0; r < 4; ++r) wv[r] = kdk[16 * w + 4 * g + r] * u[r];
            put_t(Wt[0], Wt[1], CHH, 16 * w, wv);
        }
        __syncthreads();

        // O = gamma qinv (Q_raw S) + QKm U
        acc = gemm(floatx4{0.0f, 0.0f, 0.0f, 0.0f}, Qb, nullptr, KH, St[0], St[1], KH, KD);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 16 * w + 4 * g + r;
            acc[r] *= expf(gcs[i]) * qinv[i];
        }
        acc = gemm(acc, Mb[0], Mb[1], CHH, Ut[0], Ut[1], CHH, CH);
        const floatx4 oacc = acc;   // stored after the commit below

        // S' = e^{gc_last} S + K_raw^T W: A = K^T rows d (transposed reads of
        // row-major K), B = W^T [col][token]
        const float eLast = expf(gLast);
        const int q16 = lane & 15;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int d0 = 16 * (w + 4 * t);
#pragma unroll
            for (int r = 0; r < 4; ++r) sacc[t][r] *= eLast;
#pragma unroll
            for (int ib = 0; ib < CH / 32; ++ib) {
                const int row = 32 * ib + 8 * g + (q16 >> 2), col = d0 + 4 * (q16 & 3);
                const bf16x8 kt = tr_pair(&Kb[row * KH + col], &Kb[(row + 4) * KH + col]);
                const int yo = c16 * CHH + 32 * ib + 8 * g;
                sacc[t] = mfma_bf(kt, *reinterpret_cast<const bf16x8*>(&Wt[0][yo]), sacc[t]);
                sacc[t] = mfma_bf(kt, *reinterpret_cast<const bf16x8*>(&Wt[1][yo]), sacc[t]);
            }
        }
        __syncthreads();   // every read of this chunk's LDS is done
        publish_state();
        if (chunk + 1 < a.nChunks) commit();
        // The output leaves after the commit: stores count in vmcnt with the
        // staged loads, so the commit's wait for those loads would otherwise
        // also wait out the latency of this chunk's stores.
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t i = 16 * w + 4 * g + r;
            if (i < n) p.out[((t0 + i) * Hv + h) * VD + col0 + c16] = oacc[r];
        }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            state[size_t(16 * (w + 4 * t) + 4 * g + r) * VD + col0 + c16] = sacc[t][r];
}

__device__ __forceinline__ void wait_vmcnt_all() { __builtin_amdgcn_s_waitcnt((0) | (7 << 4) | (15 << 8)); }

/* s_waitcnt vmcnt(N) alone (N < 64) */
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}



/*
    The scan for 16-byte aligned bf16 inputs with every chunk input DMA'd into
    LDS: nothing is staged in registers or converted on the scan's path.
      - raw k and q rows come straight from the input tensors, 16-byte block b
        of row r stored at b ^ (r % (KD / 8)), so A-operand reads of 16 rows
        hit distinct banks;
      - T and QKm come from the solve kernel already split into bf16 hi/lo in
        this kernel's LDS layout, with the per-row scalars;
      - the value block [64][16] bf16.
    Every input is double-buffered and fetched a whole chunk ahead, so each
    chunk waits once, at its start, for DMA issued a chunk earlier. Per chunk,
    with three barriers:
      R  = diag(beta) (V - diag(gamma kinv) K_raw S),  and Q_raw S
      U  = T R,  W = diag(kinv e^{gc_last - gc}) U
      S' = e^{gc_last} S + K_raw^T W
      O  = diag(gamma qinv) (Q_raw S) + QKm U
    S is each wave's fp32 accumulators (wave w owns key rows 16 (w + 4t) +
    0..15); its transposed hi/lo split is the B operand of both first-phase
    products, so once they are done (the barrier after R) S' can be published
    over it. Every product takes hi*hi + hi*lo (+ lo*hi) with fp32
    accumulation.
*/
template <int KD>
__global__ __launch_bounds__(256) void delta_scan_dma_kernel(DeltaArgs a) {
    constexpr int KBLK = KD / 8;                     // 16-byte blocks per k/q row
    constexpr int RPI = 1024 / (2 * KD);             // k/q rows per 1 KB DMA block
    constexpr int KI = CH / RPI / 4;                 // k (or q) DMA blocks per wave
    constexpr int TI = 2 * PMAT_BYTES / 1024 / 4;   // T (or QKm) hi+lo DMA blocks per wave: 12 KB / 4

    constexpr int KST = KD + 8;                      // S^T row stride (elements)
    constexpr int CHH = CH + 8;                      // R^T, U^T, W^T row stride
    constexpr int MT = KD / 64;                      // 16-row state tiles per wave
    static_assert(KI * 4 * RPI == CH, "k rows split evenly over the waves");
    __shared__ __attribute__((aligned(16))) __bf16 Kb[2][CH * KD];        // raw k rows, swizzled
    __shared__ __attribute__((aligned(16))) __bf16 Tb[2][2 * PMAT];       // T hi, lo (solve's packed image)
    __shared__ __attribute__((aligned(16))) float Ax[2][1024];           // v [64][16] bf16, then scalars
    __shared__ __attribute__((aligned(16))) __bf16 Qb[2][CH * KD];        // raw q rows, swizzled
    __shared__ __attribute__((aligned(16))) __bf16 Mb[2][2 * PMAT];       // QKm hi, lo
    __shared__ __attribute__((aligned(16))) __bf16 St[2][NB * KST];       // [hi/lo] S^T [col][key]
    __shared__ __attribute__((aligned(16))) __bf16 Rt[2][NB * CHH];       // R^T hi, lo
    __shared__ __attribute__((aligned(16))) __bf16 Ut[2][NB * CHH];       // U^T
    __shared__ __attribute__((aligned(16))) __bf16 Wt[2][NB * CHH];       // W^T

    const DeltaRuleParams& p = a.p;
    // keep a head's column blocks on one XCD: they read the same records
    uint32_t bid = blockIdx.x;
    const uint32_t nb = gridDim.x, nCol = uint32_t(p.valueDim / NB);
    if (nb % 8 == 0) bid = (bid % 8) * (nb / 8) + bid / 8;
    const uint32_t h = bid / nCol, cb = bid % nCol;
    const uint32_t kh = uint32_t(h / (p.valueHeads / p.keyHeads));
    const uint32_t col0 = cb * NB;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c16 = lane & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: DMA targets are scalar
    const size_t VD = p.valueDim, Hv = p.valueHeads;
    const uint32_t nChunks = a.nChunks;

    auto chunk_rows = [&](uint32_t chunk) -> uint32_t {
        const uint64_t t0 = uint64_t(chunk) * CH;
        return uint32_t(p.count - t0 < CH ? p.count - t0 : CH);
    };
    auto record = [&](uint32_t chunk) -> const float* {
        return a.work + (size_t(h) * nChunks + chunk) * WORK_SPLIT;
    };
    // DMA targets: LDS byte addresses of each buffer (uniform)
    const uint32_t ldsK = lds_address(Kb), ldsQ = lds_address(Qb), ldsT = lds_address(Tb);
    const uint32_t ldsM = lds_address(Mb), ldsA = lds_address(Ax);
    constexpr uint32_t KBUF = CH * KD * 2, TBUF = 2 * PMAT_BYTES, ABUF = 4096;   // bytes per buffer
    // per-lane byte offsets of this wave's DMA blocks within a chunk: k/q
    // rows (block j: rows RPI (w KI + j) + lane / KBLK, swizzled; rows past a
    // partial chunk's end repeat its last row, whose beta is 0), the split
    // matrices and scalars of a record, the value rows
    const uint32_t rowBytes = uint32_t(p.keyHeads * KD * 2);
    // (a row's byte offset, clamped by the uniform offset of the chunk's
    // last row: one min and one add per DMA block)
    uint32_t kqRowB[KI], kqCol[KI];
#pragma unroll
    for (int j = 0; j < KI; ++j) {
        const int row = RPI * (w * KI + j) + lane / KBLK;
        kqRowB[j] = uint32_t(row) * rowBytes;
        kqCol[j] = kh * KD * 2 + 16 * ((lane % KBLK) ^ (row % KBLK));
    }
    const uint32_t matOff = uint32_t(w * TI * 1024 + 16 * lane);
    const uint32_t vRowBytes = uint32_t(Hv * VD * 2);
    const uint32_t vRowB = uint32_t(32 * w + lane / 2) * vRowBytes + 16 * (lane & 1);

    // The next chunk's DMA is spread over the current chunk's phases, a block
    // or two between MFMAs: a wave that issues it all at once stalls on the
    // memory pipeline's queue before its next LDS read.
    struct Next {
        const uint8_t *k, *q, *rec, *v;
        uint32_t n;
        int buf;
    };
    auto next_of = [&](uint32_t chunk, int buf) __attribute__((always_inline)) {
        const uint64_t t0 = uint64_t(chunk) * CH;
        return Next{static_cast<const uint8_t*>(p.k) + t0 * rowBytes, static_cast<const uint8_t*>(p.q) + t0 * rowBytes,
                    reinterpret_cast<const uint8_t*>(record(chunk)),
                    static_cast<const uint8_t*>(p.v) + ((t0 * Hv + h) * VD + col0) * 2, chunk_rows(chunk), buf};
    };
    auto dma_rows_j = [&](const Next& nx, int j) __attribute__((always_inline)) {   // k and q block j
        const uint32_t off = min(kqRowB[j], (nx.n - 1) * rowBytes) + kqCol[j];
        dma_block(nx.k, off, ldsK + nx.buf * KBUF + (w * KI + j) * 1024);
        dma_block(nx.q, off, ldsQ + nx.buf * KBUF + (w * KI + j) * 1024);
    };
    auto dma_t_j = [&](const Next& nx, int j) __attribute__((always_inline)) {
        dma_block(nx.rec + j * 1024, matOff, ldsT + nx.buf * TBUF + (w * TI + j) * 1024);
    };
    auto dma_m_j = [&](const Next& nx, int j) __attribute__((always_inline)) {
        dma_block(nx.rec + 2 * PMAT_BYTES + j * 1024, matOff, ldsM + nx.buf * TBUF + (w * TI + j) * 1024);
    };
    auto dma_aux = [&](const Next& nx) __attribute__((always_inline)) {
        if (w < 2) {   // value block: 32 rows of 32 bytes per DMA block
            dma_block(nx.v, min(vRowB, (nx.n - 1) * vRowBytes + 16 * (lane & 1)), ldsA + nx.buf * ABUF + 1024 * w);
        } else {       // scalars
            dma_block(nx.rec + 4 * PMAT_BYTES, uint32_t(1024 * (w - 2) + 16 * lane),
                      ldsA + nx.buf * ABUF + 2048 + 1024 * (w - 2));
        }
    };

    // C-layout tile (rows row0 + 4g + r, column c16) -> transposed split [col][row]
    auto put_t = [&](__bf16* dhi, __bf16* dlo, int stride, int row0, const floatx4& x) __attribute__((always_inline)) {
        bf16x4 hv, lv;
        split_bf16x4(x, hv, lv);
        *reinterpret_cast<bf16x4*>(&dhi[c16 * stride + row0 + 4 * g]) = hv;
        *reinterpret_cast<bf16x4*>(&dlo[c16 * stride + row0 + 4 * g]) = lv;
    };
    // A operand from a swizzled k/q buffer: rows 16w + c16, k-block kb
    auto rows_a = [&](const __bf16* X, int kb) __attribute__((always_inline)) -> bf16x8 {
        const int r = 16 * w + c16, lb = 4 * kb + g;
        return *reinterpret_cast<const bf16x8*>(X + r * KD + 8 * (lb ^ (r % KBLK)));
    };
    // A operand from a packed split matrix in the solve's image (k block kb
    // of rows 16w ..; waves 0 and 1 only ever read kb = 0)
    auto mat_a = [&](const __bf16* X, int kb) __attribute__((always_inline)) -> bf16x8 {
        const int r = 16 * w + c16, lb = 4 * kb + g;
        return *reinterpret_cast<const bf16x8*>(X + pmat_offset(r, lb));
    };

    // S: wave w's tiles mt = w + 4t hold key rows 16 mt + 4g + r, column c16
    float* state = p.state + size_t(h) * KD * VD;
    floatx4 sacc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            sacc[t][r] = state[size_t(16 * (w + 4 * t) + 4 * g + r) * VD + col0 + c16];
    auto publish_state = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < MT; ++t) put_t(St[0], St[1], KST, 16 * (w + 4 * t), sacc[t]);
    };
    publish_state();
    {
        const Next first = next_of(0, 0);
#pragma unroll
        for (int j = 0; j < KI; ++j) dma_rows_j(first, j);
#pragma unroll
        for (int j = 0; j < TI; ++j) {
            dma_t_j(first, j);
            dma_m_j(first, j);
        }
        dma_aux(first);
    }

    // The wave's 16 output rows leave as one 16-byte store per lane (row
    // 16w + lane / 4, columns 4 (lane % 4) ..): the C-layout tile goes
    // through the wave's own kilobyte of the R^T buffer, which no wave uses
    // between the barrier after U and the next chunk's R phase.
    const uint32_t oOff = uint32_t(16 * w + lane / 4) * uint32_t(Hv * VD * 4) + 16 * (lane & 3);
    float* stage = reinterpret_cast<float*>(Rt[0]) + 256 * w;
    static_assert(2 * NB * CHH * 2 >= 4 * 1024, "R^T holds four waves' output tiles");
    auto store_out = [&](uint32_t chunk, const floatx4& o) __attribute__((always_inline)) {
        const uint64_t t0 = uint64_t(chunk) * CH;
        const uint32_t n = chunk_rows(chunk);
#pragma unroll
        for (int r = 0; r < 4; ++r) stage[(4 * g + r) * NB + c16] = o[r];
        wave_sync();
        const floatx4 v4 = *reinterpret_cast<const floatx4*>(stage + 4 * lane);
        uint8_t* ob = reinterpret_cast<uint8_t*>(p.out + (t0 * Hv + h) * VD + col0);
        if (uint32_t(16 * w + lane / 4) < n) *reinterpret_cast<floatx4*>(ob + oOff) = v4;
    };

    for (uint32_t chunk = 0; chunk < nChunks; ++chunk) {
        const int par = chunk & 1;
        // this chunk's inputs have landed (and every earlier store has left);
        // every read of the other buffers is done
        wait_vmcnt_all();
        __syncthreads();
        const Next nx = next_of(chunk + 1 < nChunks ? chunk + 1 : chunk, par ^ 1);   // the last chunk reloads itself

        const __bf16* K = Kb[par];
        const __bf16* Q = Qb[par];
        const __bf16* T = Tb[par];
        const __bf16* M = Mb[par];
        const __bf16* vb = reinterpret_cast<const __bf16*>(Ax[par]);
        const float* sc = Ax[par] + 512;
        const float* beta = sc;
        const float* gkinv = sc + CH;
        const float* gqinv = sc + 2 * CH;
        const float* kdk = sc + 3 * CH;
        const float eLast = sc[4 * CH];
        // R = beta (V - gamma kinv (K_raw S)), and Q_raw S for the output
        floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f}, qs = {0.0f, 0.0f, 0.0f, 0.0f};
        static_assert(KI == KD / 32, "one k/q DMA block per first-phase step");
#pragma unroll
        for (int kb = 0; kb < KD / 32; ++kb) {
            dma_rows_j(nx, kb);
            const bf16x8 x = rows_a(K, kb), xq = rows_a(Q, kb);
            const int yo = c16 * KST + 32 * kb + 8 * g;
            const bf16x8 sh = *reinterpret_cast<const bf16x8*>(&St[0][yo]);
            const bf16x8 sl = *reinterpret_cast<const bf16x8*>(&St[1][yo]);
            acc = mfma_bf(x, sh, acc);
            qs = mfma_bf(xq, sh, qs);
            acc = mfma_bf(x, sl, acc);
            qs = mfma_bf(xq, sl, qs);
        }
        {
            floatx4 rv;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 16 * w + 4 * g + r;
                rv[r] = beta[i] * (float(vb[i * NB + c16]) - gkinv[i] * acc[r]);
            }
            put_t(Rt[0], Rt[1], CHH, 16 * w, rv);
        }
        lds_barrier();

        // U = T R, W = diag(kdk) U
        floatx4 u = {0.0f, 0.0f, 0.0f, 0.0f};
        static_assert(TI == 3, "the T and QKm DMA is issued as 2 + 1 blocks each");
#pragma unroll
        for (int kb = 0; kb < CH / 32; ++kb) {
            if (kb == 0) {
                dma_t_j(nx, 0);
                dma_t_j(nx, 1);
                dma_m_j(nx, 0);
                dma_m_j(nx, 1);
            } else {
                dma_t_j(nx, 2);
                dma_m_j(nx, 2);
            }
            if (kb == 0 || w >= 2) {   // rows < 32 have no nonzero T past column 31
                const bf16x8 th = mat_a(T, kb), tl = mat_a(T + PMAT, kb);
                const int yo = c16 * CHH + 32 * kb + 8 * g;
                const bf16x8 rh = *reinterpret_cast<const bf16x8*>(&Rt[0][yo]);
                u = mfma_bf(th, rh, u);
                u = mfma_bf(th, *reinterpret_cast<const bf16x8*>(&Rt[1][yo]), u);
                u = mfma_bf(tl, rh, u);
            }
        }
        dma_aux(nx);
        put_t(Ut[0], Ut[1], CHH, 16 * w, u);
        {
            floatx4 wv;
#pragma unroll
            for (int r = 0; r < 4; ++r) wv[r] = kdk[16 * w + 4 * g + r] * u[r];
            put_t(Wt[0], Wt[1], CHH, 16 * w, wv);
        }
        lds_barrier();

        // S' = e^{gc_last} S + K_raw^T W: A = K^T rows d through transposed
        // reads of the swizzled rows, B = W^T [col][token]
        const int q16 = lane & 15;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int d0 = 16 * (w + 4 * t);
#pragma unroll
            for (int r = 0; r < 4; ++r) sacc[t][r] *= eLast;
#pragma unroll
            for (int ib = 0; ib < CH / 32; ++ib) {
                const int row = 32 * ib + 8 * g + (q16 >> 2), col = d0 + 4 * (q16 & 3);
                const int cb8 = col >> 3, co = col & 7;
                const bf16x8 kt = tr_pair(K + row * KD + 8 * (cb8 ^ (row % KBLK)) + co,
                                          K + (row + 4) * KD + 8 * (cb8 ^ ((row + 4) % KBLK)) + co);
                const int yo = c16 * CHH + 32 * ib + 8 * g;
                sacc[t] = mfma_bf(kt, *reinterpret_cast<const bf16x8*>(&Wt[0][yo]), sacc[t]);
                sacc[t] = mfma_bf(kt, *reinterpret_cast<const bf16x8*>(&Wt[1][yo]), sacc[t]);
            }
        }
        publish_state();   // every read of S^T was before the barrier after R

        // O = gamma qinv (Q_raw S) + QKm U
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = qs[r] * gqinv[16 * w + 4 * g + r];
#pragma unroll
        for (int kb = 0; kb < CH / 32; ++kb) {
            if (kb == 1 && w < 2) continue;   // QKm is zero past column 31 on rows < 32
            const bf16x8 mh = mat_a(M, kb), ml = mat_a(M + PMAT, kb);
            const int yo = c16 * CHH + 32 * kb + 8 * g;
            const bf16x8 uh = *reinterpret_cast<const bf16x8*>(&Ut[0][yo]);
            acc = mfma_bf(mh, uh, acc);
            acc = mfma_bf(mh, *reinterpret_cast<const bf16x8*>(&Ut[1][yo]), acc);
            acc = mfma_bf(ml, uh, acc);
        }
        store_out(chunk, acc);
    }
    wait_vmcnt_all();   // the last chunk's reload must land before the LDS is released
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            state[size_t(16 * (w + 4 * t) + 4 * g + r) * VD + col0 + c16] = sacc[t][r];
}


/*
    The two-level scan for long sequences (keyDim = valueDim = 128, bf16
    inputs on 16-byte boundaries). A chunk maps the state affinely,
      S' = M_c S + N_c,  M_c = e^{gc_last} I - K_raw^T diag(kdk) T diag(beta gamma kinv) K_raw,
    so a run of chunks maps it by S_end = A S_start + B, where B is the run
    from a zero state and A the same run over the 128 columns of the identity
    with zero values. Each value head's chunks are cut into P segments of L:
      pass A  delta_seg_kernel<false>, per (head, segment < P - 1): B of the
              segment and, from segment 1 on, its A (segment 0 starts from the
              given state, so its B is segment 1's start);
      join    delta_join_kernel, per (head, 16 columns): start(s + 1) =
              A_s start(s) + B_s for s = 1 .. P - 2;
      pass C  delta_seg_kernel<true>, per (head, segment): the segment's scan
              from its start state with the outputs; the last segment writes
              the final state.
    The serial chain is 2 L chunk steps and P - 2 products instead of P L
    chunk steps.

    A workgroup takes all 128 value columns of its head (pass A: and the 128
    identity columns), 16 per wave, so each wave owns whole columns of S and
    no product needs another wave's results: the chunk's inputs arrive by DMA
    into double buffers and one barrier per chunk hands them over. Every B
    operand is built in registers from the wave's own accumulators. For that,
    accumulator tile t (16 rows) holds the rows seg_row(t, m): lane (column,
    g) register r holds row seg_row(t, 4g + r), so the two tiles 2j and 2j + 1
    together hold rows 32j + 8g .. 32j + 8g + 7 in that lane, in order, which
    is what a B operand's lane holds for the contraction block j. The state's
    key rows and the chunk's token rows are both kept in this order; an A
    operand then reads 16 contiguous bytes of a row, the rows of its M side
    in the same order, and K^T's rows come from transposed reads of K whose
    lanes address the column groups of seg_row.
*/
constexpr int SEG_D = 128;                   // key and value dim of the two-level scan
constexpr int SEG_IMG = SEG_D * SEG_D;       // floats per state image

/* the row that position m (0..15) of accumulator tile t stands for */
__host__ __device__ constexpr int seg_row(int t, int m) {
    return 32 * (t >> 1) + 8 * (m >> 2) + 4 * (t & 1) + (m & 3);
}

struct SegArgs {
    DeltaArgs d;
    float* seg;          // per value head: 3 P state images
    uint32_t P, L;       // segments, chunks per segment
};

/* image slots of a head: 0 the given state, 1 + s segment s's B (s <= P - 2),
   P + s segment s's A (1 <= s <= P - 2, row-major), then the starts of
   segments 2 .. P - 1 (segment 1 starts at B_0). A state image is the
   accumulators as the waves hold them: float4 ((cb 8 + t) 64 + lane) is
   tile t of column block cb. */
__host__ __device__ constexpr uint32_t slot_b(uint32_t s) { return 1 + s; }
__host__ __device__ constexpr uint32_t slot_a(uint32_t P, uint32_t s) { return P + s; }
__host__ __device__ constexpr uint32_t slot_start(uint32_t P, uint32_t s) { return s == 0 ? 0 : s == 1 ? 1 : 2 * P - 1 + s; }
constexpr uint32_t SEG_SLOTS_PER_P = 3;

/* fp32 accumulator tiles x (slots 0-3) and y (slots 4-7) as one B operand:
   bf16 high parts and residuals */
__device__ __forceinline__ void split_pair(const floatx4& x, const floatx4& y, bf16x8& hi, bf16x8& lo) {
    bf16x4 hx, lx, hy, ly;
    split_bf16x4(x, hx, lx);
    split_bf16x4(y, hy, ly);
    const u32x2 a = __builtin_bit_cast(u32x2, hx), b = __builtin_bit_cast(u32x2, hy);
    const u32x2 c = __builtin_bit_cast(u32x2, lx), d = __builtin_bit_cast(u32x2, ly);
    hi = __builtin_bit_cast(bf16x8, u32x4{a[0], a[1], b[0], b[1]});
    lo = __builtin_bit_cast(bf16x8, u32x4{c[0], c[1], d[0], d[1]});
}

template <bool OUT>
__global__ __launch_bounds__(512, 1) void delta_seg_kernel(SegArgs sa) {
    constexpr int KD = SEG_D, VD = SEG_D;
    // 16-column blocks per wave: pass C one of the 8 value blocks; pass A two
    // of the 16 (waves 0-3 the value blocks, waves 4-7 the identity's)
    constexpr int NCB = OUT ? 1 : 2;
    constexpr uint32_t KBUF = CH * KD * 2, TBUF = 2 * PMAT_BYTES, SBUF = 2048;
    __shared__ __attribute__((aligned(16))) __bf16 Kb[2][CH * KD];
    __shared__ __attribute__((aligned(16))) __bf16 Vb[2][CH * VD];
    __shared__ __attribute__((aligned(16))) __bf16 Tb[2][2 * PMAT];
    __shared__ __attribute__((aligned(16))) float Sb[2][512];
    __shared__ __attribute__((aligned(16))) __bf16 Qb[OUT ? 2 : 1][OUT ? CH * KD : 8];
    // pass C: QKm's A operands for O, block p = (query tile i, key block jb)
    // formed by wave p: [p][hi, lo][lane] 16 bytes
    __shared__ __attribute__((aligned(16))) u32x4 Qm[OUT ? 6 : 1][2][64];

    const DeltaRuleParams& p = sa.d.p;
    const uint32_t P = sa.P, L = sa.L, nChunks = sa.d.nChunks;
    const uint32_t nSeg = OUT ? P : P - 1;
    const uint32_t h = blockIdx.x / nSeg, sg = blockIdx.x % nSeg;
    const uint32_t kh = uint32_t(h / (p.valueHeads / p.keyHeads));
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c16 = lane & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool hom = !OUT && w >= 4;                   // a wave of identity columns
    // the wave's value (or identity) columns: block cbOf(b) of 8, column colOf(b)
    auto cbOf = [&](int b) { return (NCB * w + b) & 7; };
    auto colOf = [&](int b) { return 16 * cbOf(b) + c16; };
    const uint32_t c0 = sg * L, c1 = min(c0 + L, nChunks);
    const size_t Hv = p.valueHeads;
    float* const img = sa.seg + size_t(h) * SEG_SLOTS_PER_P * P * SEG_IMG;
    auto img_tile = [&](uint32_t slot, int b, int t) -> floatx4* {
        return reinterpret_cast<floatx4*>(img + size_t(slot) * SEG_IMG + size_t((cbOf(b) * 8 + t) * 64 + lane) * 4);
    };

    // S: tile t of block b holds key rows seg_row(t, 4g + r) of column colOf(b)
    floatx4 s[NCB][8];
#pragma unroll
    for (int b = 0; b < NCB; ++b) {
        if (OUT) {
#pragma unroll
            for (int t = 0; t < 8; ++t) s[b][t] = *img_tile(slot_start(P, sg), b, t);
        } else if (hom) {
#pragma unroll
            for (int t = 0; t < 8; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) s[b][t][r] = seg_row(t, 4 * g + r) == colOf(b) ? 1.0f : 0.0f;
        } else if (sg == 0) {
            const float* st = p.state + size_t(h) * KD * VD;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
#pragma unroll
                for (int r = 0; r < 4; ++r) s[b][t][r] = st[size_t(seg_row(t, 4 * g + r)) * VD + colOf(b)];
                *img_tile(0, b, t) = s[b][t];
            }
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) s[b][t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }

    // DMA of a chunk in 1 KB blocks, the same kinds on every wave: k (and q)
    // blocks 2w, 2w + 1, value blocks 2w, 2w + 1, T blocks w and, for w < 4,
    // w + 8, scalar block w < 2. Row blocks carry rows 4 j + lane
    // / 16 with 16-byte slot lane % 16 holding the row's block slot ^ (row %
    // 16); rows past a partial chunk's end repeat its last row (whose beta is 0).
    const uint32_t rowBytes = uint32_t(p.keyHeads * KD * 2), vRowBytes = uint32_t(Hv * VD * 2);
    const uint32_t ldsK = lds_address(Kb), ldsV = lds_address(Vb), ldsT = lds_address(Tb), ldsS = lds_address(Sb);
    const uint32_t ldsQ = lds_address(Qb);
    const uint32_t lr = uint32_t(lane >> 4), ls = uint32_t(lane & 15), l16 = 16 * uint32_t(lane);
    struct Src {
        const uint8_t *k, *q, *v, *rec;
        uint32_t n, buf;
    };
    auto src_of = [&](uint32_t chunk, uint32_t buf) __attribute__((always_inline)) {
        const uint64_t t0 = uint64_t(chunk) * CH;
        const uint32_t n = uint32_t(p.count - t0 < CH ? p.count - t0 : CH);
        return Src{static_cast<const uint8_t*>(p.k) + t0 * rowBytes + kh * KD * 2,
                   static_cast<const uint8_t*>(p.q) + t0 * rowBytes + kh * KD * 2,
                   static_cast<const uint8_t*>(p.v) + (t0 * Hv + h) * VD * 2,
                   reinterpret_cast<const uint8_t*>(sa.d.work + (size_t(h) * nChunks + chunk) * WORK_SPLIT), n, buf};
    };
    auto row_off = [&](const Src& x, uint32_t j, uint32_t stride) __attribute__((always_inline)) -> uint32_t {
        const uint32_t row = 4 * j + lr;
        return min(row, x.n - 1) * stride + 16 * (ls ^ (row & 15));
    };
    auto dma_part = [&](const Src& x, int part) __attribute__((always_inline)) {
        const uint32_t bk = x.buf * KBUF, bt = x.buf * TBUF;
        if (part == 0) {
#pragma unroll
            for (uint32_t e = 0; e < 2; ++e) {
                const uint32_t j = 2 * uint32_t(w) + e;
                const uint32_t off = row_off(x, j, rowBytes);
                dma_block(x.k, off, ldsK + bk + j * 1024);
                if constexpr (OUT) dma_block(x.q, off, ldsQ + bk + j * 1024);
            }
        } else if (part == 1) {
            dma_block(x.rec + w * 1024, l16, ldsT + bt + w * 1024);
            if (w < 4) dma_block(x.rec + (w + 8) * 1024, l16, ldsT + bt + (w + 8) * 1024);
            if (w < 2) dma_block(x.rec + 2 * TBUF + w * 1024, l16, ldsS + x.buf * SBUF + w * 1024);
        } else {
#pragma unroll
            for (uint32_t e = 0; e < 2; ++e) {
                const uint32_t j = 2 * uint32_t(w) + e;
                dma_block(x.v, row_off(x, j, vRowBytes), ldsV + bk + j * 1024);
            }
        }
    };
    {
        const Src first = src_of(c0, 0);
        dma_part(first, 0);
        dma_part(first, 1);
        dma_part(first, 2);
    }
    const uint32_t oStride = uint32_t(Hv * VD * 4);      // bytes between output rows

    // The lane's LDS byte offsets within a buffer, held across the loop.
    // Tiles i and i + 2 (token rows 32 apart) and the two token-row blocks of
    // a K^T read share a row's swizzle, so they differ by immediates.
    uint32_t kOff[2][4];   // k/q A operand: token row seg_row(i, c16), block 4j + g
    uint32_t tOff[4][2];   // T/QKm A operand: token row seg_row(i, c16), block 4jb + g
    uint32_t vOff[NCB][2][4];   // value of token row 8g + 4 (i & 1) + r, column colOf(b)
    uint32_t trOff[8][2];  // K^T: token row 8g + c16 / 4 (+ 4), key columns seg_row(t, 4 (c16 % 4)) ..
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = seg_row(i, c16);
#pragma unroll
        for (int j = 0; j < 4; ++j) kOff[i][j] = uint32_t(r * KD + 8 * ((4 * j + g) ^ (r & 15))) * 2;
#pragma unroll
        for (int b = 0; b < NCB; ++b)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int row = 8 * g + 4 * i + rr, cc = colOf(b);
                vOff[b][i][rr] = uint32_t(row * VD + 8 * ((cc >> 3) ^ (row & 15)) + (cc & 7)) * 2;
            }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jb = 0; jb < 2; ++jb)
            tOff[i][jb] = (jb == 1 && i < 2) ? 0u : uint32_t(pmat_offset(seg_row(i, c16), 4 * jb + g)) * 2;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const int kc = seg_row(t, 4 * (c16 & 3));
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int r = 8 * g + (c16 >> 2) + 4 * e;
            trOff[t][e] = uint32_t(r * KD + 8 * ((kc >> 3) ^ (r & 15)) + (kc & 7)) * 2;
        }
    }
    auto lds_at = [](const void* base, uint32_t bytes) __attribute__((always_inline)) {
        return reinterpret_cast<const uint8_t*>(base) + bytes;
    };

    for (uint32_t c = c0; c < c1; ++c) {
        const uint32_t par = (c - c0) & 1;
        // this chunk's inputs have landed; every read of the other buffers is done
        wait_vmcnt_all();
        __syncthreads();
        const bool more = c + 1 < c1;
        const Src nx = src_of(more ? c + 1 : c, par ^ 1);
        const __bf16* K = Kb[par];
        const __bf16* V = Vb[par];
        const __bf16* T = Tb[par];
        const float* sc = Sb[par];
        if (more) dma_part(nx, 0);

        // R = K_raw S and, for the output, Q_raw S: A rows seg_row(i, c16),
        // 16-byte block 4j + g; each A fragment serves the wave's blocks. In
        // pass C, wave w < 6 also forms block w = (query tile i, key block jb)
        // of QKm from the same fragments: D(jt, i) = K_raw Q_raw^T over key
        // tiles jt = 2jb, 2jb + 1 (exact bf16 products), whose lane (query
        // seg_row(i, c16), g) holds the keys 32 jb + 8g .. + 7 that the A
        // operand of QKm U needs in that lane.
        constexpr int PI[6] = {0, 1, 2, 2, 3, 3}, PJB[6] = {0, 0, 0, 1, 0, 1};
        floatx4 ra[NCB][4], qa[4], d0 = {0.0f, 0.0f, 0.0f, 0.0f}, d1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            qa[i] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int b = 0; b < NCB; ++b) ra[b][i] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bf16x8 sh[NCB], sl[NCB];
#pragma unroll
            for (int b = 0; b < NCB; ++b) split_pair(s[b][2 * j], s[b][2 * j + 1], sh[b], sl[b]);
            bf16x8 x[4], xq[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t o = kOff[i & 1][j] + uint32_t(i >> 1) * 32 * KD * 2;
                x[i] = *reinterpret_cast<const bf16x8*>(lds_at(K, o));
                if constexpr (OUT) xq[i] = *reinterpret_cast<const bf16x8*>(lds_at(Qb[par], o));
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int b = 0; b < NCB; ++b) {
                    ra[b][i] = mfma_bf(x[i], sh[b], ra[b][i]);
                    ra[b][i] = mfma_bf(x[i], sl[b], ra[b][i]);
                }
                if constexpr (OUT) {
                    qa[i] = mfma_bf(xq[i], sh[0], qa[i]);
                    qa[i] = mfma_bf(xq[i], sl[0], qa[i]);
                }
            }
            if constexpr (OUT) {
#pragma unroll
                for (int pb = 0; pb < 6; ++pb)
                    if (pb == w) {
                        d0 = mfma_bf(x[2 * PJB[pb]], xq[PI[pb]], d0);
                        d1 = mfma_bf(x[2 * PJB[pb] + 1], xq[PI[pb]], d1);
                    }
            }
        }
        // QKm_ij = D_ji 2^(a_i - b_j) for keys j <= query i (the solve's
        // factors a and b carry the decays and the inverse norms), split and
        // published for every wave's output
        if constexpr (OUT) {
            if (w < 6) {
#pragma unroll
                for (int pb = 0; pb < 6; ++pb)
                    if (pb == w) {
                        const int i = PI[pb], jb = PJB[pb], qrow = seg_row(i, c16);
                        const bool diag = (i >> 1) == jb;   // keys past the query are masked
                        const float ai = sc[5 * CH + qrow];
                        const floatx4 bj0 = *reinterpret_cast<const floatx4*>(sc + 6 * CH + 32 * jb + 8 * g);
                        const floatx4 bj1 = *reinterpret_cast<const floatx4*>(sc + 6 * CH + 32 * jb + 8 * g + 4);
                        floatx4 m0, m1;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int k0 = 32 * jb + 8 * g + e, k1 = k0 + 4;
                            m0[e] = d0[e] * __builtin_amdgcn_exp2f(diag && k0 > qrow ? -INFINITY : ai - bj0[e]);
                            m1[e] = d1[e] * __builtin_amdgcn_exp2f(diag && k1 > qrow ? -INFINITY : ai - bj1[e]);
                        }
                        bf16x8 mh, ml;
                        split_pair(m0, m1, mh, ml);
                        Qm[pb][0][lane] = __builtin_bit_cast(u32x4, mh);
                        Qm[pb][1][lane] = __builtin_bit_cast(u32x4, ml);
                    }
            }
        }
        __builtin_amdgcn_sched_barrier(0);   // phases keep their own operands live
        // R = beta (V - gamma kinv R): tile i register r is token row
        // seg_row(i, 4g + r) = b + r with b = 32 (i >> 1) + 4 (i & 1) + 8g
        bf16x8 rh[NCB][2], rl[NCB][2];
#pragma unroll
        for (int b = 0; b < NCB; ++b) {
            floatx4 rv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int rb = seg_row(i, 4 * g);
                const floatx4 be = *reinterpret_cast<const floatx4*>(sc + rb);
                const floatx4 gk = *reinterpret_cast<const floatx4*>(sc + CH + rb);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float v = hom ? 0.0f
                                        : float(*reinterpret_cast<const __bf16*>(
                                              lds_at(V, vOff[b][i & 1][r] + uint32_t(i >> 1) * 32 * VD * 2)));
                    rv[i][r] = be[r] * (v - gk[r] * ra[b][i][r]);
                }
            }
            split_pair(rv[0], rv[1], rh[b][0], rl[b][0]);
            split_pair(rv[2], rv[3], rh[b][1], rl[b][1]);
        }
        if (more) dma_part(nx, 1);
        __builtin_amdgcn_sched_barrier(0);

        // U = T R (token rows < 32 have no nonzero T past column 31)
        floatx4 u[NCB][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int b = 0; b < NCB; ++b) u[b][i] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int jb = 0; jb < 2; ++jb) {
                if (jb == 1 && i < 2) continue;
                const bf16x8 th = *reinterpret_cast<const bf16x8*>(lds_at(T, tOff[i][jb]));
                const bf16x8 tl = *reinterpret_cast<const bf16x8*>(lds_at(T, tOff[i][jb] + PMAT_BYTES));
#pragma unroll
                for (int b = 0; b < NCB; ++b) {
                    u[b][i] = mfma_bf(th, rh[b][jb], u[b][i]);
                    u[b][i] = mfma_bf(th, rl[b][jb], u[b][i]);
                    u[b][i] = mfma_bf(tl, rh[b][jb], u[b][i]);
                }
            }
        }
        // W = diag(kinv e^{gc_last - gc}) U
        bf16x8 wh[NCB][2], wl[NCB][2];
#pragma unroll
        for (int b = 0; b < NCB; ++b) {
            floatx4 wv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) wv[i] = *reinterpret_cast<const floatx4*>(sc + 3 * CH + seg_row(i, 4 * g)) * u[b][i];
            split_pair(wv[0], wv[1], wh[b][0], wl[b][0]);
            split_pair(wv[2], wv[3], wh[b][1], wl[b][1]);
        }
        if (more) dma_part(nx, 2);
        __builtin_amdgcn_sched_barrier(0);

        // O = gamma qinv (Q_raw S) + QKm U, before S moves on; row b0 + r of
        // the output leaves from a uniform row address plus the lane's offset
        if constexpr (OUT) {
            bf16x8 uh[2], ul[2];
            split_pair(u[0][0], u[0][1], uh[0], ul[0]);
            split_pair(u[0][2], u[0][3], uh[1], ul[1]);
            const uint64_t t0 = uint64_t(c) * CH;
            const uint32_t n = uint32_t(p.count - t0 < CH ? p.count - t0 : CH);
            uint8_t* const ob = reinterpret_cast<uint8_t*>(p.out + (t0 * Hv + h) * VD);
            const uint32_t laneOff = uint32_t(8 * g) * oStride + uint32_t(colOf(0)) * 4;
            lds_barrier();   // every wave's QKm block is published
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int b0 = seg_row(i, 0);
                floatx4 o = *reinterpret_cast<const floatx4*>(sc + 2 * CH + b0 + 8 * g) * qa[i];
#pragma unroll
                for (int jb = 0; jb < 2; ++jb) {
                    if (jb == 1 && i < 2) continue;
                    const int pb = i < 2 ? i : 2 * i - 2 + jb;
                    const bf16x8 mh = __builtin_bit_cast(bf16x8, Qm[pb][0][lane]);
                    const bf16x8 ml = __builtin_bit_cast(bf16x8, Qm[pb][1][lane]);
                    o = mfma_bf(mh, uh[jb], o);
                    o = mfma_bf(mh, ul[jb], o);
                    o = mfma_bf(ml, uh[jb], o);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float* dst = reinterpret_cast<float*>(ob + size_t(b0 + r) * oStride + laneOff);
                    if (n == CH || uint32_t(b0 + 8 * g + r) < n) __builtin_nontemporal_store(o[r], dst);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);

        // S' = e^{gc_last} S + K_raw^T W. The transposed read of 16 lanes
        // (c16 = 4a + e) returns to lane m the 8-byte column group that lane
        // 4k + m / 4 addressed, element m % 4, for rows k = 0..3: lane c16
        // addresses token row 32 ib + 8g + c16 / 4 (and + 4), key columns
        // seg_row(t, 4 (c16 % 4)) .. + 3, so lane m receives key row
        // seg_row(t, m) over the token rows of the B operand's block ib
        const float eLast = sc[4 * CH];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
#pragma unroll
            for (int b = 0; b < NCB; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r) s[b][t][r] *= eLast;
#pragma unroll
            for (int ib = 0; ib < 2; ++ib) {
                const uint32_t ro = uint32_t(ib) * 32 * KD * 2;
                const bf16x8 kt = tr_pair(reinterpret_cast<const __bf16*>(lds_at(K, trOff[t][0] + ro)),
                                          reinterpret_cast<const __bf16*>(lds_at(K, trOff[t][1] + ro)));
#pragma unroll
                for (int b = 0; b < NCB; ++b) {
                    s[b][t] = mfma_bf(kt, wh[b][ib], s[b][t]);
                    s[b][t] = mfma_bf(kt, wl[b][ib], s[b][t]);
                }
            }
        }
    }
    wait_vmcnt_all();   // no DMA may still be landing when the LDS is released

#pragma unroll
    for (int b = 0; b < NCB; ++b) {
        if constexpr (OUT) {
            if (sg == P - 1) {
                float* st = p.state + size_t(h) * KD * VD;
#pragma unroll
                for (int t = 0; t < 8; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r) st[size_t(seg_row(t, 4 * g + r)) * VD + colOf(b)] = s[b][t][r];
            }
        } else if (!hom) {
#pragma unroll
            for (int t = 0; t < 8; ++t) *img_tile(slot_b(sg), b, t) = s[b][t];
        } else if (sg >= 1) {
            float* A = img + size_t(slot_a(P, sg)) * SEG_IMG;
#pragma unroll
            for (int t = 0; t < 8; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) A[seg_row(t, 4 * g + r) * SEG_D + colOf(b)] = s[b][t][r];
        }
    }
}

/*
    The join of the two-level scan, per (value head, 16 columns): start(s + 1)
    = A_s start(s) + B_s for s = 1 .. P - 2, from start(1) = B_0. Wave w
    computes tiles 2w and 2w + 1, key rows 32 w .. 32 w + 31, which are the
    32-row block w of the next product's contraction: it publishes their
    split in LDS for the other waves. The next step's A rows and B tiles are
    loaded while this step multiplies.
*/
__global__ __launch_bounds__(256) void delta_join_kernel(SegArgs sa) {
    const uint32_t P = sa.P, Hv = uint32_t(sa.d.p.valueHeads);
    // a head's 8 workgroups read the same A and B images: with the heads a
    // multiple of 8, they share blockIdx % 8 and so one XCD's L2
    const uint32_t h = Hv % 8 == 0 ? blockIdx.x % Hv : blockIdx.x / 8;
    const uint32_t cb = Hv % 8 == 0 ? blockIdx.x / Hv : blockIdx.x % 8;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c16 = lane & 15;
    const int w = tid >> 6;
    __shared__ __attribute__((aligned(16))) u32x4 Bs[2][4][2][64];   // [buffer][block][hi, lo][lane]
    float* const img = sa.seg + size_t(h) * SEG_SLOTS_PER_P * P * SEG_IMG;
    auto tile = [&](uint32_t slot, int t) -> floatx4* {
        return reinterpret_cast<floatx4*>(img + size_t(slot) * SEG_IMG + size_t((cb * 8 + t) * 64 + lane) * 4);
    };
    // wave w's A rows of step s: seg_row(2w + tt, c16), contraction columns 32 j + 8 g .. + 7
    struct Step {
        floatx4 a[2][4][2];
        floatx4 b[2];
    };
    auto load_step = [&](uint32_t s, Step& st) __attribute__((always_inline)) {
        const float* A = img + size_t(slot_a(P, s)) * SEG_IMG;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float* row = A + seg_row(2 * w + tt, c16) * SEG_D + 32 * j + 8 * g;
                st.a[tt][j][0] = *reinterpret_cast<const floatx4*>(row);
                st.a[tt][j][1] = *reinterpret_cast<const floatx4*>(row + 4);
            }
        st.b[0] = *tile(slot_b(s), 2 * w);
        st.b[1] = *tile(slot_b(s), 2 * w + 1);
    };
    floatx4 x0 = *tile(slot_b(0), 2 * w), x1 = *tile(slot_b(0), 2 * w + 1);
    // steps s = 1 .. P - 2; step s's loads are issued two steps ahead into a
    // ring of three named buffers (no copies, so nothing waits for them
    // before their use), and the barrier waits only for LDS
    auto step = [&](uint32_t s, const Step& cur, Step& fill) __attribute__((always_inline)) {
        const int buf = s & 1;
        {
            bf16x8 hi, lo;
            split_pair(x0, x1, hi, lo);
            Bs[buf][w][0][lane] = __builtin_bit_cast(u32x4, hi);
            Bs[buf][w][1][lane] = __builtin_bit_cast(u32x4, lo);
        }
        lds_barrier();
        if (s + 2 <= P - 2) load_step(s + 2, fill);
        x0 = cur.b[0];
        x1 = cur.b[1];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bf16x8 bh = __builtin_bit_cast(bf16x8, Bs[buf][j][0][lane]);
            const bf16x8 bl = __builtin_bit_cast(bf16x8, Bs[buf][j][1][lane]);
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                bf16x8 ah, al;
                split_pair(cur.a[tt][j][0], cur.a[tt][j][1], ah, al);
                floatx4& acc = tt ? x1 : x0;
                acc = mfma_bf(ah, bh, acc);
                acc = mfma_bf(ah, bl, acc);
                acc = mfma_bf(al, bh, acc);
            }
        }
        *tile(slot_start(P, s + 1), 2 * w) = x0;
        *tile(slot_start(P, s + 1), 2 * w + 1) = x1;
    };
    Step r0, r1, r2;
    if (P > 2) load_step(1, r0);
    if (P > 3) load_step(2, r1);
    for (uint32_t s = 1; s + 1 < P; s += 3) {
        step(s, r0, r2);
        if (s + 2 < P) step(s + 1, r1, r0);
        if (s + 3 < P) step(s + 2, r2, r1);
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
    auto aligned = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    a.vec = aligned(p.q) && aligned(p.k) && aligned(p.v) ? 1u : 0u;
    // bf16 inputs on 16-byte boundaries take the DMA scan, whose records are
    // the split form; fp32 and unaligned bf16 inputs take the register-staged
    // scans over fp32 records
    // (its per-lane DMA and store offsets within a chunk are 32-bit)
    const bool dma = p.inType == 1 && a.vec && uint64_t(CH) * p.keyHeads * p.keyDim * 2 < (1ull << 31) &&
                     uint64_t(CH) * p.valueHeads * p.valueDim * 4 < (1ull << 31);
    const size_t rec = dma ? WORK_SPLIT : WORK;
    a.work = static_cast<float*>(ctx.grow(SLOT_DELTA_WORK, size_t(p.valueHeads) * a.nChunks * rec * sizeof(float)));
    if (!a.work) return false;

    const dim3 sgrid(a.nChunks, unsigned(p.keyHeads));
    const dim3 grid{unsigned(p.valueHeads * (p.valueDim / NB))}, block{256};

    // 128 x 128 heads over many chunks: the two-level scan, P segments per
    // head so that pass C runs about one workgroup per CU, each segment at
    // least 8 chunks long
    uint32_t segP = 0, segL = 0;
    if (dma && p.keyDim == SEG_D && p.valueDim == SEG_D && ctx.cus > 0) {
        const uint64_t want = std::min<uint64_t>(16, uint64_t(ctx.cus) / p.valueHeads);
        if (want >= 3 && a.nChunks >= 8 * want) {
            segL = uint32_t((a.nChunks + want - 1) / want);
            segP = (a.nChunks + segL - 1) / segL;
        }
    }
    if (segP) {
        SegArgs sa{a, nullptr, segP, segL};
        sa.seg = static_cast<float*>(
            ctx.grow(SLOT_DELTA_SEG, size_t(p.valueHeads) * SEG_SLOTS_PER_P * segP * SEG_IMG * sizeof(float)));
        if (!sa.seg) return false;
        const unsigned Hv = unsigned(p.valueHeads);
        return ctx.launch("delta_solve_kernel", stream,
                          [&] { hipLaunchKernelGGL((delta_solve_kernel<128, false, true, false>), sgrid, dim3(256), 0, stream, a); }) &&
               ctx.launch("delta_seg_kernel<false>", stream,
                          [&] { hipLaunchKernelGGL(delta_seg_kernel<false>, dim3(Hv * (segP - 1)), dim3(512), 0, stream, sa); }) &&
               (segP < 3 || ctx.launch("delta_join_kernel", stream, [&] {
                    hipLaunchKernelGGL(delta_join_kernel, dim3(Hv * 8), dim3(256), 0, stream, sa);
                })) &&
               ctx.launch("delta_seg_kernel<true>", stream,
                          [&] { hipLaunchKernelGGL(delta_seg_kernel<true>, dim3(Hv * segP), dim3(512), 0, stream, sa); });
    }
#define AIGPU_DELTA(KD)                                                                                        \
    if (p.keyDim == KD) {                                                                                      \
        if (!ctx.launch("delta_solve_kernel", stream, [&] {                                                    \
                if (p.inType == 0)                                                                             \
                    hipLaunchKernelGGL((delta_solve_kernel<KD, true, false>), sgrid, dim3(256), 0, stream, a);  \
                else if (dma)                                                                                  \
                    hipLaunchKernelGGL((delta_solve_kernel<KD, false, true>), sgrid, dim3(256), 0, stream, a);  \
                else                                                                                           \
                    hipLaunchKernelGGL((delta_solve_kernel<KD, false, false>), sgrid, dim3(256), 0, stream, a); \
            }))                                                                                                \
            return false;                                                                                      \
        return ctx.launch("delta_scan_kernel", stream, [&] {                                                   \
            if (p.inType == 0 && a.vec)                                                                        \
                hipLaunchKernelGGL((delta_scan_f32_kernel<KD, true>), grid, block, 0, stream, a);              \
            else if (p.inType == 0)                                                                            \
                hipLaunchKernelGGL((delta_scan_f32_kernel<KD, false>), grid, block, 0, stream, a);             \
            else if (dma)                                                                                      \
                hipLaunchKernelGGL((delta_scan_dma_kernel<KD>), grid, block, 0, stream, a);                    \
            else                                                                                               \
                hipLaunchKernelGGL((delta_scan_kernel<KD, false>), grid, block, 0, stream, a);                 \
        });                                                                                                    \
    }
    AIGPU_DELTA(128)
    AIGPU_DELTA(64)
#undef AIGPU_DELTA
    return ctx.fail("delta rule: unsupported configuration");
}

} // namespace aigpu
