// prefill.hip - causal GQA prefill for gfx950.
//
// Three launches per call:
//   prefill_history_kernel  converts cached positions [0, start) of the bf16
//                           cache to the fp16 working copies (exact for every
//                           bf16 value in fp16's range; the rest raise the
//                           range flag)
//   prefill_prep_kernel     attentionMixer's QK-RMSNorm -> RoPE -> KV append
//                           (LocalModel.hpp:2608-2655) for the new tokens, in
//                           fp32; writes the bf16 cache and the fp16 copies
//   prefill_flash_kernel    flash attention on v_mfma_f32_32x32x16_f16 with
//                           fp32 accumulation and an online softmax
//
// Why fp16 operands: Q, K and P rounded to bf16 (8 significant bits) give
// max-abs errors near 6e-3 on the 8k configuration; fp16 (11 bits) keeps
// them near 1.4e-3, inside the 2e-3 bound, at the same MFMA rate. The KV
// cache itself stays bf16. Every conversion into fp16 is checked
// (to_f16_checked): a finite value that overflows sets the caller's range
// flag and the entry point fails instead of returning inf / NaN.
//
// Flash kernel layout (one workgroup = 8 waves = 256 query rows of one head,
// one wave = 32 rows; key tiles of 128, DMA'd into LDS):
//   S^T = K Q^T     A = K rows (LDS), B = Q^T (registers, loaded once, already
//                   scaled by log2(e)/sqrt(D) so the softmax is exp2 of it)
//                   -> each lane owns one query (lane % 32) and 16 keys, so
//                      the row max/sum need one exchange with lane ^ 32
//   O^T += V^T P^T  A = V^T read straight from row-major V through
//                      ds_read_b64_tr_b16, B = P^T straight from the S^T
//                      accumulators -> the softmax rescale of O is lane-local
// The K tile rows are stored permuted so that accumulator register r of the
// S^T tile holds key 16*(lane/32) + r, which makes each lane's 8-key slice of
// P^T 8 consecutive keys.
//
// Ping-pong schedule (the default for D = 128): waves 0-3 and 4-7 share the
// four SIMDs pairwise and run a tile interval apart, so while one wave of a
// pair issues MFMAs (PV of the previous tile, then QK of this one, at a
// raised wave priority) its partner runs the softmax on the VALU; each group
// issues DMA between its softmax steps (waves 4-7 the next K tile, waves 0-3
// the next V tile; K is double- and V triple-buffered, 160 KB of LDS). The
// running max is folded into the score accumulators' initial value and
// rescaling is lazy (only when the max grows by more than 8 in log2 units).
// D = 64 takes the single-phase loop: every wave computes S, the softmax and
// P.V of each tile in turn, one barrier per tile.
#include "context.hpp"
#include "device.hpp"
#include "kernels.hpp"

#include <type_traits>

namespace aigpu {

namespace {

constexpr int PREP_MAX_DIM = 256;

/* zero the pad rows that follow the last kv head's working rows: reads of
   the flash kernel's last tile run past a head's rows into the next head's
   (finite) rows, or, for the last head, into these */
__device__ __forceinline__ void zero_pad_rows(_Float16* kh, _Float16* vh, uint64_t padAt, uint32_t dim) {
    const uint32_t n8 = PREFILL_PAD_ROWS * dim / 8;
    for (uint32_t i = threadIdx.x; i < n8; i += blockDim.x) {
        reinterpret_cast<half8*>(kh + padAt)[i] = half8{0, 0, 0, 0, 0, 0, 0, 0};
        reinterpret_cast<half8*>(vh + padAt)[i] = half8{0, 0, 0, 0, 0, 0, 0, 0};
    }
}

/* grid.y = kv head; each kv head's history [0, start) is one contiguous run */
__global__ __launch_bounds__(256) void prefill_history_kernel(
    const uint16_t* __restrict__ keyCache, const uint16_t* __restrict__ valueCache,
    _Float16* __restrict__ kh, _Float16* __restrict__ vh, uint32_t per, uint64_t capacity,
    uint64_t dim, uint64_t T, uint32_t* rangeFlag) {
    const uint64_t kv = blockIdx.y;
    const uint16_t* ks = keyCache + kv * capacity * dim;
    const uint16_t* vs = valueCache + kv * capacity * dim;
    _Float16* kd = kh + kv * T * dim;
    _Float16* vd = vh + kv * T * dim;
    bool bad = false;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < per; i += gridDim.x * blockDim.x) {
        kd[i] = to_f16_checked(bf16_bits_to_float(ks[i]), bad);
        vd[i] = to_f16_checked(bf16_bits_to_float(vs[i]), bad);
    }
    raise_range_flag(rangeFlag, bad);
}

/* one workgroup per token: the token's q, k, v rows are staged in LDS with all
   loads in flight at once, its RoPE cos/sin are computed once for every row,
   then one wave per row normalises, rotates and writes */
__global__ __launch_bounds__(256) void prefill_prep_kernel(PrefillParams p, _Float16* __restrict__ qh,
                                                           _Float16* __restrict__ kh,
                                                           _Float16* __restrict__ vh, uint64_t T,
                                                           float qScale) {
    extern __shared__ float tok[];   // [heads + 2 kvHeads][dim]
    __shared__ float cs[PREP_MAX_DIM / 2], sn[PREP_MAX_DIM / 2];
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid / WAVE;
    const uint64_t t = blockIdx.x, pos = p.start + t;
    const int dim = int(p.dim), half = p.rotaryDims / 2;
    const uint64_t H = p.heads, KVH = p.kvHeads;

    if (blockIdx.x == 0) zero_pad_rows(kh, vh, KVH * T * p.dim, uint32_t(p.dim));
    const uint32_t shift = __builtin_ctz(uint32_t(p.dim));   // dim is 64 or 128
    const uint32_t nq = uint32_t(H) << shift, nk = uint32_t(KVH) << shift;
    const size_t qrow = t * H * p.qStride, krow = t * nk;
    const uint32_t nrows = p.kvReady ? nq : nq + 2 * nk;   // kvReady: the k, v rows are already written
    for (uint32_t i = tid; i < nrows; i += 256) {
        float x;
        if (i < nq) x = load_elem(p.q, qrow + size_t(i >> shift) * p.qStride + (i & (uint32_t(p.dim) - 1)), p.inType);
        else if (i < nq + nk) x = load_elem(p.k, krow + (i - nq), p.inType);
        else x = load_elem(p.v, krow + (i - nq - nk), p.inType);
        tok[i] = x;
    }
    if (p.freqs) {
        const float fpos = float(pos);   // the reference's fp32 angle (LocalModel.hpp:2632)
        for (int j = tid; j < half; j += 256) sincosf(fpos * p.freqs[j], &sn[j], &cs[j]);
    }
    __syncthreads();

    bool bad = false;   // an fp16 conversion out of range
    for (uint64_t h = w; h < (p.kvReady ? H : H + 2 * KVH); h += 4) {
        float* x = tok + h * p.dim;
        const bool isQuery = h < H, isKey = !isQuery && h < H + KVH;
        if (isQuery || isKey) {
            const float* gamma = isQuery ? p.qNorm : p.kNorm;
            if (gamma) {   // rmsNormRow (LocalModel.hpp:1341-1348)
                float ss = 0.0f;
                for (int d = lane; d < dim; d += WAVE) ss += x[d] * x[d];
                ss = wave_sum(ss);
                const float inv = 1.0f / sqrtf(ss / float(dim) + p.eps);
                for (int d = lane; d < dim; d += WAVE) x[d] = x[d] * inv * (gamma[d] + p.normOffset);
                wave_sync();
            }
            if (p.freqs) {   // rotate-half pairs (LocalModel.hpp:2636-2641)
                for (int j = lane; j < half; j += WAVE) {
                    const float a = x[j], b = x[j + half];
                    x[j] = a * cs[j] - b * sn[j];
                    x[j + half] = b * cs[j] + a * sn[j];
                }
                wave_sync();
            }
        }
        if (isQuery) {
            _Float16* dst = qh + (h * p.count + t) * p.dim;
            for (int d = lane; d < dim; d += WAVE) dst[d] = to_f16_checked(x[d] * qScale, bad);
        } else {
            const uint64_t kv = isKey ? h - H : h - H - KVH;
            const uint64_t work = (kv * T + pos) * p.dim;
            const uint64_t cache = (kv * p.capacity + pos) * p.dim;
            _Float16* wdst = isKey ? kh : vh;
            uint16_t* cdst = isKey ? p.keyCache : p.valueCache;
            for (int d = lane; d < dim; d += WAVE) {
                wdst[work + d] = to_f16_checked(x[d], bad);
                cdst[cache + d] = float_to_bf16_bits(x[d]);
            }
        }
    }
    raise_range_flag(p.rangeFlag, bad);
}

/* 8 consecutive input elements, widened to fp32 (16 B of bf16 or 32 B of f32) */
template <bool F32>
__device__ __forceinline__ void load8(const void* base, size_t i, float (&x)[8]) {
    if (F32) {
        const floatx4* s = reinterpret_cast<const floatx4*>(static_cast<const float*>(base) + i);
        const floatx4 a = s[0], b = s[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) { x[e] = a[e]; x[4 + e] = b[e]; }
    } else {
        const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[2 * e] = __uint_as_float(w[e] << 16);
            x[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
        }
    }
}

__device__ __forceinline__ void store8_f16(_Float16* dst, const float (&x)[8], float scale, bool& bad) {
    half8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = to_f16_checked(x[e] * scale, bad);
    *reinterpret_cast<half8*>(dst) = h;
}

__device__ __forceinline__ void store8_bf16(uint16_t* dst, const float (&x)[8]) {
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        w[e] = uint32_t(float_to_bf16_bits(x[2 * e])) | (uint32_t(float_to_bf16_bits(x[2 * e + 1])) << 16);
    *reinterpret_cast<u32x4*>(dst) = w;
}

/*
    The same work as prefill_prep_kernel with every row held in registers:
    one workgroup of one wave per token, D/8 lanes per row, 8 consecutive
    elements per lane (one 16-byte load of bf16). The RMS sum is a butterfly
    over the row's lanes; the rotate-half partner of element e (e +- rot/2)
    sits in lane +- rot/16 at the same slot, which needs rot % 16 == 0. Each
    lane takes four rows at a time with all four loads issued before any
    arithmetic (a wave per token measured ~1% faster over the cfg3 step than
    four waves per token, which left three of them idle in the sin/cos).
*/
constexpr int PREP_THREADS = 64;   // one wave per token: its rows four at a time per lane

template <int D, bool F32>
__global__ __launch_bounds__(PREP_THREADS) void prefill_prep_vec_kernel(PrefillParams p, _Float16* __restrict__ qh,
                                                                        _Float16* __restrict__ kh,
                                                                        _Float16* __restrict__ vh, uint32_t T,
                                                                        float qScale, uint32_t firstRow,
                                                                        float* __restrict__ rope) {
    static_assert(PREP_THREADS >= D / 2, "one thread per rotary pair");
    constexpr int LPR = D / 8, RPP = PREP_THREADS / LPR, UNROLL = 4;
    __shared__ float cs[D / 2], sn[D / 2];
    const int tid = threadIdx.x, sub = tid % LPR, lane = tid % WAVE;
    const uint32_t t = blockIdx.x, pos = uint32_t(p.start) + t;
    const uint32_t H = uint32_t(p.heads), KVH = uint32_t(p.kvHeads), rows = p.kvReady ? H : H + 2 * KVH;
    const int half = p.freqs ? p.rotaryDims / 2 : 0;
    const int e0 = 8 * sub;
    // a pass's rows: issued before the angles' sin/cos and the barrier for
    // the first pass, so that their latency overlaps that work
    auto load_pass = [&](uint32_t r0, float (&x)[UNROLL][8]) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const uint32_t r = r0 + u * RPP;
            if (r >= rows) continue;
            if (r < H) load8<F32>(p.q, (size_t(t) * H + r) * p.qStride + e0, x[u]);
            else if (r < H + KVH) load8<F32>(p.k, (size_t(t) * KVH + (r - H)) * D + e0, x[u]);
            else load8<F32>(p.v, (size_t(t) * KVH + (r - H - KVH)) * D + e0, x[u]);
        }
    };
    const uint32_t rFirst = firstRow + tid / LPR;
    float x[UNROLL][8];
    load_pass(rFirst, x);
    if (blockIdx.x == 0) zero_pad_rows(kh, vh, uint64_t(KVH) * T * D, uint32_t(D));
    if (tid < half) {
        const float fpos = float(pos);   // the reference's fp32 angle (LocalModel.hpp:2632)
        sincosf(fpos * p.freqs[tid], &sn[tid], &cs[tid]);
        if (rope) {   // the token's cos/sin for the flash kernel's own q rotation
            rope[rope_at(t, 0, tid, half, gridDim.x)] = cs[tid];
            rope[rope_at(t, 1, tid, half, gridDim.x)] = sn[tid];
        }
    }
    __syncthreads();
    // rotate-half partner lane and the sign of its term, per element slot
    const int shiftL = half / 8;
    const bool lowHalf = e0 < half, highHalf = !lowHalf && e0 < 2 * half;
    const int partner = lowHalf ? lane + shiftL : (highHalf ? lane - shiftL : lane);
    float c8[8], s8[8];
    if (lowHalf || highHalf) {
        const int j0 = lowHalf ? e0 : e0 - half;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            c8[e] = cs[j0 + e];
            s8[e] = lowHalf ? -sn[j0 + e] : sn[j0 + e];
        }
    }

    bool bad = false;   // an fp16 conversion out of range
    for (uint32_t r0 = rFirst; r0 < rows; r0 += UNROLL * RPP) {
        if (r0 != rFirst) load_pass(r0, x);
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const uint32_t r = r0 + u * RPP;
            if (r >= rows) continue;   // uniform over the row's LPR lanes
            float (&v)[8] = x[u];
            if (r < H + KVH) {
                const float* gamma = r < H ? p.qNorm : p.kNorm;
                if (gamma) {   // rmsNormRow (LocalModel.hpp:1341-1348)
                    float ss = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
#pragma unroll
                    for (int o = 1; o < LPR; o <<= 1) ss += __shfl_xor(ss, o, WAVE);
                    const float inv = 1.0f / sqrtf(ss / float(D) + p.eps);
                    const floatx4* g = reinterpret_cast<const floatx4*>(gamma + e0);
                    const floatx4 g0 = g[0], g1 = g[1];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v[e] = v[e] * inv * (g0[e] + p.normOffset);
                        v[4 + e] = v[4 + e] * inv * (g1[e] + p.normOffset);
                    }
                }
                if (half) {   // rotate-half pairs (LocalModel.hpp:2636-2641)
                    float o8[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) o8[e] = __shfl(v[e], partner, WAVE);
                    if (lowHalf || highHalf) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) v[e] = v[e] * c8[e] + o8[e] * s8[e];
                    }
                }
            }
            if (r < H) {
                store8_f16(qh + (size_t(r) * p.count + t) * D + e0, v, qScale, bad);
            } else {
                const bool isKey = r < H + KVH;
                const uint32_t kv = isKey ? r - H : r - H - KVH;
                store8_f16((isKey ? kh : vh) + (size_t(kv) * T + pos) * D + e0, v, 1.0f, bad);
                store8_bf16((isKey ? p.keyCache : p.valueCache) + (size_t(kv) * p.capacity + pos) * D + e0, v);
            }
        }
    }
    raise_range_flag(p.rangeFlag, bad);
}

/* prefill_history_kernel with 8 elements (16 B) per lane and step */
__global__ __launch_bounds__(256) void prefill_history_vec_kernel(
    const uint16_t* __restrict__ keyCache, const uint16_t* __restrict__ valueCache,
    _Float16* __restrict__ kh, _Float16* __restrict__ vh, uint32_t per8, uint64_t capacity,
    uint32_t dim, uint32_t T, uint32_t* rangeFlag) {
    const uint32_t kv = blockIdx.y;
    bool bad = false;
    const u32x4* ks = reinterpret_cast<const u32x4*>(keyCache + kv * capacity * dim);
    const u32x4* vs = reinterpret_cast<const u32x4*>(valueCache + kv * capacity * dim);
    half8* kd = reinterpret_cast<half8*>(kh + size_t(kv) * T * dim);
    half8* vd = reinterpret_cast<half8*>(vh + size_t(kv) * T * dim);
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < per8; i += gridDim.x * blockDim.x) {
        const u32x4 a = ks[i], b = vs[i];
        half8 x, y;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[2 * e] = to_f16_checked(__uint_as_float(a[e] << 16), bad);
            x[2 * e + 1] = to_f16_checked(__uint_as_float(a[e] & 0xFFFF0000u), bad);
            y[2 * e] = to_f16_checked(__uint_as_float(b[e] << 16), bad);
            y[2 * e + 1] = to_f16_checked(__uint_as_float(b[e] & 0xFFFF0000u), bad);
        }
        kd[i] = x;
        vd[i] = y;
    }
    raise_range_flag(rangeFlag, bad);
}

struct FlashArgs {
    const _Float16* qh;  // [heads][count][D], pre-scaled by log2(e)/sqrt(D)
    const _Float16* kh;  // [kvHeads][T][D]
    const _Float16* vh;  // [kvHeads][T][D]
    float* out;          // [count][heads][D]
    __bf16* outHi;       // set: out goes here as bf16 high parts ...
    __bf16* outLo;       // ... and residuals instead
    uint32_t count, start, heads, kvHeads, window, T, nQT, xcdRemap;
    // fused Q: the raw q rows are normed, rotated and scaled on load instead
    // of read from qh
    const void* qraw;    // [count][heads][qStride], inType
    const float* qNorm;  // [D] gamma or null
    const float* rope;   // cos, sin of each token (rope_at), or null
    float eps, normOffset, qScale;
    uint32_t qStride, inType, half, fuseQ;
    uint32_t outputGate;   // out *= sigmoid(qraw[row + D + d]) (LocalModel.hpp:2660-2665)
    uint32_t* rangeFlag;   // set when a q element overflows fp16 (PrefillParams::rangeFlag)
};

typedef __fp16 fp16x4 __attribute__((__vector_size__(4 * sizeof(__fp16))));

/* the S^T MFMA's A row i of a 32-key block is key pi(i) = 16((i>>2)&1) +
   4(i>>3) + (i&3): accumulator register r of lane group g then holds key
   16g + r, so each lane's P^T slice is 8 consecutive keys */
__device__ __forceinline__ int key_of_row(int i) { return 16 * ((i >> 2) & 1) + 4 * (i >> 3) + (i & 3); }

/* ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i % 4
   of the 8-byte rows addressed by lanes i/4, i/4 + 4, i/4 + 8, i/4 + 12 */
__device__ __forceinline__ half8 read_tr16x2(const _Float16* a0, const _Float16* a1) {
    typedef __attribute__((address_space(3))) fp16x4 lds_fp16x4;
    const fp16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_fp16x4*)(a0));
    const fp16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_fp16x4*)(a1));
    typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
    const u32x2v l2 = __builtin_bit_cast(u32x2v, lo), h2 = __builtin_bit_cast(u32x2v, hi);
    return __builtin_bit_cast(half8, u32x4{l2[0], l2[1], h2[0], h2[1]});
}

/* LDS swizzles: the K tile's 16-byte block c of row i sits at c ^ kswz(i),
   the V tile's block c of row r at c ^ vswz(r, D) */
__device__ __forceinline__ int kswz(int i, int D) { return (i / (128 / D)) % (D / 8); }
__device__ __forceinline__ int vswz(int r, int D) { return D == 128 ? 4 * (r & 3) : 4 * ((r >> 1) & 1); }

/* s_waitcnt vmcnt(N) leaving the other counters alone (gfx9 encoding) */
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

/* One query row into the score MFMA's B operand: this lane's half of row tq
   of head `head` (elements 16 db + 8 g + j) as fp16, scaled by
   log2(e)/sqrt(D). With fuseQ the raw row is normed (QK-RMSNorm, the other
   half's sum over one v_permlane32_swap) and rotated (RoPE pairs (e, e +
   half) within the lane, half % 16 == 0) here, as attentionMixer does
   (LocalModel.hpp:2608-2648); otherwise prep's scaled fp16 copy is read.
   Rows past the call's count give zeros. `dma()` runs after the loads of
   gamma and the cos/sin table are issued and before the q row is read: with
   qlds set (bf16 rows, fused), it has brought the wave's 32 raw rows into
   LDS at qlds (row r's 16-byte block c at c ^ (r % 16)) and waited for all
   of the wave's loads, and the row is read from there. The caller waits for
   the rest. */
template <int D, typename Dma>
__device__ __forceinline__ void load_query(const FlashArgs& a, uint32_t tq, bool rowValid, uint32_t head, int g,
                                           half8 (&qreg)[D / 16], const _Float16* qlds, Dma&& dma,
                                           float* glds = nullptr) {
    constexpr int DB = D / 16;
    if (a.fuseQ) {
        // this lane's half of its query row: elements 16 db + 8g + j. QK-RMSNorm
        // over the row (the other half is in lane ^ 32), RoPE pairs (e, e + half)
        // within the lane (half % 16 == 0), then the log2(e)/sqrt(D) scale
        // (attentionMixer, LocalModel.hpp:2608-2648)
        // Every load (gamma, the cos/sin of the rotated blocks, the q half
        // row) is issued before any is used: one memory round trip. Written
        // as loads inside the loops that use them, the compiler issued and
        // waited for them one 16-byte block at a time.
        float x[DB][8];
        bool bad = false;   // an fp16 conversion out of range
        const size_t row = (size_t(rowValid ? tq : 0) * a.heads + head) * a.qStride;
        // gamma: with glds (D = 128), one 8-byte load per lane, staged
        // through the wave's 512 B of LDS and read back by broadcast where it
        // is used, instead of 16 loads of 1 KB per wave held in 64 registers
        typedef float floatx2 __attribute__((ext_vector_type(2)));
        floatx4 gam[DB][2];
        floatx2 gpair{0.0f, 0.0f};
        if (a.qNorm) {
            if (glds) {
                gpair = reinterpret_cast<const floatx2*>(a.qNorm)[threadIdx.x & 63];
            } else {
#pragma unroll
                for (int db = 0; db < DB; ++db) {
                    const floatx4* gm = reinterpret_cast<const floatx4*>(a.qNorm + 16 * db + 8 * g);
                    gam[db][0] = gm[0];
                    gam[db][1] = gm[1];
                }
            }
        }
        // rotate-half pairs (e, e + half) sit in one lane when half % 16 == 0:
        // blocks db < hb rotate with block db + hb
        const int hb = int(a.half) / 16;
        floatx4 cs[DB / 2][4];   // cos lo, cos hi, sin lo, sin hi
        if (a.rope) {
            const uint32_t t = rowValid ? tq : 0;
#pragma unroll
            for (int db = 0; db < DB / 2; ++db) {
                // blocks past hb are not rotated: their loads read block 0 again
                const uint32_t at = db < hb ? uint32_t(16 * db + 8 * g) : 0u;
#pragma unroll
                for (int k = 0; k < 4; ++k)   // cos lo, cos hi, sin lo, sin hi
                    cs[db][k] = *reinterpret_cast<const floatx4*>(
                        a.rope + rope_at(t, uint32_t(k >> 1), at + 4 * uint32_t(k & 1), a.half, a.count));
            }
        }
        dma();
        if (a.inType == 0) {
            floatx4 raw[DB][2];
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                const floatx4* src = reinterpret_cast<const floatx4*>(static_cast<const float*>(a.qraw) + row + 16 * db + 8 * g);
                raw[db][0] = src[0];
                raw[db][1] = src[1];
            }
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[db][j] = raw[db][0][j];
                    x[db][4 + j] = raw[db][1][j];
                }
        } else {
            u32x4 raw[DB];
            if (qlds) {   // LDS-typed reads: a generic pointer would make these flat loads
                typedef __attribute__((address_space(3))) const u32x4 lds_u32x4;
                const int c = int(threadIdx.x & 31);
#pragma unroll
                for (int db = 0; db < DB; ++db)
                    raw[db] = *(lds_u32x4*)(qlds + c * D + 8 * ((2 * db + g) ^ (c & 15)));
            } else {
#pragma unroll
                for (int db = 0; db < DB; ++db)
                    raw[db] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.qraw) + row + 16 * db + 8 * g);
            }
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[db][2 * j] = __uint_as_float(raw[db][j] << 16);
                    x[db][2 * j + 1] = __uint_as_float(raw[db][j] & 0xFFFF0000u);
                }
        }
        if (a.qNorm) {   // rmsNormRow (LocalModel.hpp:1341-1348)
            float ss = 0.0f;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int j = 0; j < 8; ++j) ss += x[db][j] * x[db][j];
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
            ss = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
            const float inv = 1.0f / sqrtf(ss / float(D) + a.eps);
            if (glds) {
                static_assert(D == 128 || D == 64, "gamma staging: 64 lanes x 2 floats");
                typedef __attribute__((address_space(3))) floatx2 lds_float2;
                typedef __attribute__((address_space(3))) const floatx4 lds_floatx4c;
                *(lds_float2*)(glds + 2 * (threadIdx.x & 63)) = gpair;
#pragma unroll
                for (int db = 0; db < DB; ++db) {
                    gam[db][0] = *(lds_floatx4c*)(glds + 16 * db + 8 * g);
                    gam[db][1] = *(lds_floatx4c*)(glds + 16 * db + 8 * g + 4);
                }
            }
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[db][j] = x[db][j] * inv * (gam[db][0][j] + a.normOffset);
                    x[db][4 + j] = x[db][4 + j] * inv * (gam[db][1][j] + a.normOffset);
                }
        }
        if (a.rope) {   // rotate-half pairs (LocalModel.hpp:2636-2641)
#pragma unroll
            for (int db = 0; db < DB / 2; ++db) {
                if (db < hb) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const float cj = j < 4 ? cs[db][0][j] : cs[db][1][j - 4];
                        const float sj = j < 4 ? cs[db][2][j] : cs[db][3][j - 4];
                        const float lo = x[db][j];
                        float hi = 0.0f;
#pragma unroll
                        for (int pb = 0; pb < DB; ++pb)
                            if (pb == db + hb) hi = x[pb][j];
                        const float nlo = lo * cj - hi * sj, nhi = hi * cj + lo * sj;
                        x[db][j] = nlo;
#pragma unroll
                        for (int pb = 0; pb < DB; ++pb)
                            if (pb == db + hb) x[pb][j] = nhi;
                    }
                }
            }
        }
        // Scale and round to fp16. |y| >= 65520 rounds to infinity, and the
        // rounding is monotone, so the lane's largest magnitude decides: one
        // test in the common case (fmaxf passes over NaN; an infinite input
        // takes the element-wise check, which does not count it)
        float big = 0.0f;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int j = 0; j < 8; ++j) big = fmaxf(big, fabsf(x[db][j]));
        if (big * a.qScale < 65520.0f) {
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int j = 0; j < 8; ++j) qreg[db][j] = _Float16(x[db][j] * a.qScale);
        } else {
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int j = 0; j < 8; ++j) qreg[db][j] = to_f16_checked(x[db][j] * a.qScale, bad);
        }
        if (!rowValid) {
#pragma unroll
            for (int db = 0; db < DB; ++db) qreg[db] = half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
        raise_range_flag(a.rangeFlag, bad);
    } else {
        dma();
        const _Float16* qrow = a.qh + (size_t(head) * a.count + (rowValid ? tq : 0)) * D;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            if (rowValid) qreg[db] = *reinterpret_cast<const half8*>(qrow + 16 * db + 8 * g);
            else qreg[db] = half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
    }
}

/*
    Flash attention, one workgroup = WAVES waves of 32 query rows of one
    head; key tiles of BN = 128 keys staged in LDS by DMA (global_load_lds,
    1 KB per wave instruction). Built in two forms: the ping-pong schedule
    (PP, D = 128; described at its loop) and the single-phase loop (D = 64):
    STAGES = 2 stages, one tile ahead of the one being computed, and one
    barrier per tile: past it, tile `it` has landed for every wave and every
    wave has finished tile it - 1, whose stage is then refilled. Per tile a
    wave runs S^T = K Q^T, the online softmax, and O^T += V^T P^T, 32 keys
    at a time.

    Every wave computes every tile of the workgroup's key range; keys past a
    row's position (or outside its window) are masked, so such tiles add
    exactly nothing, and the loop stays single-path.

    LDS K tile: row i holds key pi(i % 32) + 32 (i / 32); the 16-byte column
    block c of row i sits at c ^ kswz(i, D), so the 16 rows an A-operand read
    touches hit distinct banks (a fragment-major layout reads linearly but
    makes each DMA instruction gather 32 rows x 32 bytes, which costs more
    than it saves). LDS V tile: natural rows; block c of row r at c ^ vswz(r),
    so the 4 rows x 64 bytes a 32-lane transposed read touches hit distinct
    banks.
*/
template <int D, int WAVES, int STAGES, int BN, bool PP>
__global__ __launch_bounds__(64 * WAVES, WAVES == 4 ? 2 : 1) void prefill_flash_kernel(FlashArgs a) {
    static_assert(!PP || (WAVES == 8 && STAGES == 2 && BN == 128), "ping-pong: 8 waves, 2 stages, 128-key tiles");
    constexpr int BM = 32 * WAVES;
    constexpr int NKB = BN / 32;          // 32-key blocks per tile
    constexpr int DB = D / 16;            // 16-deep d blocks of the S^T product
    constexpr int DT = D / 32;            // 32-row d tiles of the O^T accumulator
    constexpr int CPR = D / 8;            // 16-byte blocks per row
    constexpr int RPB = WAVE / CPR;       // rows per 1 KB DMA block
    constexpr int NBLK = BN / RPB;        // DMA blocks per tile (K or V)
    constexpr int BPW = NBLK / WAVES;     // DMA blocks per wave per tile (K or V)
    constexpr int TILE = BN * D;          // halfs per K or V tile
    constexpr int AHEAD = STAGES - 1;     // DMA distance in tiles
    constexpr int PER = 2 * BPW;          // DMA instructions per wave per tile
    static_assert(NBLK % WAVES == 0, "DMA blocks must split evenly over the waves");
    static_assert(STAGES >= 2 && STAGES <= 4, "2 to 4 LDS stages");
    // One LDS object per stage and operand, always indexed by a compile-time
    // stage: the compiler then tells a read of stage j from the DMA still in
    // flight into the other stages and waits on stage j's DMA only.
    // V first: its stages sit below 64 KB, inside the 16-bit offset of a DS
    // instruction, so every V read is a per-d-tile lane address plus an
    // immediate; K needs one lane address per stage
    __shared__ __attribute__((aligned(16))) _Float16 V0[TILE], V1[TILE], V2[TILE], V3[TILE];
    __shared__ __attribute__((aligned(16))) _Float16 K0[TILE], K1[TILE], K2[TILE], K3[TILE];
    // the ping-pong loop's three V stages, indexed at run time (its DMA is
    // issued and waited for explicitly, so no stage needs its own object)
    __shared__ __attribute__((aligned(16))) _Float16 VP[3 * TILE];
    auto kbuf = [&](auto j) __attribute__((always_inline)) -> _Float16* {
        if constexpr (decltype(j)::value == 0) return K0;
        else if constexpr (decltype(j)::value == 1) return K1;
        else if constexpr (decltype(j)::value == 2) return K2;
        else return K3;
    };
    auto vbuf = [&](auto j) __attribute__((always_inline)) -> _Float16* {
        if constexpr (decltype(j)::value == 0) return V0;
        else if constexpr (decltype(j)::value == 1) return V1;
        else if constexpr (decltype(j)::value == 2) return V2;
        else return V3;
    };

    // Workgroups are dealt round-robin over the 8 XCDs (blockIdx % 8), each
    // with its own L2. The logical order groups a kv head's query heads, and
    // contiguous logical ranges land on one XCD, so the G query heads sharing a
    // kv head walk the same K/V tiles from the same L2 at the same time;
    // within a kv head, the longest query tiles go first.
    const uint32_t G = a.heads / a.kvHeads;
    uint32_t lg = blockIdx.x;
    if (a.xcdRemap) lg = (blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8;
    const uint32_t kvh = lg / (G * a.nQT);
    const uint32_t rest = lg % (G * a.nQT);
    const uint32_t head = kvh * G + rest % G;
    const uint32_t qt = a.nQT - 1 - rest / G;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, c = lane & 31;
    // the wave index in a scalar register, for code after the main loop: it
    // rebuilds its lane quantities from the lane counter, so that nothing
    // computed before the loop has to stay live (or spilled) across it
    const uint32_t wsc = __builtin_amdgcn_readfirstlane(uint32_t(tid >> 6));

    const uint32_t q0 = qt * BM;
    const uint32_t wq0 = q0 + 32 * w;
    const uint32_t tq = wq0 + c;
    const bool rowValid = tq < a.count;
    const uint32_t P = a.start + tq;
    const uint32_t wLast = (wq0 + 31 < a.count ? wq0 + 31 : a.count - 1);
    const uint32_t wPosFirst = a.start + wq0, wPosLast = a.start + wLast;
    // the first key this lane's query sees (Kernels.hpp:142)
    const uint32_t firstKey = (a.window && P + 1 > a.window) ? P + 1 - a.window : 0u;

    half8 qreg[DB];
    if constexpr (!PP) {   // the ping-pong form loads Q with its first DMA
        load_query<D>(a, tq, rowValid, head, g, qreg, nullptr, [] {});
        // Q lands before any DMA is issued, so the vmcnt waits in the loop only
        // ever count DMA
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        wait_vmcnt<0>();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }

    floatx16 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] = 0.0f;
    float m = -INFINITY, lsum = 0.0f;

    // key tiles [kbeg, kend) cover every row of the workgroup; count >= 1, so
    // there is at least one
    const uint32_t tileLast = (q0 + BM < a.count ? q0 + BM : a.count) - 1;
    const uint32_t kend = a.start + tileLast + 1;
    uint32_t kbeg = 0;
    if (a.window && a.start + q0 + 1 > a.window) kbeg = a.start + q0 + 1 - a.window;
    kbeg = kbeg / BN * BN;
    const uint32_t ntiles = (kend - kbeg + BN - 1) / BN;

    const _Float16* kbase = a.kh + size_t(kvh) * a.T * D;
    const _Float16* vbase = a.vh + size_t(kvh) * a.T * D;

    // per-lane element offsets of this wave's DMA block n inside one tile,
    // recomputed at each issue (a few integer ops) rather than held in
    // registers across the loop; a tile that runs past the last key clamps
    // its rows to T - 1 instead
    auto dma_offsets = [&](int n, uint32_t& ko, uint32_t& vo) __attribute__((always_inline)) {
        const int blk = w * BPW + n;
        const int i = blk * RPB + lane / CPR, pos = lane % CPR;
        ko = uint32_t(((i & ~31) + key_of_row(i & 31)) * D + 8 * (pos ^ kswz(i, D)));
        vo = uint32_t(i * D + 8 * (pos ^ vswz(i, D)));
    };
    auto issue = [&](uint32_t k0, auto bf) __attribute__((always_inline)) {
        _Float16* kd = kbuf(bf);
        _Float16* vd = vbuf(bf);
        const _Float16* kt = kbase + size_t(k0) * D;
        const _Float16* vt = vbase + size_t(k0) * D;
        const bool tail = k0 + BN > a.T;
        uint32_t koff[BPW], voff[BPW];
#pragma unroll
        for (int n = 0; n < BPW; ++n) dma_offsets(n, koff[n], voff[n]);
#pragma unroll
        for (int n = 0; n < BPW; ++n) {
            uint32_t off = koff[n];
            if (tail) {
                const uint32_t key = k0 + off / D;
                if (key > a.T - 1) off = (a.T - 1 - k0) * D + off % D;
            }
            __builtin_amdgcn_global_load_lds(kt + off,
                                             (__attribute__((address_space(3))) void*)(kd + (w * BPW + n) * 512),
                                             16, 0, 0);
        }
#pragma unroll
        for (int n = 0; n < BPW; ++n) {
            uint32_t off = voff[n];
            if (tail) {
                const uint32_t key = k0 + off / D;
                if (key > a.T - 1) off = (a.T - 1 - k0) * D + off % D;
            }
            __builtin_amdgcn_global_load_lds(vt + off,
                                             (__attribute__((address_space(3))) void*)(vd + (w * BPW + n) * 512),
                                             16, 0, 0);
        }
    };

    // V^T rows d = 32dt + lane % 32 with keys 32kb + 16g + 8h + 0..7: lane
    // q16 of each 16-lane group addresses row 32kb + 16g + 8h + q16/4 (and the
    // row 4 below), columns 32dt + 16 (lane / 16 % 2) + 4 (q16 % 4). The
    // swizzle depends on the row only through q16 / 4 (kb, h and the +4 keep
    // row % 4), so each d tile needs one lane address and kb, h are immediates.
    int vaddr[DT];
    {
        const int q16 = lane & 15, half16 = (lane >> 4) & 1, rl = 16 * g + (q16 >> 2);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const int dbase = 32 * dt + 16 * half16 + 4 * (q16 & 3);
            vaddr[dt] = rl * D + 8 * ((dbase >> 3) ^ vswz(rl, D)) + (dbase & 7);
        }
    }
    static_assert(D == 128 || D == 64, "vswz keeps row % 4 (D 128) or row % 4 / 2 (D 64)");
    // K A-operand rows 32 kb + c, 16-byte block 2 db + g at (2 db + g) ^
    // kswz(row); kswz depends on the row only through c, so kb is an immediate
    int kaddr[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) kaddr[db] = c * D + 8 * ((2 * db + g) ^ kswz(c, D));
    // Each step passes the lane addresses through an empty asm: the compiler
    // then cannot hoist (stage base + lane address) out of the loop into one
    // register per stage and d tile, and folds each stage base, a link-time
    // constant, into the DS offset instead.
    auto opaque_addresses = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) asm volatile("" : "+v"(vaddr[dt]));
#pragma unroll
        for (int db = 0; db < DB; ++db) asm volatile("" : "+v"(kaddr[db]));
    };
    // wait for tile `it` (stage J), barrier, refill the stage of tile it - 1
    // with tile it + STAGES - 1
    auto sync = [&](uint32_t it, auto J) __attribute__((always_inline)) {
        constexpr int bf = decltype(J)::value;
        const uint32_t after = ntiles - 1 - it;   // tiles issued after `it`: min(AHEAD - 1, after)
        if (AHEAD >= 3 && after >= 2) wait_vmcnt<(AHEAD >= 3 ? 2 : 0) * PER>();
        else if (AHEAD >= 2 && after >= 1) wait_vmcnt<(AHEAD >= 2 ? 1 : 0) * PER>();
        else wait_vmcnt<0>();
        lds_barrier();
        opaque_addresses();
        if (it + AHEAD < ntiles)
            issue(kbeg + (it + AHEAD) * BN, std::integral_constant<int, (bf + AHEAD) % STAGES>{});
    };

    // S^T = K Q^T for the tile in stage J (keys from k0), masked
    auto scores = [&](uint32_t k0, auto J, floatx16 (&s)[NKB]) __attribute__((always_inline)) {
        const _Float16* ks = kbuf(J);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
            for (int r = 0; r < 16; ++r) s[kb][r] = 0.0f;
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                const half8 ka = *reinterpret_cast<const half8*>(ks + kaddr[db] + 32 * kb * D);
                s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qreg[db], s[kb], 0, 0, 0);
            }
        }
        const bool needMask = (k0 + BN - 1 > wPosFirst) ||
                              (a.window && uint64_t(k0) + a.window < uint64_t(wPosLast) + 1);
        if (needMask) {
            // register r of block kb holds key k0 + 16 g + c, c = 32 kb + r,
            // and the lane's query sees keys [firstKey, P]. The mask is built
            // without compares (whose 64 lane masks would all sit in scalar
            // registers): the sign of hi - c (and of c - lo) selects the bit
            // pattern of -inf or of +0, which is added to the score
            const int base = int(k0 + 16 * g);
            const int hi = int(P) - base;
            const int lo = a.window ? int(firstKey) - base : -(1 << 30);
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int out = (hi - (32 * kb + r)) | ((32 * kb + r) - lo);
                    s[kb][r] += __int_as_float((out >> 31) & int(0xFF800000u));
                }
        }
    };

    // 128-key tiles: the softmax and P.V go 32 keys at a time, so only one
    // block's P is live next to the scores (the register budget of two waves
    // per SIMD does not hold all four at once)
    auto softmax_pv = [&](auto J, floatx16 (&s)[NKB]) __attribute__((always_inline)) {
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
        {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
            mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
        }
        const bool grow = mx > m + 8.0f;
        const float mn = grow ? mx : m;
        const float alpha = grow ? __builtin_amdgcn_exp2f(m - mn) : 1.0f;
        const float base = mn == -INFINITY ? 0.0f : mn;
        m = mn;
        if (__any(grow)) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
        }
        const _Float16* vs = vbuf(J);
        float psum = 0.0f;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            half8 pk[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float e[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    e[j] = __builtin_amdgcn_exp2f(s[kb][8 * h + j] - base);
                    pk[h][j] = _Float16(e[j]);
                }
                psum += ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
            }
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const _Float16* a0 = vs + vaddr[dt] + (32 * kb + 8 * h) * D;
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(read_tr16x2(a0, a0 + 4 * D), pk[h], o[dt], 0, 0, 0);
                }
        }
        lsum = lsum * alpha + psum;
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    if constexpr (PP) {
        /*
            Ping-pong. Group 0 (waves 0-3) leads and group 1 (waves 4-7) runs
            one interval behind; every interval ends in a workgroup barrier.
            A wave's own steps alternate: step 2j is its MFMA phase (O += P V
            of tile j - 1, then S of tile j), step 2j + 1 the softmax of tile
            j. Waves w and w + 4 share a SIMD, so in every interval one of
            them feeds the matrix core while the other runs the softmax on
            the VALU.

            K is double-buffered by tile parity and V triple-buffered (tile j
            in stage j mod 3), 160 KB in all, so that the DMA splits evenly
            between the groups' softmax phases, the only phases that can
            absorb the ~2,100 cycles a 64 KB tile takes on the CU's memory
            path: in interval A_j (group 0 MFMA on tile j, group 1 softmax of
            j - 1) group 1 DMAs K tile j + 1, which it waits for at the end of
            B_j, the last point before group 0 reads it; in interval B_j
            (group 0 softmax of j, group 1 MFMA on j) group 0 DMAs V tile
            j + 1, needed from A_{j+2} on, and waits for it at the end of
            B_{j+1}. Each stage a DMA refills was last read in the interval
            before (K) or two intervals before (V).
        */
        const int grp = w >> 2, wq = w & 3;
        constexpr int PB = NBLK / 4;   // DMA blocks per issuing wave per tile (K or V)
        static_assert(D == 128 && RPB == 4 && PB == 8, "the ping-pong DMA offsets assume D = 128");
        // Block n of issuing wave wq holds tile rows i = 4 (8 wq + n) + r,
        // r = lane / 16, 16-byte column pos = lane % 16. K row i is key
        // 32 wq + 16 (n & 1) + 4 (n >> 1) + r (key_of_row), its column block
        // at pos ^ (4 (n & 3) + r) (kswz); V row i is key i, its block at
        // pos ^ 4 r (vswz). So every offset is a per-lane base plus a
        // compile-time constant: the K bases for the four values of n & 3
        // and one V base.
        const int rr = lane >> 4, cp = lane & 15;
        int kb0[4], vb0;   // byte offsets
#pragma unroll
        for (int m = 0; m < 4; ++m) kb0[m] = 2 * ((32 * wq + rr) * D + 8 * ((cp ^ rr) ^ (4 * m)));
        vb0 = 2 * ((32 * wq + rr) * D + 8 * (cp ^ (4 * rr)));
        // the wave's first LDS block of a stage, in a scalar register
        const uint32_t ldsWave = __builtin_amdgcn_readfirstlane(uint32_t(wq) * PB * 1024);
        // DMA blocks [n0, n1) of this wave's share of one K or V tile. The
        // per-block constant goes into the (scalar) source base, so a block
        // costs no vector instruction. A tile running past a head's last
        // row reads the next head's rows, or the zeroed pad rows after the
        // last head; the causal mask drops those keys (their finite values
        // meet P = 0).
        auto dma_rows = [&](uint32_t k0, uint32_t stage, bool isK, auto N0, auto N1) __attribute__((always_inline)) {
            constexpr int n0 = decltype(N0)::value, n1 = decltype(N1)::value;
            const uint32_t lds = __builtin_amdgcn_readfirstlane(stage + ldsWave);
            const char* src = reinterpret_cast<const char*>((isK ? kbase : vbase) + size_t(k0) * D);
            // fresh each call: the offsets are not worth registers across the loop
#pragma unroll
            for (int m = 0; m < 4; ++m) asm volatile("" : "+v"(kb0[m]));
            asm volatile("" : "+v"(vb0));
#pragma unroll
            for (int n = n0; n < n1; ++n) {
                if (isK) dma_block(src + 2 * (16 * (n & 1) + 4 * (n >> 1)) * D, uint32_t(kb0[n & 3]), lds + n * 1024);
                else dma_block(src + 2 * 4 * n * D, uint32_t(vb0), lds + n * 1024);
            }
        };
        auto active = [&](uint32_t j) __attribute__((always_inline)) {
            const uint32_t k0 = kbeg + j * BN;
            return j < ntiles && !(k0 > wPosLast || (a.window && uint64_t(k0) + BN - 1 + a.window <= uint64_t(wPosFirst)));
        };
        // The MFMA phase's two products, each software-pipelined: operand
        // fragments are read from LDS AHEAD products in advance into a ring,
        // and the four accumulator chains are interleaved, so neither the
        // LDS latency nor an accumulator dependence stalls the matrix core.
        // The scheduling groups pin that order (the default schedule waits
        // for every read just before its product).
        constexpr int AHEAD_PP = 3;
        auto pv_pp = [&](const _Float16* vs, const half8 (&pk)[NKB][2]) __attribute__((always_inline)) {
            constexpr int N = NKB * 2 * DT;   // products: (kb, h) outer, dt inner
            auto frag = [&](int i) __attribute__((always_inline)) {
                const int dt = i % DT, hh = (i / DT) % 2, kb = i / (2 * DT);
                const _Float16* a0 = vs + vaddr[dt] + (32 * kb + 8 * hh) * D;
                return read_tr16x2(a0, a0 + 4 * D);
            };
            half8 f[AHEAD_PP + 1];
#pragma unroll
            for (int i = 0; i < AHEAD_PP; ++i) f[i] = frag(i);
#pragma unroll
            for (int i = 0; i < N; ++i) {
                if (i + AHEAD_PP < N) f[(i + AHEAD_PP) % (AHEAD_PP + 1)] = frag(i + AHEAD_PP);
                const int dt = i % DT, hh = (i / DT) % 2, kb = i / (2 * DT);
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[i % (AHEAD_PP + 1)], pk[kb][hh], o[dt], 0, 0, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * AHEAD_PP, 0);
#pragma unroll
            for (int i = 0; i < N; ++i) {
                if (i + AHEAD_PP < N) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
        };
        // the causal (and window) mask of a tile's scores, arithmetic: the sign
        // of (hi - c) | (c - lo) shifted into a -inf bit pattern and added
        auto mask_scores = [&](uint32_t k0, floatx16 (&s)[NKB]) __attribute__((always_inline)) {
            const bool needMask = (k0 + BN - 1 > wPosFirst) ||
                                  (a.window && uint64_t(k0) + a.window < uint64_t(wPosLast) + 1);
            if (needMask) {
                const int base = int(k0 + 16 * g);
                const int hi = int(P) - base;
                const int lo = a.window ? int(firstKey) - base : -(1 << 30);
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int out = (hi - (32 * kb + r)) | ((32 * kb + r) - lo);
                        s[kb][r] += __int_as_float((out >> 31) & int(0xFF800000u));
                    }
            }
        };
        auto scores_pp = [&](auto J, floatx16 (&s)[NKB]) __attribute__((always_inline)) {
            const _Float16* ks = kbuf(J);
            constexpr int N = NKB * DB;   // products: db outer, kb inner
            auto frag = [&](int i) __attribute__((always_inline)) {
                const int kb = i % NKB, db = i / NKB;
                return *reinterpret_cast<const half8*>(ks + kaddr[db] + 32 * kb * D);
            };
            half8 f[AHEAD_PP + 1];
#pragma unroll
            for (int i = 0; i < AHEAD_PP; ++i) f[i] = frag(i);
#pragma unroll
            for (int i = 0; i < N; ++i) {
                if (i + AHEAD_PP < N) f[(i + AHEAD_PP) % (AHEAD_PP + 1)] = frag(i + AHEAD_PP);
                const int kb = i % NKB, db = i / NKB;
                s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[i % (AHEAD_PP + 1)], qreg[db], s[kb], 0, 0, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, AHEAD_PP, 0);
#pragma unroll
            for (int i = 0; i < N; ++i) {
                if (i + AHEAD_PP < N) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
        };
        // P.V of the previous tile and S of this one as one pipeline: the
        // first K fragments are read during the last P.V products, so the
        // matrix core does not wait for LDS between the two products
        auto pv_scores_pp = [&](const _Float16* vs, const half8 (&pk)[NKB][2], auto J, floatx16 (&s)[NKB],
                                float nb, auto PRE, const half8& pre) __attribute__((always_inline)) {
            constexpr bool prefetched = decltype(PRE)::value;   // the first fragment is `pre`
            const _Float16* ks = kbuf(J);
            constexpr int NP = NKB * 2 * DT, N = NP + NKB * DB;
            auto frag = [&](int i) __attribute__((always_inline)) {
                if (i < NP) {
                    const int dt = i % DT, hh = (i / DT) % 2, kb = i / (2 * DT);
                    const _Float16* a0 = vs + vaddr[dt] + (32 * kb + 8 * hh) * D;
                    return read_tr16x2(a0, a0 + 4 * D);
                }
                const int kb = (i - NP) % NKB, db = (i - NP) / NKB;
                return *reinterpret_cast<const half8*>(ks + kaddr[db] + 32 * kb * D);
            };
            half8 f[AHEAD_PP + 1];
#pragma unroll
            for (int i = 0; i < AHEAD_PP; ++i) f[i] = prefetched && i == 0 ? pre : frag(i);
            // S starts at -base; the moves issue beside the first P.V products
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) s[kb][r] = nb;
#pragma unroll
            for (int i = 0; i < N; ++i) {
                if (i + AHEAD_PP < N) f[(i + AHEAD_PP) % (AHEAD_PP + 1)] = frag(i + AHEAD_PP);
                if (i < NP) {
                    const int dt = i % DT, hh = (i / DT) % 2, kb = i / (2 * DT);
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[i % (AHEAD_PP + 1)], pk[kb][hh], o[dt], 0, 0, 0);
                } else {
                    const int kb = (i - NP) % NKB, db = (i - NP) / NKB;
                    s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[i % (AHEAD_PP + 1)], qreg[db], s[kb], 0, 0, 0);
                }
            }
            // DS reads per fragment: two transposed halves for P.V, one for S
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * (prefetched ? AHEAD_PP - 1 : AHEAD_PP), 0);
#pragma unroll
            for (int i = 0; i < N; ++i) {
                if (i + AHEAD_PP < NP) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                else if (i + AHEAD_PP < N) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
        };
        floatx16 s[NKB];
        half8 pk[NKB][2];
        bool haveP = false, haveS = false;
        uint32_t sK0 = 0;   // the first key of the tile whose scores s holds
        // Group 1 reads the first P.V fragment of its next MFMA phase at the
        // end of its softmax phase (that V tile is visible from the start of
        // the softmax phase), so the phase's first product does not wait for
        // the LDS: 0.4% faster. Group 0's next V tile becomes visible only at
        // the barrier that starts its MFMA phase. Two or three fragments
        // ahead held more registers across the barrier and spilled.
        half8 preV;
        auto prefetch_v = [&](const _Float16* vs) __attribute__((always_inline)) {
            const _Float16* a0 = vs + vaddr[0];   // fragment 0: dt 0, key block 0, first half
            preV = read_tr16x2(a0, a0 + 4 * D);
        };
        // MFMA phase of tile j: P.V of tile j - 1 (V stage vs), S of tile j (K
        // stage KS). The wave runs it at a raised priority: the SIMD then
        // issues its LDS reads and MFMAs ahead of the partner wave's softmax
        // (without it the younger group's MFMA phase ran a third longer than
        // the older group's, 3,380 against 2,770 cycles per interval)
        auto mphase = [&](uint32_t j, auto KS, const _Float16* vs, auto PRE) __attribute__((always_inline)) {
            __builtin_amdgcn_s_setprio(3);
            haveS = active(j);
            sK0 = kbeg + j * BN;
            // S starts at -base (the registers are free: P holds the last tile)
            const float nb = m == -INFINITY ? 0.0f : -m;
            if (haveP && haveS) {
                pv_scores_pp(vs, pk, KS, s, nb, PRE, preV);
                haveP = false;
                return;
            }
            if (haveS) {
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) s[kb][r] = nb;
            }
            if (haveP) {
                pv_pp(vs, pk);
                haveP = false;
            } else if (haveS) {
                scores_pp(KS, s);
            }
        };
        // The softmax of the ping-pong loop. The S accumulators start at
        // -base (the running max, or 0 before the row's first key), so the
        // products arrive as s - base and P = exp2 of them needs no
        // subtraction. Only when a row's maximum passes base + 8 (P would
        // exceed 2^8) does base move, to that maximum, with one subtraction
        // pass and O rescaled. `hook(kb)` runs after each 32-key block's
        // exponentials: the softmax phase's DMA goes there, two blocks at a
        // time (issued back to back, a wave's DMA instructions stall it on
        // the CU's memory queue, about 30 bytes a cycle).
        auto softmax_pp = [&](floatx16 (&s)[NKB], half8 (&pk)[NKB][2], auto hook) __attribute__((always_inline)) {
            // eight partial maxima (one per 16-key half block): short
            // independent chains instead of one of 32 dependent max3s
            float mp[NKB][2];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    mp[kb][h] = s[kb][8 * h];
#pragma unroll
                    for (int j = 1; j < 8; ++j) mp[kb][h] = fmaxf(mp[kb][h], s[kb][8 * h + j]);
                }
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) mp[kb][0] = fmaxf(mp[kb][0], mp[kb][1]);
            float mx = fmaxf(fmaxf(mp[0][0], mp[1][0]), fmaxf(mp[2][0], mp[3][0]));
            {
                const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
                mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
            }
            const bool fresh = m == -INFINITY;   // no visible key in earlier tiles
            const bool grow = fresh ? mx != -INFINITY : mx > 8.0f;
            const float shift = grow ? mx : 0.0f;
            const float alpha = fresh ? 0.0f : (grow ? __builtin_amdgcn_exp2f(-shift) : 1.0f);
            if (__any(grow)) {
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) s[kb][r] -= shift;
            }
            // eight partial row sums, one per 16-key half block, added in fp32
            // from the exponentials before their fp16 rounding: plain adds
            // issue beside the partner wave's MFMAs, where v_dot2c over the
            // fp16 P stalls the matrix core
            float ps[NKB][2];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    float e[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        e[j] = __builtin_amdgcn_exp2f(s[kb][8 * h + j]);
                        pk[kb][h][j] = _Float16(e[j]);
                    }
                    ps[kb][h] = ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
                }
                hook(kb, s, pk[kb][1]);
            }
            const float psum = ((ps[0][0] + ps[0][1]) + (ps[1][0] + ps[1][1])) + ((ps[2][0] + ps[2][1]) + (ps[3][0] + ps[3][1]));
            lsum = lsum * alpha + psum;
            if (grow) m = (fresh ? 0.0f : m) + shift;
            if (__any(grow)) {
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
            }
        };
        auto vphase = [&](auto hook) __attribute__((always_inline)) {
            __builtin_amdgcn_s_setprio(0);
            if (haveS) {
                // the mask of a diagonal tile is applied here, beside the
                // partner group's MFMAs, rather than after this wave's own
                // products, where it waited for them and held up the
                // interval (0.3% over the kernel)
                mask_scores(sK0, s);
                softmax_pp(s, pk, hook);
                haveP = true;
                haveS = false;
            } else {
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) hook(kb, s, pk[kb][1]);
            }
        };
        auto no_dma = [](int, floatx16 (&)[NKB], const half8&) __attribute__((always_inline)) {};
        using std::integral_constant;
        // the softmax phase's DMA: tile t (K or V) into the LDS stage at
        // `stage`, blocks 2 kb and 2 kb + 1 after 32-key block kb
        auto dma_hook = [&](uint32_t t, uint32_t stage, bool isK) __attribute__((always_inline)) {
            return [&, t, stage, isK](int kb, floatx16 (&sc)[NKB], const half8& last) __attribute__((always_inline)) {
                // ordering only (the asm statements emit nothing): the DMA
                // follows block kb's exponentials, whose last result it takes,
                // and precedes block kb + 1's, whose scores pass through the
                // asm after it
                asm volatile("" : : "v"(last));
                if (t < ntiles) {
                    const uint32_t k0 = kbeg + t * BN;
                    if (kb == 0) dma_rows(k0, stage, isK, integral_constant<int, 0>{}, integral_constant<int, 2>{});
                    else if (kb == 1) dma_rows(k0, stage, isK, integral_constant<int, 2>{}, integral_constant<int, 4>{});
                    else if (kb == 2) dma_rows(k0, stage, isK, integral_constant<int, 4>{}, integral_constant<int, 6>{});
                    else dma_rows(k0, stage, isK, integral_constant<int, 6>{}, integral_constant<int, 8>{});
                }
                if (kb + 1 < NKB) asm volatile("" : "+v"(sc[kb + 1 < NKB ? kb + 1 : kb]));
            };
        };
        static_assert(NKB == 4 && PB == 8, "two DMA blocks after each of four 32-key blocks");
        constexpr uint32_t VSTAGE = TILE * 2;   // bytes of one V stage
        const uint32_t ldsK0 = lds_address(K0), ldsK1 = lds_address(K1), ldsV = lds_address(VP);
        auto vstage = [&](uint32_t j) __attribute__((always_inline)) -> const _Float16* {
            return VP + (j % 3) * TILE;
        };
        // prologue: K tile 0 (group 1) or V tile 0 (group 0), the loads of
        // gamma and the cos/sin table, then the wave's 32 raw bf16 q rows by
        // DMA (1 KB, 4 rows, per instruction; a per-lane load of its own row
        // touches 32 cache lines per instruction) into V stages 1 and 2, which
        // the loop first fills in interval B_0: all in flight at once. The
        // wave then waits for all of it and reads its q rows back from LDS.
        // Without the q DMA, the compiler's waits for the q loads count only
        // its own loads, which is safe: the older DMA completes first. All of
        // it lands before the loop, whose waits then count only its DMA.
        const bool qDma = a.fuseQ && a.inType == 1 && uint64_t(a.heads) * a.qStride < (1ull << 26);   // 32-bit offsets
        const uint32_t wu = wsc;
        const _Float16* qlds = VP + TILE + wu * 32 * D;
        if (grp == 1) dma_rows(kbeg, ldsK0, true, integral_constant<int, 0>{}, integral_constant<int, PB>{});
        else dma_rows(kbeg, ldsV, false, integral_constant<int, 0>{}, integral_constant<int, PB>{});
        auto q_dma = [&]() __attribute__((always_inline)) {
            if (qDma) {
                // rows past the call's count repeat its last row (their q is zeroed)
                const uint32_t first = q0 + 32 * wu < a.count ? q0 + 32 * wu : a.count - 1;
                const char* src = static_cast<const char*>(a.qraw) + (size_t(first) * a.heads + head) * a.qStride * 2;
                const uint32_t lds = __builtin_amdgcn_readfirstlane(lds_address(qlds));
#pragma unroll
                for (int n = 0; n < 8; ++n) {
                    const uint32_t r = uint32_t(4 * n + (lane >> 4));
                    const uint32_t tr = (q0 + 32 * wu + r < a.count ? q0 + 32 * wu + r : a.count - 1) - first;
                    const uint32_t off = uint32_t((size_t(tr) * a.heads * a.qStride + 8 * ((lane & 15) ^ (r & 15))) * 2);
                    dma_block(src, off, lds + n * 1024);
                }
                wait_vmcnt<0>();
            }
        };
        // gamma staging: the wave's 512 B of K stage 1, first filled in A_0
        float* glds = D == 128 ? reinterpret_cast<float*>(K1 + wu * 256) : nullptr;
        load_query<D>(a, tq, rowValid, head, g, qreg, qDma ? qlds : nullptr, q_dma, glds);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        wait_vmcnt<0>();
        lds_barrier();
        // group 0 waits at the end of each softmax phase for the V tile it
        // issued in the previous one: the newer PB blocks may stay in flight
        auto wait_v = [&](uint32_t issuedNow) __attribute__((always_inline)) {
            if (issuedNow < ntiles) wait_vmcnt<PB>();
            else wait_vmcnt<0>();
        };
        const uint32_t nI = 2 * ntiles + 2;
        for (uint32_t i0 = 0; i0 < nI; i0 += 4) {
            const uint32_t j0 = i0 / 2;   // the even tile of this round
            // A_j0: group 0 MFMA on tile j0; group 1 softmax of j0 - 1 and
            // DMA of K j0 + 1
            opaque_addresses();
            using NoPre = std::integral_constant<bool, false>;
            using Pre = std::integral_constant<bool, true>;
            if (grp == 0) {
                mphase(j0, S0{}, vstage(j0 + 2), NoPre{});   // V of tile j0 - 1
            } else {
                vphase(dma_hook(j0 + 1, ldsK1, true));
                prefetch_v(vstage(j0 + 2));
            }
            lds_barrier();
            if (i0 + 1 >= nI) break;
            // B_j0: group 0 softmax of j0 and DMA of V j0 + 1; group 1 MFMA on j0
            opaque_addresses();
            if (grp == 0) {
                vphase(dma_hook(j0 + 1, ldsV + ((j0 + 1) % 3) * VSTAGE, false));
                wait_v(j0 + 1);
            } else {
                mphase(j0, S0{}, vstage(j0 + 2), Pre{});
                wait_vmcnt<0>();
            }
            lds_barrier();
            if (i0 + 2 >= nI) break;
            // A_j0+1: group 0 MFMA on tile j0 + 1; group 1 softmax of j0 and
            // DMA of K j0 + 2
            opaque_addresses();
            if (grp == 0) {
                mphase(j0 + 1, S1{}, vstage(j0), NoPre{});
            } else {
                vphase(dma_hook(j0 + 2, ldsK0, true));
                prefetch_v(vstage(j0));
            }
            lds_barrier();
            if (i0 + 3 >= nI) break;
            // B_j0+1: group 0 softmax of j0 + 1 and DMA of V j0 + 2; group 1
            // MFMA on j0 + 1
            opaque_addresses();
            if (grp == 0) {
                vphase(dma_hook(j0 + 2, ldsV + ((j0 + 2) % 3) * VSTAGE, false));
                wait_v(j0 + 2);
            } else {
                mphase(j0 + 1, S1{}, vstage(j0), Pre{});
                wait_vmcnt<0>();
            }
            lds_barrier();
        }
        __builtin_amdgcn_s_setprio(0);
    } else {
    issue(kbeg, S0{});
    if constexpr (AHEAD > 1)
        if (ntiles > 1) issue(kbeg + BN, S1{});
    if constexpr (AHEAD > 2)
        if (ntiles > 2) issue(kbeg + 2 * BN, S2{});

    // step `it` in stage it % STAGES: S, softmax, O += P V for one tile
    auto step = [&](uint32_t it, auto J) __attribute__((always_inline)) -> bool {
        if (it >= ntiles) return false;
        floatx16 s[NKB];
        sync(it, J);
        // a tile wholly after this wave's last row (or before the window of its
        // first) adds nothing to it: the wave only keeps the barrier and DMA
        const uint32_t k0 = kbeg + it * BN;
        if (k0 > wPosLast || (a.window && uint64_t(k0) + BN - 1 + a.window <= uint64_t(wPosFirst))) return true;
        scores(k0, J, s);
        softmax_pv(J, s);
        return true;
    };
    for (uint32_t it = 0;; it += STAGES) {
        if (!step(it, S0{})) break;
        if (!step(it + 1, S1{})) break;
        if constexpr (STAGES > 2)
            if (!step(it + 2, S2{})) break;
        if constexpr (STAGES > 3)
            if (!step(it + 3, std::integral_constant<int, 3>{})) break;
    }
    }

    lsum += __shfl_xor(lsum, 32, WAVE);
    bool direct = true;
    if constexpr (PP) {
        if (!a.outHi && !a.outputGate) {
            // The output rows leave through LDS. A lane's 16-byte pieces all
            // belong to its own row, so a store of them touches 32 cache lines
            // per instruction. Written to the wave's 16 KB of LDS (piece p of
            // row r at p ^ (r % 16): conflict-free both ways) and read back
            // two rows per instruction, each store covers 2 rows of 512 B.
            // The loop's last barrier has passed, so no wave reads K or V any
            // more.
            direct = false;
            static_assert(D == 128, "32 pieces of 16 bytes per row");
            typedef __attribute__((address_space(3))) floatx4 lds_floatx4;
            const int le = int(__lane_id()), ce = le & 31, ge = le >> 5;
            const uint32_t wqe = q0 + 32 * wsc;
            const int wv = int(wsc);
            float* ob = reinterpret_cast<float*>(wv < 6 ? VP + wv * 8192 : K0 + (wv - 6) * 8192);
            const float inv = wqe + uint32_t(ce) < a.count ? 1.0f / lsum : 0.0f;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    floatx4 val;
#pragma unroll
                    for (int i = 0; i < 4; ++i) val[i] = o[dt][4 * r4 + i] * inv;
                    const int p = 8 * dt + 2 * r4 + ge;
                    *(lds_floatx4*)(ob + ce * D + 4 * (p ^ (ce & 15))) = val;
                }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int r = 2 * i + ge, p = le & 31;
                const floatx4 val = *(lds_floatx4*)(ob + r * D + 4 * (p ^ (r & 15)));
                const uint32_t row = wqe + uint32_t(r);
                if (row < a.count)   // written once: nontemporal, so as not to displace K and V in L2
                    __builtin_nontemporal_store(val, reinterpret_cast<floatx4*>(a.out + (size_t(row) * a.heads + head) * D + 4 * p));
            }
        }
    }
    if (direct && rowValid) {
        const float inv = 1.0f / lsum;
        float* dst = a.out + (size_t(tq) * a.heads + head) * D;
        const size_t gateRow = (size_t(tq) * a.heads + head) * a.qStride + D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                floatx4 val;
#pragma unroll
                for (int i = 0; i < 4; ++i) val[i] = o[dt][4 * r4 + i] * inv;
                if (a.outputGate) {   // sigmoidOf (LocalModel.hpp:1371) of the row's gate half
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float gt = load_elem(a.qraw, gateRow + 32 * dt + 8 * r4 + 4 * g + i, int(a.inType));
                        val[i] *= 1.0f / (1.0f + expf(-gt));
                    }
                }
                if (a.outHi) {   // the o projection's operand images, as split_a_kernel writes them
                    bf16x4 h, l;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        h[i] = __bf16(val[i]);
                        l[i] = __bf16(val[i] - float(h[i]));
                    }
                    const size_t at = size_t(dst - a.out) + 32 * dt + 8 * r4 + 4 * g;
                    *reinterpret_cast<bf16x4*>(a.outHi + at) = h;
                    *reinterpret_cast<bf16x4*>(a.outLo + at) = l;
                } else {
                    *reinterpret_cast<floatx4*>(dst + 32 * dt + 8 * r4 + 4 * g) = val;
                }
            }
    }
}

} // namespace

/* the register-row kernels need 16-byte aligned rows and rot % 16 == 0
   (vec); the flash kernel normalises and rotates its own q rows when each
   lane's RoPE partners are in the lane itself (rot / 2 a multiple of 16):
   prep then handles only k and v, plus a cos/sin table for the q rotation */
static void prep_shape(const PrefillParams& p, bool* vec, bool* fuseQ) {
    const size_t inAlign = p.inType == 0 ? 4 : 8;   // elements per 16 bytes
    auto aligned = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    *vec = aligned(p.q) && aligned(p.k) && aligned(p.v) && aligned(p.keyCache) && aligned(p.valueCache) &&
           (p.qStride % inAlign) == 0 && (!p.qNorm || aligned(p.qNorm)) && (!p.kNorm || aligned(p.kNorm)) &&
           (!p.freqs || (p.rotaryDims % 16) == 0);
    *fuseQ = *vec && p.qStride < (1ull << 32) && (!p.freqs || (p.rotaryDims % 32) == 0);
}

bool prefill_prep_foldable(const PrefillParams& p, float** rope) {
    *rope = nullptr;
    bool vec = false, fuseQ = false;
    prep_shape(p, &vec, &fuseQ);
    if (!p.kvReady || !fuseQ || p.count == 0) return false;
    if (!p.freqs) return true;
    // the same slot and size launch_prefill takes for the table
    *rope = static_cast<float*>(Context::instance().grow(SLOT_PREFILL_Q, p.count * size_t(p.rotaryDims) * sizeof(float)));
    return *rope != nullptr;
}

bool prefill_work_buffers(const PrefillParams& p, void** kh, void** vh) {
    Context& ctx = Context::instance();
    const uint64_t T = p.start + p.count;
    // PREFILL_PAD_ROWS rows past the last kv head, zeroed by prep: the flash
    // kernel's last tile reads up to a tile past each head's rows unclamped
    *kh = ctx.grow(SLOT_PREFILL_K, (p.kvHeads * T + PREFILL_PAD_ROWS) * p.dim * 2);
    *vh = ctx.grow(SLOT_PREFILL_V, (p.kvHeads * T + PREFILL_PAD_ROWS) * p.dim * 2);
    return *kh && *vh;
}

bool launch_prefill(const PrefillParams& p, hipStream_t stream) {
    Context& ctx = Context::instance();
    if (p.dim != 64 && p.dim != 128) return ctx.fail("prefill: dim must be 64 or 128");
    if (p.kvHeads == 0 || p.heads % p.kvHeads) return ctx.fail("prefill: heads must be a multiple of kvHeads");
    if (p.qStride < p.dim) return ctx.fail("prefill: qStride < dim");
    if (p.outputGate && p.qStride < 2 * p.dim) return ctx.fail("prefill: the output gate needs qStride >= 2 dim");
    if (p.freqs && (p.rotaryDims == 0 || p.rotaryDims > int(p.dim) || (p.rotaryDims & 1)))
        return ctx.fail("prefill: rotaryDims must be even and within dim");
    if (p.inType != 0 && p.inType != 1) return ctx.fail("prefill: unknown input type");
    if (!p.q || (!p.kvReady && (!p.k || !p.v)) || !p.out || !p.keyCache || !p.valueCache)
        return ctx.fail("prefill: null tensor");
    if (p.count == 0) return true;
    const uint64_t T = p.start + p.count;
    if (p.capacity < T) return ctx.fail("prefill: cache capacity below start + count");
    if ((p.heads + 2 * p.kvHeads) * p.dim * sizeof(float) > 96 * 1024)
        return ctx.fail("prefill: one token's q, k, v rows exceed 96 KB of LDS");
    if (T * p.dim >= (1ull << 31) || p.heads * p.count >= (1ull << 31) || p.kvHeads > 65535)
        return ctx.fail("prefill: sequence too long");

    void* khv = nullptr;
    void* vhv = nullptr;
    if (!prefill_work_buffers(p, &khv, &vhv)) return false;
    _Float16* kh = static_cast<_Float16*>(khv);
    _Float16* vh = static_cast<_Float16*>(vhv);

    bool vec = false, fuseQ = false;
    prep_shape(p, &vec, &fuseQ);
    if (p.prepDone && !(p.kvReady && fuseQ)) return ctx.fail("prefill: prep cannot be skipped for these parameters");
    _Float16* qh = nullptr;
    float* rope = nullptr;
    if (!fuseQ) {
        qh = static_cast<_Float16*>(ctx.grow(SLOT_PREFILL_Q, p.heads * p.count * p.dim * 2));
        if (!qh) return false;
    } else if (p.freqs) {
        rope = static_cast<float*>(ctx.grow(SLOT_PREFILL_Q, p.count * size_t(p.rotaryDims) * sizeof(float)));
        if (!rope) return false;
    }
    const uint32_t firstRow = fuseQ ? uint32_t(p.heads) : 0u;

    if (p.start > 0) {
        const uint32_t per = uint32_t(p.start * p.dim);
        const uint32_t per8 = per / 8;   // dim is a multiple of 8
        const uint32_t work = vec ? per8 : per;
        const uint32_t blocks = (work + 255) / 256 < 4096 ? (work + 255) / 256 : 4096;
        if (!ctx.launch("prefill_history_kernel", stream, [&] {
                const dim3 grid{blocks, unsigned(p.kvHeads)};
                if (vec)
                    hipLaunchKernelGGL(prefill_history_vec_kernel, grid, dim3(256), 0, stream, p.keyCache,
                                       p.valueCache, kh, vh, per8, p.capacity, uint32_t(p.dim), uint32_t(T),
                                       p.rangeFlag);
                else
                    hipLaunchKernelGGL(prefill_history_kernel, grid, dim3(256), 0, stream, p.keyCache,
                                       p.valueCache, kh, vh, per, p.capacity, p.dim, T, p.rangeFlag);
            }))
            return false;
    }

    const float qScale = LOG2E / sqrtf(float(p.dim));
    // prep runs unless the caller did its work: besides q/k/v rows and the
    // cos/sin table it zeroes the working copies' pad rows
    if (!p.prepDone && !ctx.launch("prefill_prep_kernel", stream, [&] {
            const dim3 grid{unsigned(p.count)}, block{256};
            const uint32_t t32 = uint32_t(T);
            if (!vec)
                hipLaunchKernelGGL(prefill_prep_kernel, grid, block,
                                   (p.heads + 2 * p.kvHeads) * p.dim * sizeof(float), stream, p, qh, kh, vh, T,
                                   qScale);
            else if (p.dim == 128 && p.inType == 1)
                hipLaunchKernelGGL((prefill_prep_vec_kernel<128, false>), grid, dim3(PREP_THREADS), 0, stream, p, qh, kh, vh,
                                   t32, qScale, firstRow, rope);
            else if (p.dim == 128)
                hipLaunchKernelGGL((prefill_prep_vec_kernel<128, true>), grid, dim3(PREP_THREADS), 0, stream, p, qh, kh, vh,
                                   t32, qScale, firstRow, rope);
            else if (p.inType == 1)
                hipLaunchKernelGGL((prefill_prep_vec_kernel<64, false>), grid, dim3(PREP_THREADS), 0, stream, p, qh, kh, vh,
                                   t32, qScale, firstRow, rope);
            else
                hipLaunchKernelGGL((prefill_prep_vec_kernel<64, true>), grid, dim3(PREP_THREADS), 0, stream, p, qh, kh, vh,
                                   t32, qScale, firstRow, rope);
        }))
        return false;

    FlashArgs a{};
    a.qh = qh;
    a.kh = kh;
    a.vh = vh;
    a.out = p.out;
    a.outHi = reinterpret_cast<__bf16*>(p.outSplit);
    a.outLo = p.outSplit ? a.outHi + p.count * p.heads * p.dim : nullptr;
    a.count = uint32_t(p.count);
    a.start = uint32_t(p.start);
    a.heads = uint32_t(p.heads);
    a.kvHeads = uint32_t(p.kvHeads);
    a.window = uint32_t(p.window > 0xFFFFFFFFull ? 0 : p.window);
    a.T = uint32_t(T);
    a.fuseQ = fuseQ ? 1u : 0u;
    a.qraw = p.q;
    a.qNorm = p.qNorm;
    a.rope = rope;
    a.eps = p.eps;
    a.normOffset = p.normOffset;
    a.qScale = qScale;
    a.qStride = uint32_t(p.qStride);
    a.inType = uint32_t(p.inType);
    a.half = p.freqs ? uint32_t(p.rotaryDims / 2) : 0u;
    a.outputGate = p.outputGate ? 1u : 0u;
    a.rangeFlag = p.rangeFlag;
    // 8 waves of 32 query rows per workgroup, 128-key tiles: the ping-pong
    // schedule for D = 128, the single-phase loop (two stages) for D = 64
    constexpr int waves = 8;
    a.nQT = uint32_t((p.count + 32 * waves - 1) / (32 * waves));
    const uint64_t blocks = uint64_t(a.nQT) * p.heads;
    a.xcdRemap = (blocks % 8 == 0) ? 1u : 0u;
    return ctx.launch("prefill_flash_kernel", stream, [&] {
        const dim3 grid{unsigned(blocks)}, block{unsigned(64 * waves)};
        if (p.dim == 128)
            hipLaunchKernelGGL((prefill_flash_kernel<128, waves, 2, 128, true>), grid, block, 0, stream, a);
        else
            hipLaunchKernelGGL((prefill_flash_kernel<64, waves, 2, 128, false>), grid, block, 0, stream, a);
    });
}

} // namespace aigpu
