// decode.hip - batched single-token GQA decode for gfx950, HBM-bound.
//
// decode_split_kernel: one workgroup per (sequence b, kv head, chunk of CH
// positions); its 4 waves split the chunk into slabs of 64 positions.
//   - the G query heads of the kv head get QK-RMSNorm and RoPE at position
//     positions[b] on load (attentionMixer, LocalModel.hpp:2608-2648);
//   - the workgroup whose chunk ends at the new token also normalises and
//     rotates the new k, appends k and v to the bf16 cache at positions[b]
//     (LocalModel.hpp:2650-2655) and folds the new token in from registers,
//     so no workgroup reads the slot being written;
//   - scores: v_mfma_f32_16x16x32_bf16 with K rows (straight from HBM, 16-byte
//     loads, each K byte read once for all G heads) as A and q as B, q split
//     into a bf16 high part (columns 0-7) and the bf16 residual (columns 8-15)
//     so the two halves add back to ~16 significant bits;
//   - P.V: v_mfma_f32_16x16x4f32, fp32 P against widened bf16 V rows, with
//     the output columns permuted so each lane loads 16 contiguous bytes of a
//     V row;
//   - online softmax inside a wave, a cross-wave merge in LDS, then one
//     partial (m, l, acc) record per chunk.
// decode_merge_kernel combines a sequence's chunk records (the split-K merge
// algebra of the reference's Metal decoder, src/gpu/Kernels.metal:318-345).
#include "context.hpp"
#include "device.hpp"
#include "kernels.hpp"

#include <cstdlib>

namespace aigpu {

namespace {

constexpr int MAXG = 8;          // query heads per kv head handled by one workgroup
constexpr int SLAB = 64;         // positions per wave step

struct DecodeArgs {
    DecodeParams p;
    float* parts;                // [batch][kvHeads][maxChunks][RS]
    uint32_t chunkLen;           // CH
    uint32_t maxChunks;
    float scaleLog2;
};

__host__ __device__ constexpr int record_floats(int D) { return 2 * MAXG + MAXG * D; }

__device__ __forceinline__ void chunk_range(const DecodeParams& p, uint32_t L, uint32_t& first,
                                            uint32_t& nChunks, uint32_t CH) {
    first = (p.window && uint64_t(L) + 1 > p.window) ? uint32_t(uint64_t(L) + 1 - p.window) : 0u;
    nChunks = (L + 1 - first + CH - 1) / CH;
}

template <int D>
__global__ __launch_bounds__(256, 2) void decode_split_kernel(DecodeArgs a) {
    constexpr int DB = D / 32;   // 32-deep d blocks of the score MFMA
    constexpr int TPL = D / 16;  // value columns each lane carries in the P.V tiles
    constexpr int RS = record_floats(D);
    const DecodeParams& p = a.p;
    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const uint32_t G = uint32_t(p.heads / p.kvHeads);
    const uint32_t L = p.positions[b];
    if (L > p.maxPosition) return;  // outside the launch's bounds: the merge marks it NaN
    uint32_t first, nChunks;
    chunk_range(p, L, first, nChunks, a.chunkLen);
    if (chunk >= nChunks) return;  // uniform over the workgroup
    const uint32_t lo = first + chunk * a.chunkLen;
    const uint32_t hi = (lo + a.chunkLen < L + 1) ? lo + a.chunkLen : L + 1;
    const bool hasNew = hi == L + 1;
    const uint32_t cachedHi = hi < L ? hi : L;   // cached positions are [lo, cachedHi)

    __shared__ float qs[MAXG][D];
    __shared__ float rowbuf[4][D];
    __shared__ float knew[D], vnew[D];
    __shared__ float snew[MAXG];
    __shared__ float wm[4][MAXG], wl[4][MAXG];
    __shared__ float wacc[4][MAXG][D];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const size_t cacheBase = size_t(b) * p.batchStride + size_t(kvh) * p.capacity * D;
    const uint16_t* kc = p.keyCache + cacheBase;
    const uint16_t* vc = p.valueCache + cacheBase;

    // ---- queries (and the new key/value) through norm + RoPE, in fp32 ----
    const uint32_t nrows = G + (hasNew ? 1u : 0u);
    for (uint32_t r = w; r < nrows; r += 4) {
        float* x = rowbuf[w];
        if (r < G) {
            const size_t src = (size_t(b) * p.heads + size_t(kvh) * G + r) * p.qStride;
            for (int d = lane; d < D; d += WAVE) x[d] = load_elem(p.q, src + d, p.inType);
            wave_sync();
            norm_rope_row(x, D, p.qNorm, p.eps, p.normOffset, p.freqs, p.rotaryDims, L, lane);
            for (int d = lane; d < D; d += WAVE) qs[r][d] = x[d] * a.scaleLog2;
        } else {
            const size_t src = (size_t(b) * p.kvHeads + kvh) * D;
            for (int d = lane; d < D; d += WAVE) x[d] = load_elem(p.k, src + d, p.inType);
            wave_sync();
            norm_rope_row(x, D, p.kNorm, p.eps, p.normOffset, p.freqs, p.rotaryDims, L, lane);
            uint16_t* kdst = p.keyCache + cacheBase + size_t(L) * D;
            uint16_t* vdst = p.valueCache + cacheBase + size_t(L) * D;
            for (int d = lane; d < D; d += WAVE) {
                knew[d] = x[d];
                kdst[d] = float_to_bf16_bits(x[d]);
                const float vv = load_elem(p.v, src + d, p.inType);
                vnew[d] = vv;
                vdst[d] = float_to_bf16_bits(vv);
            }
        }
        wave_sync();
    }
    __syncthreads();
    if (hasNew && w == 0) {
        for (uint32_t h = 0; h < G; ++h) {
            float part = 0.0f;
            for (int d = lane; d < D; d += WAVE) part += qs[h][d] * knew[d];
            part = wave_sum(part);
            if (lane == 0) snew[h] = part;
        }
    }

    // ---- q as the B operand: column j < 8 is head j's bf16 high part, column
    //      8 + j its bf16 residual; heads >= G are zero ----
    const int g = lane >> 4, c16 = lane & 15;
    typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
    bf16x8 qb[DB];
    {
        const uint32_t h = c16 & 7;
        const bool residual = c16 >= 8;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            u16x8 bits;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const float x = h < G ? qs[h][32 * db + 8 * g + s] : 0.0f;
                const uint16_t top = float_to_bf16_bits(x);
                bits[s] = residual ? float_to_bf16_bits(x - bf16_bits_to_float(top)) : top;
            }
            qb[db] = __builtin_bit_cast(bf16x8, bits);
        }
    }

    // ---- slabs ----
    float m = -INFINITY, lsum = 0.0f;   // per lane: head c16 & 7
    floatx4 acc[TPL];
#pragma unroll
    for (int t = 0; t < TPL; ++t) acc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    for (uint32_t p0 = lo + SLAB * w; p0 < cachedHi; p0 += 4 * SLAB) {
        const uint32_t lastRow = cachedHi - 1;
        u32x4 kr[4][DB];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            uint32_t row = p0 + 16 * rb + c16;
            if (row > lastRow) row = lastRow;
#pragma unroll
            for (int db = 0; db < DB; ++db)
                kr[rb][db] = *reinterpret_cast<const u32x4*>(kc + size_t(row) * D + 32 * db + 8 * g);
        }
        typedef uint32_t vchunk __attribute__((ext_vector_type(TPL / 2)));
        vchunk vr[4][4];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t row = p0 + 16 * rb + 4 * g + i;
                if (row > lastRow) row = lastRow;
                vr[rb][i] = *reinterpret_cast<const vchunk*>(vc + size_t(row) * D + TPL * c16);
            }

        floatx4 sc[4];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            sc[rb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int db = 0; db < DB; ++db)
                sc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[rb][db]),
                                                                 qb[db], sc[rb], 0, 0, 0);
        }

        float sv[4][4];
        float mx = -INFINITY;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float x = sc[rb][i];
                x += __shfl_xor(x, 8, WAVE);   // high part + residual
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
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sv[rb][i] = exp2f(sv[rb][i] - base);
                ps += sv[rb][i];
            }
        lsum = lsum * alpha + ps;
        m = mn;

        // accumulator rows are heads 4g + r: fetch their rescale factors
        float ar[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, 4 * g + r, WAVE);
#pragma unroll
        for (int t = 0; t < TPL; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[t][r] *= ar[r];

#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int t = 0; t < TPL; ++t) {
                    const uint32_t word = vr[rb][i][t / 2];
                    const float vf = (t & 1) ? __uint_as_float(word & 0xFFFF0000u) : __uint_as_float(word << 16);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(sv[rb][i], vf, acc[t], 0, 0, 0);
                }
            }
    }

    // ---- per-wave state to LDS ----
    lsum += __shfl_xor(lsum, 16, WAVE);
    lsum += __shfl_xor(lsum, 32, WAVE);
    if (g == 0 && c16 < MAXG) {
        wm[w][c16] = m;
        wl[w][c16] = lsum;
    }
    if (g < 2) {
#pragma unroll
        for (int t = 0; t < TPL; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) wacc[w][4 * g + r][TPL * c16 + t] = acc[t][r];
    }
    __syncthreads();

    // ---- merge the waves (and the new token) into this chunk's record ----
    float* rec = a.parts + ((size_t(b) * p.kvHeads + kvh) * a.maxChunks + chunk) * RS;
    for (uint32_t idx = tid; idx < G * D; idx += 256) {
        const uint32_t h = idx / D, d = idx % D;
        float M = fmaxf(fmaxf(wm[0][h], wm[1][h]), fmaxf(wm[2][h], wm[3][h]));
        if (hasNew) M = fmaxf(M, snew[h]);
        float lt = 0.0f, at = 0.0f;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
            const float f = wm[ww][h] == -INFINITY ? 0.0f : exp2f(wm[ww][h] - M);
            lt += wl[ww][h] * f;
            at += wacc[ww][h][d] * f;
        }
        if (hasNew) {
            const float f = exp2f(snew[h] - M);
            lt += f;
            at += f * vnew[d];
        }
        rec[2 * MAXG + h * D + d] = at;
        if (d == 0) {
            rec[h] = M;
            rec[MAXG + h] = lt;
        }
    }
}

template <int D>
__global__ __launch_bounds__(128) void decode_merge_kernel(DecodeArgs a) {
    constexpr int RS = record_floats(D);
    const DecodeParams& p = a.p;
    const uint32_t hq = blockIdx.x, b = blockIdx.y;
    const uint32_t G = uint32_t(p.heads / p.kvHeads);
    const uint32_t kvh = hq / G, h = hq % G;
    const uint32_t L = p.positions[b];
    const int d = threadIdx.x;
    if (d >= D) return;
    if (L > p.maxPosition) {   // a position the caller's maxPosition did not cover
        p.out[(size_t(b) * p.heads + hq) * D + d] = __builtin_nanf("");
        return;
    }
    uint32_t first, nChunks;
    chunk_range(p, L, first, nChunks, a.chunkLen);
    const float* recs = a.parts + (size_t(b) * p.kvHeads + kvh) * a.maxChunks * RS;
    float M = -INFINITY;
    for (uint32_t c = 0; c < nChunks; ++c) M = fmaxf(M, recs[size_t(c) * RS + h]);
    float lt = 0.0f, at = 0.0f;
    for (uint32_t c = 0; c < nChunks; ++c) {
        const float* r = recs + size_t(c) * RS;
        const float f = exp2f(r[h] - M);
        lt += r[MAXG + h] * f;
        at += r[2 * MAXG + h * D + d] * f;
    }
    p.out[(size_t(b) * p.heads + hq) * D + d] = at / lt;
}

uint32_t decode_chunk_len() {
    static uint32_t len = [] {
        const char* env = std::getenv("AIGPU_DECODE_CHUNK");
        long v = env ? std::atol(env) : 512;
        if (v < 256) v = 256;
        v = v / 256 * 256;
        return uint32_t(v);
    }();
    return len;
}

} // namespace

bool launch_decode(const DecodeParams& p, hipStream_t stream) {
    Context& ctx = Context::instance();
    if (p.dim != 64 && p.dim != 128) return ctx.fail("decode: dim must be 64 or 128");
    if (p.kvHeads == 0 || p.heads % p.kvHeads) return ctx.fail("decode: heads must be a multiple of kvHeads");
    if (p.heads / p.kvHeads > MAXG) return ctx.fail("decode: at most 8 query heads per kv head");
    if (p.qStride < p.dim) return ctx.fail("decode: qStride < dim");
    if (p.freqs && (p.rotaryDims == 0 || p.rotaryDims > int(p.dim) || (p.rotaryDims & 1)))
        return ctx.fail("decode: rotaryDims must be even and within dim");
    if (p.inType != 0 && p.inType != 1) return ctx.fail("decode: unknown input type");
    if (!p.q || !p.k || !p.v || !p.out || !p.keyCache || !p.valueCache || !p.positions)
        return ctx.fail("decode: null tensor");
    if (p.batch == 0) return true;
    if (uint64_t(p.maxPosition) + 1 > p.capacity)
        return ctx.fail("decode: maxPosition + 1 exceeds the cache capacity");
    if (p.batch > 65535 || p.kvHeads > 65535) return ctx.fail("decode: batch or kvHeads too large");

    DecodeArgs a{};
    a.p = p;
    if (a.p.batchStride == 0) a.p.batchStride = p.kvHeads * p.capacity * p.dim;
    a.chunkLen = decode_chunk_len();
    a.maxChunks = (p.maxPosition + 1 + a.chunkLen - 1) / a.chunkLen;
    a.scaleLog2 = LOG2E / sqrtf(float(p.dim));
    const size_t rs = size_t(record_floats(int(p.dim)));
    a.parts = static_cast<float*>(
        ctx.grow(SLOT_DECODE_PARTS, p.batch * p.kvHeads * a.maxChunks * rs * sizeof(float)));
    if (!a.parts) return false;

    const dim3 grid(a.maxChunks, unsigned(p.kvHeads), unsigned(p.batch));
    const dim3 mgrid(unsigned(p.heads), unsigned(p.batch));
    if (p.dim == 128) {
        if (!ctx.launch("decode_split_kernel", stream, [&] {
                hipLaunchKernelGGL(decode_split_kernel<128>, grid, dim3(256), 0, stream, a);
            }))
            return false;
        return ctx.launch("decode_merge_kernel", stream, [&] {
            hipLaunchKernelGGL(decode_merge_kernel<128>, mgrid, dim3(128), 0, stream, a);
        });
    }
    if (!ctx.launch("decode_split_kernel", stream, [&] {
            hipLaunchKernelGGL(decode_split_kernel<64>, grid, dim3(256), 0, stream, a);
        }))
        return false;
    return ctx.launch("decode_merge_kernel", stream, [&] {
        hipLaunchKernelGGL(decode_merge_kernel<64>, mgrid, dim3(128), 0, stream, a);
    });
}

} // namespace aigpu
