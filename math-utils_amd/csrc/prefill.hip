// prefill.hip - causal GQA prefill for gfx950.
//
// Three launches per call:
//   prefill_history_kernel  converts cached positions [0, start) of the bf16
//                           cache to the fp16 working copies (exact: every
//                           bf16 value in fp16's range is an fp16 value)
//   prefill_prep_kernel     attentionMixer's QK-RMSNorm -> RoPE -> KV append
//                           (LocalModel.hpp:2608-2655) for the new tokens, in
//                           fp32; writes the bf16 cache and the fp16 copies
//   prefill_flash_kernel    flash attention on v_mfma_f32_32x32x16_f16 with
//                           fp32 accumulation and an online softmax
//
// Why fp16 operands: Q, K and P rounded to bf16 (8 significant bits) give
// max-abs errors near 6e-3 on the 8k configuration; fp16 (11 bits) keeps
// them near 5e-4, inside the 2e-3 bound, at the same MFMA rate. The KV cache
// itself stays bf16.
//
// Flash kernel layout (one workgroup = 4 waves = 128 query rows of one head,
// one wave = 32 rows; key tiles of 64):
//   S^T = K Q^T     A = K rows (LDS), B = Q^T (registers, loaded once)
//                   -> each lane owns one query (lane % 32) and 16 keys, so
//                      the row max/sum need one exchange with lane ^ 32
//   O^T += V^T P^T  A = V^T (LDS, stored transposed), B = P^T straight from
//                      the S^T accumulators -> the softmax rescale of O is
//                      lane-local
// The K tile rows are stored permuted so that accumulator register r of the
// S^T tile holds key 16*(lane/32) + r, which makes each lane's 8-key slice of
// P^T contiguous in Vt.
#include "context.hpp"
#include "device.hpp"
#include "kernels.hpp"

namespace aigpu {

namespace {

constexpr int PREP_MAX_DIM = 256;

__global__ __launch_bounds__(256) void prefill_history_kernel(
    const uint16_t* __restrict__ keyCache, const uint16_t* __restrict__ valueCache,
    _Float16* __restrict__ kh, _Float16* __restrict__ vh, uint64_t kvHeads, uint64_t start,
    uint64_t capacity, uint64_t dim, uint64_t T) {
    const uint64_t per = start * dim, total = kvHeads * per;
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += uint64_t(gridDim.x) * blockDim.x) {
        const uint64_t kv = i / per, rem = i % per;
        const uint64_t src = kv * capacity * dim + rem, dst = kv * T * dim + rem;
        kh[dst] = _Float16(bf16_bits_to_float(keyCache[src]));
        vh[dst] = _Float16(bf16_bits_to_float(valueCache[src]));
    }
}

/* one wave per (token, head-row); rows [0, heads) are queries, the rest KV heads */
__global__ __launch_bounds__(256) void prefill_prep_kernel(PrefillParams p, _Float16* __restrict__ qh,
                                                           _Float16* __restrict__ kh,
                                                           _Float16* __restrict__ vh, uint64_t T) {
    __shared__ float rows[4][PREP_MAX_DIM];
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const uint64_t perToken = p.heads + p.kvHeads;
    const uint64_t r = uint64_t(blockIdx.x) * 4 + w;
    if (r >= p.count * perToken) return;
    const uint64_t t = r / perToken, h = r % perToken;
    const uint64_t pos = p.start + t;
    const int dim = int(p.dim);
    float* x = rows[w];

    if (h < p.heads) {
        const uint64_t src = (t * p.heads + h) * p.qStride;
        for (int d = lane; d < dim; d += WAVE) x[d] = load_elem(p.q, src + d, p.inType);
        wave_sync();
        norm_rope_row(x, dim, p.qNorm, p.eps, p.normOffset, p.freqs, p.rotaryDims, pos, lane);
        _Float16* dst = qh + (h * p.count + t) * p.dim;
        for (int d = lane; d < dim; d += WAVE) dst[d] = _Float16(x[d]);
    } else {
        const uint64_t kv = h - p.heads;
        const uint64_t src = (t * p.kvHeads + kv) * p.dim;
        for (int d = lane; d < dim; d += WAVE) x[d] = load_elem(p.k, src + d, p.inType);
        wave_sync();
        norm_rope_row(x, dim, p.kNorm, p.eps, p.normOffset, p.freqs, p.rotaryDims, pos, lane);
        const uint64_t work = (kv * T + pos) * p.dim;
        const uint64_t cache = (kv * p.capacity + pos) * p.dim;
        for (int d = lane; d < dim; d += WAVE) {
            kh[work + d] = _Float16(x[d]);
            p.keyCache[cache + d] = float_to_bf16_bits(x[d]);
            const float vv = load_elem(p.v, src + d, p.inType);
            vh[work + d] = _Float16(vv);
            p.valueCache[cache + d] = float_to_bf16_bits(vv);
        }
    }
}

struct FlashArgs {
    const _Float16* qh;  // [heads][count][D]
    const _Float16* kh;  // [kvHeads][T][D]
    const _Float16* vh;  // [kvHeads][T][D]
    float* out;          // [count][heads][D]
    uint32_t count, start, heads, kvHeads, window, T, nQT, xcdRemap;
    float scaleLog2;
};

/* LDS row of key k (0..31) inside a 32-key block: the inverse of the A-row to
   key map pi(i) = 16*((i>>2)&1) + 4*(i>>3) + (i&3) */
__device__ __forceinline__ int key_to_lds_row(int k) {
    return 8 * ((k >> 2) & 3) + 4 * (k >> 4) + (k & 3);
}

template <int D>
__global__ __launch_bounds__(256, 2) void prefill_flash_kernel(FlashArgs a) {
    constexpr int BM = 128, BN = 64;
    constexpr int DB = D / 16;        // 16-wide d blocks of the S^T product
    constexpr int DT = D / 32;        // 32-wide d tiles of the O^T accumulator
    constexpr int KSTR = D + 8;       // halfs per K row in LDS
    constexpr int VSTR = BN + 8;      // halfs per V^T row in LDS
    constexpr int KCH = D / 8;        // 16-byte chunks per K row
    constexpr int KLOADS = BN * KCH / 256;
    __shared__ __attribute__((aligned(16))) _Float16 Ks[BN * KSTR];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[D * VSTR];

    uint32_t bid = blockIdx.x;
    if (a.xcdRemap) bid = (bid % 8) * (gridDim.x / 8) + bid / 8;
    const uint32_t head = bid % a.heads;
    const uint32_t qt = a.nQT - 1 - bid / a.heads;   // longest rows first
    const uint32_t kvh = head / (a.heads / a.kvHeads);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, c = lane & 31;

    const uint32_t q0 = qt * BM;
    const uint32_t wq0 = q0 + 32 * w;
    const uint32_t tq = wq0 + c;
    const bool rowValid = tq < a.count;
    const uint32_t P = a.start + tq;
    const bool waveActive = wq0 < a.count;
    const uint32_t wLast = (wq0 + 31 < a.count ? wq0 + 31 : a.count - 1);
    const uint32_t wPosFirst = a.start + wq0, wPosLast = a.start + wLast;

    half8 qreg[DB];
    {
        const _Float16* qrow = a.qh + (size_t(head) * a.count + (rowValid ? tq : 0)) * D;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            if (rowValid) qreg[db] = *reinterpret_cast<const half8*>(qrow + 16 * db + 8 * g);
            else qreg[db] = half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
    }

    floatx16 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] = 0.0f;
    float m = -INFINITY, lsum = 0.0f;

    const uint32_t tileLast = (q0 + BM < a.count ? q0 + BM : a.count) - 1;
    const uint32_t kend = a.start + tileLast + 1;
    uint32_t kbeg = 0;
    if (a.window && a.start + q0 + 1 > a.window) kbeg = a.start + q0 + 1 - a.window;
    kbeg = kbeg / BN * BN;

    const _Float16* kbase = a.kh + size_t(kvh) * a.T * D;
    const _Float16* vbase = a.vh + size_t(kvh) * a.T * D;
    const int vkq = tid & 15, vdq = tid >> 4;   // V^T staging: keys 4*vkq.., d 8*vdq..
    u32x4 kreg[KLOADS];
    u32x4 vreg[4];

    auto gload = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < KLOADS; ++i) {
            const int cidx = tid + 256 * i, row = cidx / KCH, col = cidx % KCH;
            uint32_t src = k0 + row;
            if (src > a.T - 1) src = a.T - 1;
            kreg[i] = *reinterpret_cast<const u32x4*>(kbase + size_t(src) * D + col * 8);
        }
        if (vdq < D / 8) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint32_t src = k0 + 4 * vkq + i;
                if (src > a.T - 1) src = a.T - 1;
                vreg[i] = *reinterpret_cast<const u32x4*>(vbase + size_t(src) * D + vdq * 8);
            }
        }
    };
    auto lstore = [&]() {
#pragma unroll
        for (int i = 0; i < KLOADS; ++i) {
            const int cidx = tid + 256 * i, row = cidx / KCH, col = cidx % KCH;
            const int lrow = (row & ~31) + key_to_lds_row(row & 31);
            *reinterpret_cast<u32x4*>(&Ks[lrow * KSTR + col * 8]) = kreg[i];
        }
        if (vdq < D / 8) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // dword e of each key row holds d = 8*vdq + 2e (low half) and +1 (high half)
                u32x2 even, odd;
                even[0] = (vreg[0][e] & 0xFFFFu) | (vreg[1][e] << 16);
                even[1] = (vreg[2][e] & 0xFFFFu) | (vreg[3][e] << 16);
                odd[0] = (vreg[0][e] >> 16) | (vreg[1][e] & 0xFFFF0000u);
                odd[1] = (vreg[2][e] >> 16) | (vreg[3][e] & 0xFFFF0000u);
                const int d = 8 * vdq + 2 * e;
                *reinterpret_cast<u32x2*>(&Vt[d * VSTR + 4 * vkq]) = even;
                *reinterpret_cast<u32x2*>(&Vt[(d + 1) * VSTR + 4 * vkq]) = odd;
            }
        }
    };

    if (kbeg < kend) gload(kbeg);
    for (uint32_t k0 = kbeg; k0 < kend; k0 += BN) {
        __syncthreads();
        lstore();
        __syncthreads();
        if (k0 + BN < kend) gload(k0 + BN);

        bool active = waveActive && k0 <= wPosLast;
        if (a.window && uint64_t(k0) + BN - 1 + a.window < uint64_t(wPosFirst) + 1) active = false;
        if (!active) continue;

        floatx16 s[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int r = 0; r < 16; ++r) s[kb][r] = 0.0f;
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                const half8 ka = *reinterpret_cast<const half8*>(&Ks[(32 * kb + c) * KSTR + 16 * db + 8 * g]);
                s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qreg[db], s[kb], 0, 0, 0);
            }
        }

        const bool needMask = (k0 + BN - 1 > wPosFirst) ||
                              (a.window && uint64_t(k0) + a.window < uint64_t(wPosLast) + 1);
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float x = s[kb][r] * a.scaleLog2;
                if (needMask) {
                    const uint32_t key = k0 + 32 * kb + 16 * g + r;
                    if (key > P || (a.window && uint64_t(key) + a.window <= P)) x = -INFINITY;
                }
                s[kb][r] = x;
                mx = fmaxf(mx, x);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 32, WAVE));
        const float mn = fmaxf(m, mx);
        const float base = mn == -INFINITY ? 0.0f : mn;
        const float alpha = exp2f(m - base);
        float ps = 0.0f;
        half8 pk[2][2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float pv = exp2f(s[kb][8 * h + j] - base);
                    ps += pv;
                    pk[kb][h][j] = _Float16(pv);
                }
        lsum = lsum * alpha + ps;
        m = mn;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
            for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const half8 va = *reinterpret_cast<const half8*>(
                        &Vt[(32 * dt + c) * VSTR + 32 * kb + 16 * g + 8 * h]);
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pk[kb][h], o[dt], 0, 0, 0);
                }
        }
    }

    lsum += __shfl_xor(lsum, 32, WAVE);
    if (rowValid) {
        const float inv = 1.0f / lsum;
        float* dst = a.out + (size_t(tq) * a.heads + head) * D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                floatx4 val;
#pragma unroll
                for (int i = 0; i < 4; ++i) val[i] = o[dt][4 * r4 + i] * inv;
                *reinterpret_cast<floatx4*>(dst + 32 * dt + 8 * r4 + 4 * g) = val;
            }
    }
}

} // namespace

bool launch_prefill(const PrefillParams& p, hipStream_t stream) {
    Context& ctx = Context::instance();
    if (p.dim != 64 && p.dim != 128) return ctx.fail("prefill: dim must be 64 or 128");
    if (p.kvHeads == 0 || p.heads % p.kvHeads) return ctx.fail("prefill: heads must be a multiple of kvHeads");
    if (p.qStride < p.dim) return ctx.fail("prefill: qStride < dim");
    if (p.freqs && (p.rotaryDims == 0 || p.rotaryDims > int(p.dim) || (p.rotaryDims & 1)))
        return ctx.fail("prefill: rotaryDims must be even and within dim");
    if (p.inType != 0 && p.inType != 1) return ctx.fail("prefill: unknown input type");
    if (!p.q || !p.k || !p.v || !p.out || !p.keyCache || !p.valueCache) return ctx.fail("prefill: null tensor");
    if (p.count == 0) return true;
    const uint64_t T = p.start + p.count;
    if (p.capacity < T) return ctx.fail("prefill: cache capacity below start + count");
    if (T >= (1ull << 31) || p.heads * p.count >= (1ull << 31))
        return ctx.fail("prefill: sequence too long");

    _Float16* qh = static_cast<_Float16*>(ctx.grow(SLOT_PREFILL_Q, p.heads * p.count * p.dim * 2));
    _Float16* kh = static_cast<_Float16*>(ctx.grow(SLOT_PREFILL_K, p.kvHeads * T * p.dim * 2));
    _Float16* vh = static_cast<_Float16*>(ctx.grow(SLOT_PREFILL_V, p.kvHeads * T * p.dim * 2));
    if (!qh || !kh || !vh) return false;

    if (p.start > 0) {
        const uint64_t total = p.kvHeads * p.start * p.dim;
        uint64_t blocks = (total + 255) / 256;
        if (blocks > 65536) blocks = 65536;
        if (!ctx.launch("prefill_history_kernel", stream, [&] {
                hipLaunchKernelGGL(prefill_history_kernel, dim3(unsigned(blocks)), dim3(256), 0, stream,
                                   p.keyCache, p.valueCache, kh, vh, p.kvHeads, p.start, p.capacity,
                                   p.dim, T);
            }))
            return false;
    }

    const uint64_t rows = p.count * (p.heads + p.kvHeads);
    if (!ctx.launch("prefill_prep_kernel", stream, [&] {
            hipLaunchKernelGGL(prefill_prep_kernel, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, stream,
                               p, qh, kh, vh, T);
        }))
        return false;

    FlashArgs a{};
    a.qh = qh;
    a.kh = kh;
    a.vh = vh;
    a.out = p.out;
    a.count = uint32_t(p.count);
    a.start = uint32_t(p.start);
    a.heads = uint32_t(p.heads);
    a.kvHeads = uint32_t(p.kvHeads);
    a.window = uint32_t(p.window > 0xFFFFFFFFull ? 0 : p.window);
    a.T = uint32_t(T);
    a.nQT = uint32_t((p.count + 127) / 128);
    a.scaleLog2 = LOG2E / sqrtf(float(p.dim));
    const uint64_t blocks = uint64_t(a.nQT) * p.heads;
    a.xcdRemap = (blocks % 8 == 0) ? 1u : 0u;
    if (p.dim == 128)
        return ctx.launch("prefill_flash_kernel", stream, [&] {
            hipLaunchKernelGGL(prefill_flash_kernel<128>, dim3(unsigned(blocks)), dim3(256), 0, stream, a);
        });
    return ctx.launch("prefill_flash_kernel", stream, [&] {
        hipLaunchKernelGGL(prefill_flash_kernel<64>, dim3(unsigned(blocks)), dim3(256), 0, stream, a);
    });
}

} // namespace aigpu
