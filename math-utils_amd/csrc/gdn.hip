// gdn.hip - the Gated DeltaNet steps either side of the recurrence
// (gatedDeltaNetMixer, LocalModel.hpp:2724-2844) for gfx950. Both are
// HBM-bound streams, so the kernels are laid out for coalesced 8- or 16-byte
// accesses and nothing else:
//   gdn_conv_kernel        the linFusedQKVZ de-interleave (:2739-2776) fused
//                          with causalConvolution + SiLU (:2678-2708): reads
//                          the projection rows once, writes dense q, k, v (the
//                          delta rule's inputs) and, for the fused layout, z
//                          and the b/a gate inputs
//   gdn_window_kernel      the carried window (the last K-1 inputs), after
//                          the convolution has read the old one
//   gdn_gated_norm_kernel  rmsNormRow of each (token, value head) row times
//                          SiLU(z) (:2833-2841), or times sigmoid(z) as
//                          kimiDeltaMixer gates its rows (:2936-2945)
#include "context.hpp"
#include "device.hpp"
#include "kernels.hpp"

namespace aigpu {

namespace {

constexpr int MAXK = 8;    // largest convolution kernel
constexpr int TB = 16;     // tokens per convolution thread (16 measured 5% faster than 32)
constexpr int UNROLL = 16; // tokens whose loads a thread has in flight together

/* siluOf (LocalModel.hpp:1369), x / (1 + e^-x), with the hardware exp2 and
   reciprocal (about 2 ulp) in place of a correctly rounded exp and divide:
   these kernels are otherwise VALU-bound on the exact forms. e^-x overflows
   to infinity for x < -88 and the reciprocal to 0, so SiLU goes to -0 there. */
__device__ __forceinline__ float fast_sigmoid(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * LOG2E));
}
__device__ __forceinline__ float silu_of(float x) { return x * fast_sigmoid(x); }

/* N (4 or 8) consecutive elements at element index i of an fp32 or bf16
   tensor, as fp32 */
template <bool BF16, int N>
__device__ __forceinline__ void loadN(const void* base, size_t i, float (&x)[N]) {
    if constexpr (BF16) {
        if constexpr (N == 8) {
            const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + i);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[2 * e] = __uint_as_float(w[e] << 16);
                x[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
            }
        } else {
            const u32x2 w = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(base) + i);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                x[2 * e] = __uint_as_float(w[e] << 16);
                x[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
            }
        }
    } else {
#pragma unroll
        for (int h = 0; h < N / 4; ++h) {
            const floatx4 v = *reinterpret_cast<const floatx4*>(static_cast<const float*>(base) + i + 4 * h);
#pragma unroll
            for (int e = 0; e < 4; ++e) x[4 * h + e] = v[e];
        }
    }
}

template <bool BF16, int N>
__device__ __forceinline__ void storeN(void* base, size_t i, const float (&x)[N]) {
    if constexpr (BF16) {
        // round to nearest even in hardware (v_cvt_pk_bf16_f32)
        uint32_t w[N / 2];
#pragma unroll
        for (int e = 0; e < N / 2; ++e) {
            typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
            w[e] = __builtin_bit_cast(uint32_t, bf16x2{__bf16(x[2 * e]), __bf16(x[2 * e + 1])});
        }
        if constexpr (N == 8)
            *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(base) + i) = u32x4{w[0], w[1], w[2], w[3]};
        else
            *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(base) + i) = u32x2{w[0], w[1]};
    } else {
#pragma unroll
        for (int h = 0; h < N / 4; ++h)
            *reinterpret_cast<floatx4*>(static_cast<float*>(base) + i + 4 * h) =
                floatx4{x[4 * h], x[4 * h + 1], x[4 * h + 2], x[4 * h + 3]};
    }
}

struct ConvArgs {
    GdnConvParams p;
    uint32_t KW, VW, CW, groups;   // groups: 8-channel groups of CW (+ VW for z, + b/a heads, fused)
};

/* element index, within the input rows, of convolution channel c (q | k | v
   order) of token t; the fused layout holds per key head q, k, the group's v
   and the group's z (LocalModel.hpp:2739-2776). Split into a per-channel
   offset and a per-token row start. */
template <bool FUSED>
__device__ __forceinline__ size_t channel_offset(const ConvArgs& a, uint32_t c) {
    const GdnConvParams& p = a.p;
    if constexpr (!FUSED) return c;
    const uint32_t KD = uint32_t(p.keyDim), VD = uint32_t(p.valueDim);
    const uint32_t G = uint32_t(p.valueHeads / p.keyHeads);
    const size_t stride = 2 * KD + 2 * size_t(G) * VD;
    if (c < a.KW) return (c / KD) * stride + c % KD;
    if (c < 2 * a.KW) return ((c - a.KW) / KD) * stride + KD + (c - a.KW) % KD;
    const uint32_t vc = c - 2 * a.KW, vh = vc / VD;
    return (vh / G) * stride + 2 * KD + (vh % G) * VD + vc % VD;
}
template <bool FUSED>
__device__ __forceinline__ size_t row_elems(const ConvArgs& a) {
    const GdnConvParams& p = a.p;
    if constexpr (!FUSED) return a.CW;
    return p.keyHeads * (2 * p.keyDim + 2 * (p.valueHeads / p.keyHeads) * p.valueDim);
}

/*
    Thread = 8 consecutive channels x TB consecutive tokens (one 16-byte bf16
    load per token). The K-1 previous inputs of each channel stay in registers
    as the thread walks its tokens, so every input is read once (plus a K-1
    row halo per block); the first block reads its halo from the carried
    window. KT is the kernel size when fixed at compile time (4, the models'
    value), 0 for any size up to MAXK. Channel groups past CW copy the fused
    layout's z rows; one more range de-interleaves b and a.
*/
template <bool IN_BF16, bool OUT_BF16, bool FUSED, int KT>
__global__ __launch_bounds__(256) void gdn_conv_kernel(ConvArgs a) {
    constexpr int CPT = 8;
    constexpr int KM = KT ? KT : MAXK;   // register taps
    const GdnConvParams& p = a.p;
    const uint32_t grp = blockIdx.x * 256 + threadIdx.x;
    const uint64_t t0 = uint64_t(blockIdx.y) * TB;
    const uint32_t K = KT ? uint32_t(KT) : uint32_t(p.kernelSize);
    const uint64_t tEnd = t0 + TB < p.count ? t0 + TB : p.count;
    const size_t rowE = row_elems<FUSED>(a);
    if (grp < a.CW / CPT) {
        const uint32_t c = CPT * grp;
        const size_t off = channel_offset<FUSED>(a, c);
        float w[CPT][KM];
#pragma unroll
        for (int e = 0; e < CPT; ++e)
#pragma unroll
            for (int j = 0; j < KM; ++j) w[e][j] = uint32_t(j) < K ? p.kernel[(c + e) * K + j] : 0.0f;
        float wcur[CPT];   // the current token's tap, K - 1
#pragma unroll
        for (int e = 0; e < CPT; ++e) {
            wcur[e] = w[e][0];
#pragma unroll
            for (int j = 1; j < KM; ++j)
                if (uint32_t(j) == K - 1) wcur[e] = w[e][j];
        }
        // hist[j]: input of token t - (K-1) + j, j < K-1, before token t
        float hist[KM > 1 ? KM - 1 : 1][CPT];
#pragma unroll
        for (int j = 0; j < KM - 1; ++j) {
#pragma unroll
            for (int e = 0; e < CPT; ++e) hist[j][e] = 0.0f;
            if (uint32_t(j) < K - 1) {
                const int64_t at = int64_t(t0) - int64_t(K - 1) + j;
                if (at >= 0) {
                    loadN<IN_BF16, CPT>(p.in, uint64_t(at) * rowE + off, hist[j]);
                } else {
                    const float* src = p.window + size_t(int64_t(K - 1) + at) * a.CW + c;
#pragma unroll
                    for (int e = 0; e < CPT; ++e) hist[j][e] = src[e];
                }
            }
        }
        // the dense output this channel range feeds
        void* dst;
        uint32_t dc, dw;
        if (c < a.KW) dst = p.q, dc = c, dw = a.KW;
        else if (c < 2 * a.KW) dst = p.k, dc = c - a.KW, dw = a.KW;
        else dst = p.v, dc = c - 2 * a.KW, dw = a.VW;
        // UNROLL tokens' loads go out together (rows past the end re-read the
        // last row), then the tokens are computed in order
        for (uint64_t tb = t0; tb < tEnd; tb += UNROLL) {
            float xs[UNROLL][CPT];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u)
                loadN<IN_BF16, CPT>(p.in, (tb + u < p.count ? tb + u : p.count - 1) * rowE + off, xs[u]);
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                if (tb + u >= tEnd) break;   // uniform over the workgroup
                float o[CPT];
#pragma unroll
                for (int e = 0; e < CPT; ++e) {
                    // taps in the reference's order: j = 0 (oldest) .. K-1 (current)
                    float acc = 0.0f;
#pragma unroll
                    for (int j = 0; j < KM - 1; ++j)
                        if (uint32_t(j) < K - 1) acc += w[e][j] * hist[j][e];
                    acc += wcur[e] * xs[u][e];
                    o[e] = silu_of(acc);
                }
                storeN<OUT_BF16, CPT>(dst, (tb + u) * dw + dc, o);
#pragma unroll
                for (int j = 0; j + 1 < KM - 1; ++j)
                    if (uint32_t(j) + 1 < K - 1)
#pragma unroll
                        for (int e = 0; e < CPT; ++e) hist[j][e] = hist[j + 1][e];
#pragma unroll
                for (int j = 0; j < KM - 1; ++j)
                    if (uint32_t(j) == K - 2)
#pragma unroll
                        for (int e = 0; e < CPT; ++e) hist[j][e] = xs[u][e];
            }
        }
        return;
    }
    if constexpr (FUSED) {
        const uint32_t KD = uint32_t(p.keyDim), VD = uint32_t(p.valueDim);
        const uint32_t G = uint32_t(p.valueHeads / p.keyHeads);
        const size_t stride = 2 * KD + 2 * size_t(G) * VD;
        if (grp < (a.CW + a.VW) / CPT) {   // z: copied, not convolved
            const uint32_t zc = CPT * grp - a.CW, vh = zc / VD, kh = vh / G;
            const size_t zoff = kh * stride + 2 * KD + size_t(G) * VD + (vh % G) * VD + zc % VD;
            for (uint64_t tb = t0; tb < tEnd; tb += UNROLL) {
                float xs[UNROLL][CPT];
#pragma unroll
                for (int u = 0; u < UNROLL; ++u)
                    loadN<IN_BF16, CPT>(p.in, (tb + u < p.count ? tb + u : p.count - 1) * rowE + zoff, xs[u]);
#pragma unroll
                for (int u = 0; u < UNROLL; ++u)
                    if (tb + u < tEnd) storeN<OUT_BF16, CPT>(p.z, (tb + u) * a.VW + zc, xs[u]);
            }
            return;
        }
        const uint32_t vh = grp - (a.CW + a.VW) / CPT;   // b, a of one value head
        if (vh < p.valueHeads) {
            const uint32_t kh = vh / G, j = vh % G;
            for (uint64_t t = t0; t < tEnd; ++t) {
                const size_t pair = (t * p.keyHeads + kh) * 2 * G;
                p.b[t * p.valueHeads + vh] = load_elem(p.ba, pair + j, IN_BF16 ? 1 : 0);
                p.a[t * p.valueHeads + vh] = load_elem(p.ba, pair + G + j, IN_BF16 ? 1 : 0);
            }
        }
    }
}

/* the window after the call: the last K-1 inputs of window ++ in, in fp32
   (LocalModel.hpp:2700-2707); one thread per channel reads its K-1 values
   before writing any, so the in-place shift of a short call is safe */
template <bool IN_BF16, bool FUSED>
__global__ __launch_bounds__(256) void gdn_window_kernel(ConvArgs a) {
    const GdnConvParams& p = a.p;
    const uint32_t c = blockIdx.x * 256 + threadIdx.x;
    if (c >= a.CW) return;
    const uint32_t K = uint32_t(p.kernelSize);
    const size_t off = channel_offset<FUSED>(a, c), rowE = row_elems<FUSED>(a);
    float next[MAXK - 1];
#pragma unroll
    for (int i = 0; i < MAXK - 1; ++i) {
        next[i] = 0.0f;
        if (uint32_t(i) < K - 1) {
            const int64_t at = int64_t(p.count) - int64_t(K - 1) + i;
            next[i] = at >= 0 ? load_elem(p.in, uint64_t(at) * rowE + off, IN_BF16 ? 1 : 0)
                              : p.window[size_t(int64_t(K - 1) + at) * a.CW + c];
        }
    }
#pragma unroll
    for (int i = 0; i < MAXK - 1; ++i)
        if (uint32_t(i) < K - 1) p.window[size_t(i) * a.CW + c] = next[i];
}

/* rmsNormRow with the weight stored directly (offset 0), then x SiLU(z)
   (LocalModel.hpp:2833-2841). LPR lanes per (token, value head) row, 4
   elements per lane and step: a wave takes 64 / LPR rows at once, so short
   rows (valueDim 128: 32 lanes) still use every lane. */
template <bool Z_BF16, bool OUT_BF16, int LPR>
__global__ __launch_bounds__(256) void gdn_gated_norm_kernel(GdnGatedNormParams p) {
    constexpr int RPW = WAVE / LPR;
    const int lane = threadIdx.x & 63;
    const uint64_t row = (uint64_t(blockIdx.x) * 4 + (threadIdx.x >> 6)) * RPW + lane / LPR;
    const int sub = lane % LPR;
    const bool live = row < p.count * p.valueHeads;
    const uint32_t VD = uint32_t(p.valueDim);
    const uint64_t r = live ? row : 0;
    const float* x = p.x + r * VD;
    // the first piece's x, gamma and z are requested together, before the
    // reduction waits (at VD = 4 LPR that is the whole row)
    const uint32_t d0 = 4 * sub;
    const floatx4 v0 = *reinterpret_cast<const floatx4*>(x + d0);
    const floatx4 g0 = *reinterpret_cast<const floatx4*>(p.gamma + d0);
    float z0[4];
    loadN<Z_BF16, 4>(p.z, r * VD + d0, z0);
    float ss = v0[0] * v0[0] + v0[1] * v0[1] + v0[2] * v0[2] + v0[3] * v0[3];
    for (uint32_t d = d0 + 4 * LPR; d < VD; d += 4 * LPR) {
        const floatx4 v = *reinterpret_cast<const floatx4*>(x + d);
        ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
    }
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) ss += __shfl_xor(ss, o, WAVE);
    const float inv = 1.0f / sqrtf(ss / float(VD) + p.eps);
    if (!live) return;
    {
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float s = fast_sigmoid(z0[e]);
            o[e] = v0[e] * inv * g0[e] * (p.sigmoidGate ? s : z0[e] * s);
        }
        storeN<OUT_BF16, 4>(p.out, r * VD + d0, o);
    }
    for (uint32_t d = d0 + 4 * LPR; d < VD; d += 4 * LPR) {
        const floatx4 v = *reinterpret_cast<const floatx4*>(x + d);
        const floatx4 gm = *reinterpret_cast<const floatx4*>(p.gamma + d);
        float z[4], o[4];
        loadN<Z_BF16, 4>(p.z, r * VD + d, z);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float s = fast_sigmoid(z[e]);
            o[e] = v[e] * inv * gm[e] * (p.sigmoidGate ? s : z[e] * s);
        }
        storeN<OUT_BF16, 4>(p.out, r * VD + d, o);
    }
}

} // namespace

bool launch_gdn_conv(const GdnConvParams& p, hipStream_t stream) {
    Context& ctx = Context::instance();
    if (p.inType > 1 || p.outType > 1) return ctx.fail("gdn conv: unknown tensor type");
    if (p.keyHeads == 0 || p.valueHeads % p.keyHeads) return ctx.fail("gdn conv: valueHeads must be a multiple of keyHeads");
    if (p.keyDim == 0 || p.valueDim == 0 || p.keyDim % 8 || p.valueDim % 8)
        return ctx.fail("gdn conv: keyDim and valueDim must be multiples of 8");
    if (p.kernelSize < 1 || p.kernelSize > MAXK) return ctx.fail("gdn conv: kernel size must be 1 to 8");
    if (!p.in || !p.kernel || !p.q || !p.k || !p.v || (p.kernelSize > 1 && !p.window))
        return ctx.fail("gdn conv: null tensor");
    if (p.fused && (!p.ba || !p.z || !p.a || !p.b)) return ctx.fail("gdn conv: the fused layout needs ba, z, a and b");
    if (p.count == 0) return true;
    auto aligned = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) % 16) == 0; };
    if (!aligned(p.in) || !aligned(p.q) || !aligned(p.k) || !aligned(p.v) || (p.fused && !aligned(p.z)) ||
        (p.window && !aligned(p.window)))
        return ctx.fail("gdn conv: tensors must be 16-byte aligned");
    ConvArgs a{};
    a.p = p;
    const uint64_t KW = p.keyHeads * p.keyDim, VW = p.valueHeads * p.valueDim, CW = 2 * KW + VW;
    if (CW + VW >= (1ull << 31) || p.count >= (1ull << 37)) return ctx.fail("gdn conv: tensors too large");
    a.KW = uint32_t(KW);
    a.VW = uint32_t(VW);
    a.CW = uint32_t(CW);
    a.groups = uint32_t(CW / 8 + (p.fused ? VW / 8 + p.valueHeads : 0));
    const dim3 grid{(a.groups + 255) / 256, unsigned((p.count + TB - 1) / TB)};
    if (grid.y > 65535) return ctx.fail("gdn conv: sequence too long for one call");
#define AIGPU_CONV(I, O, F)                                                                                    \
    if (p.inType == I && p.outType == O && p.fused == F) {                                                    \
        if (!ctx.launch("gdn_conv_kernel", stream, [&] {                                                      \
                if (p.kernelSize == 4)                                                                        \
                    hipLaunchKernelGGL((gdn_conv_kernel<I == 1, O == 1, F == 1, 4>), grid, dim3(256), 0, stream, a); \
                else                                                                                          \
                    hipLaunchKernelGGL((gdn_conv_kernel<I == 1, O == 1, F == 1, 0>), grid, dim3(256), 0, stream, a); \
            }))                                                                                               \
            return false;                                                                                     \
        if (p.kernelSize == 1) return true;                                                                   \
        return ctx.launch("gdn_window_kernel", stream, [&] {                                                  \
            hipLaunchKernelGGL((gdn_window_kernel<I == 1, F == 1>), dim3((a.CW + 255) / 256), dim3(256), 0,   \
                               stream, a);                                                                    \
        });                                                                                                   \
    }
    AIGPU_CONV(0, 0, 0) AIGPU_CONV(0, 1, 0) AIGPU_CONV(1, 0, 0) AIGPU_CONV(1, 1, 0)
    AIGPU_CONV(0, 0, 1) AIGPU_CONV(0, 1, 1) AIGPU_CONV(1, 0, 1) AIGPU_CONV(1, 1, 1)
#undef AIGPU_CONV
    return ctx.fail("gdn conv: unsupported configuration");
}

bool launch_gdn_gated_norm(const GdnGatedNormParams& p, hipStream_t stream) {
    Context& ctx = Context::instance();
    if (p.zType > 1 || p.outType > 1) return ctx.fail("gdn gated norm: unknown tensor type");
    if (p.valueDim == 0 || p.valueDim % 4) return ctx.fail("gdn gated norm: valueDim must be a multiple of 4");
    if (!p.x || !p.z || !p.gamma || !p.out) return ctx.fail("gdn gated norm: null tensor");
    if (p.count == 0) return true;
    auto aligned = [](const void* ptr, size_t n) { return (reinterpret_cast<uintptr_t>(ptr) % n) == 0; };
    if (!aligned(p.x, 16) || !aligned(p.gamma, 16) || !aligned(p.z, p.zType ? 8 : 16) ||
        !aligned(p.out, p.outType ? 8 : 16))
        return ctx.fail("gdn gated norm: tensors must be aligned to 4 elements");
    const uint64_t rows = p.count * p.valueHeads;
    // lanes per row: valueDim / 4 up to a wave, a power of two dividing it
    int lpr = 64;
    while (lpr > 1 && (p.valueDim < 4u * lpr || p.valueDim % (4u * lpr))) lpr >>= 1;
    if (p.valueDim / 4 >= 64) lpr = 64;
    const uint64_t perBlock = 4ull * (WAVE / lpr);
    if ((rows + perBlock - 1) / perBlock > 0x7FFFFFFFull) return ctx.fail("gdn gated norm: too many rows");
    const dim3 grid{unsigned((rows + perBlock - 1) / perBlock)};
    return ctx.launch("gdn_gated_norm_kernel", stream, [&] {
#define AIGPU_NORM(L)                                                                                           \
    if (lpr == L) {                                                                                          \
        if (p.zType == 0 && p.outType == 0) hipLaunchKernelGGL((gdn_gated_norm_kernel<false, false, L>), grid, dim3(256), 0, stream, p); \
        else if (p.zType == 0) hipLaunchKernelGGL((gdn_gated_norm_kernel<false, true, L>), grid, dim3(256), 0, stream, p); \
        else if (p.outType == 0) hipLaunchKernelGGL((gdn_gated_norm_kernel<true, false, L>), grid, dim3(256), 0, stream, p); \
        else hipLaunchKernelGGL((gdn_gated_norm_kernel<true, true, L>), grid, dim3(256), 0, stream, p); \
    }
        AIGPU_NORM(64) AIGPU_NORM(32) AIGPU_NORM(16) AIGPU_NORM(8) AIGPU_NORM(4) AIGPU_NORM(2) AIGPU_NORM(1)
#undef AIGPU_NORM
    });
}

} // namespace aigpu
