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
//                          SiLU(z) (:2833-2841)
#include "context.hpp"
#include "device.hpp"
#include "kernels.hpp"

namespace aigpu {

namespace {

constexpr int MAXK = 8;    // largest convolution kernel
constexpr int TB = 32;     // tokens per convolution thread
constexpr int UNROLL = 8;  // tokens whose loads a thread has in flight together

__device__ __forceinline__ float silu_of(float x) { return x / (1.0f + expf(-x)); }   // LocalModel.hpp:1369

/* 4 consecutive elements at element index i of an fp32 (T = false) or bf16
   tensor, as fp32 */
template <bool BF16>
__device__ __forceinline__ floatx4 load4(const void* base, size_t i) {
    if constexpr (BF16) {
        const u32x2 w = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(base) + i);
        return floatx4{__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xFFFF0000u),
                       __uint_as_float(w[1] << 16), __uint_as_float(w[1] & 0xFFFF0000u)};
    } else {
        return *reinterpret_cast<const floatx4*>(static_cast<const float*>(base) + i);
    }
}

template <bool BF16>
__device__ __forceinline__ void store4(void* base, size_t i, const floatx4& x) {
    if constexpr (BF16) {
        u32x2 w;
        w[0] = uint32_t(float_to_bf16_bits(x[0])) | (uint32_t(float_to_bf16_bits(x[1])) << 16);
        w[1] = uint32_t(float_to_bf16_bits(x[2])) | (uint32_t(float_to_bf16_bits(x[3])) << 16);
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(base) + i) = w;
    } else {
        *reinterpret_cast<floatx4*>(static_cast<float*>(base) + i) = x;
    }
}

struct ConvArgs {
    GdnConvParams p;
    uint32_t KW, VW, CW, quads;   // quads: 4-channel groups of CW (+ VW for z when fused)
};

/* element index, within the input rows, of convolution channel c (q | k | v
   order) of token t; the fused layout holds per key head q, k, the group's v
   and the group's z (LocalModel.hpp:2739-2776) */
template <bool FUSED>
__device__ __forceinline__ size_t in_index(const ConvArgs& a, uint64_t t, uint32_t c) {
    const GdnConvParams& p = a.p;
    if constexpr (!FUSED) return t * a.CW + c;
    const uint32_t KD = uint32_t(p.keyDim), VD = uint32_t(p.valueDim);
    const uint32_t G = uint32_t(p.valueHeads / p.keyHeads);
    const size_t stride = 2 * KD + 2 * size_t(G) * VD;
    uint32_t kh, off;
    if (c < a.KW) {
        kh = c / KD;
        off = c % KD;
    } else if (c < 2 * a.KW) {
        kh = (c - a.KW) / KD;
        off = KD + (c - a.KW) % KD;
    } else {
        const uint32_t vc = c - 2 * a.KW, vh = vc / VD;
        kh = vh / G;
        off = 2 * KD + (vh % G) * VD + vc % VD;
    }
    return (t * p.keyHeads + kh) * stride + off;
}

/*
    Thread = 4 consecutive channels x TB consecutive tokens. The K-1 previous
    inputs of each channel stay in registers as the thread walks its tokens,
    so every input is read once (plus a K-1 row halo per block); the first
    block reads its halo from the carried window. Channel quads past CW copy
    the fused layout's z rows; one more range de-interleaves b and a.
*/
template <bool IN_BF16, bool OUT_BF16, bool FUSED>
__global__ __launch_bounds__(256) void gdn_conv_kernel(ConvArgs a) {
    const GdnConvParams& p = a.p;
    const uint32_t quad = blockIdx.x * 256 + threadIdx.x;
    const uint64_t t0 = uint64_t(blockIdx.y) * TB;
    const uint32_t K = uint32_t(p.kernelSize);
    const uint64_t tEnd = t0 + TB < p.count ? t0 + TB : p.count;
    if (quad < a.CW / 4) {
        const uint32_t c = 4 * quad;
        float w[4][MAXK];
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int j = 0; j < MAXK; ++j) w[e][j] = uint32_t(j) < K ? p.kernel[(c + e) * K + j] : 0.0f;
        // hist[j]: input of token t - (K-1) + j, j < K-1, before token t
        floatx4 hist[MAXK - 1];
#pragma unroll
        for (int j = 0; j < MAXK - 1; ++j) {
            hist[j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            if (uint32_t(j) < K - 1) {
                const int64_t at = int64_t(t0) - int64_t(K - 1) + j;
                if (at >= 0) hist[j] = load4<IN_BF16>(p.in, in_index<FUSED>(a, uint64_t(at), c));
                else hist[j] = *reinterpret_cast<const floatx4*>(p.window + size_t(int64_t(K - 1) + at) * a.CW + c);
            }
        }
        // the dense output this channel range feeds
        float wcur[4];   // the current token's tap, K - 1
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            wcur[e] = w[e][0];
#pragma unroll
            for (int j = 1; j < MAXK; ++j)
                if (uint32_t(j) == K - 1) wcur[e] = w[e][j];
        }
        void* dst;
        uint32_t dc, dw;
        if (c < a.KW) dst = p.q, dc = c, dw = a.KW;
        else if (c < 2 * a.KW) dst = p.k, dc = c - a.KW, dw = a.KW;
        else dst = p.v, dc = c - 2 * a.KW, dw = a.VW;
        // UNROLL tokens' loads go out together (rows past the end re-read the
        // last row), then the tokens are computed in order
        for (uint64_t tb = t0; tb < tEnd; tb += UNROLL) {
            floatx4 xs[UNROLL];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u)
                xs[u] = load4<IN_BF16>(p.in, in_index<FUSED>(a, tb + u < p.count ? tb + u : p.count - 1, c));
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                if (tb + u >= tEnd) break;   // uniform over the workgroup
                const floatx4 x = xs[u];
                floatx4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // taps in the reference's order: j = 0 (oldest) .. K-1 (current)
                    float acc = 0.0f;
#pragma unroll
                    for (int j = 0; j < MAXK - 1; ++j)
                        if (uint32_t(j) < K - 1) acc += w[e][j] * hist[j][e];
                    acc += wcur[e] * x[e];
                    o[e] = silu_of(acc);
                }
                store4<OUT_BF16>(dst, (tb + u) * dw + dc, o);
#pragma unroll
                for (int j = 0; j < MAXK - 2; ++j)
                    if (uint32_t(j) + 1 < K - 1) hist[j] = hist[j + 1];
#pragma unroll
                for (int j = 0; j < MAXK - 1; ++j)
                    if (uint32_t(j) == K - 2) hist[j] = x;
            }
        }
        return;
    }
    if constexpr (FUSED) {
        const uint32_t KD = uint32_t(p.keyDim), VD = uint32_t(p.valueDim);
        const uint32_t G = uint32_t(p.valueHeads / p.keyHeads);
        const size_t stride = 2 * KD + 2 * size_t(G) * VD;
        if (quad < (a.CW + a.VW) / 4) {   // z: copied, not convolved
            const uint32_t zc = 4 * quad - a.CW, vh = zc / VD, kh = vh / G;
            const size_t off = 2 * KD + size_t(G) * VD + (vh % G) * VD + zc % VD;
            for (uint64_t tb = t0; tb < tEnd; tb += UNROLL) {
                floatx4 xs[UNROLL];
#pragma unroll
                for (int u = 0; u < UNROLL; ++u) {
                    const uint64_t t = tb + u < p.count ? tb + u : p.count - 1;
                    xs[u] = load4<IN_BF16>(p.in, (t * p.keyHeads + kh) * stride + off);
                }
#pragma unroll
                for (int u = 0; u < UNROLL; ++u)
                    if (tb + u < tEnd) store4<OUT_BF16>(p.z, (tb + u) * a.VW + zc, xs[u]);
            }
            return;
        }
        const uint32_t vh = quad - (a.CW + a.VW) / 4;   // b, a of one value head
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
    float next[MAXK - 1];
#pragma unroll
    for (int i = 0; i < MAXK - 1; ++i) {
        next[i] = 0.0f;
        if (uint32_t(i) < K - 1) {
            const int64_t at = int64_t(p.count) - int64_t(K - 1) + i;
            next[i] = at >= 0 ? load_elem(p.in, in_index<FUSED>(a, uint64_t(at), c), IN_BF16 ? 1 : 0)
                              : p.window[size_t(int64_t(K - 1) + at) * a.CW + c];
        }
    }
#pragma unroll
    for (int i = 0; i < MAXK - 1; ++i)
        if (uint32_t(i) < K - 1) p.window[size_t(i) * a.CW + c] = next[i];
}

/* one wave per (token, value head) row: rmsNormRow with the weight stored
   directly (offset 0), then x SiLU(z) (LocalModel.hpp:2833-2841) */
template <bool Z_BF16, bool OUT_BF16>
__global__ __launch_bounds__(256) void gdn_gated_norm_kernel(GdnGatedNormParams p) {
    const uint64_t row = uint64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= p.count * p.valueHeads) return;
    const uint32_t VD = uint32_t(p.valueDim);
    const float* x = p.x + row * VD;
    float ss = 0.0f;
    for (uint32_t d = 4 * lane; d < VD; d += 4 * WAVE) {
        const floatx4 v = *reinterpret_cast<const floatx4*>(x + d);
        ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / float(VD) + p.eps);
    for (uint32_t d = 4 * lane; d < VD; d += 4 * WAVE) {
        const floatx4 v = *reinterpret_cast<const floatx4*>(x + d);
        const floatx4 gm = *reinterpret_cast<const floatx4*>(p.gamma + d);
        const floatx4 z = load4<Z_BF16>(p.z, row * VD + d);
        floatx4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = v[e] * inv * gm[e] * silu_of(z[e]);
        store4<OUT_BF16>(p.out, row * VD + d, o);
    }
}

} // namespace

bool launch_gdn_conv(const GdnConvParams& p, hipStream_t stream) {
    Context& ctx = Context::instance();
    if (p.inType > 1 || p.outType > 1) return ctx.fail("gdn conv: unknown tensor type");
    if (p.keyHeads == 0 || p.valueHeads % p.keyHeads) return ctx.fail("gdn conv: valueHeads must be a multiple of keyHeads");
    if (p.keyDim == 0 || p.valueDim == 0 || p.keyDim % 4 || p.valueDim % 4)
        return ctx.fail("gdn conv: keyDim and valueDim must be multiples of 4");
    if (p.kernelSize < 1 || p.kernelSize > MAXK) return ctx.fail("gdn conv: kernel size must be 1 to 8");
    if (!p.in || !p.kernel || !p.q || !p.k || !p.v || (p.kernelSize > 1 && !p.window))
        return ctx.fail("gdn conv: null tensor");
    if (p.fused && (!p.ba || !p.z || !p.a || !p.b)) return ctx.fail("gdn conv: the fused layout needs ba, z, a and b");
    if (p.count == 0) return true;
    auto aligned = [](const void* ptr, size_t n) { return (reinterpret_cast<uintptr_t>(ptr) % n) == 0; };
    const size_t io = p.inType ? 8 : 16, oo = p.outType ? 8 : 16;
    if (!aligned(p.in, io) || !aligned(p.q, oo) || !aligned(p.k, oo) || !aligned(p.v, oo) ||
        (p.fused && !aligned(p.z, oo)) || (p.window && !aligned(p.window, 16)))
        return ctx.fail("gdn conv: tensors must be aligned to 4 elements");
    ConvArgs a{};
    a.p = p;
    const uint64_t KW = p.keyHeads * p.keyDim, VW = p.valueHeads * p.valueDim, CW = 2 * KW + VW;
    if (CW + VW >= (1ull << 31) || p.count >= (1ull << 37)) return ctx.fail("gdn conv: tensors too large");
    a.KW = uint32_t(KW);
    a.VW = uint32_t(VW);
    a.CW = uint32_t(CW);
    a.quads = uint32_t(CW / 4 + (p.fused ? VW / 4 + (p.valueHeads + 3) / 4 * 4 : 0));
    const dim3 grid{(a.quads + 255) / 256, unsigned((p.count + TB - 1) / TB)};
    if (grid.y > 65535) return ctx.fail("gdn conv: sequence too long for one call");
#define AIGPU_CONV(I, O, F)                                                                                    \
    if (p.inType == I && p.outType == O && p.fused == F) {                                                    \
        if (!ctx.launch("gdn_conv_kernel", stream, [&] {                                                      \
                hipLaunchKernelGGL((gdn_conv_kernel<I == 1, O == 1, F == 1>), grid, dim3(256), 0, stream, a); \
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
    if ((rows + 3) / 4 > 0x7FFFFFFFull) return ctx.fail("gdn gated norm: too many rows");
    const dim3 grid{unsigned((rows + 3) / 4)};
    return ctx.launch("gdn_gated_norm_kernel", stream, [&] {
        if (p.zType == 0 && p.outType == 0) hipLaunchKernelGGL((gdn_gated_norm_kernel<false, false>), grid, dim3(256), 0, stream, p);
        else if (p.zType == 0) hipLaunchKernelGGL((gdn_gated_norm_kernel<false, true>), grid, dim3(256), 0, stream, p);
        else if (p.outType == 0) hipLaunchKernelGGL((gdn_gated_norm_kernel<true, false>), grid, dim3(256), 0, stream, p);
        else hipLaunchKernelGGL((gdn_gated_norm_kernel<true, true>), grid, dim3(256), 0, stream, p);
    });
}

} // namespace aigpu
