// matmul.hip - out[m][n] = a[m][k] . w[n][k] (+ bias[n]) (+ out), the
// projection every mixer and MLP applies (LocalModel.hpp:1044-1078 apply,
// behind gpu::matmulNT*), for the reference's four weight encodings:
//   F32    [n][k] fp32
//   BF16   [n][k] bf16 (widened by a 16-bit shift, Kernels.hip widenBF16)
//   Q8     [n][k] int8 codes, one fp32 scale per 32 codes (Quant.hpp:528-538)
//   Q4     [n][k/2] bytes, one fp32 scale per 32 codes; byte j of a block
//          holds code j in its low nibble and code j+16 in its high nibble,
//          each offset by 8 (Quant.hpp:540-549)
//
// gemv_kernel serves up to 8 rows of a (decode, small batches): it is bound
// by the weight bytes, so every lane streams 16-byte pieces of a weight row
// (4, 8, 16 or 32 weights), one wave owns GEMV_ROWS weight rows and keeps an
// fp32 accumulator per (weight row, a row), and a shuffle tree reduces the
// lanes. More rows of a run as blocks of 8 along grid.y.
#include "context.hpp"
#include "device.hpp"
#include "gemv.hpp"
#include "kernels.hpp"

namespace aigpu {

namespace {

constexpr int GEMV_ROWS = 2;   // weight rows per wave
constexpr int GEMV_MAX_M = 8;  // rows of a per launch block

template <int TYPE, int M>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams p) {
    constexpr int E = piece_elems<TYPE>();
    const int lane = threadIdx.x & 63;
    const uint32_t row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * GEMV_ROWS;
    if (row0 >= p.n) return;   // whole wave leaves; no block barriers below
    const uint32_t m0 = blockIdx.y * M;
    const uint32_t pieces = p.k / E;
    const size_t rowBytes = size_t(p.k) * row_bytes_per_k_x2<TYPE>() / 2;
    const uint32_t blocks = p.k / 32;

    const char* wrow[GEMV_ROWS];
    const float* srow[GEMV_ROWS];
#pragma unroll
    for (int r = 0; r < GEMV_ROWS; ++r) {
        const uint32_t rr = row0 + r < p.n ? row0 + r : p.n - 1;
        wrow[r] = static_cast<const char*>(p.w) + rr * rowBytes;
        srow[r] = TYPE >= 2 ? p.scales + size_t(rr) * blocks : nullptr;
    }
    float acc[GEMV_ROWS][M];
#pragma unroll
    for (int r = 0; r < GEMV_ROWS; ++r)
#pragma unroll
        for (int i = 0; i < M; ++i) acc[r][i] = 0.0f;

#pragma unroll 2
    for (uint32_t c = lane; c < pieces; c += WAVE) {
        u32x4 wv[GEMV_ROWS];
#pragma unroll
        for (int r = 0; r < GEMV_ROWS; ++r) wv[r] = *reinterpret_cast<const u32x4*>(wrow[r] + size_t(c) * 16);
        float sc[GEMV_ROWS];
#pragma unroll
        for (int r = 0; r < GEMV_ROWS; ++r) sc[r] = TYPE == 2 ? srow[r][c >> 1] : (TYPE == 3 ? srow[r][c] : 1.0f);
#pragma unroll
        for (int i = 0; i < M; ++i) {
            if (m0 + i < p.m) {
                const float* x = p.a + size_t(m0 + i) * p.k + size_t(c) * E;
#pragma unroll
                for (int r = 0; r < GEMV_ROWS; ++r) {
                    const float d = piece_dot<TYPE>(wv[r], x);
                    acc[r][i] = TYPE >= 2 ? fmaf(d, sc[r], acc[r][i]) : acc[r][i] + d;
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < GEMV_ROWS; ++r)
#pragma unroll
        for (int i = 0; i < M; ++i) acc[r][i] = wave_sum(acc[r][i]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < GEMV_ROWS; ++r) {
            const uint32_t n = row0 + r;
            if (n >= p.n) continue;
            const float b = p.bias ? p.bias[n] : 0.0f;
#pragma unroll
            for (int i = 0; i < M; ++i) {
                if (m0 + i >= p.m) continue;
                float* o = p.out + size_t(m0 + i) * p.ldo + n;
                *o = (p.accumulate ? *o : 0.0f) + acc[r][i] + b;
            }
        }
    }
}

/* any k for F32 and BF16 (rows not on 16-byte boundaries): one wave per
   weight row and a row of a, element by element */
template <int TYPE>
__global__ __launch_bounds__(256) void gemv_scalar_kernel(GemvParams p) {
    const int lane = threadIdx.x & 63;
    const uint64_t task = uint64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (task >= uint64_t(p.n) * p.m) return;
    const uint32_t n = uint32_t(task % p.n), i = uint32_t(task / p.n);
    const float* x = p.a + size_t(i) * p.k;
    float s = 0.0f;
    for (uint32_t t = lane; t < p.k; t += WAVE) {
        const float wv = TYPE == 0 ? static_cast<const float*>(p.w)[size_t(n) * p.k + t]
                                   : bf16_bits_to_float(static_cast<const uint16_t*>(p.w)[size_t(n) * p.k + t]);
        s = fmaf(x[t], wv, s);
    }
    s = wave_sum(s);
    if (lane == 0) {
        float* o = p.out + size_t(i) * p.ldo + n;
        *o = (p.accumulate ? *o : 0.0f) + s + (p.bias ? p.bias[n] : 0.0f);
    }
}

template <int TYPE>
bool launch_type(Context& ctx, const GemvParams& p, hipStream_t stream) {
    constexpr int E = piece_elems<TYPE>();
    if (p.k % E || (reinterpret_cast<uintptr_t>(p.w) % 16) || (reinterpret_cast<uintptr_t>(p.a) % 16)) {
        if constexpr (TYPE <= 1) {
            const uint64_t tasks = uint64_t(p.n) * p.m;
            if ((tasks + 3) / 4 > 0x7FFFFFFFull) return ctx.fail("matmul: too many outputs");
            return ctx.launch("gemv_scalar_kernel", stream, [&] {
                hipLaunchKernelGGL((gemv_scalar_kernel<TYPE>), dim3(unsigned((tasks + 3) / 4)), dim3(256), 0, stream, p);
            });
        }
        return ctx.fail("matmul: quantised weights need k a multiple of 32 and 16-byte aligned rows");
    }
    const unsigned gx = unsigned((p.n + 4 * GEMV_ROWS - 1) / (4 * GEMV_ROWS));
    const int M = p.m <= 1 ? 1 : (p.m <= 2 ? 2 : (p.m <= 4 ? 4 : GEMV_MAX_M));
    const unsigned gy = unsigned((p.m + M - 1) / M);
    if (gy > 65535u) return ctx.fail("matmul: too many rows of a");
    return ctx.launch("gemv_kernel", stream, [&] {
        const dim3 grid(gx, gy);
        if (M == 1) hipLaunchKernelGGL((gemv_kernel<TYPE, 1>), grid, dim3(256), 0, stream, p);
        else if (M == 2) hipLaunchKernelGGL((gemv_kernel<TYPE, 2>), grid, dim3(256), 0, stream, p);
        else if (M == 4) hipLaunchKernelGGL((gemv_kernel<TYPE, 4>), grid, dim3(256), 0, stream, p);
        else hipLaunchKernelGGL((gemv_kernel<TYPE, 8>), grid, dim3(256), 0, stream, p);
    });
}

} // namespace

bool launch_gemv(const GemvParams& p, hipStream_t stream) {
    Context& ctx = Context::instance();
    if (p.m == 0 || p.n == 0) return true;
    if (!p.a || !p.w || !p.out) return ctx.fail("matmul: null tensor");
    if (p.k == 0) return ctx.fail("matmul: k must be positive");
    if (p.ldo < p.n) return ctx.fail("matmul: output row stride below n");
    if (p.type >= 2 && !p.scales) return ctx.fail("matmul: quantised weights need scales");
    if (p.type >= 2 && p.k % 32) return ctx.fail("matmul: quantised weights need k a multiple of 32");
    switch (p.type) {
        case 0: return launch_type<0>(ctx, p, stream);
        case 1: return launch_type<1>(ctx, p, stream);
        case 2: return launch_type<2>(ctx, p, stream);
        case 3: return launch_type<3>(ctx, p, stream);
        default: return ctx.fail("matmul: unknown weight type");
    }
}

} // namespace aigpu
