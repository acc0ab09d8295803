// copy.hip - a plain streaming device copy: what HBM delivers on this part,
// the ceiling beside the 8 TB/s spec peak that the HBM-bound kernels' roofline
// fractions use. No counterpart in the reference's kernels; its GPU testing
// measures bandwidth with a bf16 GEMV (src/gpu-testing.cpp:298-351), which
// the bench runs too.
//
// Each thread moves UNROLL 16-byte pieces per step, all loads issued before
// any store, with the nontemporal cache policy (each byte is touched once).
// Workgroups stride over the buffer, four per CU.
#include "context.hpp"
#include "device.hpp"
#include "kernels.hpp"

namespace aigpu {

namespace {

constexpr int COPY_THREADS = 256, COPY_UNROLL = 8;

__global__ __launch_bounds__(COPY_THREADS) void copy_kernel(u32x4* __restrict__ dst, const u32x4* __restrict__ src,
                                                            uint64_t pieces) {
    const uint64_t stride = uint64_t(gridDim.x) * COPY_THREADS * COPY_UNROLL;
    for (uint64_t base = uint64_t(blockIdx.x) * COPY_THREADS * COPY_UNROLL + threadIdx.x; base < pieces;
         base += stride) {
        u32x4 v[COPY_UNROLL];
#pragma unroll
        for (int u = 0; u < COPY_UNROLL; ++u) {
            const uint64_t i = base + uint64_t(u) * COPY_THREADS;
            if (i < pieces) v[u] = __builtin_nontemporal_load(src + i);
        }
#pragma unroll
        for (int u = 0; u < COPY_UNROLL; ++u) {
            const uint64_t i = base + uint64_t(u) * COPY_THREADS;
            if (i < pieces) __builtin_nontemporal_store(v[u], dst + i);
        }
    }
}

/* the last bytes % 16 bytes, one thread each */
__global__ void copy_tail_kernel(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src, uint32_t n) {
    if (threadIdx.x < n) dst[threadIdx.x] = src[threadIdx.x];
}

} // namespace

bool launch_copy(void* dst, const void* src, uint64_t bytes, hipStream_t stream) {
    Context& ctx = Context::instance();
    if (bytes == 0) return true;
    if (!dst || !src) return ctx.fail("copy: null pointer");
    if ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15)
        return ctx.fail("copy: pointers must be 16-byte aligned");
    const uint8_t* s = static_cast<const uint8_t*>(src);
    uint8_t* d = static_cast<uint8_t*>(dst);
    if ((s < d + bytes) && (d < s + bytes)) return ctx.fail("copy: the buffers overlap");
    const uint64_t pieces = bytes / 16;
    const uint32_t tail = uint32_t(bytes % 16);
    if (pieces) {
        const uint64_t want = (pieces + COPY_THREADS * COPY_UNROLL - 1) / (COPY_THREADS * COPY_UNROLL);
        const unsigned grid = unsigned(want < 1024 ? want : 1024);
        if (!ctx.launch("copy_kernel", stream, [&] {
                hipLaunchKernelGGL(copy_kernel, dim3(grid), dim3(COPY_THREADS), 0, stream,
                                   reinterpret_cast<u32x4*>(d), reinterpret_cast<const u32x4*>(s), pieces);
            }))
            return false;
    }
    if (tail && !ctx.launch("copy_tail_kernel", stream, [&] {
            hipLaunchKernelGGL(copy_tail_kernel, dim3(1), dim3(16), 0, stream, d + pieces * 16, s + pieces * 16, tail);
        }))
        return false;
    return true;
}

} // namespace aigpu
