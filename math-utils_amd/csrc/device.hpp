// device.hpp - gfx950 device helpers shared by the attention kernels:
// element conversions, wave64 reductions and the MFMA operand types.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aigpu {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int WAVE = 64;
constexpr float LOG2E = 1.4426950408889634f;

/* bfloat16 is the top half of a float32: widening is a shift */
__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

/* round to nearest even; NaN stays NaN */
__device__ __forceinline__ uint16_t float_to_bf16_bits(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return uint16_t((u >> 16) | 0x40);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}

/* element i of a tensor tagged F32 (0) or BF16 (1) */
__device__ __forceinline__ float load_elem(const void* base, size_t i, int type) {
    if (type == 0) return static_cast<const float*>(base)[i];
    return bf16_bits_to_float(static_cast<const uint16_t*>(base)[i]);
}

/* wave64 butterflies */
/* softplusOf and sigmoidOf (LocalModel.hpp:1371-1376) with the library exp */
__device__ __forceinline__ float softplus_of(float x) { return x > 20.0f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float sigmoid_of(float x) { return 1.0f / (1.0f + expf(-x)); }

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, WAVE);
    return x;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, WAVE));
    return x;
}

/* orders LDS traffic between the lanes of one wave without a workgroup barrier */
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

/* s_waitcnt lgkmcnt(0) (vmcnt and expcnt left alone), then s_barrier. Unlike
   __syncthreads() it carries no workgroup release fence, which on gfx950 waits
   for every outstanding vector-memory operation (vmcnt(0)) and so would also
   wait for loads or DMA issued for later work; those are ordered by the
   waits the compiler places before their uses. The signal fences keep the
   compiler from moving LDS accesses across the barrier. */
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

/*
    QK-RMSNorm then rotate-half RoPE of one row held in LDS (`x`, dim floats),
    done by one wave. Restates attentionMixer (LocalModel.hpp:2608-2648):
    inv = 1/sqrt(sum(x^2)/dim + eps); x = x*inv*(gamma + offset); then for
    j < rot/2 the pair (j, j+rot/2) turns by angle = float(pos)*freq[j],
    computed in fp32 as the reference does. gamma == nullptr skips the norm,
    freqs == nullptr skips the rotation.
*/
__device__ __forceinline__ void norm_rope_row(float* x, int dim, const float* gamma, float eps,
                                              float offset, const float* freqs, int rot,
                                              uint64_t pos, int lane) {
    if (gamma) {
        float ss = 0.0f;
        for (int d = lane; d < dim; d += WAVE) ss += x[d] * x[d];
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / float(dim) + eps);
        for (int d = lane; d < dim; d += WAVE) x[d] = x[d] * inv * (gamma[d] + offset);
        wave_sync();
    }
    if (freqs) {
        const int half = rot / 2;
        const float fpos = float(pos);
        for (int j = lane; j < half; j += WAVE) {
            const float angle = fpos * freqs[j];
            float sn, cs;
            sincosf(angle, &sn, &cs);
            const float a = x[j], b = x[j + half];
            x[j] = a * cs - b * sn;
            x[j + half] = b * cs + a * sn;
        }
        wave_sync();
    }
}

/* fp16 of a finite fp32 value, noting in `bad` when it does not fit fp16's
   range (|x| >= 65520 rounds to infinity); infinite or NaN inputs stay what
   they are and are not noted (a NaN converts to a NaN, never to an infinity) */
__device__ __forceinline__ _Float16 to_f16_checked(float x, bool& bad) {
    const _Float16 h = _Float16(x);
    bad |= __builtin_isinf(float(h)) && !__builtin_isinf(x);
    return h;
}

/* a vector store of 1 into the range flag (a benign race: every writer
   stores the same value) */
__device__ __forceinline__ void raise_range_flag(uint32_t* flag, bool bad) {
    if (bad && flag) *reinterpret_cast<volatile uint32_t*>(flag) = 1u;
}

/* One 1 KB DMA block: each lane's 16 bytes from `src` into LDS at
   lds + 16 * lane. Written as asm so the compiler's wait analysis does not
   track it: it cannot tell double-buffered stages apart, and a pending
   global_load_lds (a FLAT-family load that also counts in lgkmcnt) makes
   it wait for every LDS read with lgkmcnt(0). Callers order their DMA with
   explicit vmcnt waits and barriers. One wait state separates the M0 write
   from the DMA that reads it; no other code of these kernels uses M0. */
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"   // M0 is reserved, and clobbered on purpose
__device__ __forceinline__ void dma_block(const void* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "s"(lds)
                 : "memory", "m0");
}
/* the same from a uniform base plus a 32-bit per-lane byte offset */
__device__ __forceinline__ void dma_block(const void* base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(base), "s"(lds)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

/* The flash kernel's table of each new token's RoPE cos and sin (rot / 2
   each, rot % 32 == 0): element i of token t's cos (which = 0) or sin
   (which = 1) at ((which * rot / 8 + i / 4) * count + t) * 4 + i % 4. The
   16-byte groups of consecutive tokens are adjacent, so a load in which
   each lane reads one token's group touches the fewest cache lines. */
__device__ __forceinline__ size_t rope_at(uint32_t t, uint32_t which, uint32_t i, uint32_t half, uint32_t count) {
    return ((size_t(which) * (half / 4) + i / 4) * count + t) * 4 + i % 4;
}

/* LDS byte address of a __shared__ object */
__device__ __forceinline__ uint32_t lds_address(const void* p) {
    return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}

} // namespace aigpu
