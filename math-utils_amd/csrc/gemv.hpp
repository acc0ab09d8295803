// gemv.hpp - decoding 16-byte pieces of a weight row in the reference's four
// encodings (F32, BF16, Q8, Q4; Quant.hpp:528-549) against fp32
// activations; shared by the projections and the resident decoder.
#pragma once

#include "device.hpp"

namespace aigpu {

template <int TYPE>
__host__ __device__ constexpr int piece_elems() {   // weights in 16 bytes
    return TYPE == 0 ? 4 : (TYPE == 1 ? 8 : (TYPE == 2 ? 16 : 32));
}
template <int TYPE>
__host__ __device__ constexpr int row_bytes_per_k_x2() {   // 2 x bytes per weight
    return TYPE == 0 ? 8 : (TYPE == 1 ? 4 : (TYPE == 2 ? 2 : 1));
}

/* the dot of E weights from one 16-byte piece with a's matching E values */
template <int TYPE>
__device__ __forceinline__ float piece_dot(const u32x4 w, const float* x) {
    float s = 0.0f;
    if constexpr (TYPE == 0) {
        const floatx4 a = *reinterpret_cast<const floatx4*>(x);
#pragma unroll
        for (int e = 0; e < 4; ++e) s = fmaf(a[e], __uint_as_float(w[e]), s);
    } else if constexpr (TYPE == 1) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const floatx4 a = *reinterpret_cast<const floatx4*>(x + 4 * e);
            s = fmaf(a[0], __uint_as_float(w[2 * e] << 16), s);
            s = fmaf(a[1], __uint_as_float(w[2 * e] & 0xFFFF0000u), s);
            s = fmaf(a[2], __uint_as_float(w[2 * e + 1] << 16), s);
            s = fmaf(a[3], __uint_as_float(w[2 * e + 1] & 0xFFFF0000u), s);
        }
    } else if constexpr (TYPE == 2) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const floatx4 a = *reinterpret_cast<const floatx4*>(x + 4 * e);
#pragma unroll
            for (int j = 0; j < 4; ++j) s = fmaf(a[j], float(int32_t(w[e] << (24 - 8 * j)) >> 24), s);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const floatx4 lo = *reinterpret_cast<const floatx4*>(x + 4 * e);
            const floatx4 hi = *reinterpret_cast<const floatx4*>(x + 16 + 4 * e);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t byte = (w[e] >> (8 * j)) & 0xFFu;
                s = fmaf(lo[j], float(int(byte & 0xFu) - 8), s);
                s = fmaf(hi[j], float(int(byte >> 4) - 8), s);
            }
        }
    }
    return s;
}

} // namespace aigpu
