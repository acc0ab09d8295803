// attention_f32.hip - fp32 causal GQA attention with kernels::attention's
// semantics (include/ai/Kernels.hpp:130-168): for token t and head h at
// position start+t, keys [first, start+t] of kv head h/(heads/kvHeads), with
// first = start+t+1-window when a window is set; out = softmax(q.K/sqrt(D)) V.
//
// This is the exact-arithmetic path behind the drop-in aigpu_attention: fp32
// loads, fp32 FMAs, expf. One wave owns one (token, head) and walks the keys
// in blocks of 64 with an online softmax: lane j scores key j of the block,
// then the lanes switch to owning dimensions for the P.V accumulation. Both
// loops issue their loads in batches before using them (a key row as up to
// 16 16-byte pieces per lane with four partial sums when rows are 16-byte
// aligned; value rows as 16-byte pieces, several rows per load instruction,
// or else eight rows at a time), so that a block costs a few memory round
// trips rather than one per dimension or per key.
#include "context.hpp"
#include "device.hpp"
#include "kernels.hpp"

namespace aigpu {

namespace {

constexpr int MAX_DIM = 256;

__global__ __launch_bounds__(256) void attention_f32_kernel(AttentionF32Params p) {
    __shared__ __align__(16) float qs[4][MAX_DIM];
    __shared__ float ps[4][WAVE];

    const int lane = threadIdx.x & (WAVE - 1);
    const int w = threadIdx.x / WAVE;
    const uint64_t task = uint64_t(blockIdx.x) * 4 + w;
    if (task >= p.count * p.heads) return;  // whole wave leaves; no block barriers below

    const uint64_t token = task / p.heads, head = task % p.heads;
    const uint64_t position = p.start + token;
    const uint64_t first = p.window && position + 1 > p.window ? position + 1 - p.window : 0;
    const uint64_t kv = head / (p.heads / p.kvHeads);
    const int dim = int(p.dim);
    const float scale = 1.0f / sqrtf(float(dim));

    for (int d = lane; d < dim; d += WAVE)
        qs[w][d] = load_elem(p.q, (token * p.heads + head) * p.qStride + d, p.qType);
    wave_sync();

    const size_t kvBase = kv * p.headStride;
    float m = -INFINITY, l = 0.0f;
    float acc[MAX_DIM / WAVE] = {0.0f, 0.0f, 0.0f, 0.0f};
    // key rows in 16-byte pieces: every row start (and q's copy in LDS) on a
    // 16-byte boundary, which fp32 rows with dim % 4 == 0 and bf16 rows with
    // dim % 8 == 0 and strides to match give
    const size_t esz = p.kvType == 0 ? 4 : 2, per = 16 / esz;
    const bool vec = dim % int(per) == 0 && (reinterpret_cast<uintptr_t>(p.keys) % 16) == 0 &&
                     (kvBase * esz) % 16 == 0 && (p.posStride * esz) % 16 == 0;
    // fp32 value rows of dim / 4 16-byte pieces, a power of two: LPR lanes per
    // row, RPI = 64 / LPR rows per load instruction, each lane a four-float
    // accumulator for its piece and its group of rows (summed across the
    // groups at the end); up to 16 pieces per lane in flight
    const int LPR = dim / 4;
    const bool vecv = p.kvType == 0 && dim % 4 == 0 && (LPR & (LPR - 1)) == 0 &&
                      (reinterpret_cast<uintptr_t>(p.values) % 16) == 0 && (kvBase * 4) % 16 == 0 &&
                      (p.posStride * 4) % 16 == 0;
    const int RPI = vecv ? WAVE / LPR : 1, vg = vecv ? lane / LPR : 0, vc = vecv ? lane % LPR : 0;
    floatx4 acc2 = {0.0f, 0.0f, 0.0f, 0.0f};

    for (uint64_t j0 = first; j0 <= position; j0 += WAVE) {
        const uint64_t j = j0 + lane;
        const bool ok = j <= position;
        float s = -INFINITY;
        if (ok) {
            const size_t row = kvBase + j * p.posStride;
            float dot = 0.0f;
            if (vec && p.kvType == 0) {
                // up to 64 dimensions per batch: 16 pieces in flight, four partial sums
                const floatx4* kr = reinterpret_cast<const floatx4*>(static_cast<const float*>(p.keys) + row);
                const floatx4* q4 = reinterpret_cast<const floatx4*>(qs[w]);
                floatx4 part = {0.0f, 0.0f, 0.0f, 0.0f};
                for (int c0 = 0; c0 < dim / 4; c0 += 16) {
                    floatx4 kp[16];
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (c0 + i < dim / 4) kp[i] = kr[c0 + i];
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (c0 + i < dim / 4) {
                            const floatx4 qv = q4[c0 + i];
#pragma unroll
                            for (int e = 0; e < 4; ++e) part[e] = fmaf(qv[e], kp[i][e], part[e]);
                        }
                }
                dot = (part[0] + part[1]) + (part[2] + part[3]);
            } else if (vec) {
                // bf16: eight elements per piece, up to 128 dimensions per batch
                const u32x4* kr = reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p.keys) + row);
                const floatx4* q4 = reinterpret_cast<const floatx4*>(qs[w]);
                floatx4 part = {0.0f, 0.0f, 0.0f, 0.0f};
                for (int c0 = 0; c0 < dim / 8; c0 += 16) {
                    u32x4 kp[16];
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (c0 + i < dim / 8) kp[i] = kr[c0 + i];
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (c0 + i < dim / 8) {
                            const floatx4 qa = q4[2 * (c0 + i)], qb = q4[2 * (c0 + i) + 1];
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const uint32_t wv = kp[i][e];
                                const float lo = __uint_as_float(wv << 16), hi = __uint_as_float(wv & 0xFFFF0000u);
                                const float q0 = e < 2 ? qa[2 * e] : qb[2 * e - 4];
                                const float q1 = e < 2 ? qa[2 * e + 1] : qb[2 * e - 3];
                                part[e] = fmaf(q1, hi, fmaf(q0, lo, part[e]));
                            }
                        }
                }
                dot = (part[0] + part[1]) + (part[2] + part[3]);
            } else if (p.kvType == 0) {
                const float* kr = static_cast<const float*>(p.keys) + row;
                for (int d = 0; d < dim; ++d) dot = fmaf(qs[w][d], kr[d], dot);
            } else {
                const uint16_t* kr = static_cast<const uint16_t*>(p.keys) + row;
                for (int d = 0; d < dim; ++d) dot = fmaf(qs[w][d], bf16_bits_to_float(kr[d]), dot);
            }
            s = dot * scale;
        }
        const float mn = fmaxf(m, wave_max(s));  // finite: the block holds key j0
        const float alpha = expf(m - mn);
        const float pj = ok ? expf(s - mn) : 0.0f;
        l = l * alpha + wave_sum(pj);
        m = mn;
#pragma unroll
        for (int i = 0; i < MAX_DIM / WAVE; ++i) acc[i] *= alpha;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc2[e] *= alpha;

        ps[w][lane] = pj;
        wave_sync();
        const int nb = int(position + 1 - j0 < WAVE ? position + 1 - j0 : WAVE);
        if (vecv) {
            const floatx4* vb = reinterpret_cast<const floatx4*>(static_cast<const float*>(p.values) + kvBase) + vc;
            const size_t rs = p.posStride / 4;
            for (int t0 = 0; t0 < LPR; t0 += 16) {
                floatx4 vp[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const int r = (t0 + u) * RPI + vg;
                    vp[u] = t0 + u < LPR && r < nb ? vb[(j0 + uint64_t(r)) * rs] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
                }
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const int r = (t0 + u) * RPI + vg;
                    if (t0 + u < LPR && r < nb) {
                        const float pv = ps[w][r];
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc2[e] = fmaf(pv, vp[u][e], acc2[e]);
                    }
                }
            }
        }
        for (int jb = 0; !vecv && jb < nb; jb += 8) {   // eight value rows' loads in flight
            float vr[8][MAX_DIM / WAVE];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const size_t row = kvBase + (j0 + jb + u) * p.posStride;
#pragma unroll
                for (int i = 0; i < MAX_DIM / WAVE; ++i) {
                    const int d = lane + i * WAVE;
                    vr[u][i] = jb + u < nb && d < dim ? load_elem(p.values, row + d, p.kvType) : 0.0f;
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (jb + u >= nb) break;   // uniform
                const float pv = ps[w][jb + u];
#pragma unroll
                for (int i = 0; i < MAX_DIM / WAVE; ++i) acc[i] = fmaf(pv, vr[u][i], acc[i]);
            }
        }
        wave_sync();
    }

    const float inv = 1.0f / l;
    float* dst = p.out + task * p.dim;
    if (vecv) {
        for (int off = LPR; off < WAVE; off <<= 1)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc2[e] += __shfl_xor(acc2[e], off, WAVE);
        if (vg == 0) {
#pragma unroll
            for (int e = 0; e < 4; ++e) dst[4 * vc + e] = acc2[e] * inv;
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < MAX_DIM / WAVE; ++i) {
        const int d = lane + i * WAVE;
        if (d < dim) dst[d] = acc[i] * inv;
    }
}

} // namespace

bool launch_attention_f32(const AttentionF32Params& p, hipStream_t stream) {
    Context& ctx = Context::instance();
    if (p.dim == 0 || p.dim > MAX_DIM) return ctx.fail("attention: dim must be 1..256");
    if (p.kvHeads == 0 || p.heads % p.kvHeads) return ctx.fail("attention: heads must be a multiple of kvHeads");
    if (p.qStride < p.dim) return ctx.fail("attention: qStride < dim");
    const uint64_t tasks = p.count * p.heads;
    if (tasks == 0) return true;
    const uint64_t blocks = (tasks + 3) / 4;
    if (blocks > 0x7FFFFFFFull) return ctx.fail("attention: too many tasks");
    return ctx.launch("attention_f32_kernel", stream, [&] {
        hipLaunchKernelGGL(attention_f32_kernel, dim3(unsigned(blocks)), dim3(256), 0, stream, p);
    });
}

} // namespace aigpu
