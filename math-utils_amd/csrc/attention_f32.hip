// attention_f32.hip - fp32 causal GQA attention with kernels::attention's
// semantics (include/ai/Kernels.hpp:130-168): for token t and head h at
// position start+t, keys [first, start+t] of kv head h/(heads/kvHeads), with
// first = start+t+1-window when a window is set; out = softmax(q.K/sqrt(D)) V.
//
// This is the exact-arithmetic path behind the drop-in aigpu_attention: fp32
// loads, fp32 FMAs, expf. One wave owns one (token, head) and walks the keys
// in blocks of 64 with an online softmax: lane j scores key j of the block,
// then the lanes switch to owning dimensions for the P.V accumulation.
#include "context.hpp"
#include "device.hpp"
#include "kernels.hpp"

namespace aigpu {

namespace {

constexpr int MAX_DIM = 256;

__global__ __launch_bounds__(256) void attention_f32_kernel(AttentionF32Params p) {
    __shared__ float qs[4][MAX_DIM];
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

    for (uint64_t j0 = first; j0 <= position; j0 += WAVE) {
        const uint64_t j = j0 + lane;
        const bool ok = j <= position;
        float s = -INFINITY;
        if (ok) {
            const size_t row = kvBase + j * p.posStride;
            float dot = 0.0f;
            if (p.kvType == 0) {
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

        ps[w][lane] = pj;
        wave_sync();
        const int nb = int(position + 1 - j0 < WAVE ? position + 1 - j0 : WAVE);
        for (int jj = 0; jj < nb; ++jj) {
            const float pv = ps[w][jj];
            const size_t row = kvBase + (j0 + jj) * p.posStride;
#pragma unroll
            for (int i = 0; i < MAX_DIM / WAVE; ++i) {
                const int d = lane + i * WAVE;
                if (d < dim) acc[i] = fmaf(pv, load_elem(p.values, row + d, p.kvType), acc[i]);
            }
        }
        wave_sync();
    }

    const float inv = 1.0f / l;
    float* dst = p.out + task * p.dim;
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
