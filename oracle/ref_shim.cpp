/*
    ref_shim.cpp - C entry points over the reference's own CPU kernels.

    TEST INFRASTRUCTURE ONLY. Compiled by oracle/Makefile from the reference
    headers where they lie under $(REF) (the read-only hday200202/math-utils
    checkout); nothing from the reference is copied into this repository. The
    resulting oracle/_ref/libref_*.so validates the C restatement in
    oracle.c and may serve as the CPU baseline ("kind": "reference").

    Wrapped, unchanged:
      ai::kernels::attention   include/ai/Kernels.hpp:132-168
      ai::kernels::deltaStep   include/ai/Kernels.hpp:105-128 (also driven by
                               ref_gated_delta_rule, the mixer's token loop)
      ai::kernels::Pool        include/ai/ThreadPool.hpp:33-124
      math::random::Random     include/math/Random.hpp:15-89
      ai::quant::quantize, dequantRow   include/ai/Quant.hpp:420-450, 528-558
*/
#include <sched.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "ai/Kernels.hpp"
#include "math/Random.hpp"

extern "C" {

/* Restricts the reference pool to the first `n` CPUs of this process's
   affinity mask, through the reference's own Pool::configure. Must run before
   the first threaded call; returns the pool size afterwards. */
int ref_configure_pool(int n) {
    cpu_set_t set;
    std::vector<size_t> cpus;
    if (sched_getaffinity(0, sizeof(set), &set) == 0)
        for (int c = 0; c < CPU_SETSIZE && (int)cpus.size() < n; ++c)
            if (CPU_ISSET(c, &set)) cpus.push_back(size_t(c));
    if (!cpus.empty()) ai::kernels::Pool::configure(cpus);
    return int(ai::kernels::Pool::instance().size());
}

void ref_attention(const float* q, const float* keys, const float* values, float* out,
                   uint64_t count, uint64_t start, uint64_t heads, uint64_t kvHeads,
                   uint64_t dim, uint64_t qStride, uint64_t window, int threaded) {
    ai::kernels::attention(q, keys, values, out, count, start, heads, kvHeads, dim, qStride,
                           window, threaded != 0);
}

void ref_delta_step(float* state, const float* key, const float* query, const float* value,
                    const float* decay, int perKeyDecay, float beta, uint64_t keys,
                    uint64_t values, float* out, float* prediction, float* delta) {
    ai::kernels::deltaStep(state, key, query, value, decay, perKeyDecay != 0, beta, keys, values,
                           out, prediction, delta);
}

float ref_dot(const float* a, const float* b, uint64_t n) { return ai::kernels::dot(a, b, n); }

/* the reference's matmulNTBF16 (Kernels.hpp:243-257), the kernel its
   bandwidth test times (gpu-testing.cpp:298-351) */
void ref_matmul_nt_bf16(const float* a, const uint16_t* b, float* c, uint64_t m, uint64_t k, uint64_t n,
                        int threaded) {
    ai::kernels::matmulNTBF16(a, b, c, m, k, n, threaded != 0);
}

/* gatedDeltaNetMixer's per-token loop (LocalModel.hpp:2802-2830) around the
   reference's own deltaStep, single-threaded as the mixer runs it. The l2
   normalisation with eps inside the square root (LocalModel.hpp:1380-1386)
   and the 1/sqrt(KD) q scale (:2817-2818) are restated here: LocalModel.hpp
   does not compile with this toolchain. g is the log decay, beta the gate. */
void ref_gated_delta_rule(const float* q, const float* k, const float* v, const float* g,
                          const float* beta, float* state, float* out, uint64_t count,
                          uint64_t keyHeads, uint64_t valueHeads, uint64_t KD, uint64_t VD,
                          int normalize) {
    std::vector<float> qh(KD), kh(KD), prediction(VD), delta(VD);
    const uint64_t group = valueHeads / keyHeads;
    const float qScale = 1.0f / std::sqrt(float(KD));
    auto l2 = [](float* x, uint64_t n) {
        float sum = 0.0f;
        for (uint64_t i = 0; i < n; ++i) sum += x[i] * x[i];
        const float inv = 1.0f / std::sqrt(sum + 1e-6f);
        for (uint64_t i = 0; i < n; ++i) x[i] *= inv;
    };
    for (uint64_t t = 0; t < count; ++t)
        for (uint64_t h = 0; h < valueHeads; ++h) {
            const uint64_t kHead = h / group;
            std::memcpy(qh.data(), q + (t * keyHeads + kHead) * KD, sizeof(float) * KD);
            std::memcpy(kh.data(), k + (t * keyHeads + kHead) * KD, sizeof(float) * KD);
            if (normalize) {
                l2(qh.data(), KD);
                l2(kh.data(), KD);
                for (uint64_t i = 0; i < KD; ++i) qh[i] *= qScale;
            }
            const float decay = std::exp(g[t * valueHeads + h]);
            ai::kernels::deltaStep(state + h * KD * VD, kh.data(), qh.data(), v + (t * valueHeads + h) * VD,
                                   &decay, false, beta[t * valueHeads + h], KD, VD,
                                   out + (t * valueHeads + h) * VD, prediction.data(), delta.data());
        }
}

/* Draws `n` values from Random(seed): kind 0 next() as raw bits, 1 u01,
   2 normal(0,1), 3 randInt(lo, hi), 4 randDouble(lo, hi). */
void ref_random(uint64_t seed, int kind, uint64_t n, double lo, double hi, void* out) {
    math::random::Random rng(seed);
    for (uint64_t i = 0; i < n; ++i) {
        switch (kind) {
        case 0: static_cast<uint64_t*>(out)[i] = rng(); break;
        case 1: static_cast<double*>(out)[i] = rng.u01(); break;
        case 2: static_cast<double*>(out)[i] = rng.normal(); break;
        case 3: static_cast<int64_t*>(out)[i] = rng.randInt(int64_t(lo), int64_t(hi)); break;
        default: static_cast<double*>(out)[i] = rng.randDouble(lo, hi); break;
        }
    }
}

} // extern "C"

extern "C" {
/* kimiDeltaMixer's per-head token loop (LocalModel.hpp:2928-2947) around the
   reference's own deltaStep with perKeyDecay: g is the log decay per key
   channel [count][valueHeads][KD]; normalisation as ref_gated_delta_rule */
void ref_kda_rule(const float* q, const float* k, const float* v, const float* g, const float* beta,
                  float* state, float* out, uint64_t count, uint64_t keyHeads, uint64_t valueHeads,
                  uint64_t KD, uint64_t VD, int normalize) {
    std::vector<float> qh(KD), kh(KD), prediction(VD), delta(VD), decay(KD);
    const uint64_t group = valueHeads / keyHeads;
    const float qScale = 1.0f / std::sqrt(float(KD));
    auto l2 = [](float* x, uint64_t n) {
        float sum = 0.0f;
        for (uint64_t i = 0; i < n; ++i) sum += x[i] * x[i];
        const float inv = 1.0f / std::sqrt(sum + 1e-6f);
        for (uint64_t i = 0; i < n; ++i) x[i] *= inv;
    };
    for (uint64_t t = 0; t < count; ++t)
        for (uint64_t h = 0; h < valueHeads; ++h) {
            const uint64_t kHead = h / group;
            std::memcpy(qh.data(), q + (t * keyHeads + kHead) * KD, sizeof(float) * KD);
            std::memcpy(kh.data(), k + (t * keyHeads + kHead) * KD, sizeof(float) * KD);
            if (normalize) {
                l2(qh.data(), KD);
                l2(kh.data(), KD);
                for (uint64_t i = 0; i < KD; ++i) qh[i] *= qScale;
            }
            for (uint64_t i = 0; i < KD; ++i) decay[i] = std::exp(g[(t * valueHeads + h) * KD + i]);
            ai::kernels::deltaStep(state + h * KD * VD, kh.data(), qh.data(), v + (t * valueHeads + h) * VD,
                                   decay.data(), true, beta[t * valueHeads + h], KD, VD,
                                   out + (t * valueHeads + h) * VD, prediction.data(), delta.data());
        }
}
/* ai::quant::quantize (Quant.hpp:420-450) of a float [outDim][inDim]
   matrix: codes (Q8 one int8 per weight, Q4 two per byte) and scales
   [outDim][inDim/32]. Returns 0 when the reference declines (inDim not a
   multiple of 32). */
int ref_quantize(const float* src, uint64_t outDim, uint64_t inDim, int q4, void* codes, float* scales) {
    const auto t = ai::quant::quantize(src, size_t(outDim), size_t(inDim),
                                       q4 ? ai::quant::Type::Q4 : ai::quant::Type::Q8);
    if (!t.valid()) return 0;
    const size_t stored = q4 ? size_t(outDim * inDim / 2) : size_t(outDim * inDim);
    std::memcpy(codes, t.quants.get(), stored);
    std::memcpy(scales, t.scales.get(), sizeof(float) * size_t(outDim * (inDim / 32)));
    return 1;
}

/* ai::quant::dequantRow (Quant.hpp:528-558) of every row of a quantised
   matrix given as codes and scales */
void ref_dequant_rows(const void* codes, const float* scales, uint64_t outDim, uint64_t inDim, int q4, float* out) {
    ai::quant::QuantTensor t;
    t.type = q4 ? ai::quant::Type::Q4 : ai::quant::Type::Q8;
    t.outDim = size_t(outDim);
    t.inDim = size_t(inDim);
    const size_t stored = q4 ? size_t(outDim * inDim / 2) : size_t(outDim * inDim);
    t.quants = std::shared_ptr<int8_t[]>(new int8_t[stored]);
    t.scales = std::shared_ptr<float[]>(new float[size_t(outDim * (inDim / 32))]);
    std::memcpy(t.quants.get(), codes, stored);
    std::memcpy(t.scales.get(), scales, sizeof(float) * size_t(outDim * (inDim / 32)));
    for (size_t r = 0; r < size_t(outDim); ++r) ai::quant::dequantRow(t, r, out + r * size_t(inDim));
}

}
