/*
    oracle.c - CPU restatement of the reference attention hot path.

    TEST INFRASTRUCTURE ONLY: the checker the HIP backend is compared with,
    and the CPU baseline bench.py times. The product never links it.
    Every function names the reference file:line it restates; paths are
    relative to the hday200202/math-utils tree.
*/
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdlib.h>
#include <string.h>

/* ========================================================================= //
    Static-split thread pool (include/ai/ThreadPool.hpp:69-124)

    Persistent workers; thread i always takes slice(count, i, threads), the
    calling thread is thread 0. The split is contiguous and static, as the
    reference's Pool::run is, so per-thread work (and its imbalance on causal
    attention) is the reference's.
// ========================================================================= */

typedef void (*or_body)(size_t begin, size_t end, void* ctx);

typedef struct {
    pthread_t* workers;
    int size; /* including the caller */
    pthread_mutex_t mutex;
    pthread_cond_t wake, done;
    unsigned long epoch;
    int remaining, stopping;
    or_body body;
    void* ctx;
    size_t count;
} or_pool;

static or_pool g_pool;
static pthread_once_t g_pool_once = PTHREAD_ONCE_INIT;
static pthread_mutex_t g_run_mutex = PTHREAD_MUTEX_INITIALIZER;
static int g_pool_requested = 0;

/* ThreadPool.hpp:69-73 */
static void or_slice(size_t count, size_t index, size_t threads, size_t* b, size_t* e) {
    const size_t span = (count + threads - 1) / threads;
    size_t begin = index * span;
    if (begin > count) begin = count;
    size_t end = begin + span;
    if (end > count) end = count;
    *b = begin;
    *e = end;
}

static void* or_worker(void* arg) {
    const int index = (int)(intptr_t)arg;
    unsigned long seen = 0;
    for (;;) {
        pthread_mutex_lock(&g_pool.mutex);
        while (g_pool.epoch == seen && !g_pool.stopping)
            pthread_cond_wait(&g_pool.wake, &g_pool.mutex);
        if (g_pool.stopping) { pthread_mutex_unlock(&g_pool.mutex); return NULL; }
        seen = g_pool.epoch;
        or_body body = g_pool.body;
        void* ctx = g_pool.ctx;
        const size_t count = g_pool.count;
        pthread_mutex_unlock(&g_pool.mutex);

        size_t b, e;
        or_slice(count, (size_t)index, (size_t)g_pool.size, &b, &e);
        if (b < e) body(b, e, ctx);

        pthread_mutex_lock(&g_pool.mutex);
        if (--g_pool.remaining == 0) pthread_cond_signal(&g_pool.done);
        pthread_mutex_unlock(&g_pool.mutex);
    }
}

int or_threads(int requested) {
    if (requested > 0) return requested;
    cpu_set_t set;
    if (sched_getaffinity(0, sizeof(set), &set) == 0) {
        const int n = CPU_COUNT(&set);
        if (n > 0) return n;
    }
    return 1;
}

static void or_pool_start(void) {
    const int n = or_threads(g_pool_requested);
    g_pool.size = n;
    pthread_mutex_init(&g_pool.mutex, NULL);
    pthread_cond_init(&g_pool.wake, NULL);
    pthread_cond_init(&g_pool.done, NULL);
    g_pool.workers = (pthread_t*)calloc((size_t)(n > 1 ? n - 1 : 1), sizeof(pthread_t));
    for (int i = 1; i < n; ++i)
        pthread_create(&g_pool.workers[i - 1], NULL, or_worker, (void*)(intptr_t)i);
}

/* Runs body over [0, count) on `threads` threads (<= pool size), statically. */
static void or_pool_run(size_t count, int threads, or_body body, void* ctx) {
    if (count == 0) return;
    if (threads <= 1) { body(0, count, ctx); return; }
    if (g_pool_requested == 0) g_pool_requested = threads;
    pthread_once(&g_pool_once, or_pool_start);
    pthread_mutex_lock(&g_run_mutex);
    const int size = g_pool.size;
    if (size <= 1) { pthread_mutex_unlock(&g_run_mutex); body(0, count, ctx); return; }
    pthread_mutex_lock(&g_pool.mutex);
    g_pool.body = body;
    g_pool.ctx = ctx;
    g_pool.count = count;
    g_pool.remaining = size - 1;
    g_pool.epoch++;
    pthread_cond_broadcast(&g_pool.wake);
    pthread_mutex_unlock(&g_pool.mutex);

    size_t b, e;
    or_slice(count, 0, (size_t)size, &b, &e);
    if (b < e) body(b, e, ctx);

    pthread_mutex_lock(&g_pool.mutex);
    while (g_pool.remaining > 0) pthread_cond_wait(&g_pool.done, &g_pool.mutex);
    pthread_mutex_unlock(&g_pool.mutex);
    pthread_mutex_unlock(&g_run_mutex);
}

/* ========================================================================= //
    Random (include/math/Random.hpp:15-89)
// ========================================================================= */

static inline uint64_t or_rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

/* Random.hpp:81-86 */
static inline uint64_t or_splitmix64(uint64_t* x) {
    uint64_t z = (*x += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* Random.hpp:23-26: the four state words are consecutive splitmix64 outputs */
void or_rng_seed(or_rng* r, uint64_t seed) {
    for (int i = 0; i < 4; ++i) r->s[i] = or_splitmix64(&seed);
    r->has_spare = 0;
    r->spare = 0.0;
}

/* xoshiro256++ (Random.hpp:67-79) */
uint64_t or_rng_next(or_rng* r) {
    uint64_t* s = r->s;
    const uint64_t result = or_rotl(s[0] + s[3], 23) + s[0];
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = or_rotl(s[3], 45);
    return result;
}

/* Random.hpp:28 */
double or_rng_u01(or_rng* r) { return (double)(or_rng_next(r) >> 11) * 0x1.0p-53; }

/* Random.hpp:30 */
double or_rng_uniform(or_rng* r, double lo, double hi) { return lo + or_rng_u01(r) * (hi - lo); }

/* Random.hpp:32-39: rejection sampling against the largest multiple of span */
int64_t or_rng_int(or_rng* r, int64_t lo, int64_t hi) {
    const uint64_t span = (uint64_t)hi - (uint64_t)lo + 1;
    if (span == 0) return (int64_t)or_rng_next(r);
    const uint64_t limit = UINT64_MAX - (UINT64_MAX % span);
    uint64_t x;
    do { x = or_rng_next(r); } while (x >= limit);
    return lo + (int64_t)(x % span);
}

/* Box-Muller with a cached spare (Random.hpp:41-57) */
double or_rng_normal(or_rng* r, double mean, double stddev) {
    if (r->has_spare) {
        r->has_spare = 0;
        return mean + stddev * r->spare;
    }
    const double u1 = 1.0 - or_rng_u01(r);
    const double u2 = or_rng_u01(r);
    const double rad = sqrt(-2.0 * log(u1));
    const double theta = 2.0 * 3.14159265358979323846 * u2;
    r->spare = rad * sin(theta);
    r->has_spare = 1;
    return mean + stddev * (rad * cos(theta));
}

/* LocalModel.hpp:1621-1630 */
uint64_t or_fnv1a(const char* text) {
    uint64_t h = 0xCBF29CE484222325ULL;
    for (const unsigned char* c = (const unsigned char*)text; *c; ++c) {
        h ^= *c;
        h *= 0x100000001B3ULL;
    }
    return h;
}

enum { OR_FILL_CHUNK = 1 << 14 };

typedef struct {
    float* out;
    size_t n;
    uint64_t base;
    double a, b;
    int uniform;
} or_fill_ctx;

/* LocalModel.hpp:1555-1573: one generator per 2^14-element chunk */
static void or_fill_body(size_t begin, size_t end, void* p) {
    const or_fill_ctx* c = (const or_fill_ctx*)p;
    for (size_t chunk = begin; chunk < end; ++chunk) {
        or_rng r;
        or_rng_seed(&r, c->base + (uint64_t)chunk * 0x9E3779B97F4A7C15ULL);
        const size_t from = chunk * OR_FILL_CHUNK;
        const size_t to = from + OR_FILL_CHUNK < c->n ? from + OR_FILL_CHUNK : c->n;
        if (c->uniform)
            for (size_t i = from; i < to; ++i) c->out[i] = (float)or_rng_uniform(&r, c->a, c->b);
        else
            for (size_t i = from; i < to; ++i) c->out[i] = (float)or_rng_normal(&r, c->a, c->b);
    }
}

static void or_fill(float* out, size_t n, uint64_t seed, const char* name, double a, double b,
                    int uniform, int threads) {
    or_fill_ctx c = {out, n, seed ^ or_fnv1a(name), a, b, uniform};
    const size_t chunks = (n + OR_FILL_CHUNK - 1) / OR_FILL_CHUNK;
    or_pool_run(chunks, threads, or_fill_body, &c);
}

void or_fill_normal(float* out, size_t n, uint64_t seed, const char* name, double mean,
                    double stddev, int threads) {
    or_fill(out, n, seed, name, mean, stddev, 0, threads);
}

void or_fill_uniform(float* out, size_t n, uint64_t seed, const char* name, double lo,
                     double hi, int threads) {
    or_fill(out, n, seed, name, lo, hi, 1, threads);
}

/* ========================================================================= //
    bfloat16
// ========================================================================= */

uint16_t or_bf16_from_float(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float or_bf16_to_float(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float x;
    memcpy(&x, &u, 4);
    return x;
}

void or_round_to_bf16(float* x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = or_bf16_to_float(or_bf16_from_float(x[i]));
}

void or_pack_bf16(const float* x, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = or_bf16_from_float(x[i]);
}

void or_unpack_bf16(const uint16_t* x, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = or_bf16_to_float(x[i]);
}

/* ========================================================================= //
    Attention (include/ai/Kernels.hpp:39-70, 130-168)
// ========================================================================= */

enum { OR_LANES = 32 }; /* Kernels.hpp:55 */

/* Kernels.hpp:57-70: 32 interleaved accumulators, summed in order, then the tail */
float or_dot(const float* a, const float* b, size_t n) {
    float acc[OR_LANES] = {0};
    size_t i = 0;
    for (; i + OR_LANES <= n; i += OR_LANES)
        for (size_t j = 0; j < OR_LANES; ++j) acc[j] += a[i + j] * b[i + j];
    float sum = 0.0f;
    for (size_t j = 0; j < OR_LANES; ++j) sum += acc[j];
    for (; i < n; ++i) sum += a[i] * b[i];
    return sum;
}

typedef struct {
    const float *q, *keys, *values;
    float* out;
    size_t count, start, heads, kvHeads, dim, qStride, posStride, headStride, window;
    const uint32_t* rows;
} or_attn_ctx;

/* Kernels.hpp:137-162: per (token, head) task, scores row, max, exp-sum, PV */
static void or_attn_body(size_t begin, size_t end, void* p) {
    const or_attn_ctx* c = (const or_attn_ctx*)p;
    const float scale = 1.0f / sqrtf((float)c->dim);
    float* scores = (float*)malloc(sizeof(float) * (c->start + c->count + 1));
    for (size_t task = begin; task < end; ++task) {
        const size_t slot = task / c->heads, head = task % c->heads;
        const size_t token = c->rows ? c->rows[slot] : slot;
        const size_t position = c->start + token;
        const size_t first =
            c->window && position + 1 > c->window ? position + 1 - c->window : 0;
        const size_t kv = head / (c->heads / c->kvHeads);
        const float* query = c->q + (token * c->heads + head) * c->qStride;
        float maximum = -INFINITY;
        for (size_t j = first; j <= position; ++j) {
            scores[j] = or_dot(query, c->keys + j * c->posStride + kv * c->headStride, c->dim) * scale;
            if (scores[j] > maximum) maximum = scores[j];
        }
        float sum = 0;
        for (size_t j = first; j <= position; ++j) {
            scores[j] = expf(scores[j] - maximum);
            sum += scores[j];
        }
        float* dst = c->out + task * c->dim;
        for (size_t d = 0; d < c->dim; ++d) dst[d] = 0.0f;
        const float inv = 1.0f / sum;
        for (size_t j = first; j <= position; ++j) {
            const float w = scores[j] * inv;
            const float* v = c->values + j * c->posStride + kv * c->headStride;
            for (size_t d = 0; d < c->dim; ++d) dst[d] += w * v[d];
        }
    }
    free(scores);
}

void or_attention_strided(const float* q, const float* keys, const float* values, float* out,
                          size_t count, size_t start, size_t heads, size_t kvHeads, size_t dim,
                          size_t qStride, size_t posStride, size_t headStride, size_t window,
                          const uint32_t* rows, size_t nrows, int threads) {
    or_attn_ctx c = {q, keys, values, out, count, start, heads, kvHeads, dim,
                     qStride, posStride, headStride, window, rows};
    const size_t n = rows ? nrows : count;
    const size_t tasks = n * heads;
    /* Kernels.hpp:164-166: the pool only for substantial work */
    if (threads > 1 && tasks > 1 &&
        (double)n * (double)heads * (double)(start + (count + 1) / 2) * (double)dim >= 262144.0)
        or_pool_run(tasks, threads, or_attn_body, &c);
    else
        or_attn_body(0, tasks, &c);
}

void or_attention(const float* q, const float* keys, const float* values, float* out,
                  size_t count, size_t start, size_t heads, size_t kvHeads, size_t dim,
                  size_t qStride, size_t window, int threads) {
    or_attention_strided(q, keys, values, out, count, start, heads, kvHeads, dim, qStride,
                         kvHeads * dim, dim, window, NULL, 0, threads);
}

/* ========================================================================= //
    QK-RMSNorm and RoPE (include/ai/LocalModel.hpp:807-820, 1341-1348, 2608-2648)
// ========================================================================= */

/* LocalModel.hpp:1341-1348 */
void or_rms_norm_row(const float* x, const float* w, float* out, size_t n, float eps,
                     float weightOffset) {
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) sum += x[i] * x[i];
    const float inv = 1.0f / sqrtf(sum / (float)n + eps);
    for (size_t i = 0; i < n; ++i) out[i] = x[i] * inv * (w[i] + weightOffset);
}

/* LocalModel.hpp:807-820, with the parameter validation of :800-806 */
int or_rotary_frequencies(float* out, size_t rotaryDims, float theta, int type, float factor,
                          float lowFreq, float highFreq, float original) {
    if (!isfinite(theta) || theta <= 0 || !isfinite(factor) || factor < 1) return 0;
    if (type == 2 && (!isfinite(original) || original <= 0 || !isfinite(lowFreq) ||
                      !isfinite(highFreq) || lowFreq <= 0 || highFreq <= lowFreq))
        return 0;
    for (size_t j = 0; j < rotaryDims / 2; ++j) {
        float frequency = 1.0f / powf(theta, (float)(2 * j) / (float)rotaryDims);
        if (type == 1) frequency /= factor;
        if (type == 2) {
            const float wavelength = 6.283185307179586f / frequency;
            if (wavelength > original / lowFreq)
                frequency /= factor;
            else if (wavelength >= original / highFreq) {
                const float blend = (original / wavelength - lowFreq) / (highFreq - lowFreq);
                frequency *= (1 - blend) / factor + blend;
            }
        }
        out[j] = frequency;
    }
    return 1;
}

/* LocalModel.hpp:2608-2618 (norm) then :2624-2643 (rotate-half RoPE, fp32 angle) */
void or_qk_norm_rope(float* q, float* k, size_t count, size_t startPos, size_t heads,
                     size_t kvHeads, size_t dim, size_t qStride, const float* qGamma,
                     const float* kGamma, float eps, float weightOffset, const float* freqs,
                     size_t rotaryDims) {
    const size_t KW = kvHeads * dim;
    for (size_t t = 0; t < count; ++t) {
        if (qGamma)
            for (size_t h = 0; h < heads; ++h) {
                float* qh = q + t * heads * qStride + h * qStride;
                or_rms_norm_row(qh, qGamma, qh, dim, eps, weightOffset);
            }
        if (kGamma)
            for (size_t h = 0; h < kvHeads; ++h)
                or_rms_norm_row(k + t * KW + h * dim, kGamma, k + t * KW + h * dim, dim, eps,
                                weightOffset);
    }
    if (!freqs) return;
    const size_t half = rotaryDims / 2;
    for (size_t t = 0; t < count; ++t) {
        for (size_t j = 0; j < half; ++j) {
            const float angle = (float)(startPos + t) * freqs[j];
            const float cs = cosf(angle), sn = sinf(angle);
            for (size_t h = 0; h < heads; ++h) {
                float* x = q + t * heads * qStride + h * qStride;
                const float a = x[j], b = x[j + half];
                x[j] = a * cs - b * sn;
                x[j + half] = b * cs + a * sn;
            }
            for (size_t h = 0; h < kvHeads; ++h) {
                float* x = k + t * KW + h * dim;
                const float a = x[j], b = x[j + half];
                x[j] = a * cs - b * sn;
                x[j + half] = b * cs + a * sn;
            }
        }
    }
}

/* ========================================================================= //
    Gated delta rule (Kernels.hpp:102-128, LocalModel.hpp:1371-1386, 2797-2830)
// ========================================================================= */

float or_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

float or_softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

void or_l2normalise(float* v, size_t n, float eps) {
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) sum += v[i] * v[i];
    const float inv = 1.0f / sqrtf(sum + eps);
    for (size_t i = 0; i < n; ++i) v[i] *= inv;
}

/* Kernels.hpp:105-128: decay fused with prediction, rank-one update fused with
   the readout (out reads the updated state) */
void or_delta_step(float* state, const float* key, const float* query, const float* value,
                   const float* decay, int perKeyDecay, float beta, size_t keys, size_t values,
                   float* out, float* prediction, float* delta) {
    for (size_t d = 0; d < values; ++d) prediction[d] = 0.0f;
    for (size_t i = 0; i < keys; ++i) {
        float* row = state + i * values;
        const float a = decay[perKeyDecay ? i : 0], k = key[i];
        for (size_t d = 0; d < values; ++d) {
            row[d] *= a;
            prediction[d] += row[d] * k;
        }
    }
    for (size_t d = 0; d < values; ++d) delta[d] = (value[d] - prediction[d]) * beta;
    for (size_t d = 0; d < values; ++d) out[d] = 0.0f;
    for (size_t i = 0; i < keys; ++i) {
        float* row = state + i * values;
        const float k = key[i], q = query[i];
        for (size_t d = 0; d < values; ++d) {
            row[d] += k * delta[d];
            out[d] += row[d] * q;
        }
    }
}

/* LocalModel.hpp:2820-2823 */
void or_gdn_gates(const float* a, const float* b, const float* aLog, const float* dtBias,
                  float* g, float* beta, size_t count, size_t valueHeads) {
    for (size_t t = 0; t < count; ++t)
        for (size_t h = 0; h < valueHeads; ++h) {
            const size_t i = t * valueHeads + h;
            const float aPlusBias = a[i] + dtBias[h];
            g[i] = -expf(aLog[h]) * or_softplus(aPlusBias);
            beta[i] = or_sigmoid(b[i]);
        }
}

typedef struct {
    const float *q, *k, *v, *g, *beta;
    float *state, *out;
    size_t count, keyHeads, valueHeads, KD, VD;
    int normalize;
} or_gdn_ctx;

/* LocalModel.hpp:2802-2830, restricted to value heads [begin, end); with
   perKey set, the decay is one per key channel, g [count][valueHeads][KD] as
   kimiDeltaMixer's loop (LocalModel.hpp:2928-2947) */
static void or_gdn_body_impl(size_t begin, size_t end, void* p, int perKey) {
    const or_gdn_ctx* c = (const or_gdn_ctx*)p;
    const size_t KD = c->KD, VD = c->VD, nV = c->valueHeads;
    const size_t group = c->valueHeads / c->keyHeads;
    float* qh = (float*)malloc(sizeof(float) * KD);
    float* kh = (float*)malloc(sizeof(float) * KD);
    float* kv = (float*)malloc(sizeof(float) * VD);
    float* delta = (float*)malloc(sizeof(float) * VD);
    float* decays = (float*)malloc(sizeof(float) * KD);
    const float qScale = 1.0f / sqrtf((float)KD);
    for (size_t t = 0; t < c->count; ++t) {
        for (size_t vHead = begin; vHead < end; ++vHead) {
            const size_t kHead = vHead / group;
            memcpy(qh, c->q + (t * c->keyHeads + kHead) * KD, sizeof(float) * KD);
            memcpy(kh, c->k + (t * c->keyHeads + kHead) * KD, sizeof(float) * KD);
            if (c->normalize) {
                or_l2normalise(qh, KD, 1e-6f);
                or_l2normalise(kh, KD, 1e-6f);
                for (size_t i = 0; i < KD; ++i) qh[i] *= qScale;
            }
            const float beta = c->beta[t * nV + vHead];
            if (perKey) {
                for (size_t i = 0; i < KD; ++i) decays[i] = expf(c->g[(t * nV + vHead) * KD + i]);
            } else {
                decays[0] = expf(c->g[t * nV + vHead]);
            }
            or_delta_step(c->state + vHead * KD * VD, kh, qh, c->v + (t * nV + vHead) * VD, decays,
                          perKey, beta, KD, VD, c->out + (t * nV + vHead) * VD, kv, delta);
        }
    }
    free(decays);
    free(qh);
    free(kh);
    free(kv);
    free(delta);
}

static void or_gdn_body(size_t begin, size_t end, void* p) { or_gdn_body_impl(begin, end, p, 0); }
static void or_kda_body(size_t begin, size_t end, void* p) { or_gdn_body_impl(begin, end, p, 1); }

void or_kda_rule(const float* q, const float* k, const float* v, const float* g, const float* beta,
                 float* state, float* out, size_t count, size_t keyHeads, size_t valueHeads, size_t KD,
                 size_t VD, int normalize, int threads) {
    or_gdn_ctx c = {q, k, v, g, beta, state, out, count, keyHeads, valueHeads, KD, VD, normalize};
    if (threads > 1)
        or_pool_run(valueHeads, threads, or_kda_body, &c);
    else
        or_kda_body(0, valueHeads, &c);
}

void or_gated_delta_rule(const float* q, const float* k, const float* v, const float* g,
                         const float* beta, float* state, float* out, size_t count,
                         size_t keyHeads, size_t valueHeads, size_t KD, size_t VD,
                         int normalize, int threads) {
    or_gdn_ctx c = {q, k, v, g, beta, state, out, count, keyHeads, valueHeads, KD, VD, normalize};
    if (threads > 1)
        or_pool_run(valueHeads, threads, or_gdn_body, &c);
    else
        or_gdn_body(0, valueHeads, &c);
}


/* ========================================================================= //
    Gated DeltaNet neighbours of the recurrence (include/ai/LocalModel.hpp)
// ========================================================================= */

/* siluOf, LocalModel.hpp:1369 */
float or_silu(float x) { return x / (1.0f + expf(-x)); }

/* causalConvolution, LocalModel.hpp:2678-2708: channel c of token t mixes
   inputs t-K+1 .. t with kernel[c][0..K-1] (tap K-1 the current token),
   reaching back into `window` ([K-1][CW], its last row the most recent input)
   for t-K+1+j < 0, then SiLU. The window then holds the last K-1 inputs of
   window ++ in. */
void or_gdn_conv(const float* in, size_t count, size_t CW, size_t K, const float* kernel,
                 float* window, float* out) {
    for (size_t t = 0; t < count; ++t)
        for (size_t c = 0; c < CW; ++c) {
            float acc = 0.0f;
            for (size_t j = 0; j < K; ++j) {
                const long at = (long)t - (long)(K - 1) + (long)j;
                const float xv = at >= 0 ? in[(size_t)at * CW + c] : window[(size_t)((long)K - 1 + at) * CW + c];
                acc += kernel[c * K + j] * xv;
            }
            out[t * CW + c] = or_silu(acc);
        }
    if (K < 2) return;
    float* next = (float*)malloc((K - 1) * CW * sizeof(float));
    for (size_t i = 0; i < K - 1; ++i) {
        const long at = (long)count - (long)(K - 1) + (long)i;
        const float* src = at >= 0 ? &in[(size_t)at * CW] : &window[(size_t)((long)K - 1 + at) * CW];
        memcpy(&next[i * CW], src, CW * sizeof(float));
    }
    memcpy(window, next, (K - 1) * CW * sizeof(float));
    free(next);
}

/* the linFusedQKVZ de-interleave of gatedDeltaNetMixer, LocalModel.hpp:2739-2776.
   fused [count][nK][2 KD + 2 G VD]: per key head its q, its k, its G value
   heads' v, then the same heads' z; ba [count][nK][2 G]: the G heads' b,
   then their a. Out: qkv [count][CW] (all q, all k, all v), z [count][nV][VD],
   b, a [count][nV]. */
void or_gdn_deinterleave(const float* fused, const float* ba, size_t count, size_t nK, size_t nV,
                         size_t KD, size_t VD, float* qkv, float* z, float* b, float* a) {
    const size_t G = nV / nK, KW = nK * KD, VW = nV * VD, CW = 2 * KW + VW;
    const size_t stride = 2 * KD + 2 * G * VD, baStride = 2 * G;
    for (size_t t = 0; t < count; ++t)
        for (size_t kh = 0; kh < nK; ++kh) {
            const float* head = &fused[(t * nK + kh) * stride];
            const float* pair = &ba[(t * nK + kh) * baStride];
            memcpy(&qkv[t * CW + kh * KD], head, KD * sizeof(float));
            memcpy(&qkv[t * CW + KW + kh * KD], head + KD, KD * sizeof(float));
            for (size_t j = 0; j < G; ++j) {
                const size_t vh = kh * G + j;
                const float* vSrc = head + 2 * KD + j * VD;
                const float* zSrc = vSrc + G * VD;
                memcpy(&qkv[t * CW + 2 * KW + vh * VD], vSrc, VD * sizeof(float));
                memcpy(&z[t * VW + vh * VD], zSrc, VD * sizeof(float));
                b[t * nV + vh] = pair[j];
                a[t * nV + vh] = pair[G + j];
            }
        }
}

/* the gated norm after the recurrence, LocalModel.hpp:2833-2841: per token
   and value head, rmsNormRow(x, gamma, VD, eps) (weight stored directly,
   offset 0), then times siluOf(z) elementwise; kimiDeltaMixer (:2936-2945)
   multiplies by sigmoidOf(z) instead. x, z, out [count][nV][VD]. */
void or_gdn_gated_norm(const float* x, const float* z, const float* gamma, float eps, float* out,
                       size_t count, size_t nV, size_t VD, int sigmoidGate) {
    for (size_t r = 0; r < count * nV; ++r) {
        or_rms_norm_row(&x[r * VD], gamma, &out[r * VD], VD, eps, 0.0f);
        for (size_t d = 0; d < VD; ++d)
            out[r * VD + d] *= sigmoidGate ? or_sigmoid(z[r * VD + d]) : or_silu(z[r * VD + d]);
    }
}

/* kimiDeltaMixer's gate loop, LocalModel.hpp:2894-2905, kept as the log
   decay g (the reference goes on to store exp(g)) */
void or_kda_gates(const float* f, const float* b, const float* aLog, const float* dtBias, int safeGate,
                  float lowerBound, float* g, float* beta, size_t count, size_t valueHeads, size_t KD) {
    for (size_t t = 0; t < count; ++t)
        for (size_t h = 0; h < valueHeads; ++h) {
            const float rate = expf(aLog[h]);
            for (size_t i = 0; i < KD; ++i) {
                const size_t c = (t * valueHeads + h) * KD + i;
                const float x = f[c] + dtBias[h * KD + i];
                g[c] = safeGate ? lowerBound * or_sigmoid(rate * x) : -rate * or_softplus(x);
            }
            beta[t * valueHeads + h] = or_sigmoid(b[t * valueHeads + h]);
        }
}

/* the attention output gate of attentionMixer, LocalModel.hpp:2660-2665:
   out[t][h][d] *= sigmoidOf(q[(t heads + h) qStride + dim + d]) */
void or_output_gate(float* out, const float* q, size_t count, size_t heads, size_t dim, size_t qStride) {
    for (size_t t = 0; t < count; ++t)
        for (size_t h = 0; h < heads; ++h) {
            const float* g = &q[(t * heads + h) * qStride + dim];
            float* o = &out[(t * heads + h) * dim];
            for (size_t d = 0; d < dim; ++d) o[d] *= or_sigmoid(g[d]);
        }
}

/* ---- projections ---- */

void or_dequant(const void* codes, const float* scales, size_t outDim, size_t inDim, int type, float* out) {
    const size_t blocks = inDim / 32;
    for (size_t r = 0; r < outDim; ++r) {
        const float* s = scales + r * blocks;
        if (type == 2) {
            const int8_t* q = (const int8_t*)codes + r * inDim;
            for (size_t i = 0; i < blocks * 32; ++i) out[r * inDim + i] = (float)q[i] * s[i / 32];
        } else {
            const uint8_t* q = (const uint8_t*)codes + r * (inDim / 2);
            for (size_t b = 0; b < blocks; ++b)
                for (size_t j = 0; j < 16; ++j) {
                    const uint8_t packed = q[b * 16 + j];
                    out[r * inDim + b * 32 + j] = (float)((int)(packed & 0x0F) - 8) * s[b];
                    out[r * inDim + b * 32 + j + 16] = (float)((int)(packed >> 4) - 8) * s[b];
                }
        }
    }
}

void or_matmul_nt(const float* a, const void* w, const float* scales, const float* bias, float* out,
                  size_t m, size_t k, size_t n, int type) {
    float* row = (float*)malloc(sizeof(float) * k);
    for (size_t j = 0; j < n; ++j) {
        if (type == 0) {
            memcpy(row, (const float*)w + j * k, sizeof(float) * k);
        } else if (type == 1) {
            const uint16_t* b = (const uint16_t*)w + j * k;
            for (size_t t = 0; t < k; ++t) {
                const uint32_t bits = (uint32_t)b[t] << 16;
                memcpy(&row[t], &bits, 4);
            }
        } else {
            const size_t bytes = type == 2 ? k : k / 2;
            or_dequant((const uint8_t*)w + j * bytes, scales + j * (k / 32), 1, k, type, row);
        }
        for (size_t i = 0; i < m; ++i) {
            double s = 0.0;
            for (size_t t = 0; t < k; ++t) s += (double)a[i * k + t] * (double)row[t];
            out[i * n + j] = (float)s + (bias ? bias[j] : 0.0f);
        }
    }
    free(row);
}

/* ---- multi-head latent attention ---- */

void or_latent_attention(const float* q, const float* latent, const float* wkv, const uint32_t* selStart,
                         const uint32_t* selCount, const uint32_t* selKeys, float* out, size_t count,
                         size_t startPos, size_t nH, size_t Dn, size_t Dv, size_t C, float scale) {
    const size_t perHead = Dn + Dv;
    float* folded = (float*)malloc(sizeof(float) * C);
    float* context = (float*)malloc(sizeof(float) * C);
    float* scores = (float*)malloc(sizeof(float) * (startPos + count + 1));
    for (size_t job = 0; job < count * nH; ++job) {
        const size_t t = job / nH, head = job % nH;
        const size_t pos = startPos + t;
        const float* qh = &q[(t * nH + head) * Dn];
        const float* Wk = wkv + head * perHead * C;
        const float* Wv = Wk + Dn * C;
        for (size_t c = 0; c < C; ++c) folded[c] = 0.0f;
        for (size_t d = 0; d < Dn; ++d) {
            const float qd = qh[d];
            const float* row = Wk + d * C;
            for (size_t c = 0; c < C; ++c) folded[c] += qd * row[c];
        }
        const int dense = !selCount || selCount[t] == 0xFFFFFFFFu;
        const size_t n = dense ? pos + 1 : selCount[t];
        float best = -1e30f;
        for (size_t i = 0; i < n; ++i) {
            const size_t key = dense ? i : selKeys[selStart[t] + i];
            scores[i] = or_dot(folded, latent + key * C, C) * scale;
            if (scores[i] > best) best = scores[i];
        }
        float sum = 0.0f;
        for (size_t i = 0; i < n; ++i) {
            scores[i] = expf(scores[i] - best);
            sum += scores[i];
        }
        const float inv = 1.0f / sum;
        for (size_t c = 0; c < C; ++c) context[c] = 0.0f;
        for (size_t i = 0; i < n; ++i) {
            const size_t key = dense ? i : selKeys[selStart[t] + i];
            const float p = scores[i] * inv;
            const float* cr = latent + key * C;
            for (size_t j = 0; j < C; ++j) context[j] += p * cr[j];
        }
        float* o = &out[(t * nH + head) * Dv];
        for (size_t v = 0; v < Dv; ++v) o[v] = or_dot(Wv + v * C, context, C);
    }
    free(folded);
    free(context);
    free(scores);
}

/* ---- the sparse-attention indexer (selectKeys, LocalModel.hpp:2971-3068) ---- */

/* layerNormRow (LocalModel.hpp:1355-1367): mean, then the mean square of the
   deviations, both summed in order in fp32 */
static void or_layer_norm_row(const float* x, const float* w, const float* b, float* out, size_t n, float eps) {
    float mean = 0.0f;
    for (size_t i = 0; i < n; ++i) mean += x[i];
    mean /= (float)n;
    float var = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        const float d = x[i] - mean;
        var += d * d;
    }
    var /= (float)n;
    const float inv = 1.0f / sqrtf(var + eps);
    for (size_t i = 0; i < n; ++i) out[i] = (x[i] - mean) * inv * w[i] + (b ? b[i] : 0.0f);
}

void or_index_update(const float* k, const float* kNorm, const float* kNormBias, const float* ape, float* keys,
                     const float* gates, float* pools, size_t count, size_t startPos, size_t Di, size_t P) {
    float* weight = (float*)malloc(sizeof(float) * (P ? P : 1));
    for (size_t t = 0; t < count; ++t) {
        const size_t pos = startPos + t;
        or_layer_norm_row(k + t * Di, kNorm, kNormBias, keys + pos * Di, Di, 1e-6f);   /* :2988-2990 */
        if ((pos + 1) % P != 0) continue;                                               /* :2994 */
        const size_t first = pos + 1 - P;
        float* pooled = pools + (pos / P) * Di;
        for (size_t d = 0; d < Di; ++d) {                                               /* :2998-3009 */
            float best = -1e30f;
            for (size_t i = 0; i < P; ++i) {
                weight[i] = gates[(first + i) * Di + d] + ape[i * Di + d];
                if (weight[i] > best) best = weight[i];
            }
            float sum = 0.0f;
            for (size_t i = 0; i < P; ++i) {
                weight[i] = expf(weight[i] - best);
                sum += weight[i];
            }
            float acc = 0.0f;
            for (size_t i = 0; i < P; ++i) acc += weight[i] / sum * keys[(first + i) * Di + d];
            pooled[d] = acc;
        }
    }
    free(weight);
}

void or_select_keys(const float* q, const float* w, const float* pools, uint32_t* selStart, uint32_t* selCount,
                    uint32_t* selKeys, float* scores, size_t count, size_t startPos, size_t nI, size_t Di,
                    size_t P, size_t topK, int tail) {
    const size_t budget = topK / P, stride = budget * P + P;
    const size_t maxPools = (startPos + count) / P;
    const float headScale = 1.0f / sqrtf((float)nI), dimScale = 1.0f / sqrtf((float)Di);   /* :3024-3025 */
    float* score = (float*)malloc(sizeof(float) * (maxPools ? maxPools : 1));
    uint8_t* chosen = (uint8_t*)malloc(maxPools ? maxPools : 1);
    for (size_t t = 0; t < count; ++t) {
        const size_t pos = startPos + t, complete = (pos + 1) / P;
        selStart[t] = (uint32_t)(t * stride);
        if (complete <= budget && tail) {   /* :3036: sees everything */
            selCount[t] = 0xFFFFFFFFu;
            continue;
        }
        for (size_t p = 0; p < complete; ++p) {   /* :3038-3047 */
            float total = 0.0f;
            for (size_t h = 0; h < nI; ++h) {
                const float logit = or_dot(&q[(t * nI + h) * Di], pools + p * Di, Di) * dimScale;
                total += w[t * nI + h] * headScale * (logit > 0.0f ? logit : 0.0f);
            }
            score[p] = total;
            if (scores) scores[t * maxPools + p] = total;
        }
        /* the keep best (:3049-3053); among equal scores the lower pool index
           (nth_element leaves that order unspecified) */
        const size_t keep = budget < complete ? budget : complete;
        for (size_t p = 0; p < complete; ++p) {
            size_t above = 0;
            for (size_t o = 0; o < complete && above < keep; ++o)
                if (score[o] > score[p] || (score[o] == score[p] && o < p)) ++above;
            chosen[p] = above < keep;
        }
        size_t n = 0;
        for (size_t p = 0; p < complete; ++p)   /* :3055-3059, in key order (the sort, :3066) */
            if (chosen[p])
                for (size_t j = 0; j < P; ++j) selKeys[t * stride + n++] = (uint32_t)(p * P + j);
        if (tail)                               /* :3062-3064 */
            for (size_t j = complete * P; j <= pos; ++j) selKeys[t * stride + n++] = (uint32_t)j;
        selCount[t] = (uint32_t)n;
    }
    free(score);
    free(chosen);
}

