/*
    oracle.h - CPU restatement of the reference attention hot path.

    TEST INFRASTRUCTURE ONLY. Nothing in the product (math-utils_amd/) links,
    loads or calls this code. It is the checker for the HIP backend: tests/
    compare the GPU results with it, bench.py times it as the CPU baseline,
    and __graft_entry__.smoke() uses it to check one small GPU invocation.

    Each function cites the reference file:line it restates (paths relative to
    the hday200202/math-utils tree). The arithmetic follows the reference's
    order of operations: 32-accumulator dot, two-pass softmax, fp32 everywhere,
    static contiguous split across threads.

    Pinning (what checks each function, beyond retyping it):
      or_rng_*                 known-answer stream of the published
                               splitmix64/xoshiro256++ generators, plus the
                               reference's own Random compiled into oracle/_ref
      or_attention*            bit-compared against the reference's
                               kernels::attention compiled from its own header
                               (oracle/_ref), and against an fp64 closed form
                               (llm-testing.cpp:106-134 restated)
      or_delta_step            bit-compared against kernels::deltaStep (_ref),
                               and against the four-pass restatement of
                               llm-testing.cpp:813-851
      or_rms_norm_row,
      or_qk_norm_rope          closed forms and invariants: rms of normed/gamma
                               is 1, RoPE keeps pair norms, position 0 is the
                               identity, fp64 rotation matches
      or_rotary_frequencies    closed form 1/theta^(2j/rot); linear and llama3
                               scaling against llm-testing.cpp:141-145's
                               expected values
      or_gated_delta_rule      bit-compared against the reference's deltaStep
                               driven token by token (ref_gated_delta_rule in
                               oracle/_ref); equals or_delta_step applied step
                               by step; beta=0 and decay=1 special cases; one
                               token equals one deltaStep; l2norm closed form
      or_gdn_gates             closed form of softplus / sigmoid
      or_kda_rule              bit-compared against the reference's deltaStep
                               with perKeyDecay driven token by token
                               (ref_kda_rule in oracle/_ref); equal decays in
                               every channel reduce it to or_gated_delta_rule
      or_gdn_conv              the reference's header (LocalModel.hpp) needs
                               <format>, absent from this image's libstdc++,
                               so it cannot be compiled into oracle/_ref.
                               Pinned by: an fp64 per-channel convolution with
                               asymmetric taps and a nonzero carried window;
                               a one-hot current tap reduces to SiLU(x); and
                               window continuity, token-by-token calls equal
                               one call (llm-testing.cpp:853-890 checks the
                               same of the reference's window)
      or_gdn_deinterleave      round trip: the fused rows are built per key
                               head by concatenation as the reference's comment
                               states (q, k, the group's v, the group's z; b
                               then a), and come back as the plain layout
      or_gdn_gated_norm,
      or_silu                  fp64 closed form (both gate kinds); a constant
                               row normalises to sign * gamma; SiLU(0) = 0 and
                               SiLU(x) -> x
      or_kda_gates             fp64 closed forms of both gate forms, including
                               softplus's x > 20 branch; the safe gate stays in
                               [lowerBound, 0]; the bias is per channel and the
                               rate sits inside the sigmoid
      or_output_gate           fp64 closed form; a zero gate halves the output,
                               a large one leaves it, and only the second half
                               of each q row is read
*/
#ifndef ORACLE_H
#define ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- seeded inputs: math::random::Random (include/math/Random.hpp:15-89) ---- */
typedef struct or_rng {
    uint64_t s[4];
    double spare;
    int has_spare;
} or_rng;

void     or_rng_seed(or_rng* r, uint64_t seed);
uint64_t or_rng_next(or_rng* r);
double   or_rng_u01(or_rng* r);
double   or_rng_uniform(or_rng* r, double lo, double hi);
int64_t  or_rng_int(or_rng* r, int64_t lo, int64_t hi);
double   or_rng_normal(or_rng* r, double mean, double stddev);

/* FNV-1a as LocalModel::stableHash (include/ai/LocalModel.hpp:1621-1630) */
uint64_t or_fnv1a(const char* text);

/* chunked, named fill as the random initialiser (LocalModel.hpp:1555-1573):
   chunk c of 2^14 elements draws from Random(seed ^ fnv1a(name) + c*golden) */
void or_fill_normal(float* out, size_t n, uint64_t seed, const char* name,
                    double mean, double stddev, int threads);
void or_fill_uniform(float* out, size_t n, uint64_t seed, const char* name,
                     double lo, double hi, int threads);

/* bfloat16 round-to-nearest-even and widening (a shift, Kernels.hpp:84-99) */
uint16_t or_bf16_from_float(float x);
float    or_bf16_to_float(uint16_t b);
void     or_round_to_bf16(float* x, size_t n);                 /* in place */
void     or_pack_bf16(const float* x, uint16_t* out, size_t n);
void     or_unpack_bf16(const uint16_t* x, float* out, size_t n);

/* ---- attention: kernels::attention (include/ai/Kernels.hpp:130-168) ---- */
float or_dot(const float* a, const float* b, size_t n);       /* Kernels.hpp:55-70 */

/* Same argument list and layouts as kernels::attention: q [count][heads][qStride],
   keys/values position-major [pos][kvHeads][dim], out [count][heads][dim].
   threads>1 uses a static contiguous split (ThreadPool.hpp:69-124) under the
   same work threshold as Kernels.hpp:165. */
void or_attention(const float* q, const float* keys, const float* values, float* out,
                  size_t count, size_t start, size_t heads, size_t kvHeads, size_t dim,
                  size_t qStride, size_t window, int threads);

/* The same arithmetic with an explicit key/value layout (element strides per
   position and per kv head) and an optional subset of query tokens: tokens
   [rows[i]] for i < nrows (rows == NULL means all `count`). out is
   [nrows][heads][dim]. Used for head-major caches and for sampled rows of
   large problems. */
void or_attention_strided(const float* q, const float* keys, const float* values,
                          float* out, size_t count, size_t start, size_t heads,
                          size_t kvHeads, size_t dim, size_t qStride,
                          size_t posStride, size_t headStride, size_t window,
                          const uint32_t* rows, size_t nrows, int threads);

/* ---- norm and RoPE glue of LocalModel::attentionMixer ---- */
/* rmsNormRow (LocalModel.hpp:1341-1348) */
void or_rms_norm_row(const float* x, const float* w, float* out, size_t n, float eps,
                     float weightOffset);

/* LocalConfig rotary table (LocalModel.hpp:807-820). type 0 default, 1 linear,
   2 llama3. Returns 0 on invalid parameters. */
int or_rotary_frequencies(float* out, size_t rotaryDims, float theta, int type,
                          float factor, float lowFreq, float highFreq, float original);

/* attentionMixer QK-RMSNorm then RoPE, in place (LocalModel.hpp:2608-2648).
   q [count][heads][qStride], k [count][kvHeads][dim]. qGamma/kGamma NULL skips
   the norm; freqs NULL skips RoPE. */
void or_qk_norm_rope(float* q, float* k, size_t count, size_t startPos, size_t heads,
                     size_t kvHeads, size_t dim, size_t qStride, const float* qGamma,
                     const float* kGamma, float eps, float weightOffset,
                     const float* freqs, size_t rotaryDims);

/* ---- gated delta rule ---- */
float or_sigmoid(float x);                                   /* LocalModel.hpp:1371 */
float or_softplus(float x);                                  /* LocalModel.hpp:1374-1376 */
void  or_l2normalise(float* v, size_t n, float eps);         /* LocalModel.hpp:1380-1386 */

/* kernels::deltaStep (Kernels.hpp:102-128) */
void or_delta_step(float* state, const float* key, const float* query, const float* value,
                   const float* decay, int perKeyDecay, float beta, size_t keys,
                   size_t values, float* out, float* prediction, float* delta);

/* gate computation of gatedDeltaNetMixer (LocalModel.hpp:2820-2823):
   g = -exp(aLog[h]) * softplus(a + dtBias[h]); beta = sigmoid(b). a, b, g,
   beta are [count][valueHeads]. */
void or_gdn_gates(const float* a, const float* b, const float* aLog, const float* dtBias,
                  float* g, float* beta, size_t count, size_t valueHeads);

/* The recurrence loop of gatedDeltaNetMixer (LocalModel.hpp:2802-2830).
   q,k [count][keyHeads][KD]; v [count][valueHeads][VD]; g (log decay) and
   beta [count][valueHeads]; state [valueHeads][KD][VD] in/out; out
   [count][valueHeads][VD]. normalize != 0 applies l2normalise to q and k and
   scales q by 1/sqrt(KD) as the mixer does; 0 takes q,k as given.
   threads > 1 splits value heads statically (the reference runs this loop on
   one thread; heads are independent so the split changes no arithmetic). */
void or_gated_delta_rule(const float* q, const float* k, const float* v, const float* g,
                         const float* beta, float* state, float* out, size_t count,
                         size_t keyHeads, size_t valueHeads, size_t KD, size_t VD,
                         int normalize, int threads);

/* ---- Gated DeltaNet neighbours ---- */
float or_silu(float x);                                      /* LocalModel.hpp:1369 */
/* causalConvolution (LocalModel.hpp:2678-2708): in, out [count][CW]; kernel
   [CW][K]; window [K-1][CW] read, then replaced by the last K-1 inputs */
void or_gdn_conv(const float* in, size_t count, size_t CW, size_t K, const float* kernel,
                 float* window, float* out);
/* the linFusedQKVZ de-interleave (LocalModel.hpp:2739-2776) */
void or_gdn_deinterleave(const float* fused, const float* ba, size_t count, size_t nK, size_t nV,
                         size_t KD, size_t VD, float* qkv, float* z, float* b, float* a);
/* rmsNormRow then x SiLU(z) per (token, value head) (LocalModel.hpp:2833-2841);
   sigmoidGate != 0: x sigmoid(z) instead, kimiDeltaMixer's form (:2936-2945) */
void or_gdn_gated_norm(const float* x, const float* z, const float* gamma, float eps, float* out,
                       size_t count, size_t nV, size_t VD, int sigmoidGate);

/* attentionMixer's output gate (LocalModel.hpp:2660-2665): out [count][heads][dim]
   times sigmoid of the second dim elements of each q row (qStride >= 2 dim) */
void or_output_gate(float* out, const float* q, size_t count, size_t heads, size_t dim, size_t qStride);

/* Kimi Delta Attention's recurrence (kimiDeltaMixer, LocalModel.hpp:2928-2947):
   as or_gated_delta_rule, but the decay is one per key channel: g is the log
   decay [count][valueHeads][KD], and deltaStep runs with perKeyDecay */
void or_kda_rule(const float* q, const float* k, const float* v, const float* g, const float* beta,
                 float* state, float* out, size_t count, size_t keyHeads, size_t valueHeads, size_t KD,
                 size_t VD, int normalize, int threads);

/* kimiDeltaMixer's gates (LocalModel.hpp:2894-2905) as log decays: with
   rate = exp(aLog[h]) and x = f[t][h][i] + dtBias[h][i],
   g = safeGate ? lowerBound sigmoid(rate x) : -rate softplus(x); beta =
   sigmoid(b). f, g [count][valueHeads][KD]; b, beta [count][valueHeads]. The
   reference stores exp(g); the recurrence here takes g and exponentiates it. */
void or_kda_gates(const float* f, const float* b, const float* aLog, const float* dtBias, int safeGate,
                  float lowerBound, float* g, float* beta, size_t count, size_t valueHeads, size_t KD);

/* ---- projections ---- */
/* dequantRange (Quant.hpp:528-549) of every row: type 2 (Q8) code * scale;
   type 3 (Q4) byte j of a 32-block gives code j (low nibble) and code j+16
   (high nibble), each minus 8, times the block's scale. codes [outDim][inDim]
   (Q8) or [outDim][inDim/2] (Q4), scales [outDim][inDim/32]. */
void or_dequant(const void* codes, const float* scales, size_t outDim, size_t inDim, int type, float* out);
/* apply (LocalModel.hpp:1052-1078): out[m][n] = sum_k a[m][k] w[n][k] (+ bias[n]),
   the weight widened (type 0 fp32, 1 bf16 bits << 16) or dequantised (2 Q8,
   3 Q4) first; the products of fp32 values are summed in double, so the
   result is the rounded exact sum (the reference's CPU and GPU paths each
   sum in their own order). */
void or_matmul_nt(const float* a, const void* w, const float* scales, const float* bias, float* out,
                  size_t m, size_t k, size_t n, int type);

/* ---- multi-head latent attention ---- */
/* latentAttentionMixer's attention (LocalModel.hpp:3118-3158), per token t
   and head h: folded = sum_d q[t][h][d] Wk_h[d] (Wk_h the first Dn rows of
   head h's Dn + Dv rows of wkv, each C wide); scores against the cached
   latents latent[pos][C] by or_dot, times `scale`; the reference's softmax
   (max, exp, sum, then p = e * (1/sum)); context = sum p * latent; out[v] =
   or_dot(Wv_h[v], context). Token t sees positions 0..startPos+t (dense),
   or when selCount[t] != UINT32_MAX the sorted list selKeys[selStart[t] ..
   + selCount[t]) (KeySelection, :1203-1206). */
void or_latent_attention(const float* q, const float* latent, const float* wkv, const uint32_t* selStart,
                         const uint32_t* selCount, const uint32_t* selKeys, float* out, size_t count,
                         size_t startPos, size_t nH, size_t Dn, size_t Dv, size_t C, float scale);

/* selectKeys's cache update (LocalModel.hpp:2982-3011): layerNormRow (eps
   1e-6, :1355-1367) of each new token's index key k[t] into keys[pos], and
   every pool a token of the call completes folded from its P members, channel
   by channel, by the softmax of gates + ape. gates[pos] hold the caller's
   idxGate projection already. */
void or_index_update(const float* k, const float* kNorm, const float* kNormBias, const float* ape, float* keys,
                     const float* gates, float* pools, size_t count, size_t startPos, size_t Di, size_t P);

/* selectKeys's choice (:3013-3067): per token, relu-scored pools summed over
   the nI heads under w, the topK / P best (equal scores: the lower pool
   index), expanded to their keys in order, then the unfinished pool when
   tail. selStart[t] = t * (topK / P * P + P); selCount[t] = UINT32_MAX for a
   token that sees every key. scores, if not NULL, receives [count][(startPos
   + count) / P] (entries past a token's complete pools untouched). */
void or_select_keys(const float* q, const float* w, const float* pools, uint32_t* selStart, uint32_t* selCount,
                    uint32_t* selKeys, float* scores, size_t count, size_t startPos, size_t nI, size_t Di,
                    size_t P, size_t topK, int tail);

/* number of threads the static pool would use given a request (<=0: all
   online CPUs in this process's affinity mask) */
int or_threads(int requested);

#ifdef __cplusplus
}
#endif

#endif
