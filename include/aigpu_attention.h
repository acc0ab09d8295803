#ifndef AIGPU_ATTENTION_H
#define AIGPU_ATTENTION_H

/*
    aigpu_attention.h - the C ABI of the MI355X (gfx950) attention backend.

    Same conventions as the reference's device boundary
    (include/ai/gpu/DeviceABI.h in hday200202/math-utils):
      - plain C symbols with the aigpu_ prefix; scalars, pointers and POD
        structs only; structs go in by pointer, never by value
        (DeviceABI.h:59-65);
      - strings are borrowed from the backend (DeviceABI.h:79-83);
      - the allocator frees: device memory comes from aigpu_upload /
        aigpu_allocate and goes back through aigpu_release
        (DeviceABI.h:89-99);
      - every entry returns 1 on success and 0 on failure with the reason in
        aigpu_last_error(); aigpu_available() is safe to call first
        (DeviceABI.h:75-77);
      - calls are serialised on one process-wide lock, as the reference
        backend's Context::gate does (src/gpu/Kernels.hip:48-63);
      - AiGpuCounters separate kernel time from transfer time
        (DeviceABI.h:66-72).

    The attention entries replace these CPU call sites of the reference:
      kernels::attention     include/ai/Kernels.hpp:132-134, called at
                             include/ai/LocalModel.hpp:2657-2659
      norm -> RoPE -> append -> attention of attentionMixer
                             include/ai/LocalModel.hpp:2608-2659
      the per-token deltaStep loop of gatedDeltaNetMixer
                             include/ai/LocalModel.hpp:2802-2830 (deltaStep at
                             include/ai/Kernels.hpp:105-128)

    Layouts. Host-side tensors keep the reference's layouts: q
    [count][heads][qStride], k/v [count][kvHeads][dim], out
    [count][heads][dim] (Kernels.hpp:143-154). The device KV cache is
    head-major bf16: [kvHeads][capacity][dim] per sequence, so each KV head's
    history is one contiguous run in HBM.
*/

#include <stddef.h>
#include <stdint.h>

/*
    Shared with the reference's boundary. include/ai/gpu/DeviceABI.h
    (guard AI_GPU_DEVICE_ABI_H) defines AiGpuCounters, the AiGpuDense*
    structs and the device-management, projection and resident-decoder entry
    points that this backend implements too. Where that header is reachable
    (on the include path as ai/gpu/DeviceABI.h, or beside this file) it is
    included here and those definitions are taken from it, so both headers
    can share a translation unit in either order. Elsewhere this file
    declares the same types, with the same layouts, and the same entry
    points itself.
*/
#if !defined(AI_GPU_DEVICE_ABI_H) && defined(__has_include)
#if __has_include("ai/gpu/DeviceABI.h")
#include "ai/gpu/DeviceABI.h"
#elif __has_include("DeviceABI.h")
#include "DeviceABI.h"
#endif
#endif

#if defined(_WIN32)
#define AIGPU_ABI __declspec(dllexport)
#else
#define AIGPU_ABI __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* element types of tensors crossing the boundary */
enum { AIGPU_F32 = 0, AIGPU_BF16 = 1 };

#ifndef AI_GPU_DEVICE_ABI_H
/* DeviceABI.h:66-72 */
typedef struct AiGpuCounters {
    uint64_t launches;
    uint64_t hostToDeviceBytes;
    uint64_t deviceToHostBytes;
    double kernelSeconds;
    double transferSeconds;
} AiGpuCounters;

/* ---- device entry points, as DeviceABI.h:75-118 ---- */
AIGPU_ABI int aigpu_available(void);                               /* DeviceABI.h:77 */
AIGPU_ABI const char* aigpu_device_name(void);                     /* DeviceABI.h:82 */
AIGPU_ABI const char* aigpu_last_error(void);                      /* DeviceABI.h:83 */
AIGPU_ABI uint64_t aigpu_total_memory(void);                       /* DeviceABI.h:85 */
AIGPU_ABI uint64_t aigpu_free_memory(void);                        /* DeviceABI.h:86 */
AIGPU_ABI uint64_t aigpu_allocated_bytes(void);                    /* DeviceABI.h:87 */
AIGPU_ABI void* aigpu_upload(const void* host, uint64_t bytes);    /* DeviceABI.h:97 */
AIGPU_ABI void aigpu_release(void* device, uint64_t bytes);        /* DeviceABI.h:98 */
AIGPU_ABI int aigpu_download(void* host, const void* device, uint64_t bytes); /* DeviceABI.h:99 */
AIGPU_ABI void aigpu_synchronize(void);                            /* DeviceABI.h:115 */
AIGPU_ABI void aigpu_counters(AiGpuCounters* out);                 /* DeviceABI.h:117 */
AIGPU_ABI void aigpu_reset_counters(void);                         /* DeviceABI.h:118 */
#endif /* !AI_GPU_DEVICE_ABI_H */

/* New beside aigpu_upload: a zero-filled device allocation (KV caches,
   recurrent states) released by aigpu_release, and a host->device copy into
   an existing allocation at a byte offset. */
AIGPU_ABI void* aigpu_allocate(uint64_t bytes);
AIGPU_ABI int aigpu_write(void* device, uint64_t offset, const void* host, uint64_t bytes);

/* ------------------------------------------------------------------------ */
/* 1. Drop-in for kernels::attention (Kernels.hpp:132-134).                  */
/*    Host pointers, fp32, the reference's position-major KV                 */
/*    [pos][kvHeads][dim]; same argument list and meaning. Staged in,         */
/*    computed in fp32 on the GPU, copied back. Replaces the call at          */
/*    LocalModel.hpp:2657-2659 line for line.                                 */
/* ------------------------------------------------------------------------ */
AIGPU_ABI int aigpu_attention(const float* q, const float* keys, const float* values,
                              float* out, uint64_t count, uint64_t start, uint64_t heads,
                              uint64_t kvHeads, uint64_t dim, uint64_t qStride,
                              uint64_t window);

/* 2. The same computation on device pointers, with a dtype tag for q and for
      the KV history and explicit KV element strides, so one entry serves the
      reference's position-major layout (posStride = kvHeads*dim,
      headStride = dim) and the head-major cache (posStride = dim,
      headStride = capacity*dim). fp32 arithmetic; out is fp32. */
typedef struct AiGpuAttention {
    const void* q;            /* [count][heads][qStride], qType */
    const void* keys;         /* kvType, element (pos, head) at pos*posStride + head*headStride */
    const void* values;
    float* out;               /* [count][heads][dim] */
    uint32_t qType, kvType;
    uint64_t count, start, heads, kvHeads, dim, qStride, window;
    uint64_t posStride, headStride;
    void* stream;             /* hipStream_t; NULL = default stream */
} AiGpuAttention;
AIGPU_ABI int aigpu_attention_device(const AiGpuAttention* args);

/* ------------------------------------------------------------------------ */
/* 3. Prefill: attentionMixer's QK-RMSNorm -> RoPE -> KV append -> causal    */
/*    attention (LocalModel.hpp:2608-2659) for `count` new tokens at          */
/*    positions start..start+count-1, against a head-major bf16 cache that    */
/*    already holds positions [0, start). Flash-style kernel on fp16 MFMA     */
/*    with fp32 accumulation. dim must be 64 or 128. q, k, v (after norm,     */
/*    RoPE and q's scale) and the cached history go through fp16. A value     */
/*    fp16 cannot hold (|x| >= 65520) raises the call's range flag (below);   */
/*    the call has still written out and the new k, v rows of the cache.     */
/*    The device form is asynchronous: it launches on its stream and         */
/*    returns without waiting, and aigpu_range_status reports its flag. The   */
/*    host form waits for its kernels anyway and returns 0 with a reason.     */
/* ------------------------------------------------------------------------ */
typedef struct AiGpuPrefill {
    const void* q;            /* [count][heads][qStride], inType */
    const void* k;            /* [count][kvHeads][dim], inType */
    const void* v;            /* [count][kvHeads][dim], inType */
    float* out;               /* [count][heads][dim] fp32 */
    void* keyCache;           /* bf16 [kvHeads][capacity][dim] */
    void* valueCache;         /* bf16 [kvHeads][capacity][dim] */
    const float* qNorm;       /* [dim] gamma, NULL = no QK-norm (LocalModel.hpp:2609-2617) */
    const float* kNorm;       /* [dim] gamma, NULL = no QK-norm */
    const float* rotaryFrequencies; /* [rotaryDims/2] (LocalModel.hpp:807-820); NULL = no RoPE */
    float epsilon;            /* cfg.normEps */
    float normOffset;         /* spec.normWeightOffset (0 for qwen3) */
    uint32_t rotaryDims;
    uint32_t inType;
    uint32_t outputGate;      /* 1: out *= sigmoid(q[.. + dim + d]), the gate half of each q row
                                 (spec.attnOutputGate, LocalModel.hpp:2660-2665); needs qStride >= 2 dim */
    uint32_t reserved;
    uint64_t count, start, heads, kvHeads, dim, qStride, window, capacity;
    void* stream;
} AiGpuPrefill;
/* device pointers throughout */
AIGPU_ABI int aigpu_prefill_attention(const AiGpuPrefill* args);
/* q, k, v, out, qNorm, kNorm, rotaryFrequencies are host pointers (fp32 or
   bf16 per inType); the caches are device allocations. Staged in and out. */
AIGPU_ABI int aigpu_prefill_attention_host(const AiGpuPrefill* args);

/* A plain streaming copy of `bytes` between two device buffers (16-byte
   aligned, not overlapping) on `stream`. No counterpart in the reference's
   ABI: it measures what HBM delivers on this part, the ceiling beside the
   spec peak for the HBM-bound kernels (the reference's GPU testing measures
   bandwidth with a bf16 GEMV, src/gpu-testing.cpp:298-351). Asynchronous. */
AIGPU_ABI int aigpu_copy_device(void* dst, const void* src, uint64_t bytes, void* stream);

/* fp16 range flags of the asynchronous prefill calls (aigpu_prefill_attention,
   aigpu_prefill_mixer). No counterpart in the reference, whose calls are all
   synchronous on the host. Every prefill call takes the next ticket (1, 2,
   ...; aigpu_range_ticket returns the latest) and a flag word of its own,
   which its kernels raise when a value overflows fp16. aigpu_range_status
   waits for the device and returns 1 when no call since the previous query
   raised its flag; otherwise 0, with *ticket (when not NULL) the earliest
   raising call's ticket and aigpu_last_error naming it. Either way the flags
   are clear afterwards. A call captured into a graph has no ticket of its
   own: its replays raise a shared flag, reported as ticket UINT64_MAX. 255
   tickets share the flag words in turn, so a flag is lost only if 255 later
   calls are queued before its call runs. */
AIGPU_ABI uint64_t aigpu_range_ticket(void);
AIGPU_ABI int aigpu_range_status(uint64_t* ticket);

/* ------------------------------------------------------------------------ */
/* 4. Decode: one new token for each of `batch` sequences with ragged         */
/*    cached lengths. The new q and k get QK-RMSNorm and RoPE at position     */
/*    positions[b] inside the kernel ("on load"); the new k, v are appended   */
/*    to sequence b's cache at positions[b]; attention covers positions       */
/*    [first, positions[b]] (first from the window as Kernels.hpp:142).       */
/*    For batch 1 this is exactly attentionMixer with count = 1. Split-K,     */
/*    HBM-bound kernel; heads/kvHeads must be 1..8 and dim 64 or 128.         */
/* ------------------------------------------------------------------------ */
typedef struct AiGpuDecode {
    const void* q;            /* [batch][heads][qStride], inType */
    const void* k;            /* [batch][kvHeads][dim], inType */
    const void* v;            /* [batch][kvHeads][dim], inType */
    float* out;               /* [batch][heads][dim] fp32 */
    void* keyCache;           /* bf16, sequence b at b*batchStride: [kvHeads][capacity][dim] */
    void* valueCache;
    const uint32_t* positions;/* [batch] cached length of each sequence = new token position */
    const float* qNorm;
    const float* kNorm;
    const float* rotaryFrequencies;
    float epsilon;
    float normOffset;
    uint32_t rotaryDims;
    uint32_t inType;
    uint32_t maxPosition;     /* >= every positions[b]; sizes the launch */
    uint32_t outputGate;      /* as AiGpuPrefill::outputGate */
    uint64_t batch, heads, kvHeads, dim, qStride, window, capacity;
    uint64_t batchStride;     /* elements between sequences' caches; 0 = kvHeads*capacity*dim */
    void* stream;
} AiGpuDecode;
AIGPU_ABI int aigpu_decode_attention(const AiGpuDecode* args);
/* q, k, v, out, positions, qNorm, kNorm, rotaryFrequencies are host
   pointers; the caches are device allocations. */
AIGPU_ABI int aigpu_decode_attention_host(const AiGpuDecode* args);
/* aigpu_decode_attention without any allocation. No counterpart in the
   reference: it is for callers that cannot allocate device memory (code
   under HIP graph capture, serving loops that forbid hipMalloc). Its
   split-K records live in a fixed 32 MiB device array per GPU, held until
   the process ends; larger batches run in slices that fit it, and a call
   whose single sequence does not fit returns 0 with the reason. Every call
   on a GPU shares that array: calls on different streams are ordered by the
   backend, but replays of graphs captured from it that overlap on one GPU
   race on it. Make one call (or aigpu_available) before a capture: the
   first call of a process sets up the backend and looks up the array's
   address, which capture does not allow. Same arguments, kernels and
   results as aigpu_decode_attention. */
AIGPU_ABI int aigpu_decode_attention_static(const AiGpuDecode* args);

/* ------------------------------------------------------------------------ */
/* 5. Gated delta rule over a token range (the recurrence of                  */
/*    gatedDeltaNetMixer, LocalModel.hpp:2802-2830): for each token t and     */
/*    value head h (key head h / (valueHeads/keyHeads)):                      */
/*      S *= exp(g); delta = beta*(v - S^T k); S += k delta^T; out = S^T q    */
/*    computed as a chunked scan (WY form) with fp32 state.                   */
/* ------------------------------------------------------------------------ */
typedef struct AiGpuDeltaRule {
    const void* q;            /* [count][keyHeads][keyDim], inType */
    const void* k;            /* [count][keyHeads][keyDim], inType */
    const void* v;            /* [count][valueHeads][valueDim], inType */
    const float* g;           /* [count][valueHeads] log decay (used when aLog is NULL) */
    const float* beta;        /* [count][valueHeads] (used when aLog is NULL) */
    const float* a;           /* raw gate inputs [count][valueHeads] (used when aLog is set): */
    const float* b;           /*   g = -exp(aLog[h])*softplus(a + dtBias[h]), beta = sigmoid(b) */
    const float* aLog;        /* [valueHeads] (LocalModel.hpp:2820-2823) */
    const float* dtBias;      /* [valueHeads] */
    float* state;             /* [valueHeads][keyDim][valueDim] fp32, in/out */
    float* out;               /* [count][valueHeads][valueDim] fp32 */
    uint32_t inType;
    uint32_t normalize;       /* 1: l2normalise q,k (eps 1e-6) and q *= 1/sqrt(keyDim) */
    uint32_t chunk;           /* 64 (0 = 64) */
    uint32_t reserved;
    uint64_t count, keyHeads, valueHeads, keyDim, valueDim;
    void* stream;
} AiGpuDeltaRule;
AIGPU_ABI int aigpu_gated_delta_rule(const AiGpuDeltaRule* args);
/* every tensor a host pointer; state updated in place on the host */
AIGPU_ABI int aigpu_gated_delta_rule_host(const AiGpuDeltaRule* args);

/* ------------------------------------------------------------------------ */
/* 5b. Kimi Delta Attention's recurrence (kimiDeltaMixer,                    */
/*     LocalModel.hpp:2928-2947): the gated delta rule with one decay per    */
/*     KEY CHANNEL, deltaStep(perKeyDecay = true) (Kernels.hpp:105-128).     */
/* ------------------------------------------------------------------------ */
typedef struct AiGpuKda {
    const void* q;            /* [count][keyHeads][keyDim], inType */
    const void* k;            /* [count][keyHeads][keyDim], inType */
    const void* v;            /* [count][valueHeads][valueDim], inType */
    const float* g;           /* [count][valueHeads][keyDim] log decay (decay = exp(g) <= 1) */
    const float* beta;        /* [count][valueHeads] */
    /* raw gates, used when g and beta are NULL (LocalModel.hpp:2894-2905):  */
    /*   g = safeGate ? lowerBound sigmoid(exp(aLog) (f + dtBias))            */
    /*                : -exp(aLog) softplus(f + dtBias),  beta = sigmoid(b)   */
    const float* f;           /* [count][valueHeads][keyDim] decay projection (f_b output) */
    const float* b;           /* [count][valueHeads] write-strength projection */
    const float* aLog;        /* [valueHeads] */
    const float* dtBias;      /* [valueHeads][keyDim] */
    float lowerBound;         /* LocalConfig::linLowerBound, <= 0 */
    uint32_t safeGate;        /* LocalConfig::linSafeGate */
    float* state;             /* [valueHeads][keyDim][valueDim] fp32, in/out */
    float* out;               /* [count][valueHeads][valueDim] fp32 */
    uint32_t inType;
    uint32_t normalize;       /* 1: l2normalise q,k (eps 1e-6) and q *= 1/sqrt(keyDim) */
    uint64_t count, keyHeads, valueHeads, keyDim, valueDim;
    void* stream;
} AiGpuKda;
AIGPU_ABI int aigpu_kda_rule(const AiGpuKda* args);

/* ------------------------------------------------------------------------ */
/* 6. The Gated DeltaNet steps either side of the recurrence                 */
/*    (gatedDeltaNetMixer, LocalModel.hpp:2724-2844). No reference kernel    */
/*    exists for them: the mixer runs them inline on the host.               */
/* ------------------------------------------------------------------------ */
/* causalConvolution + SiLU (LocalModel.hpp:2678-2708) over the projection    */
/* rows, with the linFusedQKVZ de-interleave (:2739-2776) when `fused` is     */
/* set, writing the recurrence's dense inputs. The window carries the last   */
/* kernelSize-1 inputs between calls (LocalCache::convWindow), as fp32.      */
typedef struct AiGpuGdnConv {
    const void* in;           /* fused == 0: [count][CW] rows q | k | v (CW = 2 keyHeads keyDim
                                 + valueHeads valueDim); fused: [count][keyHeads][2 keyDim +
                                 2 G valueDim] (per key head q, k, its G value heads' v, their z) */
    const void* ba;           /* fused: [count][keyHeads][2 G], the G heads' b then their a */
    const float* kernel;      /* [CW][kernelSize] (LocalLayer::linConv) */
    float* window;            /* [kernelSize-1][CW] fp32, read then replaced */
    void* q;                  /* out [count][keyHeads][keyDim], outType */
    void* k;                  /* out [count][keyHeads][keyDim], outType */
    void* v;                  /* out [count][valueHeads][valueDim], outType */
    void* z;                  /* fused: out [count][valueHeads][valueDim], outType (not convolved) */
    float* a;                 /* fused: out [count][valueHeads] fp32 */
    float* b;                 /* fused: out [count][valueHeads] fp32 */
    uint32_t inType, outType; /* AIGPU_F32 / AIGPU_BF16 */
    uint32_t fused, reserved;
    uint64_t count, keyHeads, valueHeads, keyDim, valueDim, kernelSize;
    void* stream;
} AiGpuGdnConv;
AIGPU_ABI int aigpu_gdn_conv(const AiGpuGdnConv* args);

/* rmsNormRow of each (token, value head) row of the recurrence output, its  */
/* weight stored directly, then times SiLU(z) (LocalModel.hpp:2833-2841), or */
/* with gateKind 1 times sigmoid(z), kimiDeltaMixer's form (:2936-2945)      */
typedef struct AiGpuGdnGatedNorm {
    const float* x;           /* [count][valueHeads][valueDim] fp32 */
    const void* z;            /* [count][valueHeads][valueDim], zType */
    const float* gamma;       /* [valueDim] (LocalLayer::linNorm) */
    void* out;                /* [count][valueHeads][valueDim], outType */
    float epsilon;            /* LocalConfig::normEps */
    uint32_t zType, outType, gateKind; /* gateKind 0: SiLU, 1: sigmoid */
    uint64_t count, valueHeads, valueDim;
    void* stream;
} AiGpuGdnGatedNorm;
AIGPU_ABI int aigpu_gdn_gated_norm(const AiGpuGdnGatedNorm* args);

/* ------------------------------------------------------------------------ */
/* 5c. Multi-head latent attention (latentAttentionMixer,                    */
/*     LocalModel.hpp:3118-3158): per token and head, q folded through the  */
/*     head's key rows of kv_b_proj, softmax against the cached latents     */
/*     (all positions up to the token, or the indexer's sorted selection,   */
/*     KeySelection :1203-1206), the weighted latents through the value     */
/*     rows. Device pointers.                                               */
/* ------------------------------------------------------------------------ */
typedef struct AiGpuLatentAttention {
    const float* q;           /* [count][heads][nopeDim] (q_b_proj output, :3106) */
    const float* latent;      /* [startPos + count][kvLoraRank] cache, this call's rows included */
    const void* kvB;          /* [heads * (nopeDim + vDim)][kvLoraRank] kv_b_proj, kvBType */
    uint32_t kvBType;         /* AIGPU_F32 / AIGPU_BF16 */
    uint32_t reserved;
    const uint32_t* selStart; /* [count] or NULL (every token dense) */
    const uint32_t* selCount; /* [count], 0xFFFFFFFF for a dense token */
    const uint32_t* selKeys;  /* the concatenated sorted key lists */
    float* out;               /* [count][heads][vDim] fp32 */
    float scale;              /* 1/sqrt(qk_nope_head_dim + qk_rope_head_dim), :3116 */
    uint64_t count, startPos, heads, nopeDim, vDim, kvLoraRank;
    void* stream;
} AiGpuLatentAttention;
AIGPU_ABI int aigpu_latent_attention(const AiGpuLatentAttention* args);

/* ------------------------------------------------------------------------ */
/* 7. Projections (DeviceABI.h:101-112): c[m][n] = a[m][k] . b[n][k]^T, with */
/*    a and c host fp32 and b a device weight from aigpu_upload, in the     */
/*    reference's four encodings (Quant.hpp): fp32, bf16, Q8 (int8 codes,   */
/*    one fp32 scale per 32) and Q4 (two codes a byte, byte j of a block    */
/*    holding codes j and j+16, offset 8; one fp32 scale per 32). They      */
/*    return nothing, as the reference's do; failures set aigpu_last_error.  */
/* ------------------------------------------------------------------------ */
#ifndef AI_GPU_DEVICE_ABI_H
AIGPU_ABI void aigpu_matmul_nt(const float* a, const void* b, float* c,
                               uint64_t m, uint64_t k, uint64_t n);            /* DeviceABI.h:101 */
AIGPU_ABI void aigpu_matmul_nt_bf16(const float* a, const void* b, float* c,
                                    uint64_t m, uint64_t k, uint64_t n);       /* DeviceABI.h:104 */
AIGPU_ABI void aigpu_matmul_nt_q8(const float* a, const void* b, const void* scales, float* c,
                                  uint64_t m, uint64_t k, uint64_t n);         /* DeviceABI.h:107 */
AIGPU_ABI void aigpu_matmul_nt_q4(const float* a, const void* b, const void* scales, float* c,
                                  uint64_t m, uint64_t k, uint64_t n);         /* DeviceABI.h:111 */
#endif /* !AI_GPU_DEVICE_ABI_H */

/* The device form of the same product (no counterpart in the reference,
   whose matmul stages a and c through the host every call): every pointer
   is device memory, the bias is optional, and accumulate = 1 adds the
   product into c (a residual add). */
enum { AIGPU_W_F32 = 0, AIGPU_W_BF16 = 1, AIGPU_W_Q8 = 2, AIGPU_W_Q4 = 3 };
typedef struct AiGpuMatmul {
    const float* a;           /* [m][k] fp32 */
    const void* b;            /* [n][k] weights in `type` */
    const float* scales;      /* [n][k/32] for Q8 / Q4 */
    const float* bias;        /* [n] or NULL */
    float* c;                 /* [m][ldc] fp32 */
    uint32_t type;            /* AIGPU_W_* (AiGpuDenseWeight::type) */
    uint32_t accumulate;
    uint64_t m, k, n, ldc;    /* ldc 0 means n */
    void* stream;
} AiGpuMatmul;
AIGPU_ABI int aigpu_matmul_device(const AiGpuMatmul* args);

/* ------------------------------------------------------------------------ */
/* 8. The resident single-token decoder (DeviceABI.h:119-152), the same     */
/*    structs and entry points: a dense RMSNorm / RoPE / SwiGLU model kept   */
/*    on the device; LocalModel::residentDecode (LocalModel.hpp:3598-3645)   */
/*    is the caller. Weight codes and scales are device pointers (from      */
/*    aigpu_upload) and stay the caller's; norms, biases, rotary            */
/*    frequencies and the cache arrays are host pointers, copied in.        */
/* ------------------------------------------------------------------------ */
#ifndef AI_GPU_DEVICE_ABI_H
typedef struct AiGpuDenseWeight {       /* DeviceABI.h:122-127 */
    const void* codes;
    const void* scales;
    uint32_t type, inDim, outDim;       /* F32=0, BF16=1, Q8=2, Q4=3 */
    const float* bias;                  /* optional, copied at creation */
} AiGpuDenseWeight;
typedef struct AiGpuDenseLayer {        /* DeviceABI.h:128-135 */
    AiGpuDenseWeight q, k, v, o, gate, up, down;
    const float* inputNorm;
    const float* postNorm;
    const float* qNorm;
    const float* kNorm;
    uint32_t window;                    /* 0 = full causal attention */
} AiGpuDenseLayer;
typedef struct AiGpuDenseConfig {       /* DeviceABI.h:136-143 */
    uint32_t hidden, layers, heads, kvHeads, headDim, intermediate;
    uint32_t capacity, rotaryDims, vocab;
    float epsilon, theta;
    const float* finalNorm;
    AiGpuDenseWeight head;
    const float* rotaryFrequencies;     /* rotaryDims/2 entries; optional */
} AiGpuDenseConfig;
AIGPU_ABI int aigpu_dense_supported(void);                                      /* DeviceABI.h:144 */
AIGPU_ABI void* aigpu_dense_create(const AiGpuDenseConfig* config,
                                   const AiGpuDenseLayer* layers, const float* const* keys,
                                   const float* const* values, uint32_t length);  /* DeviceABI.h:145 */
AIGPU_ABI void aigpu_dense_release(void* context);                             /* DeviceABI.h:148 */
AIGPU_ABI void aigpu_dense_decode(void* context, const float* embedding,
                                  float* logits, uint32_t position);           /* DeviceABI.h:149 */
AIGPU_ABI void aigpu_dense_read_cache(void* context, float* const* keys,
                                      float* const* values, uint32_t length);  /* DeviceABI.h:151 */
#endif /* !AI_GPU_DEVICE_ABI_H */

/* ------------------------------------------------------------------------ */
/* 9. attentionMixer for a prefill in one call (LocalModel.hpp:2577-2667):  */
/*    the q, k, v projections of x (apply, :2604-2606), QK-RMSNorm -> RoPE  */
/*    -> KV append (:2608-2655) as the k and v projections' epilogue, the   */
/*    causal attention over the cache (:2657-2659), the output gate         */
/*    (:2660-2665) and the o projection (:2667) into out. The weights are   */
/*    AiGpuDenseWeight with every pointer on the device (bias included);    */
/*    qStride is dim, or 2 dim with outputGate (q_proj's per-head gate      */
/*    half). dim 64 or 128; codes 16-byte aligned.                          */
/* ------------------------------------------------------------------------ */
typedef struct AiGpuPrefillMixer {
    const float* x;                 /* [count][hidden] fp32, the normed hidden states */
    AiGpuDenseWeight q, k, v, o;    /* q [heads*qStride][hidden], k and v [kvHeads*dim][hidden],
                                       o [hidden][heads*dim] */
    float* out;                     /* [count][hidden] fp32 */
    void* keyCache;                 /* bf16 [kvHeads][capacity][dim], positions [0, start) valid */
    void* valueCache;
    const float* qNorm;             /* [dim] gamma or NULL (LocalModel.hpp:2609-2617) */
    const float* kNorm;
    const float* rotaryFrequencies; /* [rotaryDims/2] or NULL = no RoPE */
    float epsilon, normOffset;
    uint32_t rotaryDims, outputGate;
    uint32_t accumulate;            /* 1: out += the mixer's output (the residual add) */
    uint32_t reserved;
    uint64_t count, start, hidden, heads, kvHeads, dim, window, capacity;
    void* stream;
} AiGpuPrefillMixer;
/* asynchronous like aigpu_prefill_attention: values outside fp16's range
   raise the call's range flag (aigpu_range_status) */
AIGPU_ABI int aigpu_prefill_mixer(const AiGpuPrefillMixer* args);

/* ------------------------------------------------------------------------ */
/* 10. The sparse-attention indexer (selectKeys, LocalModel.hpp:2971-3068),  */
/*    GLM-5.3's pooled form: the call's index keys layer-normed into the     */
/*    key cache and folded, pool by pool, into pooled keys; each query token */
/*    scoring the pools wholly at or before it and keeping the topK / pool   */
/*    best, plus the unfinished pool with indexTail. The result is the       */
/*    selection aigpu_latent_attention takes. Among equal scores at the      */
/*    boundary the lower pool is kept (the reference's nth_element leaves    */
/*    that order unspecified). Device pointers throughout.                   */
/* ------------------------------------------------------------------------ */
typedef struct AiGpuSelectKeys {
    const float* h;                 /* [count][hidden], latentAttentionMixer's input (the call, :3110) */
    const float* qResid;            /* [count][qRank], q_a_proj's normed output (:3097-3099) */
    AiGpuDenseWeight idxK;          /* [dim][hidden] */
    AiGpuDenseWeight idxGate;       /* [dim][hidden] */
    AiGpuDenseWeight idxQB;         /* [heads*dim][qRank] */
    AiGpuDenseWeight idxWeights;    /* [heads][hidden] */
    const float* kNorm;             /* [dim] layerNorm weight */
    const float* kNormBias;         /* [dim] or NULL */
    const float* ape;               /* [pool][dim] */
    float* indexKeys;               /* [capacity][dim]; positions < startPos valid */
    float* indexGates;              /* [capacity][dim] */
    float* poolKeys;                /* [capacity/pool + 1][dim] */
    uint32_t* selStart;             /* [count] */
    uint32_t* selCount;             /* [count]; UINT32_MAX: the token sees every key */
    uint32_t* selKeys;              /* [count][topK/pool*pool + pool], each token's keys sorted */
    float* scores;                  /* optional [count][(startPos+count)/pool]: sparse tokens' pool scores */
    uint32_t indexTail, reserved;
    uint64_t count, startPos, hidden, qRank, heads, dim, topK, pool, capacity;
    void* stream;
} AiGpuSelectKeys;
AIGPU_ABI int aigpu_select_keys(const AiGpuSelectKeys* args);

/* ------------------------------------------------------------------------ */
/* Per-kernel timing. With profiling on, every launch is bracketed by a pair */
/* of hipEvents on the stream it runs on; aigpu_profile_read synchronises    */
/* and reports the summed device time and launch count of kernels whose name */
/* contains `kernel` since the last reset.                                   */
/* ------------------------------------------------------------------------ */
AIGPU_ABI void aigpu_profile(int enable);
AIGPU_ABI int aigpu_profile_read(const char* kernel, double* milliseconds, uint64_t* launches);
AIGPU_ABI void aigpu_profile_reset(void);

#ifdef __cplusplus
}
#endif

#endif /* AIGPU_ATTENTION_H */
