// kernels.hpp - host-side launchers of the gfx950 kernels. Each takes device
// pointers only, validates what its kernel's grid and indexing assume, and
// launches on the given stream. The extern "C" layer (abi.hip) stages host
// data and calls these.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aigpu {

// ---- generic fp32 attention (kernels::attention semantics) ---------------
struct AttentionF32Params {
    const void* q;
    const void* keys;
    const void* values;
    float* out;
    int qType, kvType;
    uint64_t count, start, heads, kvHeads, dim, qStride, window, posStride, headStride;
};
bool launch_attention_f32(const AttentionF32Params& p, hipStream_t stream);

// ---- prefill: norm + RoPE + append, then fp16 MFMA flash attention --------
struct PrefillParams {
    const void* q;
    const void* k;
    const void* v;
    float* out;
    uint16_t* keyCache;
    uint16_t* valueCache;
    const float* qNorm;
    const float* kNorm;
    const float* freqs;
    float eps, normOffset;
    int rotaryDims, inType, outputGate;
    // 1: k and v are not read; the new rows [start, start + count) are already
    // in the caches and in the working buffers of prefill_work_buffers (the k
    // and v projections' epilogue wrote them)
    int kvReady;
    uint64_t count, start, heads, kvHeads, dim, qStride, window, capacity;
    // set to 1 by any conversion into the fp16 working copies that overflows
    // fp16's range (device address of the call's flag word; null: not tracked)
    uint32_t* rangeFlag;
    // when set, out is not written: each output row goes as bf16 high parts
    // here ([count][heads·dim]) and as bf16 residuals x - hi right after them
    // (the operand images of gemm_split_image)
    uint16_t* outSplit;
    // 1 (with kvReady): the caller has written the q rotation's cos/sin table
    // (prefill_prep_foldable) and zeroed the working copies' pad rows, all
    // that prep would do: it is not launched
    int prepDone;
};
bool launch_prefill(const PrefillParams& p, hipStream_t stream);
// rows of zeros after the last kv head in the flash kernel's working copies
constexpr uint32_t PREFILL_PAD_ROWS = 128;
// the flash kernel's fp16 copies of the cache, [kvHeads][start + count][dim]
bool prefill_work_buffers(const PrefillParams& p, void** kh, void** vh);
// whether launch_prefill's prep, for these kvReady parameters, would only
// write the cos/sin table of the flash kernel's q rotation and zero the pad
// rows; *rope is then that table (count * rotaryDims floats in the layout of
// rope_at in device.hpp), grown, or null without RoPE
bool prefill_prep_foldable(const PrefillParams& p, float** rope);

// ---- decode: norm + RoPE on load, append, split-K attention, merge --------
struct DecodeParams {
    const void* q;
    const void* k;
    const void* v;
    float* out;
    uint16_t* keyCache;
    uint16_t* valueCache;
    const uint32_t* positions;
    const float* qNorm;
    const float* kNorm;
    const float* freqs;
    float eps, normOffset;
    int rotaryDims, inType, outputGate;
    uint32_t maxPosition;
    uint64_t batch, heads, kvHeads, dim, qStride, window, capacity, batchStride;
};
// caller-provided scratch in place of the context's growable slots
struct FixedScratch {
    void* base;
    size_t bytes;
};
bool launch_decode(const DecodeParams& p, hipStream_t stream, const FixedScratch* fixed = nullptr);
// the address and size of the decode path's fixed device scratch on the
// current device (hipGetSymbolAddress, taken once per device)
bool decode_static_scratch(void** base, size_t* bytes);

// ---- gated delta rule: chunked scan --------------------------------------
struct DeltaRuleParams {
    const void* q;
    const void* k;
    const void* v;
    const float* g;
    const float* beta;
    const float* a;
    const float* b;
    const float* aLog;
    const float* dtBias;
    float* state;
    float* out;
    int inType, normalize, chunk;
    uint64_t count, keyHeads, valueHeads, keyDim, valueDim;
};
bool launch_delta_rule(const DeltaRuleParams& p, hipStream_t stream);

// ---- projections: out[m][n] = a[m][k] . w[n][k] (+ bias) (+ out) ----
struct GemvParams {
    const float* a;       // [m][k] fp32
    const void* w;        // [n][k] in `type`
    const float* scales;  // [n][k/32] for Q8 and Q4
    const float* bias;    // [n] or null
    float* out;           // [m][ldo]
    int type;             // 0 F32, 1 BF16, 2 Q8, 3 Q4 (AiGpuDenseWeight::type)
    int accumulate;       // 1: out += a . w^T
    uint32_t m, k, n, ldo;
};
bool launch_gemv(const GemvParams& p, hipStream_t stream);

// the k or v projection of a prefill with attentionMixer's per-token work
// as its epilogue: QK-RMSNorm (gamma), rotate-half RoPE (freqs), then the
// row appended to the bf16 cache and to the flash kernel's fp16 copy
struct KvEpilogue {
    uint16_t* cache;      // bf16 [kvHeads][capacity][dim]
    void* work;           // fp16 [kvHeads][T][dim]
    const float* gamma;   // [dim] or null
    const float* freqs;   // [rot / 2] or null
    float eps, offset;
    uint32_t dim, rot, start, T;
    uint64_t capacity;
    uint32_t* rangeFlag;  // as PrefillParams::rangeFlag
};
bool launch_gemm_kv(const GemvParams& p, const KvEpilogue& e, hipStream_t stream);
// whether launch_gemv splits p.a into the bf16 images a following
// launch_gemm_kv_pair can reuse (aSplit)
bool gemm_splits_a(const GemvParams& p);
// the DMA GEMM's operand images of p.a (bf16 high parts [m][k], then the
// residuals), grown for p, when p takes that GEMM; null otherwise
uint16_t* gemm_split_image(const GemvParams& p);
// launch_gemv for a p that takes the DMA GEMM, with gemm_split_image(p)
// already written (p.a is not read)
bool launch_gemv_presplit(const GemvParams& p, hipStream_t stream);
// the k and v projections of the same rows: one GEMM over both weights, then
// the epilogue as its own kernel, where the shapes allow; otherwise two
// launch_gemm_kv calls
// fold: also write prep's cos/sin table (rope, may be null) and zero the
// working copies' pad rows; *folded says whether that was done
bool launch_gemm_kv_pair(const GemvParams& pk, const GemvParams& pv, const KvEpilogue& ek, const KvEpilogue& ev,
                         bool aSplit, bool fold, float* rope, bool* folded, hipStream_t stream);

// ---- attentionMixer for a prefill: projections, norm/RoPE/append, flash
// attention, output gate, o projection ----
struct MixerWeight {
    const void* codes;
    const float* scales;
    const float* bias;
    int type;
    uint32_t in, out;
};
struct MixerParams {
    const float* x;
    MixerWeight q, k, v, o;
    float* out;
    uint16_t* keyCache;
    uint16_t* valueCache;
    const float* qNorm;
    const float* kNorm;
    const float* freqs;
    float eps, normOffset;
    int rotaryDims, outputGate, accumulate;
    uint64_t count, start, hidden, heads, kvHeads, dim, qStride, window, capacity;
    uint32_t* rangeFlag;  // as PrefillParams::rangeFlag
};
bool launch_prefill_mixer(const MixerParams& p, hipStream_t stream);

// ---- the sparse-attention indexer (selectKeys) ----
struct IndexerParams {
    const float* h;          // [count][hidden]
    const float* qResid;     // [count][qRank]
    MixerWeight wk, wgate, wq, ww;   // idxK, idxGate, idxQB, idxWeights
    const float* kNorm;      // [dim] layerNorm weight
    const float* kNormBias;  // [dim] or null
    const float* ape;        // [pool][dim]
    float* keys;             // [capacity][dim]
    float* gates;            // [capacity][dim]
    float* pools;            // [capacity / pool + 1][dim]
    uint32_t* selStart;
    uint32_t* selCount;
    uint32_t* selKeys;       // [count][topK / pool * pool + pool]
    float* scores;           // optional [count][(startPos + count) / pool]
    int tail;
    uint64_t count, startPos, hidden, qRank, heads, dim, topK, pool, capacity;
};
bool launch_select_keys(const IndexerParams& p, hipStream_t stream);

// ---- multi-head latent attention ----
struct LatentParams {
    const float* q;          // [count][heads][nope]
    const float* latent;     // [positions][rank]
    const void* wkv;         // [heads * (nope + vdim)][rank], wType
    int wType;               // 0 fp32, 1 bf16
    const uint32_t* selStart;   // per token, or null (all dense)
    const uint32_t* selCount;   // UINT32_MAX: dense
    const uint32_t* selKeys;
    float* out;              // [count][heads][vdim]
    float scale;
    uint64_t count, startPos, heads, nope, vdim, rank;
};
bool launch_latent_attention(const LatentParams& p, hipStream_t stream);

// ---- Kimi Delta Attention: the delta rule with per-key-channel decay ----
struct KdaParams {
    const void* q;        // [count][keyHeads][keyDim], inType
    const void* k;
    const void* v;        // [count][valueHeads][valueDim], inType
    const float* g;       // [count][valueHeads][keyDim] log decay per key channel
    const float* beta;    // [count][valueHeads]
    const float* f;       // raw gates instead of g/beta: [count][valueHeads][keyDim]
    const float* b;       // [count][valueHeads]
    const float* aLog;    // [valueHeads]
    const float* dtBias;  // [valueHeads][keyDim]
    float lowerBound;
    int safeGate;
    float* state;         // [valueHeads][keyDim][valueDim]
    float* out;           // [count][valueHeads][valueDim]
    int inType, normalize;
    uint64_t count, keyHeads, valueHeads, keyDim, valueDim;
};
bool launch_kda(const KdaParams& p, hipStream_t stream);

// ---- Gated DeltaNet neighbours: de-interleave + causal conv, gated norm --
struct GdnConvParams {
    const void* in;       // plain [count][CW] or fused [count][keyHeads][2KD + 2G VD]
    const void* ba;       // fused: [count][keyHeads][2G]
    const float* kernel;  // [CW][kernelSize]
    float* window;        // [kernelSize - 1][CW], in/out
    void* q;
    void* k;
    void* v;
    void* z;              // fused: [count][valueHeads][valueDim]
    float* a;             // fused: [count][valueHeads]
    float* b;
    uint32_t inType, outType, fused;
    uint64_t count, keyHeads, valueHeads, keyDim, valueDim, kernelSize;
};
bool launch_gdn_conv(const GdnConvParams& p, hipStream_t stream);

struct GdnGatedNormParams {
    const float* x;       // [count][valueHeads][valueDim]
    const void* z;
    const float* gamma;   // [valueDim]
    void* out;
    float eps;
    uint32_t zType, outType;
    uint32_t sigmoidGate;  // 0: x SiLU(z) (Gated DeltaNet), 1: x sigmoid(z) (Kimi)
    uint64_t count, valueHeads, valueDim;
};
bool launch_gdn_gated_norm(const GdnGatedNormParams& p, hipStream_t stream);

// ---- a plain streaming device copy (the bench's achievable-bandwidth line) ----
bool launch_copy(void* dst, const void* src, uint64_t bytes, hipStream_t stream);

} // namespace aigpu
