// mixer.hip - attentionMixer for a prefill (LocalModel.hpp:2577-2667) as one
// call on the device: the q, k, v projections of the normed hidden states,
// QK-RMSNorm -> RoPE -> KV append, causal attention over the cache, the
// output gate, and the o projection.
//
// The k and v projections carry the per-token work as their GEMM's epilogue
// (launch_gemm_kv): the normed, rotated rows go straight from the MFMA
// accumulators to the bf16 cache and to the flash kernel's fp16 copy, with
// no fp32 k / v round trip through HBM and no separate prep pass over them.
// The q projection is stored raw: the flash kernel normalises and rotates
// its own q rows on load (or prep does, when the shape rules that out).
#include "context.hpp"
#include "kernels.hpp"

namespace aigpu {

namespace {

GemvParams projection(const MixerWeight& w, const float* a, float* out, uint64_t m, int accumulate) {
    GemvParams g{};
    g.a = a;
    g.w = w.codes;
    g.scales = w.scales;
    g.bias = w.bias;
    g.out = out;
    g.type = w.type;
    g.accumulate = accumulate;
    g.m = uint32_t(m);
    g.k = w.in;
    g.n = w.out;
    g.ldo = w.out;
    return g;
}

} // namespace

bool launch_prefill_mixer(const MixerParams& p, hipStream_t stream) {
    Context& ctx = Context::instance();
    const uint64_t H = p.heads, KV = p.kvHeads, D = p.dim;
    if (!p.x || !p.out || !p.keyCache || !p.valueCache || !p.q.codes || !p.k.codes || !p.v.codes || !p.o.codes)
        return ctx.fail("prefill mixer: null tensor");
    if (D != 64 && D != 128) return ctx.fail("prefill mixer: dim must be 64 or 128");
    if (KV == 0 || H % KV) return ctx.fail("prefill mixer: heads must be a multiple of kvHeads");
    if (p.qStride != (p.outputGate ? 2 * D : D))
        return ctx.fail("prefill mixer: qStride must be dim, or 2 dim with the output gate");
    if (p.q.in != p.hidden || p.k.in != p.hidden || p.v.in != p.hidden || p.q.out != H * p.qStride ||
        p.k.out != KV * D || p.v.out != KV * D || p.o.in != H * D || p.o.out != p.hidden)
        return ctx.fail("prefill mixer: weight shapes do not match hidden, heads, kvHeads, dim");
    if (p.count == 0) return true;
    const uint64_t T = p.start + p.count;
    if (p.capacity < T) return ctx.fail("prefill mixer: cache capacity below start + count");
    if (p.count >= (1ull << 31) || T >= (1ull << 31)) return ctx.fail("prefill mixer: sequence too long");

    float* q = static_cast<float*>(ctx.grow(SLOT_MIXER_Q, p.count * H * p.qStride * sizeof(float)));
    float* attn = static_cast<float*>(ctx.grow(SLOT_MIXER_ATTN, p.count * H * D * sizeof(float)));
    if (!q || !attn) return false;

    PrefillParams pp{};
    pp.q = q;
    pp.out = attn;
    pp.keyCache = p.keyCache;
    pp.valueCache = p.valueCache;
    pp.qNorm = p.qNorm;
    pp.kNorm = p.kNorm;
    pp.freqs = p.freqs;
    pp.eps = p.eps;
    pp.normOffset = p.normOffset;
    pp.rotaryDims = p.rotaryDims;
    pp.inType = 0;
    pp.outputGate = p.outputGate;
    pp.kvReady = 1;
    pp.count = p.count;
    pp.start = p.start;
    pp.heads = H;
    pp.kvHeads = KV;
    pp.dim = D;
    pp.qStride = p.qStride;
    pp.window = p.window;
    pp.capacity = p.capacity;
    pp.rangeFlag = p.rangeFlag;
    void* kh = nullptr;
    void* vh = nullptr;
    if (!prefill_work_buffers(pp, &kh, &vh)) return false;

    const GemvParams pq = projection(p.q, p.x, q, p.count, 0);
    if (!launch_gemv(pq, stream)) return false;
    KvEpilogue ek{};
    ek.cache = p.keyCache;
    ek.work = kh;
    ek.gamma = p.kNorm;
    ek.freqs = p.freqs;
    ek.eps = p.eps;
    ek.offset = p.normOffset;
    ek.dim = uint32_t(D);
    ek.rot = uint32_t(p.rotaryDims);
    ek.start = uint32_t(p.start);
    ek.T = uint32_t(T);
    ek.capacity = p.capacity;
    ek.rangeFlag = p.rangeFlag;
    KvEpilogue ev = ek;
    ev.cache = p.valueCache;
    ev.work = vh;
    ev.gamma = nullptr;
    ev.freqs = nullptr;
    // the q projection left x's bf16 split in scratch when it took the DMA GEMM;
    // the k / v pass after the pair's GEMM can also do all that prep would
    float* rope = nullptr;
    const bool foldable = prefill_prep_foldable(pp, &rope);
    bool folded = false;
    if (!launch_gemm_kv_pair(projection(p.k, p.x, nullptr, p.count, 0), projection(p.v, p.x, nullptr, p.count, 0), ek,
                             ev, gemm_splits_a(pq), foldable, rope, &folded, stream))
        return false;
    pp.prepDone = folded ? 1 : 0;
    // when the o projection takes the DMA GEMM, the flash kernel writes its
    // bf16 operand images directly (no fp32 round trip and split pass)
    const GemvParams po = projection(p.o, attn, p.out, p.count, p.accumulate ? 1 : 0);
    pp.outSplit = gemm_split_image(po);
    if (!launch_prefill(pp, stream)) return false;
    return pp.outSplit ? launch_gemv_presplit(po, stream) : launch_gemv(po, stream);
}

} // namespace aigpu
