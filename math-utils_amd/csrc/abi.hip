// abi.hip - the extern "C" entry points of include/aigpu_attention.h and the
// process-wide Context behind them.
//
// Host forms stage their host tensors into device scratch, launch, and copy
// the results back, timing kernels and transfers apart as the reference's
// dispatch does (src/gpu/Kernels.hip:387-426). Device forms launch on the
// caller's stream and return without synchronising.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstring>
#include <string>

#include "context.hpp"
#include "kernels.hpp"

namespace aigpu {

using Clock = std::chrono::steady_clock;

static double since(Clock::time_point t) {
    return std::chrono::duration<double>(Clock::now() - t).count();
}

Context& Context::instance() {
    static Context ctx;
    return ctx;
}

Context::Context() {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
        (void)hipGetLastError();
        error = "no HIP device found";
        return;
    }
    if (hipSetDevice(0) != hipSuccess) {
        error = "hipSetDevice(0) failed";
        return;
    }
    hipDeviceProp_t props{};
    if (hipGetDeviceProperties(&props, 0) != hipSuccess) {
        error = "hipGetDeviceProperties failed";
        return;
    }
    if (std::strncmp(props.gcnArchName, "gfx950", 6) != 0) {
        error = std::string("this backend is built for gfx950, found ") + props.gcnArchName;
        return;
    }
    name = props.name;
    cus = props.multiProcessorCount;
    if (hipHostMalloc(reinterpret_cast<void**>(&rangeHost), RANGE_SLOTS * sizeof(uint32_t), hipHostMallocMapped) !=
            hipSuccess ||
        hipHostGetDevicePointer(reinterpret_cast<void**>(&rangeDev), rangeHost, 0) != hipSuccess) {
        (void)hipGetLastError();
        error = "hipHostMalloc of the fp16 range flags failed";
        return;
    }
    for (int i = 0; i < RANGE_SLOTS; ++i) rangeHost[i] = 0;
    if (hipEventCreateWithFlags(&handoff, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        error = "hipEventCreate of the stream handoff event failed";
        return;
    }
    ok = true;
}

static bool capturing(hipStream_t stream) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &capture) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return capture != hipStreamCaptureStatusNone;
}

uint32_t* Context::rangeSlot(hipStream_t stream, uint64_t* ticket) {
    if (capturing(stream)) {
        *ticket = UINT64_MAX;
        return rangeDev;   // slot 0: not cleared, a replay of an earlier capture may have raised it
    }
    const uint64_t t = ++rangeTickets;
    const int slot = 1 + int((t - 1) % (RANGE_SLOTS - 1));
    // the slot's previous ticket (RANGE_SLOTS - 1 calls ago) has long
    // completed unless that many calls are queued; a flag it raised is kept
    if (__atomic_load_n(rangeHost + slot, __ATOMIC_ACQUIRE) != 0) rangeRaised.push_back(slotTicket[slot]);
    __atomic_store_n(rangeHost + slot, 0u, __ATOMIC_RELEASE);
    slotTicket[slot] = t;
    *ticket = t;
    return rangeDev + slot;
}

bool Context::rangeRaisedFor(uint64_t ticket) {
    const int slot = ticket == UINT64_MAX ? 0 : 1 + int((ticket - 1) % (RANGE_SLOTS - 1));
    if (slot != 0 && slotTicket[slot] != ticket) return false;
    if (__atomic_load_n(rangeHost + slot, __ATOMIC_ACQUIRE) == 0) return false;
    __atomic_store_n(rangeHost + slot, 0u, __ATOMIC_RELEASE);
    return true;
}

int Context::rangeStatus(uint64_t* ticket) {
    if (ticket) *ticket = 0;
    const hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return fail(std::string("range status: ") + hipGetErrorString(e)), 0;
    std::vector<uint64_t> raised;
    raised.swap(rangeRaised);
    for (int slot = 0; slot < RANGE_SLOTS; ++slot) {
        if (__atomic_load_n(rangeHost + slot, __ATOMIC_ACQUIRE) == 0) continue;
        __atomic_store_n(rangeHost + slot, 0u, __ATOMIC_RELEASE);
        raised.push_back(slot == 0 ? UINT64_MAX : slotTicket[slot]);
    }
    if (raised.empty()) return 1;
    uint64_t first = raised[0];
    for (uint64_t t : raised) first = t < first ? t : first;
    if (ticket) *ticket = first;
    const std::string who = first == UINT64_MAX ? std::string("a prefill call captured into a graph (a replay)")
                                                : "prefill call ticket " + std::to_string(first);
    fail(who + (raised.size() > 1 ? " (and " + std::to_string(raised.size() - 1) + " more)" : std::string()) +
         ": a q, k or v element (after its norm, rotation and scale) or a cached key or value lies outside "
         "fp16's range (|x| > 65504): the fp16 working copies cannot hold it");
    return 0;
}

Context::~Context() {
    // process teardown: the runtime reclaims device memory itself
}

void* Context::grow(ScratchSlot slot, size_t bytes) {
    if (bytes == 0) bytes = 256;
    if (scratchBytes[slot] >= bytes) return scratch[slot];
    if (scratch[slot]) {
        (void)hipDeviceSynchronize();   // the old buffer may still be in use by queued work
        (void)hipFree(scratch[slot]);
        allocated -= scratchBytes[slot];
        scratch[slot] = nullptr;
        scratchBytes[slot] = 0;
    }
    void* fresh = nullptr;
    if (hipMalloc(&fresh, bytes) != hipSuccess) {
        (void)hipGetLastError();
        error = "hipMalloc failed for " + std::to_string(bytes) + " scratch bytes";
        return nullptr;
    }
    scratch[slot] = fresh;
    scratchBytes[slot] = bytes;
    allocated += bytes;
    return fresh;
}

void* Context::growZeroed(ScratchSlot slot, size_t bytes) {
    const bool fresh = scratchBytes[slot] < (bytes ? bytes : 256);
    void* p = grow(slot, bytes);
    if (p && fresh && hipMemset(p, 0, scratchBytes[slot]) != hipSuccess) {
        (void)hipGetLastError();
        error = "hipMemset of scratch failed";
        return nullptr;
    }
    return p;
}

hipEvent_t Context::takeEvent() {
    if (!spareEvents.empty()) {
        hipEvent_t e = spareEvents.back();
        spareEvents.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

void Context::resolveProfile() {
    for (Pending& rec : pending) {
        float ms = 0.0f;
        if (hipEventSynchronize(rec.end) == hipSuccess && hipEventElapsedTime(&ms, rec.begin, rec.end) == hipSuccess) {
            auto& slot = totals[rec.kernel];
            slot.first += ms;
            slot.second += 1;
        }
        spareEvents.push_back(rec.begin);
        spareEvents.push_back(rec.end);
    }
    pending.clear();
}

} // namespace aigpu

using aigpu::Clock;
using aigpu::Context;
using aigpu::since;

namespace {

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

/* Orders a call after the previous call when the two use different streams:
   every call shares the backend's scratch, so the new stream first waits for
   the event recorded after the previous call's launches, and this call's own
   launches are followed by the event in turn. A stream being captured into a
   graph is left alone (the caller orders captured work); so is the case of
   one stream, where stream order already holds. */
struct StreamOrder {
    Context& ctx;
    hipStream_t stream;
    bool active = true;
    StreamOrder(Context& c, hipStream_t s) : ctx(c), stream(s) {
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(s, &capture) != hipSuccess) {
            (void)hipGetLastError();
            capture = hipStreamCaptureStatusNone;
        }
        if (capture != hipStreamCaptureStatusNone) {
            active = false;
            return;
        }
        if (ctx.handoffValid && ctx.handoffStream != s && hipStreamWaitEvent(s, ctx.handoff, 0) != hipSuccess)
            (void)hipGetLastError();
    }
    ~StreamOrder() {
        if (!active) return;
        if (hipEventRecord(ctx.handoff, stream) == hipSuccess) {
            ctx.handoffStream = stream;
            ctx.handoffValid = true;
        } else {
            (void)hipGetLastError();
        }
    }
    StreamOrder(const StreamOrder&) = delete;
    StreamOrder& operator=(const StreamOrder&) = delete;
};

size_t elem_bytes(uint32_t type) { return type == AIGPU_BF16 ? 2 : 4; }

/* copies `bytes` from the host into scratch at byte offset `at`; returns the device address */
void* stage_in(Context& ctx, char* base, size_t& at, const void* host, size_t bytes) {
    if (!host || bytes == 0) return nullptr;
    at = (at + 255) & ~size_t(255);
    void* dst = base + at;
    const Clock::time_point mark = Clock::now();
    if (hipMemcpy(dst, host, bytes, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipGetLastError();
        ctx.error = "hipMemcpy host to device failed";
        return nullptr;
    }
    ctx.stats.transferSeconds += since(mark);
    ctx.stats.hostToDeviceBytes += bytes;
    at += bytes;
    return dst;
}

size_t padded(size_t bytes) { return bytes ? ((bytes + 255) & ~size_t(255)) + 256 : 0; }

bool copy_out(Context& ctx, void* host, const void* dev, size_t bytes) {
    const Clock::time_point mark = Clock::now();
    if (hipMemcpy(host, dev, bytes, hipMemcpyDeviceToHost) != hipSuccess) {
        (void)hipGetLastError();
        return ctx.fail("hipMemcpy device to host failed");
    }
    ctx.stats.transferSeconds += since(mark);
    ctx.stats.deviceToHostBytes += bytes;
    return true;
}

bool finish(Context& ctx, Clock::time_point mark) {
    const hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return ctx.fail(std::string("kernel execution failed: ") + hipGetErrorString(e));
    ctx.stats.kernelSeconds += since(mark);
    return true;
}

} // namespace

extern "C" {

AIGPU_ABI int aigpu_available(void) { return Context::instance().ok ? 1 : 0; }

AIGPU_ABI const char* aigpu_device_name(void) { return Context::instance().name.c_str(); }

AIGPU_ABI const char* aigpu_last_error(void) { return Context::instance().error.c_str(); }

AIGPU_ABI uint64_t aigpu_total_memory(void) {
    size_t free = 0, total = 0;
    if (!Context::instance().ok || hipMemGetInfo(&free, &total) != hipSuccess) return 0;
    return total;
}

AIGPU_ABI uint64_t aigpu_free_memory(void) {
    size_t free = 0, total = 0;
    if (!Context::instance().ok || hipMemGetInfo(&free, &total) != hipSuccess) return 0;
    return free;
}

AIGPU_ABI uint64_t aigpu_allocated_bytes(void) { return Context::instance().allocated; }

AIGPU_ABI void* aigpu_upload(const void* host, uint64_t bytes) {
    Context& ctx = Context::instance();
    if (!ctx.ok || bytes == 0) return nullptr;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    void* device = nullptr;
    if (hipMalloc(&device, bytes) != hipSuccess) {
        (void)hipGetLastError();
        ctx.error = "out of VRAM: hipMalloc(" + std::to_string(bytes) + ") failed";
        return nullptr;
    }
    if (host && hipMemcpy(device, host, bytes, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(device);
        ctx.error = "hipMemcpy host to device failed during upload";
        return nullptr;
    }
    ctx.allocated += bytes;
    ctx.stats.hostToDeviceBytes += host ? bytes : 0;
    return device;
}

AIGPU_ABI void* aigpu_allocate(uint64_t bytes) {
    Context& ctx = Context::instance();
    if (!ctx.ok || bytes == 0) return nullptr;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    void* device = nullptr;
    if (hipMalloc(&device, bytes) != hipSuccess) {
        (void)hipGetLastError();
        ctx.error = "out of VRAM: hipMalloc(" + std::to_string(bytes) + ") failed";
        return nullptr;
    }
    if (hipMemset(device, 0, bytes) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(device);
        ctx.error = "hipMemset failed";
        return nullptr;
    }
    ctx.allocated += bytes;
    return device;
}

AIGPU_ABI void aigpu_release(void* device, uint64_t bytes) {
    if (!device) return;
    Context& ctx = Context::instance();
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    (void)hipFree(device);
    ctx.allocated -= bytes;
}

AIGPU_ABI int aigpu_download(void* host, const void* device, uint64_t bytes) {
    Context& ctx = Context::instance();
    if (!ctx.ok || !device || !host) return 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    return copy_out(ctx, host, device, bytes) ? 1 : 0;
}

AIGPU_ABI int aigpu_write(void* device, uint64_t offset, const void* host, uint64_t bytes) {
    Context& ctx = Context::instance();
    if (!ctx.ok || !device || !host) return 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    if (hipMemcpy(static_cast<char*>(device) + offset, host, bytes, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipGetLastError();
        ctx.error = "hipMemcpy host to device failed";
        return 0;
    }
    ctx.stats.hostToDeviceBytes += bytes;
    return 1;
}

AIGPU_ABI void aigpu_synchronize(void) {
    if (Context::instance().ok) (void)hipDeviceSynchronize();
}

AIGPU_ABI void aigpu_counters(AiGpuCounters* out) {
    if (out) *out = Context::instance().stats;
}

AIGPU_ABI void aigpu_reset_counters(void) { Context::instance().stats = AiGpuCounters{}; }

AIGPU_ABI int aigpu_copy_device(void* dst, const void* src, uint64_t bytes, void* stream) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, as_stream(stream));
    return aigpu::launch_copy(dst, src, bytes, order.stream) ? 1 : 0;
}

AIGPU_ABI uint64_t aigpu_range_ticket(void) {
    Context& ctx = Context::instance();
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    return ctx.rangeTickets;
}

AIGPU_ABI int aigpu_range_status(uint64_t* ticket) {
    Context& ctx = Context::instance();
    if (ticket) *ticket = 0;
    if (!ctx.ok) return 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    return ctx.rangeStatus(ticket);
}

AIGPU_ABI void aigpu_profile(int enable) {
    Context& ctx = Context::instance();
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    ctx.profiling = enable != 0;
}

AIGPU_ABI void aigpu_profile_reset(void) {
    Context& ctx = Context::instance();
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    ctx.resolveProfile();
    ctx.totals.clear();
}

AIGPU_ABI int aigpu_profile_read(const char* kernel, double* milliseconds, uint64_t* launches) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    ctx.resolveProfile();
    double ms = 0.0;
    uint64_t n = 0;
    for (const auto& kv : ctx.totals)
        if (!kernel || kv.first.find(kernel) != std::string::npos) {
            ms += kv.second.first;
            n += kv.second.second;
        }
    if (milliseconds) *milliseconds = ms;
    if (launches) *launches = n;
    return n > 0 ? 1 : 0;
}

/* ---------------------------------------------------------------- 1 + 2 */

AIGPU_ABI int aigpu_attention_device(const AiGpuAttention* args) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    if (!args) return ctx.fail("attention: null arguments"), 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, as_stream(args->stream));
    aigpu::AttentionF32Params p{};
    p.q = args->q;
    p.keys = args->keys;
    p.values = args->values;
    p.out = args->out;
    p.qType = int(args->qType);
    p.kvType = int(args->kvType);
    p.count = args->count;
    p.start = args->start;
    p.heads = args->heads;
    p.kvHeads = args->kvHeads;
    p.dim = args->dim;
    p.qStride = args->qStride;
    p.window = args->window;
    p.posStride = args->posStride;
    p.headStride = args->headStride;
    if (!p.q || !p.keys || !p.values || !p.out) return ctx.fail("attention: null tensor"), 0;
    return aigpu::launch_attention_f32(p, order.stream) ? 1 : 0;
}

AIGPU_ABI int aigpu_attention(const float* q, const float* keys, const float* values, float* out,
                              uint64_t count, uint64_t start, uint64_t heads, uint64_t kvHeads,
                              uint64_t dim, uint64_t qStride, uint64_t window) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    if (!q || !keys || !values || !out) return ctx.fail("attention: null tensor"), 0;
    if (count == 0) return 1;
    if (kvHeads == 0 || heads % kvHeads) return ctx.fail("attention: heads must be a multiple of kvHeads"), 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, nullptr);
    const size_t qBytes = ((count - 1) * heads * qStride + (heads - 1) * qStride + dim) * 4;
    const size_t kvBytes = (start + count) * kvHeads * dim * 4;
    const size_t outBytes = count * heads * dim * 4;
    char* in = static_cast<char*>(ctx.grow(aigpu::SLOT_STAGE_IN, padded(qBytes) + 2 * padded(kvBytes)));
    float* dOut = static_cast<float*>(ctx.grow(aigpu::SLOT_STAGE_OUT, outBytes));
    if (!in || !dOut) return 0;
    size_t at = 0;
    const void* dq = stage_in(ctx, in, at, q, qBytes);
    const void* dk = stage_in(ctx, in, at, keys, kvBytes);
    const void* dv = stage_in(ctx, in, at, values, kvBytes);
    if (!dq || !dk || !dv) return 0;
    aigpu::AttentionF32Params p{dq, dk, dv, dOut, AIGPU_F32, AIGPU_F32, count, start, heads,
                                kvHeads, dim, qStride, window, kvHeads * dim, dim};
    const Clock::time_point mark = Clock::now();
    if (!aigpu::launch_attention_f32(p, nullptr) || !finish(ctx, mark)) return 0;
    return copy_out(ctx, out, dOut, outBytes) ? 1 : 0;
}

/* ------------------------------------------------------------------ 3 */

static aigpu::PrefillParams prefill_params(const AiGpuPrefill* a) {
    aigpu::PrefillParams p{};
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
    p.out = a->out;
    p.keyCache = static_cast<uint16_t*>(a->keyCache);
    p.valueCache = static_cast<uint16_t*>(a->valueCache);
    p.qNorm = a->qNorm;
    p.kNorm = a->kNorm;
    p.freqs = a->rotaryFrequencies;
    p.eps = a->epsilon;
    p.normOffset = a->normOffset;
    p.rotaryDims = int(a->rotaryDims);
    p.inType = int(a->inType);
    p.outputGate = a->outputGate ? 1 : 0;
    p.count = a->count;
    p.start = a->start;
    p.heads = a->heads;
    p.kvHeads = a->kvHeads;
    p.dim = a->dim;
    p.qStride = a->qStride;
    p.window = a->window;
    p.capacity = a->capacity;
    return p;
}

AIGPU_ABI int aigpu_prefill_attention(const AiGpuPrefill* args) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    if (!args) return ctx.fail("prefill: null arguments"), 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, as_stream(args->stream));
    aigpu::PrefillParams p = prefill_params(args);
    uint64_t ticket = 0;
    p.rangeFlag = ctx.rangeSlot(order.stream, &ticket);
    return aigpu::launch_prefill(p, order.stream) ? 1 : 0;
}

AIGPU_ABI int aigpu_prefill_attention_host(const AiGpuPrefill* args) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    if (!args || !args->q || !args->k || !args->v || !args->out) return ctx.fail("prefill: null tensor"), 0;
    if (args->count == 0) return 1;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, nullptr);
    const size_t es = elem_bytes(args->inType);
    const size_t qBytes = args->count * args->heads * args->qStride * es;
    const size_t kvBytes = args->count * args->kvHeads * args->dim * es;
    const size_t gBytes = args->dim * 4, fBytes = (args->rotaryDims / 2) * 4;
    const size_t outBytes = args->count * args->heads * args->dim * 4;
    char* in = static_cast<char*>(ctx.grow(aigpu::SLOT_STAGE_IN, padded(qBytes) + 2 * padded(kvBytes) +
                                                                       2 * padded(gBytes) + padded(fBytes)));
    float* dOut = static_cast<float*>(ctx.grow(aigpu::SLOT_STAGE_OUT, outBytes));
    if (!in || !dOut) return 0;
    AiGpuPrefill dev = *args;
    size_t at = 0;
    dev.q = stage_in(ctx, in, at, args->q, qBytes);
    dev.k = stage_in(ctx, in, at, args->k, kvBytes);
    dev.v = stage_in(ctx, in, at, args->v, kvBytes);
    dev.qNorm = static_cast<const float*>(stage_in(ctx, in, at, args->qNorm, gBytes));
    dev.kNorm = static_cast<const float*>(stage_in(ctx, in, at, args->kNorm, gBytes));
    dev.rotaryFrequencies = static_cast<const float*>(
        args->rotaryFrequencies ? stage_in(ctx, in, at, args->rotaryFrequencies, fBytes) : nullptr);
    dev.out = dOut;
    if (!dev.q || !dev.k || !dev.v) return 0;
    const Clock::time_point mark = Clock::now();
    aigpu::PrefillParams p = prefill_params(&dev);
    uint64_t ticket = 0;
    p.rangeFlag = ctx.rangeSlot(nullptr, &ticket);
    if (!aigpu::launch_prefill(p, nullptr) || !finish(ctx, mark)) return 0;
    if (ctx.rangeRaisedFor(ticket))
        return ctx.fail("prefill: a q, k or v element (after its norm, rotation and scale) or a cached key or value "
                        "lies outside fp16's range (|x| > 65504): the fp16 working copies cannot hold it"),
               0;
    return copy_out(ctx, args->out, dOut, outBytes) ? 1 : 0;
}

/* ------------------------------------------------------------------ 4 */

static aigpu::DecodeParams decode_params(const AiGpuDecode* a) {
    aigpu::DecodeParams p{};
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
    p.out = a->out;
    p.keyCache = static_cast<uint16_t*>(a->keyCache);
    p.valueCache = static_cast<uint16_t*>(a->valueCache);
    p.positions = a->positions;
    p.qNorm = a->qNorm;
    p.kNorm = a->kNorm;
    p.freqs = a->rotaryFrequencies;
    p.eps = a->epsilon;
    p.normOffset = a->normOffset;
    p.rotaryDims = int(a->rotaryDims);
    p.inType = int(a->inType);
    p.outputGate = a->outputGate ? 1 : 0;
    p.maxPosition = a->maxPosition;
    p.batch = a->batch;
    p.heads = a->heads;
    p.kvHeads = a->kvHeads;
    p.dim = a->dim;
    p.qStride = a->qStride;
    p.window = a->window;
    p.capacity = a->capacity;
    p.batchStride = a->batchStride;
    return p;
}

AIGPU_ABI int aigpu_decode_attention(const AiGpuDecode* args) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    if (!args) return ctx.fail("decode: null arguments"), 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, as_stream(args->stream));
    return aigpu::launch_decode(decode_params(args), order.stream) ? 1 : 0;
}

AIGPU_ABI int aigpu_decode_attention_static(const AiGpuDecode* args) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    if (!args) return ctx.fail("decode (no allocation): null arguments"), 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, as_stream(args->stream));
    aigpu::FixedScratch fixed{};
    if (!aigpu::decode_static_scratch(&fixed.base, &fixed.bytes)) return 0;
    struct NoAlloc {
        Context& c;
        explicit NoAlloc(Context& x) : c(x) { c.noAlloc = true; }
        ~NoAlloc() { c.noAlloc = false; }
    } guard(ctx);
    return aigpu::launch_decode(decode_params(args), order.stream, &fixed) ? 1 : 0;
}

AIGPU_ABI int aigpu_decode_attention_host(const AiGpuDecode* args) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    if (!args || !args->q || !args->k || !args->v || !args->out || !args->positions)
        return ctx.fail("decode: null tensor"), 0;
    if (args->batch == 0) return 1;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, nullptr);
    const size_t es = elem_bytes(args->inType);
    const size_t qBytes = args->batch * args->heads * args->qStride * es;
    const size_t kvBytes = args->batch * args->kvHeads * args->dim * es;
    const size_t pBytes = args->batch * 4;
    const size_t gBytes = args->dim * 4, fBytes = (args->rotaryDims / 2) * 4;
    const size_t outBytes = args->batch * args->heads * args->dim * 4;
    char* in = static_cast<char*>(ctx.grow(aigpu::SLOT_STAGE_IN, padded(qBytes) + 2 * padded(kvBytes) + padded(pBytes) +
                                                                       2 * padded(gBytes) + padded(fBytes)));
    float* dOut = static_cast<float*>(ctx.grow(aigpu::SLOT_STAGE_OUT, outBytes));
    if (!in || !dOut) return 0;
    AiGpuDecode dev = *args;
    uint32_t maxPos = 0;
    for (uint64_t b = 0; b < args->batch; ++b) maxPos = args->positions[b] > maxPos ? args->positions[b] : maxPos;
    dev.maxPosition = maxPos;
    size_t at = 0;
    dev.q = stage_in(ctx, in, at, args->q, qBytes);
    dev.k = stage_in(ctx, in, at, args->k, kvBytes);
    dev.v = stage_in(ctx, in, at, args->v, kvBytes);
    dev.positions = static_cast<const uint32_t*>(stage_in(ctx, in, at, args->positions, pBytes));
    dev.qNorm = static_cast<const float*>(stage_in(ctx, in, at, args->qNorm, gBytes));
    dev.kNorm = static_cast<const float*>(stage_in(ctx, in, at, args->kNorm, gBytes));
    dev.rotaryFrequencies = static_cast<const float*>(
        args->rotaryFrequencies ? stage_in(ctx, in, at, args->rotaryFrequencies, fBytes) : nullptr);
    dev.out = dOut;
    if (!dev.q || !dev.k || !dev.v || !dev.positions) return 0;
    const Clock::time_point mark = Clock::now();
    if (!aigpu::launch_decode(decode_params(&dev), nullptr) || !finish(ctx, mark)) return 0;
    return copy_out(ctx, args->out, dOut, outBytes) ? 1 : 0;
}

/* ------------------------------------------------------------------ 5 */

static aigpu::DeltaRuleParams delta_params(const AiGpuDeltaRule* a) {
    aigpu::DeltaRuleParams p{};
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
    p.g = a->g;
    p.beta = a->beta;
    p.a = a->a;
    p.b = a->b;
    p.aLog = a->aLog;
    p.dtBias = a->dtBias;
    p.state = a->state;
    p.out = a->out;
    p.inType = int(a->inType);
    p.normalize = int(a->normalize);
    p.chunk = int(a->chunk);
    p.count = a->count;
    p.keyHeads = a->keyHeads;
    p.valueHeads = a->valueHeads;
    p.keyDim = a->keyDim;
    p.valueDim = a->valueDim;
    return p;
}

AIGPU_ABI int aigpu_gated_delta_rule(const AiGpuDeltaRule* args) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    if (!args) return ctx.fail("delta rule: null arguments"), 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, as_stream(args->stream));
    return aigpu::launch_delta_rule(delta_params(args), order.stream) ? 1 : 0;
}

AIGPU_ABI int aigpu_gated_delta_rule_host(const AiGpuDeltaRule* args) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    if (!args || !args->q || !args->k || !args->v || !args->state || !args->out)
        return ctx.fail("delta rule: null tensor"), 0;
    if (args->count == 0) return 1;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, nullptr);
    const size_t es = elem_bytes(args->inType);
    const size_t qkBytes = args->count * args->keyHeads * args->keyDim * es;
    const size_t vBytes = args->count * args->valueHeads * args->valueDim * es;
    const size_t gateBytes = args->count * args->valueHeads * 4;
    const size_t headBytes = args->valueHeads * 4;
    const size_t stateBytes = args->valueHeads * args->keyDim * args->valueDim * 4;
    const size_t outBytes = args->count * args->valueHeads * args->valueDim * 4;
    char* in = static_cast<char*>(ctx.grow(aigpu::SLOT_STAGE_IN, 2 * padded(qkBytes) + padded(vBytes) + 2 * padded(gateBytes) +
                                                                       2 * padded(headBytes) + padded(stateBytes)));
    float* dOut = static_cast<float*>(ctx.grow(aigpu::SLOT_STAGE_OUT, outBytes));
    if (!in || !dOut) return 0;
    AiGpuDeltaRule dev = *args;
    size_t at = 0;
    dev.q = stage_in(ctx, in, at, args->q, qkBytes);
    dev.k = stage_in(ctx, in, at, args->k, qkBytes);
    dev.v = stage_in(ctx, in, at, args->v, vBytes);
    if (args->aLog) {
        dev.a = static_cast<const float*>(stage_in(ctx, in, at, args->a, gateBytes));
        dev.b = static_cast<const float*>(stage_in(ctx, in, at, args->b, gateBytes));
        dev.aLog = static_cast<const float*>(stage_in(ctx, in, at, args->aLog, headBytes));
        dev.dtBias = static_cast<const float*>(stage_in(ctx, in, at, args->dtBias, headBytes));
        dev.g = dev.beta = nullptr;
    } else {
        dev.g = static_cast<const float*>(stage_in(ctx, in, at, args->g, gateBytes));
        dev.beta = static_cast<const float*>(stage_in(ctx, in, at, args->beta, gateBytes));
    }
    dev.state = static_cast<float*>(stage_in(ctx, in, at, args->state, stateBytes));
    dev.out = dOut;
    if (!dev.q || !dev.k || !dev.v || !dev.state) return 0;
    const Clock::time_point mark = Clock::now();
    if (!aigpu::launch_delta_rule(delta_params(&dev), nullptr) || !finish(ctx, mark)) return 0;
    if (!copy_out(ctx, args->out, dOut, outBytes)) return 0;
    return copy_out(ctx, args->state, dev.state, stateBytes) ? 1 : 0;
}

} // extern "C"

AIGPU_ABI int aigpu_gdn_conv(const AiGpuGdnConv* args) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    if (!args) return ctx.fail("gdn conv: null arguments"), 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, as_stream(args->stream));
    aigpu::GdnConvParams p{};
    p.in = args->in;
    p.ba = args->ba;
    p.kernel = args->kernel;
    p.window = args->window;
    p.q = args->q;
    p.k = args->k;
    p.v = args->v;
    p.z = args->z;
    p.a = args->a;
    p.b = args->b;
    p.inType = args->inType == AIGPU_BF16 ? 1 : (args->inType == AIGPU_F32 ? 0 : 2);
    p.outType = args->outType == AIGPU_BF16 ? 1 : (args->outType == AIGPU_F32 ? 0 : 2);
    p.fused = args->fused ? 1 : 0;
    p.count = args->count;
    p.keyHeads = args->keyHeads;
    p.valueHeads = args->valueHeads;
    p.keyDim = args->keyDim;
    p.valueDim = args->valueDim;
    p.kernelSize = args->kernelSize;
    return aigpu::launch_gdn_conv(p, order.stream) ? 1 : 0;
}

AIGPU_ABI int aigpu_gdn_gated_norm(const AiGpuGdnGatedNorm* args) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    if (!args) return ctx.fail("gdn gated norm: null arguments"), 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, as_stream(args->stream));
    aigpu::GdnGatedNormParams p{};
    p.x = args->x;
    p.z = args->z;
    p.gamma = args->gamma;
    p.out = args->out;
    p.eps = args->epsilon;
    p.zType = args->zType == AIGPU_BF16 ? 1 : (args->zType == AIGPU_F32 ? 0 : 2);
    p.outType = args->outType == AIGPU_BF16 ? 1 : (args->outType == AIGPU_F32 ? 0 : 2);
    if (args->gateKind > 1) return ctx.fail("gdn gated norm: gateKind must be 0 (SiLU) or 1 (sigmoid)"), 0;
    p.sigmoidGate = args->gateKind;
    p.count = args->count;
    p.valueHeads = args->valueHeads;
    p.valueDim = args->valueDim;
    return aigpu::launch_gdn_gated_norm(p, order.stream) ? 1 : 0;
}

AIGPU_ABI int aigpu_kda_rule(const AiGpuKda* args) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    if (!args) return ctx.fail("kda: null arguments"), 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, as_stream(args->stream));
    aigpu::KdaParams p{};
    p.q = args->q;
    p.k = args->k;
    p.v = args->v;
    p.g = args->g;
    p.beta = args->beta;
    p.f = args->f;
    p.b = args->b;
    p.aLog = args->aLog;
    p.dtBias = args->dtBias;
    p.lowerBound = args->lowerBound;
    p.safeGate = args->safeGate ? 1 : 0;
    p.state = args->state;
    p.out = args->out;
    p.inType = int(args->inType);
    p.normalize = args->normalize ? 1 : 0;
    p.count = args->count;
    p.keyHeads = args->keyHeads;
    p.valueHeads = args->valueHeads;
    p.keyDim = args->keyDim;
    p.valueDim = args->valueDim;
    return aigpu::launch_kda(p, order.stream) ? 1 : 0;
}

namespace {

/* the host-staged product of DeviceABI.h's aigpu_matmul_nt* (Kernels.hip
   dispatch: a in, kernel, c out, each timed into the counters) */
void matmul_host(const float* a, const void* b, const void* scales, float* c, uint64_t m, uint64_t k, uint64_t n,
                 int type) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return;
    if (!a || !b || !c || (type >= 2 && !scales)) {
        ctx.error = "matmul: null tensor";
        return;
    }
    if (m == 0 || n == 0) return;
    if (m > 0xFFFFFFFFull || k > 0xFFFFFFFFull || n > 0xFFFFFFFFull || k == 0) {
        ctx.error = "matmul: dimensions out of range";
        return;
    }
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, nullptr);
    const size_t inBytes = m * k * 4, outBytes = m * n * 4;
    char* in = static_cast<char*>(ctx.grow(aigpu::SLOT_STAGE_IN, padded(inBytes)));
    float* dC = static_cast<float*>(ctx.grow(aigpu::SLOT_STAGE_OUT, outBytes));
    if (!in || !dC) return;
    size_t at = 0;
    const float* dA = static_cast<const float*>(stage_in(ctx, in, at, a, inBytes));
    if (!dA) return;
    aigpu::GemvParams p{};
    p.a = dA;
    p.w = b;
    p.scales = static_cast<const float*>(scales);
    p.out = dC;
    p.type = type;
    p.m = uint32_t(m);
    p.k = uint32_t(k);
    p.n = uint32_t(n);
    p.ldo = uint32_t(n);
    const Clock::time_point mark = Clock::now();
    if (!aigpu::launch_gemv(p, nullptr) || !finish(ctx, mark)) return;
    if (copy_out(ctx, c, dC, outBytes)) ctx.error.clear();
}

} // namespace

extern "C" {

AIGPU_ABI void aigpu_matmul_nt(const float* a, const void* b, float* c, uint64_t m, uint64_t k, uint64_t n) {
    matmul_host(a, b, nullptr, c, m, k, n, 0);
}

AIGPU_ABI void aigpu_matmul_nt_bf16(const float* a, const void* b, float* c, uint64_t m, uint64_t k, uint64_t n) {
    matmul_host(a, b, nullptr, c, m, k, n, 1);
}

AIGPU_ABI void aigpu_matmul_nt_q8(const float* a, const void* b, const void* scales, float* c, uint64_t m,
                                  uint64_t k, uint64_t n) {
    matmul_host(a, b, scales, c, m, k, n, 2);
}

AIGPU_ABI void aigpu_matmul_nt_q4(const float* a, const void* b, const void* scales, float* c, uint64_t m,
                                  uint64_t k, uint64_t n) {
    matmul_host(a, b, scales, c, m, k, n, 3);
}

AIGPU_ABI int aigpu_matmul_device(const AiGpuMatmul* args) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    if (!args) return ctx.fail("matmul: null arguments"), 0;
    if (args->m > 0xFFFFFFFFull || args->k > 0xFFFFFFFFull || args->n > 0xFFFFFFFFull ||
        args->ldc > 0xFFFFFFFFull)
        return ctx.fail("matmul: dimensions out of range"), 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, as_stream(args->stream));
    aigpu::GemvParams p{};
    p.a = args->a;
    p.w = args->b;
    p.scales = args->scales;
    p.bias = args->bias;
    p.out = args->c;
    p.type = int(args->type);
    p.accumulate = args->accumulate ? 1 : 0;
    p.m = uint32_t(args->m);
    p.k = uint32_t(args->k);
    p.n = uint32_t(args->n);
    p.ldo = uint32_t(args->ldc ? args->ldc : args->n);
    return aigpu::launch_gemv(p, order.stream) ? 1 : 0;
}

} // extern "C"

extern "C" {

AIGPU_ABI int aigpu_prefill_mixer(const AiGpuPrefillMixer* args) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    if (!args) return ctx.fail("prefill mixer: null arguments"), 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, as_stream(args->stream));
    auto weight = [](const AiGpuDenseWeight& w) {
        aigpu::MixerWeight m{};
        m.codes = w.codes;
        m.scales = static_cast<const float*>(w.scales);
        m.bias = w.bias;
        m.type = int(w.type);
        m.in = w.inDim;
        m.out = w.outDim;
        return m;
    };
    for (const AiGpuDenseWeight* w : {&args->q, &args->k, &args->v, &args->o})
        if (w->type > AIGPU_W_Q4 || (w->type >= AIGPU_W_Q8 && !w->scales))
            return ctx.fail("prefill mixer: unknown weight type or missing scales"), 0;
    if (args->hidden > 0xFFFFFFFFull || args->heads * args->dim * 2 > 0xFFFFFFFFull)
        return ctx.fail("prefill mixer: dimensions out of range"), 0;
    aigpu::MixerParams p{};
    p.x = args->x;
    p.q = weight(args->q);
    p.k = weight(args->k);
    p.v = weight(args->v);
    p.o = weight(args->o);
    p.out = args->out;
    p.keyCache = static_cast<uint16_t*>(args->keyCache);
    p.valueCache = static_cast<uint16_t*>(args->valueCache);
    p.qNorm = args->qNorm;
    p.kNorm = args->kNorm;
    p.freqs = args->rotaryFrequencies;
    p.eps = args->epsilon;
    p.normOffset = args->normOffset;
    p.rotaryDims = args->rotaryFrequencies ? int(args->rotaryDims) : 0;
    p.outputGate = args->outputGate ? 1 : 0;
    p.accumulate = args->accumulate ? 1 : 0;
    p.count = args->count;
    p.start = args->start;
    p.hidden = args->hidden;
    p.heads = args->heads;
    p.kvHeads = args->kvHeads;
    p.dim = args->dim;
    p.qStride = args->outputGate ? 2 * args->dim : args->dim;
    p.window = args->window;
    p.capacity = args->capacity;
    uint64_t ticket = 0;
    p.rangeFlag = ctx.rangeSlot(order.stream, &ticket);
    return aigpu::launch_prefill_mixer(p, order.stream) ? 1 : 0;
}

AIGPU_ABI int aigpu_select_keys(const AiGpuSelectKeys* args) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    if (!args) return ctx.fail("select keys: null arguments"), 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, as_stream(args->stream));
    auto weight = [](const AiGpuDenseWeight& w) {
        aigpu::MixerWeight m{};
        m.codes = w.codes;
        m.scales = static_cast<const float*>(w.scales);
        m.bias = w.bias;
        m.type = int(w.type);
        m.in = w.inDim;
        m.out = w.outDim;
        return m;
    };
    for (const AiGpuDenseWeight* w : {&args->idxK, &args->idxGate, &args->idxQB, &args->idxWeights})
        if (w->type > AIGPU_W_Q4 || (w->type >= AIGPU_W_Q8 && !w->scales))
            return ctx.fail("select keys: unknown weight type or missing scales"), 0;
    aigpu::IndexerParams p{};
    p.h = args->h;
    p.qResid = args->qResid;
    p.wk = weight(args->idxK);
    p.wgate = weight(args->idxGate);
    p.wq = weight(args->idxQB);
    p.ww = weight(args->idxWeights);
    p.kNorm = args->kNorm;
    p.kNormBias = args->kNormBias;
    p.ape = args->ape;
    p.keys = args->indexKeys;
    p.gates = args->indexGates;
    p.pools = args->poolKeys;
    p.selStart = args->selStart;
    p.selCount = args->selCount;
    p.selKeys = args->selKeys;
    p.scores = args->scores;
    p.tail = args->indexTail ? 1 : 0;
    p.count = args->count;
    p.startPos = args->startPos;
    p.hidden = args->hidden;
    p.qRank = args->qRank;
    p.heads = args->heads;
    p.dim = args->dim;
    p.topK = args->topK;
    p.pool = args->pool;
    p.capacity = args->capacity;
    return aigpu::launch_select_keys(p, order.stream) ? 1 : 0;
}

AIGPU_ABI int aigpu_latent_attention(const AiGpuLatentAttention* args) {
    Context& ctx = Context::instance();
    if (!ctx.ok) return 0;
    if (!args) return ctx.fail("latent attention: null arguments"), 0;
    std::lock_guard<std::recursive_mutex> lock(ctx.gate);
    const StreamOrder order(ctx, as_stream(args->stream));
    aigpu::LatentParams p{};
    p.q = args->q;
    p.latent = args->latent;
    p.wkv = args->kvB;
    p.wType = args->kvBType == AIGPU_BF16 ? 1 : (args->kvBType == AIGPU_F32 ? 0 : 2);
    p.selStart = args->selStart;
    p.selCount = args->selStart ? args->selCount : nullptr;
    p.selKeys = args->selKeys;
    p.out = args->out;
    p.scale = args->scale;
    p.count = args->count;
    p.startPos = args->startPos;
    p.heads = args->heads;
    p.nope = args->nopeDim;
    p.vdim = args->vDim;
    p.rank = args->kvLoraRank;
    return aigpu::launch_latent_attention(p, order.stream) ? 1 : 0;
}

} // extern "C"
