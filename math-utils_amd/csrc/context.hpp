// context.hpp - process-wide backend state behind the C ABI.
//
// One device context per process, as the reference HIP backend keeps
// (src/gpu/Kernels.hip:43-124): device selection, the last error string,
// the allocation total, counters, growable scratch buffers and the lock every
// entry point takes. Scratch buffers are allocated once and grown, never per
// call: hipMalloc serialises against the device.
#pragma once

#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/aigpu_attention.h"

namespace aigpu {

enum ScratchSlot {
    SLOT_STAGE_IN = 0,   // host-form staging of inputs
    SLOT_STAGE_OUT,      // host-form staging of outputs
    SLOT_PREFILL_Q,      // fp16 head-major q of a prefill
    SLOT_PREFILL_K,      // fp16 head-major k history of a prefill
    SLOT_PREFILL_V,      // fp16 head-major v history of a prefill
    SLOT_DECODE_PARTS,   // split-K partial softmax records
    SLOT_DELTA_WORK,     // per-chunk solve products of the delta rule
    SLOT_LATENT,         // folded queries, contexts and split records of latent attention
    SLOT_MIXER_Q,        // fp32 q projection of a prefill mixer
    SLOT_MIXER_ATTN,     // fp32 attention output of a prefill mixer
    SLOT_INDEXER,        // index keys, queries, head weights and scores of selectKeys
    SLOT_GEMM_SPLIT,     // the K slices' partial tiles of a split GEMM
    SLOT_GEMM_A,         // a split into bf16 high parts and residuals for gemm_dma_kernel
    SLOT_MIXER_KV,       // fp32 k and v projections of a prefill mixer before their epilogue
    SLOT_ATTN_PARTS,     // split records of the tiled fp32 attention
    SLOT_DELTA_SEG,      // segment maps and start states of the two-level delta-rule scan
    SLOT_COUNT
};

struct Context {
    bool ok = false;
    std::string name;
    int cus = 0;         // compute units of the device
    std::string error;
    std::recursive_mutex gate;

    size_t allocated = 0;
    AiGpuCounters stats{};

    void* scratch[SLOT_COUNT] = {};
    size_t scratchBytes[SLOT_COUNT] = {};

    // profiling: events bracketing each launch, resolved on read
    bool profiling = false;
    // set during a call that must allocate nothing: no profiling events
    bool noAlloc = false;

    // fp16 range flags: RANGE_SLOTS words of mapped pinned host memory
    // (rangeDev is their device address). Every prefill call takes a ticket
    // and the word of its slot; kernels converting into the fp16 working
    // copies store 1 there when a finite value overflows fp16. Slot 0 belongs
    // to calls captured into a graph (their replays have no ticket of their
    // own); tickets 1, 2, ... cycle through slots 1 .. RANGE_SLOTS - 1.
    static constexpr int RANGE_SLOTS = 256;
    uint32_t* rangeHost = nullptr;
    uint32_t* rangeDev = nullptr;
    uint64_t rangeTickets = 0;                 // tickets issued so far
    uint64_t slotTicket[RANGE_SLOTS] = {};     // the ticket that last took each slot
    std::vector<uint64_t> rangeRaised;         // raised tickets found when their slot was taken again
    // a ticket for a call on `stream` and the device address of its flag word
    // (cleared); a stream being captured gets slot 0 and ticket UINT64_MAX
    uint32_t* rangeSlot(hipStream_t stream, uint64_t* ticket);
    // whether `ticket`'s word is raised, clearing it (its call has completed)
    bool rangeRaisedFor(uint64_t ticket);
    // waits for the device; 1 when no call since the last query raised its
    // word, else 0 with the error naming the earliest ticket that did
    int rangeStatus(uint64_t* ticket);

    // calls on different streams share the scratch slots (and the fixed
    // decode scratch): an event recorded on the stream of each call, which
    // a call on another stream waits for before its first launch
    hipEvent_t handoff = nullptr;
    hipStream_t handoffStream = nullptr;
    bool handoffValid = false;
    struct Pending { std::string kernel; hipEvent_t begin, end; };
    std::vector<Pending> pending;
    std::vector<hipEvent_t> spareEvents;
    std::map<std::string, std::pair<double, uint64_t>> totals;

    static Context& instance();

    // a scratch slot of at least `bytes`; nullptr (and error set) on failure
    void* grow(ScratchSlot slot, size_t bytes);
    // the same, zero-filled whenever it is (re)allocated; kernels that use it
    // must leave it zero again
    void* growZeroed(ScratchSlot slot, size_t bytes);

    bool fail(const std::string& why) {
        error = why;
        return false;
    }

    // records a launch: with profiling on, hipEvents bracket it on `stream`
    template <typename Launch>
    bool launch(const char* kernel, hipStream_t stream, Launch body) {
        hipEvent_t a = nullptr, b = nullptr;
        const bool timed = profiling && !noAlloc;
        if (timed) {
            a = takeEvent();
            b = takeEvent();
            if (a) (void)hipEventRecord(a, stream);
        }
        body();
        const hipError_t e = hipGetLastError();
        if (timed && a && b) {
            (void)hipEventRecord(b, stream);
            pending.push_back({kernel, a, b});
        }
        ++stats.launches;
        if (e != hipSuccess) return fail(std::string("launch of ") + kernel + " failed: " + hipGetErrorString(e));
        return true;
    }

    hipEvent_t takeEvent();
    void resolveProfile();

private:
    Context();
    ~Context();
};

} // namespace aigpu
