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
    SLOT_COUNT
};

struct Context {
    bool ok = false;
    std::string name;
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

    // one word of mapped pinned host memory that kernels converting into the
    // prefill's fp16 working copies set to 1 when a finite value overflows
    // fp16; rangeDev is its device address
    uint32_t* rangeHost = nullptr;
    uint32_t* rangeDev = nullptr;

    // calls on different streams share the scratch slots (and the fixed
    // decode scratch): an event recorded on the stream of each call, which
    // a call on another stream waits for before its first launch
    hipEvent_t handoff = nullptr;
    hipStream_t handoffStream = nullptr;
    bool handoffValid = false;
    // waits for `stream` and reports (and clears) a raised range flag as a
    // failure of `what`; a stream being captured into a graph is not waited
    // for and the flag stays for the next checked call
    bool checkRange(const char* what, hipStream_t stream);
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
