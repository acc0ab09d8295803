// stub.cpp - the no-device backend: every entry point of
// include/aigpu_attention.h answers "unavailable" (0 or null) and
// aigpu_last_error() says why, as the reference's src/gpu/Stub.cpp:18-66 does
// for DeviceABI.h. Linked in place of libaigpu.so where there is no ROCm, so
// callers take their CPU path through the same availability check they need
// anyway when a card is absent at run time.
#include "../../include/aigpu_attention.h"

extern "C" {

namespace {
const char NO_NAME[] = "";
const char NO_DEVICE[] = "built without the HIP attention backend: no device";
}

AIGPU_ABI int aigpu_available(void) { return 0; }
AIGPU_ABI const char* aigpu_device_name(void) { return NO_NAME; }
AIGPU_ABI const char* aigpu_last_error(void) { return NO_DEVICE; }
AIGPU_ABI uint64_t aigpu_total_memory(void) { return 0; }
AIGPU_ABI uint64_t aigpu_free_memory(void) { return 0; }
AIGPU_ABI uint64_t aigpu_allocated_bytes(void) { return 0; }
AIGPU_ABI void* aigpu_upload(const void*, uint64_t) { return nullptr; }
AIGPU_ABI void* aigpu_allocate(uint64_t) { return nullptr; }
AIGPU_ABI void aigpu_release(void*, uint64_t) {}
AIGPU_ABI int aigpu_download(void*, const void*, uint64_t) { return 0; }
AIGPU_ABI int aigpu_write(void*, uint64_t, const void*, uint64_t) { return 0; }
AIGPU_ABI void aigpu_synchronize(void) {}
AIGPU_ABI void aigpu_counters(AiGpuCounters* out) {
    if (out) *out = AiGpuCounters{};
}
AIGPU_ABI void aigpu_reset_counters(void) {}

AIGPU_ABI int aigpu_attention(const float*, const float*, const float*, float*, uint64_t, uint64_t,
                              uint64_t, uint64_t, uint64_t, uint64_t, uint64_t) {
    return 0;
}
AIGPU_ABI int aigpu_attention_device(const AiGpuAttention*) { return 0; }
AIGPU_ABI int aigpu_prefill_attention(const AiGpuPrefill*) { return 0; }
AIGPU_ABI int aigpu_prefill_attention_host(const AiGpuPrefill*) { return 0; }
AIGPU_ABI int aigpu_copy_device(void*, const void*, uint64_t, void*) { return 0; }
AIGPU_ABI uint64_t aigpu_range_ticket(void) { return 0; }
AIGPU_ABI int aigpu_range_status(uint64_t* ticket) {
    if (ticket) *ticket = 0;
    return 0;
}
AIGPU_ABI int aigpu_decode_attention(const AiGpuDecode*) { return 0; }
AIGPU_ABI int aigpu_decode_attention_host(const AiGpuDecode*) { return 0; }
AIGPU_ABI int aigpu_decode_attention_static(const AiGpuDecode*) { return 0; }
AIGPU_ABI int aigpu_gated_delta_rule(const AiGpuDeltaRule*) { return 0; }
AIGPU_ABI int aigpu_gated_delta_rule_host(const AiGpuDeltaRule*) { return 0; }
AIGPU_ABI int aigpu_gdn_conv(const AiGpuGdnConv*) { return 0; }
AIGPU_ABI int aigpu_kda_rule(const AiGpuKda*) { return 0; }
AIGPU_ABI void aigpu_matmul_nt(const float*, const void*, float*, uint64_t, uint64_t, uint64_t) {}
AIGPU_ABI void aigpu_matmul_nt_bf16(const float*, const void*, float*, uint64_t, uint64_t, uint64_t) {}
AIGPU_ABI void aigpu_matmul_nt_q8(const float*, const void*, const void*, float*, uint64_t, uint64_t, uint64_t) {}
AIGPU_ABI void aigpu_matmul_nt_q4(const float*, const void*, const void*, float*, uint64_t, uint64_t, uint64_t) {}
AIGPU_ABI int aigpu_matmul_device(const AiGpuMatmul*) { return 0; }
AIGPU_ABI int aigpu_latent_attention(const AiGpuLatentAttention*) { return 0; }
AIGPU_ABI int aigpu_prefill_mixer(const AiGpuPrefillMixer*) { return 0; }
AIGPU_ABI int aigpu_select_keys(const AiGpuSelectKeys*) { return 0; }
AIGPU_ABI int aigpu_dense_supported(void) { return 0; }
AIGPU_ABI void* aigpu_dense_create(const AiGpuDenseConfig*, const AiGpuDenseLayer*, const float* const*,
                                   const float* const*, uint32_t) { return nullptr; }
AIGPU_ABI void aigpu_dense_release(void*) {}
AIGPU_ABI void aigpu_dense_decode(void*, const float*, float*, uint32_t) {}
AIGPU_ABI void aigpu_dense_read_cache(void*, float* const*, float* const*, uint32_t) {}
AIGPU_ABI int aigpu_gdn_gated_norm(const AiGpuGdnGatedNorm*) { return 0; }

AIGPU_ABI void aigpu_profile(int) {}
AIGPU_ABI int aigpu_profile_read(const char*, double* ms, uint64_t* n) {
    if (ms) *ms = 0.0;
    if (n) *n = 0;
    return 0;
}
AIGPU_ABI void aigpu_profile_reset(void) {}

} // extern "C"
