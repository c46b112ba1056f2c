// Paged chunked-prefill attention on MFMA (placeholder until the bf16 tile
// kernel lands; the f32 path of tvara_attn_prefill does not use this file).
#include "common.hpp"

namespace tvara_amd {

bool prefill_bf16_supported(const BlockLayout&, int) { return false; }

void launch_prefill_bf16(const PrefillArgs&, int, int, hipStream_t) {
    throw std::runtime_error("bf16 prefill is not available in this build");
}

}  // namespace tvara_amd
