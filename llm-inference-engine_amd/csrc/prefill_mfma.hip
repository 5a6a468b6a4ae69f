// MFMA prefill attention for 16-bit KV caches (gfx950). Not yet enabled:
// prefill_mfma_enabled() returns false and the VALU kernel runs.
#include "common.hpp"
#include "prefill.hpp"

namespace iehip {

bool prefill_mfma_enabled() { return false; }

int prefill_mfma_launch(float*, const float*, const void*, const void*, int, const int32_t*,
                        const int32_t*, const ie_kv_layout&, int, int, hipStream_t) {
  return fail(IE_HIP_EINVAL, "attention_prefill: MFMA path not built");
}

}  // namespace iehip
