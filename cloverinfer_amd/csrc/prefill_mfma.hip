// prefill_mfma.hip - MFMA chunked prefill (fp16/bf16).
#include "attn_common.h"

namespace clv {

bool prefill_mfma_supported(DType, int, int) { return false; }

hipError_t launch_prefill_mfma(const PrefillParams &, DType, hipStream_t) {
  return hipErrorInvalidValue;
}

}  // namespace clv
