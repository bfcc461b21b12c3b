// Attention forward (placeholder until the MFMA kernel lands).
#include "common.hpp"

namespace intent_hip {
int attention_resources(int64_t, int64_t, IntentHipKernelResources *) {
  return fail(INTENT_HIP_ERR_UNSUPPORTED, "attention is not built yet");
}
}  // namespace intent_hip

extern "C" int intent_hip_attention_fwd_f16(const void *, const void *, const void *, void *, int64_t, int64_t,
                                            int64_t, int64_t, int64_t, int64_t, const int64_t *, float, int,
                                            void *) {
  return intent_hip::fail(INTENT_HIP_ERR_UNSUPPORTED, "attention is not built yet");
}
