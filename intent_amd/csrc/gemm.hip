// bf16 GEMM (placeholder until the MFMA kernel lands).
#include "common.hpp"

namespace intent_hip {
int gemm_resources(int64_t, int64_t, IntentHipKernelResources *) {
  return fail(INTENT_HIP_ERR_UNSUPPORTED, "bf16 GEMM is not built yet");
}
}  // namespace intent_hip

extern "C" int intent_hip_gemm_bf16(const void *, const void *, void *, int64_t, int64_t, int64_t, int64_t,
                                    int64_t, int64_t, void *) {
  return intent_hip::fail(INTENT_HIP_ERR_UNSUPPORTED, "bf16 GEMM is not built yet");
}
