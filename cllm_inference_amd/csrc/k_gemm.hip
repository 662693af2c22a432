// k_gemm.hip -- int8-MFMA prefill GEMM (not yet implemented: every type routes to the GEMV).
#include "launch.h"

namespace cllm_hip {

bool gemm_supported(uint32_t) { return false; }

hipError_t launch_gemm(uint32_t, const uint8_t*, int, int, int, const int8_t*, const float*,
                       const int32_t*, const float*, float*, hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace cllm_hip
