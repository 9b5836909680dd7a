// okq_gemm.hip -- MFMA dequant-GEMM for prefill (placeholder until the
// MFMA kernels land; gemm_supported() reports no shape).
#include "okq_device.h"
#include "okq_internal.h"

namespace okq {

bool gemm_supported(int, int64_t, int64_t) { return false; }

hipError_t launch_gemm(int, const void *, bool, int64_t, int64_t, const void *, int64_t, const float *, float *, int,
                       hipStream_t) {
  return hipErrorNotSupported;
}

}  // namespace okq
