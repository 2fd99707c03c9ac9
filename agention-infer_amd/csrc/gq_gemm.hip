// gq_gemm.hip -- batched prefill GEMM (placeholder until the MFMA kernels land).
#include "gq_device.h"
#include "gq_internal.h"

namespace gq {
size_t gemm_workspace_bytes(const gq_weight *, int, int) { return (size_t)-1; }
hipError_t launch_gemm(const gq_weight *, const float *, int, float *, int, void *, size_t, int,
                       hipStream_t) {
  return hipErrorNotSupported;
}
}  // namespace gq
