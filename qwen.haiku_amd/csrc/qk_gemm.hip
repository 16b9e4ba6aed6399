// qk_gemm.hip -- chunked-prefill GEMM (int8 MFMA). Placeholder until the
// MFMA kernel lands: reports "not supported".
#include "qk_dev.h"
#include "qk_kernels.h"

namespace qk {
hipError_t launch_gemm(int, const uint8_t *, int64_t, int64_t, const uint8_t *, int64_t, float *,
                       int, hipStream_t) {
    return hipErrorNotSupported;
}
}  // namespace qk
