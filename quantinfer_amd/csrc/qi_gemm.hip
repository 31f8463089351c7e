// Prefill GEMM (M >= 128) on MFMA. Not yet enabled: every call falls back to
// the f32 GEMV path until the kernel lands.
#include "qi_internal.h"

namespace qi {

bool gemm_supported(int32_t, int32_t, uint64_t, uint64_t) { return false; }

hipError_t launch_gemm(const Image&, const GemmArgs&, hipStream_t) { return hipErrorNotSupported; }

}  // namespace qi
