// Stage A launcher: row log-sum-exp (kernel_A.py:232-263).
#include "stage_kernels.h"
#include "stage_dispatch.h"
#include "stage_f32.h"

namespace lard {

hipError_t launch_row_lse(const RelArgs& a, int dps, hipStream_t stream) {
  if (a.s.f32) return launch_row_lse_f32(a, stream);  // float32 inputs (both sides)
  const dim3 grid((a.T + kStageRows - 1) / kStageRows, a.B * a.Hq);
  switch (dps) {
#define X(DP, unused) \
  case DP: hipLaunchKernelGGL((row_kernel<MODE_LSE, DP, 16>), grid, dim3(kStageThreads), 0, stream, a); break;
    LARD_DP_CASES(X, 0)
#undef X
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace lard
