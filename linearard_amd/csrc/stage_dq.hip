// Stage C row-side launcher: dq (kernel_C.py:388-447).
#include "stage_kernels.h"
#include "stage_dispatch.h"
#include "stage_f32.h"

namespace lard {

template <int DPS>
static hipError_t launch_dq(const RelArgs& a, int dpt, dim3 grid, hipStream_t stream) {
  switch (dpt) {
#define X(DP, unused) \
  case DP: hipLaunchKernelGGL((row_kernel<MODE_DQ, DPS, DP>), grid, dim3(kStageThreads), 0, stream, a); break;
    LARD_DP_CASES(X, 0)
#undef X
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_row_dq(const RelArgs& a, int dps, int dpt, hipStream_t stream) {
  if (a.s.f32) return launch_row_dq_f32(a, stream);  // float32 inputs (both sides)
  const dim3 grid((a.T + kStageRows - 1) / kStageRows, a.B * a.Hq);
  switch (dps) {
#define X(DP, unused) \
  case DP: return launch_dq<DP>(a, dpt, grid, stream);
    LARD_DP_CASES(X, 0)
#undef X
    default: return hipErrorInvalidValue;
  }
}

}  // namespace lard
