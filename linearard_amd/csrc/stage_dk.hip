// Stage C column-side launcher: dk summed over the GQA group, one owner per
// key tile, no atomics (replaces the atomic_add of kernel_C.py:242-253).
#include "stage_kernels.h"
#include "stage_dispatch.h"
#include "stage_f32.h"

namespace lard {

template <int DPS>
static hipError_t launch_dk(const RelArgs& a, int dpt, dim3 grid, hipStream_t stream) {
  switch (dpt) {
#define X(DP, unused) \
  case DP: hipLaunchKernelGGL((col_kernel<DPS, DP>), grid, dim3(kStageThreads), 0, stream, a); break;
    LARD_DP_CASES(X, 0)
#undef X
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_col_dk(const RelArgs& a, int dps, int dpt, hipStream_t stream) {
  if (a.s.f32) return launch_col_dk_f32(a, stream);  // float32 inputs (both sides)
  const dim3 grid((a.T + kStageRows - 1) / kStageRows, a.B * a.s.hkv);
  switch (dps) {
#define X(DP, unused) \
  case DP: return launch_dk<DP>(a, dpt, grid, stream);
    LARD_DP_CASES(X, 0)
#undef X
    default: return hipErrorInvalidValue;
  }
}

}  // namespace lard
