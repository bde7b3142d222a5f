// Launcher of the generic fused forward (LSEs and KL in one pass) used for
// head dims the throughput kernels do not cover (Ds == Dt == 256).
#include "fused_kernels.h"

namespace lard {

bool fused_fwd_supported(int ds, int dt, bool same_dtype) { return same_dtype && ds == dt; }

template <bool BF>
static hipError_t launch_fused(const FusedArgs& f, int dp, dim3 grid, hipStream_t stream) {
  switch (dp) {
    case 16: hipLaunchKernelGGL((fused_fwd_kernel<16, BF>), grid, dim3(kStageThreads), 0, stream, f); break;
    case 32: hipLaunchKernelGGL((fused_fwd_kernel<32, BF>), grid, dim3(kStageThreads), 0, stream, f); break;
    case 64: hipLaunchKernelGGL((fused_fwd_kernel<64, BF>), grid, dim3(kStageThreads), 0, stream, f); break;
    case 128: hipLaunchKernelGGL((fused_fwd_kernel<128, BF>), grid, dim3(kStageThreads), 0, stream, f); break;
    case 256: hipLaunchKernelGGL((fused_fwd_kernel<256, BF>), grid, dim3(kStageThreads), 0, stream, f); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_fused_fwd(const FusedArgs& f, int dp, bool bf16, hipStream_t stream) {
  const dim3 grid((f.r.T + kStageRows - 1) / kStageRows, f.r.B * f.r.Hq);
  return bf16 ? launch_fused<true>(f, dp, grid, stream) : launch_fused<false>(f, dp, grid, stream);
}

}  // namespace lard
