// Launcher of the fused forward (AttnKLAlignFn.forward, integration.py:8-45).
#include "fused_kernels.h"

namespace lard {

bool fused_fwd_supported(int ds, int dt, bool same_dtype) { return same_dtype && ds == dt; }

bool fused_fwd_grad_supported(int d) { return d <= 128; }

template <bool BF, bool GRAD>
static hipError_t launch_fused(const FusedArgs& f, int dp, dim3 grid, hipStream_t stream) {
  switch (dp) {
    case 16: hipLaunchKernelGGL((fused_fwd_kernel<16, BF, GRAD>), grid, dim3(kStageThreads), 0, stream, f); break;
    case 32: hipLaunchKernelGGL((fused_fwd_kernel<32, BF, GRAD>), grid, dim3(kStageThreads), 0, stream, f); break;
    case 64: hipLaunchKernelGGL((fused_fwd_kernel<64, BF, GRAD>), grid, dim3(kStageThreads), 0, stream, f); break;
    case 128: hipLaunchKernelGGL((fused_fwd_kernel<128, BF, GRAD>), grid, dim3(kStageThreads), 0, stream, f); break;
    case 256:
      // the two fp32 gradient accumulators do not fit the register file at
      // D = 256; that shape takes its dq from the stage C row kernel instead
      if constexpr (GRAD) return hipErrorInvalidValue;
      hipLaunchKernelGGL((fused_fwd_kernel<256, BF, false>), grid, dim3(kStageThreads), 0, stream, f);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_fused_fwd(const FusedArgs& f, int dp, bool bf16, bool grad, hipStream_t stream) {
  const dim3 grid((f.r.T + kStageRows - 1) / kStageRows, f.r.B * f.r.Hq);
  if (bf16) return grad ? launch_fused<true, true>(f, dp, grid, stream) : launch_fused<true, false>(f, dp, grid, stream);
  return grad ? launch_fused<false, true>(f, dp, grid, stream) : launch_fused<false, false>(f, dp, grid, stream);
}

}  // namespace lard
