// Deterministic sum of the per-row KL terms into the 0-d loss.  The
// reference adds one fp32 atomic per program into a shared scalar
// (kernel_B.py:216-218), whose order is nondeterministic; here one
// workgroup sums in a fixed order in double precision.
#include "stage_kernels.h"

namespace lard {

constexpr int kReduceThreads = 1024;

__global__ __launch_bounds__(kReduceThreads) void reduce_sum_kernel(const float* __restrict__ x, int64_t n,
                                                                    float* __restrict__ out) {
  __shared__ double part[kReduceThreads];
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += kReduceThreads) s += (double)x[i];
  part[threadIdx.x] = s;
  __syncthreads();
  for (int stride = kReduceThreads / 2; stride > 0; stride >>= 1) {
    if ((int)threadIdx.x < stride) part[threadIdx.x] += part[threadIdx.x + stride];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[0] = (float)part[0];
}

hipError_t launch_reduce_sum(const float* x, int64_t n, float* out, hipStream_t stream) {
  hipLaunchKernelGGL(reduce_sum_kernel, dim3(1), dim3(kReduceThreads), 0, stream, x, n, out);
  return hipGetLastError();
}

}  // namespace lard
