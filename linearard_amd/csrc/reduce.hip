// Deterministic sum of the per-row KL terms into the 0-d loss.  The
// reference adds one fp32 atomic per program into a shared scalar
// (kernel_B.py:216-218), whose order is nondeterministic; here the sum runs
// in a fixed order in double precision: kReduceBlocks workgroups each sum a
// contiguous slice into one partial, then one workgroup sums the partials.
#include "stage_kernels.h"

namespace lard {

constexpr int kReduceThreads = 256;

__device__ __forceinline__ double block_sum(double s, double* part) {
  part[threadIdx.x] = s;
  __syncthreads();
  for (int stride = kReduceThreads / 2; stride > 0; stride >>= 1) {
    if ((int)threadIdx.x < stride) part[threadIdx.x] += part[threadIdx.x + stride];
    __syncthreads();
  }
  return part[0];
}

__global__ __launch_bounds__(kReduceThreads) void reduce_partial_kernel(const float* __restrict__ x, int64_t n,
                                                                        double* __restrict__ partial) {
  __shared__ double part[kReduceThreads];
  const int64_t per = (n + kReduceBlocks - 1) / kReduceBlocks;
  const int64_t lo = per * blockIdx.x;
  const int64_t hi = lo + per < n ? lo + per : n;
  double s = 0.0;
  for (int64_t i = lo + threadIdx.x; i < hi; i += kReduceThreads) s += (double)x[i];
  const double total = block_sum(s, part);
  if (threadIdx.x == 0) partial[blockIdx.x] = total;
}

__global__ __launch_bounds__(kReduceThreads) void reduce_final_kernel(const double* __restrict__ partial,
                                                                      float* __restrict__ out) {
  __shared__ double part[kReduceThreads];
  double s = 0.0;
  for (int i = threadIdx.x; i < kReduceBlocks; i += kReduceThreads) s += partial[i];
  const double total = block_sum(s, part);
  if (threadIdx.x == 0) out[0] = (float)total;
}

__global__ __launch_bounds__(kReduceThreads) void reduce_zero_kernel(float* __restrict__ out) {
  if (threadIdx.x == 0) out[0] = 0.f;
}

hipError_t launch_reduce_sum(const float* x, int64_t n, double* partial, float* out, hipStream_t stream) {
  if (n <= 0) {
    hipLaunchKernelGGL(reduce_zero_kernel, dim3(1), dim3(kReduceThreads), 0, stream, out);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(reduce_partial_kernel, dim3(kReduceBlocks), dim3(kReduceThreads), 0, stream, x, n, partial);
  hipLaunchKernelGGL(reduce_final_kernel, dim3(1), dim3(kReduceThreads), 0, stream, partial, out);
  return hipGetLastError();
}

__global__ __launch_bounds__(kReduceThreads) void scale_inplace_kernel(float* __restrict__ x, int64_t n4,
                                                                        const float* __restrict__ dscale) {
  const float s = *dscale;
  f32x4* v = reinterpret_cast<f32x4*>(x);
  for (int64_t i = (int64_t)blockIdx.x * kReduceThreads + threadIdx.x; i < n4; i += (int64_t)gridDim.x * kReduceThreads)
    v[i] *= s;
}

hipError_t launch_scale_inplace(float* x, int64_t n, const float* dscale, hipStream_t stream) {
  if (n <= 0 || dscale == nullptr) return hipSuccess;
  const int64_t n4 = n / 4;
  const int64_t want = (n4 + kReduceThreads - 1) / kReduceThreads;
  const int blocks = (int)(want < 4096 ? want : 4096);
  hipLaunchKernelGGL(scale_inplace_kernel, dim3(blocks), dim3(kReduceThreads), 0, stream, x, n4, dscale);
  return hipGetLastError();
}

}  // namespace lard
