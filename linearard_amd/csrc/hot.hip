// Launchers of the throughput kernels and the transposed-key pre-pass.
#include "hot_kernels.h"

namespace lard {

// xT[bh][d][t'] = x[bh][t][d] with t' the sigma-permuted position of t inside
// its group of 16 keys; positions >= T are zero.  One workgroup per 64 keys.
__global__ __launch_bounds__(256) void transpose_keys_kernel(const u16* __restrict__ x, int64_t sb, int64_t sh,
                                                             int64_t st, int H, int T, int D, int Tp,
                                                             u16* __restrict__ xT) {
  constexpr int LDS_W = 128 + 8;
  __shared__ __attribute__((aligned(16))) u16 tile[kTile * LDS_W];
  const int t0 = blockIdx.x * kTile;
  const int bh = blockIdx.y;
  const int b = bh / H, h = bh - b * H;
  const u16* src = x + (int64_t)b * sb + (int64_t)h * sh;
  const int cpr = D / 8;
  for (int c = threadIdx.x; c < kTile * cpr; c += 256) {
    const int r = c / cpr, dc = (c % cpr) * 8;
    const int t = t0 + r;
    u16x8 v = (u16x8)(0);
    if (t < T) v = *reinterpret_cast<const u16x8*>(src + (int64_t)t * st + dc);
    *reinterpret_cast<u16x8*>(tile + r * LDS_W + dc) = v;
  }
  __syncthreads();
  u16* dst = xT + (int64_t)bh * D * Tp + t0;
  for (int c = threadIdx.x; c < D * 8; c += 256) {
    const int d = c >> 3, p0 = (c & 7) * 8;  // 8 output positions p0..p0+7
    u16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int p = p0 + e;
      const int q = p & 15;
      const int key = (p & ~15) + (q < 4 || q >= 12 ? q : (q < 8 ? q + 4 : q - 4));
      v[e] = tile[key * LDS_W + d];
    }
    *reinterpret_cast<u16x8*>(dst + (int64_t)d * Tp + p0) = v;
  }
}

bool hot_supported(int ds, int dt, bool same_dtype) { return same_dtype && ds == dt && ds <= 128; }

hipError_t launch_transpose_keys(const u16* x, int64_t sb, int64_t sh, int64_t st, int B, int H, int T, int D, int Tp,
                                 u16* xT, hipStream_t stream) {
  hipLaunchKernelGGL(transpose_keys_kernel, dim3(Tp / kTile, B * H), dim3(256), 0, stream, x, sb, sh, st, H, T, D,
                     Tp, xT);
  return hipGetLastError();
}

template <bool BF>
static hipError_t fwd_dispatch(const HotArgs& f, int dp, dim3 grid, hipStream_t stream) {
  const dim3 block(kFwdWaves * 64);
  switch (dp) {
    case 16: hipLaunchKernelGGL((hot_fwd_kernel<16, BF>), grid, block, 0, stream, f); break;
    case 32: hipLaunchKernelGGL((hot_fwd_kernel<32, BF>), grid, block, 0, stream, f); break;
    case 64: hipLaunchKernelGGL((hot_fwd_kernel<64, BF>), grid, block, 0, stream, f); break;
    case 128: hipLaunchKernelGGL((hot_fwd_kernel<128, BF>), grid, block, 0, stream, f); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_hot_fwd(const HotArgs& f, int dp, bool bf16, hipStream_t stream) {
  const int rows = kFwdWaves * 32;
  const dim3 grid((f.r.T + rows - 1) / rows, f.r.B * f.r.Hq);
  return bf16 ? fwd_dispatch<true>(f, dp, grid, stream) : fwd_dispatch<false>(f, dp, grid, stream);
}

template <bool BF>
static hipError_t dq_dispatch(const HotArgs& f, int dp, dim3 grid, hipStream_t stream) {
  const dim3 block(kDqWaves * 64);
  switch (dp) {
    case 16: hipLaunchKernelGGL((hot_dq_kernel<16, BF>), grid, block, 0, stream, f); break;
    case 32: hipLaunchKernelGGL((hot_dq_kernel<32, BF>), grid, block, 0, stream, f); break;
    case 64: hipLaunchKernelGGL((hot_dq_kernel<64, BF>), grid, block, 0, stream, f); break;
    case 128: hipLaunchKernelGGL((hot_dq_kernel<128, BF>), grid, block, 0, stream, f); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_hot_dq(const HotArgs& f, int dp, bool bf16, hipStream_t stream) {
  const int rows = kDqWaves * 32;
  const dim3 grid((f.r.T + rows - 1) / rows, f.r.B * f.r.Hq);
  return bf16 ? dq_dispatch<true>(f, dp, grid, stream) : dq_dispatch<false>(f, dp, grid, stream);
}

template <bool BF>
static hipError_t bwd_dispatch(const HotArgs& f, int dp, dim3 grid, hipStream_t stream) {
  const dim3 block(kBwdWaves * 64);
  switch (dp) {
    case 16: hipLaunchKernelGGL((hot_bwd_kernel<16, BF>), grid, block, 0, stream, f); break;
    case 32: hipLaunchKernelGGL((hot_bwd_kernel<32, BF>), grid, block, 0, stream, f); break;
    case 64: hipLaunchKernelGGL((hot_bwd_kernel<64, BF>), grid, block, 0, stream, f); break;
    case 128: hipLaunchKernelGGL((hot_bwd_kernel<128, BF>), grid, block, 0, stream, f); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_hot_bwd(const HotArgs& f, int dp, bool bf16, hipStream_t stream) {
  const dim3 grid((f.r.T + kBwdWaves * 32 - 1) / (kBwdWaves * 32), f.r.B * f.r.s.hkv);
  return bf16 ? bwd_dispatch<true>(f, dp, grid, stream) : bwd_dispatch<false>(f, dp, grid, stream);
}

}  // namespace lard
