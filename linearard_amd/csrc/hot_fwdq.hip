// Launchers of the fused forward with the row-side gradient (hot_fwdq.h).
#include "hot_fwdq.h"

namespace lard {

namespace {

template <bool BF>
hipError_t fwdq_dispatch(const HotArgs& f, int dp, int nblocks, hipStream_t stream) {
  const dim3 grid(nblocks), block(kWavesQ * 64);
  switch (dp) {
    case 16: hipLaunchKernelGGL((hot_fwdq_kernel<16, BF>), grid, block, 0, stream, f); break;
    case 32: hipLaunchKernelGGL((hot_fwdq_kernel<32, BF>), grid, block, 0, stream, f); break;
    case 64: hipLaunchKernelGGL((hot_fwdq_kernel<64, BF>), grid, block, 0, stream, f); break;
    case 128: hipLaunchKernelGGL((hot_fwdq_kernel<128, BF>), grid, block, 0, stream, f); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <bool BF>
hipError_t fwdq_batch_dispatch(const HotBatch& m, int dp, hipStream_t stream) {
  const dim3 grid(m.first[m.n]), block(kWavesQ * 64);
  switch (dp) {
    case 16: hipLaunchKernelGGL((hot_fwdq_batch_kernel<16, BF>), grid, block, 0, stream, m); break;
    case 32: hipLaunchKernelGGL((hot_fwdq_batch_kernel<32, BF>), grid, block, 0, stream, m); break;
    case 64: hipLaunchKernelGGL((hot_fwdq_batch_kernel<64, BF>), grid, block, 0, stream, m); break;
    case 128: hipLaunchKernelGGL((hot_fwdq_batch_kernel<128, BF>), grid, block, 0, stream, m); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_hot_fwdq(const HotArgs& f, int dp, bool bf16, hipStream_t stream) {
  const int n = fwdq_items(f);
  return bf16 ? fwdq_dispatch<true>(f, dp, n, stream) : fwdq_dispatch<false>(f, dp, n, stream);
}

// first[] from the relations' work items; an error if the batch is empty,
// too large or its grid would not fit an int.
hipError_t launch_hot_fwdq_batch(HotBatch& m, int dp, bool bf16, hipStream_t stream) {
  if (m.n < 1 || m.n > kMaxRelations) return hipErrorInvalidValue;
  int64_t total = 0;
  for (int r = 0; r < m.n; ++r) {
    m.first[r] = (int)total;
    total += fwdq_items(m.rel[r]);
    if (total > INT32_MAX) return hipErrorInvalidValue;
  }
  m.first[m.n] = (int)total;
  if (total == 0) return hipErrorInvalidValue;
  return bf16 ? fwdq_batch_dispatch<true>(m, dp, stream) : fwdq_batch_dispatch<false>(m, dp, stream);
}

}  // namespace lard
