// Launchers of the throughput kernels and their pre-passes.
#include "hot_kernels.h"

namespace lard {

// tok_ok[b][j] = (j < T && mask[b][j] != 0) for j < Tp.
__global__ __launch_bounds__(256) void token_prep_kernel(const RelArgs a, int Tp, unsigned char* __restrict__ tok_ok) {
  const int j = blockIdx.x * 256 + (int)threadIdx.x;
  const int b = blockIdx.y;
  if (j >= Tp) return;
  const bool v = j < a.T && mask_at(a.mask, a.mask_kind, (int64_t)b * a.mask_sb + j);
  tok_ok[(int64_t)b * Tp + j] = v ? 1 : 0;
}

// nl_x[bh][i] = -lse_x[bh][i] * log2(e) for rows in the valid set (token valid
// and both LSEs finite, kernel_C.py:155-161), -inf otherwise and for i >= T.
__global__ __launch_bounds__(256) void row_prep_kernel(const RelArgs a, int Tp, const unsigned char* __restrict__ tok_ok,
                                                       float* __restrict__ nl_s, float* __restrict__ nl_t) {
  const int i = blockIdx.x * 256 + (int)threadIdx.x;
  const int64_t bh = blockIdx.y;
  if (i >= Tp) return;
  const int b = (int)(bh / a.Hq);
  bool ok = false;
  float ls = 0.f, lt = 0.f;
  if (i < a.T) {
    ls = a.lse_s_in[bh * a.T + i];
    lt = a.lse_t_in[bh * a.T + i];
    ok = tok_ok[(int64_t)b * Tp + i] != 0 && ls != kNegInf && lt != kNegInf;
  }
  nl_s[bh * Tp + i] = ok ? -ls * kLog2e : kNegInf;
  nl_t[bh * Tp + i] = ok ? -lt * kLog2e : kNegInf;
}

bool hot_supported(int ds, int dt, bool same_dtype) { return same_dtype && ds == dt && ds <= 128; }

hipError_t launch_token_prep(const RelArgs& a, int Tp, unsigned char* tok_ok, hipStream_t stream) {
  hipLaunchKernelGGL(token_prep_kernel, dim3((Tp + 255) / 256, a.B), dim3(256), 0, stream, a, Tp, tok_ok);
  return hipGetLastError();
}

hipError_t launch_row_prep(const RelArgs& a, int Tp, const unsigned char* tok_ok, float* nl_s, float* nl_t,
                           hipStream_t stream) {
  hipLaunchKernelGGL(row_prep_kernel, dim3((Tp + 255) / 256, a.B * a.Hq), dim3(256), 0, stream, a, Tp, tok_ok, nl_s,
                     nl_t);
  return hipGetLastError();
}

// One flat grid; the kernels map blockIdx.x to work items with xcd_item().
#define LARD_HOT_DISPATCH(KERNEL)                                                                    \
  template <bool BF>                                                                                 \
  static hipError_t KERNEL##_dispatch(const HotArgs& f, int dp, int nblocks, hipStream_t stream) {  \
    const dim3 grid(nblocks), block(kWaves * 64);                                                    \
    switch (dp) {                                                                                    \
      case 16: hipLaunchKernelGGL((KERNEL<16, BF>), grid, block, 0, stream, f); break;               \
      case 32: hipLaunchKernelGGL((KERNEL<32, BF>), grid, block, 0, stream, f); break;               \
      case 64: hipLaunchKernelGGL((KERNEL<64, BF>), grid, block, 0, stream, f); break;               \
      case 128: hipLaunchKernelGGL((KERNEL<128, BF>), grid, block, 0, stream, f); break;             \
      default: return hipErrorInvalidValue;                                                          \
    }                                                                                                \
    return hipGetLastError();                                                                        \
  }

LARD_HOT_DISPATCH(hot_fwd_kernel)
LARD_HOT_DISPATCH(hot_dq_kernel)
LARD_HOT_DISPATCH(hot_bwd_kernel)
#undef LARD_HOT_DISPATCH

#define LARD_HOT_BATCH_DISPATCH(KERNEL)                                                              \
  template <bool BF>                                                                                 \
  static hipError_t KERNEL##_dispatch(const HotBatch& m, int dp, hipStream_t stream) {              \
    const dim3 grid(m.first[m.n]), block(kWaves * 64);                                               \
    switch (dp) {                                                                                    \
      case 16: hipLaunchKernelGGL((KERNEL<16, BF>), grid, block, 0, stream, m); break;               \
      case 32: hipLaunchKernelGGL((KERNEL<32, BF>), grid, block, 0, stream, m); break;               \
      case 64: hipLaunchKernelGGL((KERNEL<64, BF>), grid, block, 0, stream, m); break;               \
      case 128: hipLaunchKernelGGL((KERNEL<128, BF>), grid, block, 0, stream, m); break;             \
      default: return hipErrorInvalidValue;                                                          \
    }                                                                                                \
    return hipGetLastError();                                                                        \
  }

LARD_HOT_BATCH_DISPATCH(hot_fwd_batch_kernel)
LARD_HOT_BATCH_DISPATCH(hot_dq_batch_kernel)
LARD_HOT_BATCH_DISPATCH(hot_bwd_batch_kernel)
#undef LARD_HOT_BATCH_DISPATCH

// first[] from the relations' work items; false if the batch is empty,
// too large or its grid would not fit an int.
static bool batch_prefix(HotBatch& m, bool column_side) {
  if (m.n < 1 || m.n > kMaxRelations) return false;
  int64_t total = 0;
  for (int r = 0; r < m.n; ++r) {
    m.first[r] = (int)total;
    total += column_side ? bwd_items(m.rel[r]) : fwd_items(m.rel[r]);
    if (total > INT32_MAX) return false;
  }
  m.first[m.n] = (int)total;
  return total > 0;
}

hipError_t launch_hot_fwd_batch(HotBatch& m, int dp, bool bf16, hipStream_t stream) {
  if (!batch_prefix(m, false)) return hipErrorInvalidValue;
  return bf16 ? hot_fwd_batch_kernel_dispatch<true>(m, dp, stream) : hot_fwd_batch_kernel_dispatch<false>(m, dp, stream);
}

hipError_t launch_hot_dq_batch(HotBatch& m, int dp, bool bf16, hipStream_t stream) {
  if (!batch_prefix(m, false)) return hipErrorInvalidValue;
  return bf16 ? hot_dq_batch_kernel_dispatch<true>(m, dp, stream) : hot_dq_batch_kernel_dispatch<false>(m, dp, stream);
}

hipError_t launch_hot_bwd_batch(HotBatch& m, int dp, bool bf16, hipStream_t stream) {
  if (!batch_prefix(m, true)) return hipErrorInvalidValue;
  return bf16 ? hot_bwd_batch_kernel_dispatch<true>(m, dp, stream) : hot_bwd_batch_kernel_dispatch<false>(m, dp, stream);
}

static int row_blocks(const RelArgs& a, int heads) { return (a.T + kRows - 1) / kRows * a.B * heads; }

hipError_t launch_hot_fwd(const HotArgs& f, int dp, bool bf16, hipStream_t stream) {
  const int n = row_blocks(f.r, f.r.Hq);
  return bf16 ? hot_fwd_kernel_dispatch<true>(f, dp, n, stream) : hot_fwd_kernel_dispatch<false>(f, dp, n, stream);
}

hipError_t launch_hot_dq(const HotArgs& f, int dp, bool bf16, hipStream_t stream) {
  const int n = row_blocks(f.r, f.r.Hq);
  return bf16 ? hot_dq_kernel_dispatch<true>(f, dp, n, stream) : hot_dq_kernel_dispatch<false>(f, dp, n, stream);
}

hipError_t launch_hot_bwd(const HotArgs& f, int dp, bool bf16, hipStream_t stream) {
  const int n = row_blocks(f.r, f.r.s.hkv);
  return bf16 ? hot_bwd_kernel_dispatch<true>(f, dp, n, stream) : hot_bwd_kernel_dispatch<false>(f, dp, n, stream);
}

}  // namespace lard
