// Launchers of the throughput kernels and their pre-passes.
#include "hot_kernels.h"

namespace lard {

// One workgroup per sequence b: tok_ok[b][j] = (j < T && mask[b][j] != 0)
// for j < Tp (four tokens per thread and store), and first2[b] = the first
// and second valid token of the sequence (T where there is none).
constexpr int kPrepThreads = 1024;

__device__ __forceinline__ void two_smallest(int& f0, int& f1, int g0, int g1) {  // merge two sorted pairs
  const int lo = min(f0, g0);
  f1 = min(max(f0, g0), min(f1, g1));
  f0 = lo;
}

__global__ __launch_bounds__(kPrepThreads) void token_prep_kernel(const RelArgs a, int Tp,
                                                                  unsigned char* __restrict__ tok_ok,
                                                                  int* __restrict__ first2) {
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  int f0 = a.T, f1 = a.T;  // this thread's two smallest valid tokens (it visits them in order)
  for (int j0 = 4 * tid; j0 < Tp; j0 += 4 * kPrepThreads) {
    unsigned word = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = j0 + e;
      if (j < a.T && mask_at(a.mask, a.mask_kind, (int64_t)b * a.mask_sb + j)) {
        word |= 1u << (8 * e);
        if (f0 == a.T)
          f0 = j;
        else if (f1 == a.T)
          f1 = j;
      }
    }
    *reinterpret_cast<unsigned*>(tok_ok + (int64_t)b * Tp + j0) = word;  // Tp is a multiple of 64
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) two_smallest(f0, f1, __shfl_xor(f0, o, 64), __shfl_xor(f1, o, 64));
  __shared__ int part[2][kPrepThreads / 64];
  if ((tid & 63) == 0) {
    part[0][tid >> 6] = f0;
    part[1][tid >> 6] = f1;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kPrepThreads / 64; ++w) two_smallest(f0, f1, part[0][w], part[1][w]);
    first2[2 * b] = f0;
    first2[2 * b + 1] = f1;
  }
}

// nl_x[bh][i] = -lse_x[bh][i] * log2(e) for rows in the valid set (token valid
// and both LSEs finite, kernel_C.py:155-161), -inf otherwise and for i >= T.
// A row with exactly one valid key also gets -inf: there P_s = P_t = 1, so
// its D is exactly 0 (kernel_C.py:224-233 with lse == S), which the
// normalisers then give without any rounding of S * c2 - lse * log2(e).
__global__ __launch_bounds__(256) void row_prep_kernel(const RelArgs a, int Tp, const unsigned char* __restrict__ tok_ok,
                                                       const int* __restrict__ first2, float* __restrict__ nl_s,
                                                       float* __restrict__ nl_t) {
  const int i = blockIdx.x * 256 + (int)threadIdx.x;
  const int64_t bh = blockIdx.y;
  if (i >= Tp) return;
  const int b = (int)(bh / a.Hq);
  bool ok = false;
  float ls = 0.f, lt = 0.f;
  if (i < a.T) {
    ls = a.lse_s_in[bh * a.T + i];
    lt = a.lse_t_in[bh * a.T + i];
    const bool one_key = a.causal ? i == first2[2 * b] : first2[2 * b + 1] >= a.T;
    ok = tok_ok[(int64_t)b * Tp + i] != 0 && ls != kNegInf && lt != kNegInf && !one_key;
  }
  nl_s[bh * Tp + i] = ok ? -ls * kLog2e : kNegInf;
  nl_t[bh * Tp + i] = ok ? -lt * kLog2e : kNegInf;
}

bool hot_supported(int ds, int dt, bool same_dtype) { return same_dtype && ds == dt && ds <= 128; }

hipError_t launch_token_prep(const RelArgs& a, int Tp, unsigned char* tok_ok, int* first2, hipStream_t stream) {
  hipLaunchKernelGGL(token_prep_kernel, dim3(a.B), dim3(kPrepThreads), 0, stream, a, Tp, tok_ok, first2);
  return hipGetLastError();
}

hipError_t launch_row_prep(const RelArgs& a, int Tp, const unsigned char* tok_ok, const int* first2, float* nl_s,
                           float* nl_t, hipStream_t stream) {
  hipLaunchKernelGGL(row_prep_kernel, dim3((Tp + 255) / 256, a.B * a.Hq), dim3(256), 0, stream, a, Tp, tok_ok, first2,
                     nl_s, nl_t);
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
