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

// ---- the keys as float16 (bfloat16 inputs) ----
//
// One scale per side (student, teacher): s = 2^-e, the smallest e >= 0 with
// max |x| * s < 2^15 over q and k, so the float16 operands stay finite (a
// bfloat16 value below 2^15 is exactly a float16 value, down to 2^-17 in
// magnitude), e <= kMaxScaleExp (values of 2^55 and more are beyond this
// path: they would overflow float16 even scaled).
// Three launches, all plain kernels (no memset, valid under graph capture):
// clear the maximum, fold max |x| of q and k into it, convert k.
constexpr int kPrepBlock = 256;
constexpr int kMaxScaleExp = 40;

__global__ __launch_bounds__(64) void clear_u32_kernel(unsigned* p) {
  if (threadIdx.x == 0) *p = 0u;
}

// max of |x| as bfloat16 bit patterns (ordered like the magnitudes) over a
// [B, H, T, D] view with element strides (sb, sh, st, 1); D % 8 == 0.
__global__ __launch_bounds__(kPrepBlock) void absmax_bf16_kernel(const u16* __restrict__ x, int H, int T, int D,
                                                                  int64_t sb, int64_t sh, int64_t st, int64_t nchunk,
                                                                  unsigned* __restrict__ out) {
  const int cpr = D / 8;
  unsigned m = 0;
  for (int64_t c = (int64_t)blockIdx.x * kPrepBlock + threadIdx.x; c < nchunk; c += (int64_t)gridDim.x * kPrepBlock) {
    const int64_t row = c / cpr;
    const int d0 = (int)(c - row * cpr) * 8;
    const int64_t t = row % T, bh = row / T;
    const int64_t h = bh % H, b = bh / H;
    const u16x8 v = *reinterpret_cast<const u16x8*>(x + b * sb + h * sh + t * st + d0);
#pragma unroll
    for (int e = 0; e < 8; ++e) m = max(m, (unsigned)(v[e] & 0x7fffu));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = max(m, (unsigned)__shfl_xor((int)m, o, 64));
  if ((threadIdx.x & 63) == 0) atomicMax(out, m);
}

__device__ __forceinline__ float student_scale(unsigned maxbits) {
  if (maxbits >= 0x7f80u) return 1.f;  // inf / NaN: nothing to scale against
  const float m = __builtin_bit_cast(float, maxbits << 16);
  int ex = 0;
  (void)frexpf(m, &ex);  // m < 2^ex
  const int e = min(max(ex - 15, 0), kMaxScaleExp);
  return ldexpf(1.f, -e);
}

// y[b, h, t, :] = float16(x[b, h, t, :] * s), y contiguous [B, H, T, D].
__global__ __launch_bounds__(kPrepBlock) void to_f16_kernel(const u16* __restrict__ x, int H, int T, int D, int64_t sb,
                                                             int64_t sh, int64_t st, int64_t nchunk,
                                                             const unsigned* __restrict__ maxbits,
                                                             u16* __restrict__ y, float* __restrict__ scale_out) {
  const float s = student_scale(*maxbits);
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = s;
  const int cpr = D / 8;
  for (int64_t c = (int64_t)blockIdx.x * kPrepBlock + threadIdx.x; c < nchunk; c += (int64_t)gridDim.x * kPrepBlock) {
    const int64_t row = c / cpr;
    const int d0 = (int)(c - row * cpr) * 8;
    const int64_t t = row % T, bh = row / T;
    const int64_t h = bh % H, b = bh / H;
    const u16x8 v = *reinterpret_cast<const u16x8*>(x + b * sb + h * sh + t * st + d0);
    *reinterpret_cast<u16x8*>(y + row * D + d0) = bf16_to_f16_scaled(v, s);
  }
}

static int prep_blocks(int64_t nchunk) {
  const int64_t want = (nchunk + kPrepBlock - 1) / kPrepBlock;
  return (int)(want < 2048 ? (want > 0 ? want : 1) : 2048);
}

hipError_t launch_keys_f16(const SideArgs& s, int B, int Hq, int T, unsigned* maxbits, float* scale, u16* k16,
                           hipStream_t stream) {
  const int D = s.dim;
  const int64_t nk = (int64_t)B * s.hkv * T * (D / 8);
  const int64_t nq = (int64_t)B * Hq * T * (D / 8);
  hipLaunchKernelGGL(clear_u32_kernel, dim3(1), dim3(64), 0, stream, maxbits);
  hipLaunchKernelGGL(absmax_bf16_kernel, dim3(prep_blocks(nk)), dim3(kPrepBlock), 0, stream, s.k, s.hkv, T, D, s.k_sb,
                     s.k_sh, s.k_st, nk, maxbits);
  if (s.q != s.k)
    hipLaunchKernelGGL(absmax_bf16_kernel, dim3(prep_blocks(nq)), dim3(kPrepBlock), 0, stream, s.q, Hq, T, D, s.q_sb,
                       s.q_sh, s.q_st, nq, maxbits);
  hipLaunchKernelGGL(to_f16_kernel, dim3(prep_blocks(nk)), dim3(kPrepBlock), 0, stream, s.k, s.hkv, T, D, s.k_sb, s.k_sh,
                     s.k_st, nk, (const unsigned*)maxbits, k16, scale);
  return hipGetLastError();
}

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
