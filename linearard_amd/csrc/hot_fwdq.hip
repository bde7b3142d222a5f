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
//   clear_u32_kernel       the maximum := 0;
//   keys_f16_kernel        converts k with s = 1 (the scale of every input
//                          below 2^15) and folds max |x| of k, and of q when
//                          it is another tensor, into the maximum;
//   keys_f16_fixup_kernel  writes s; when s < 1 (rare) converts k again.
// Grid: x = one (b, head) of k, then (q != k) one (b, head) of q; y = blocks
// of kKeyRows rows of that head (strided by gridDim.y beyond 65535 blocks).
constexpr int kPrepBlock = 256;
constexpr int kKeyRows = 64;
constexpr int kMaxScaleExp = 40;

__global__ __launch_bounds__(64) void clear_u32_kernel(unsigned* p) {
  if (threadIdx.x == 0) *p = 0u;
}

struct KeyPrep {
  const u16* k;
  const u16* q;        // null: q is k
  int64_t k_sb, k_sh, k_st, q_sb, q_sh, q_st;
  int hkv, hq, T, D;   // D % 8 == 0
  unsigned* maxbits;
  float* scale;
  u16* k16;            // [B, hkv, T, D] contiguous
};

__device__ __forceinline__ float side_scale(unsigned maxbits) {
  if (maxbits >= 0x7f80u) return 1.f;  // inf / NaN: nothing to scale against
  const float m = __builtin_bit_cast(float, maxbits << 16);
  int ex = 0;
  (void)frexpf(m, &ex);  // m < 2^ex
  const int e = min(max(ex - 15, 0), kMaxScaleExp);
  return ldexpf(1.f, -e);
}

// The rows of this block: (b, head) and the first row, for k (or q) heads.
struct KeyRows {
  const u16* base;
  int64_t st;
  int head;
  bool is_q;
  int64_t b;
};

__device__ __forceinline__ KeyRows key_rows(const KeyPrep& p, int nbk) {
  KeyRows r;
  const int x = (int)blockIdx.x;
  r.is_q = x >= nbk;
  const int bh = r.is_q ? x - nbk : x;
  const int H = r.is_q ? p.hq : p.hkv;
  r.b = bh / H;
  r.head = bh - (int)r.b * H;
  r.base = r.is_q ? p.q + r.b * p.q_sb + (int64_t)r.head * p.q_sh : p.k + r.b * p.k_sb + (int64_t)r.head * p.k_sh;
  r.st = r.is_q ? p.q_st : p.k_st;
  return r;
}

__global__ __launch_bounds__(kPrepBlock) void keys_f16_kernel(const KeyPrep p, int nbk) {
  const KeyRows r = key_rows(p, nbk);
  const int cpr = p.D / 8;
  u16* out = p.k16 + ((r.b * p.hkv + r.head) * (int64_t)p.T) * p.D;
  unsigned m = 0;
  for (int t0 = (int)blockIdx.y * kKeyRows; t0 < p.T; t0 += (int)gridDim.y * kKeyRows) {
    const int n = min(kKeyRows, p.T - t0) * cpr;
    for (int c = (int)threadIdx.x; c < n; c += kPrepBlock) {
      const int t = t0 + c / cpr;
      const int d0 = (c - (t - t0) * cpr) * 8;
      const u16x8 v = *reinterpret_cast<const u16x8*>(r.base + t * r.st + d0);
#pragma unroll
      for (int e = 0; e < 8; ++e) m = max(m, (unsigned)(v[e] & 0x7fffu));
      if (!r.is_q) *reinterpret_cast<u16x8*>(out + (int64_t)t * p.D + d0) = bf16_to_f16_scaled(v, 1.f);
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = max(m, (unsigned)__shfl_xor((int)m, o, 64));
  __shared__ unsigned red[kPrepBlock / 64];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < kPrepBlock / 64; ++w) m = max(m, red[w]);
    // the maximum only grows: a block below what is already there skips the
    // atomic (a stale read only costs an atomic that changes nothing)
    if (m > __hip_atomic_load(p.maxbits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) atomicMax(p.maxbits, m);
  }
}

__global__ __launch_bounds__(kPrepBlock) void keys_f16_fixup_kernel(const KeyPrep p, int nbk) {
  const float s = side_scale(*p.maxbits);
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *p.scale = s;
  if (s == 1.f || (int)blockIdx.x >= nbk) return;  // the first pass converted with s = 1
  const KeyRows r = key_rows(p, nbk);
  const int cpr = p.D / 8;
  u16* out = p.k16 + ((r.b * p.hkv + r.head) * (int64_t)p.T) * p.D;
  for (int t0 = (int)blockIdx.y * kKeyRows; t0 < p.T; t0 += (int)gridDim.y * kKeyRows) {
    const int n = min(kKeyRows, p.T - t0) * cpr;
    for (int c = (int)threadIdx.x; c < n; c += kPrepBlock) {
      const int t = t0 + c / cpr;
      const int d0 = (c - (t - t0) * cpr) * 8;
      const u16x8 v = *reinterpret_cast<const u16x8*>(r.base + t * r.st + d0);
      *reinterpret_cast<u16x8*>(out + (int64_t)t * p.D + d0) = bf16_to_f16_scaled(v, s);
    }
  }
}

hipError_t launch_keys_f16(const SideArgs& s, int B, int Hq, int T, unsigned* maxbits, float* scale, u16* k16,
                           hipStream_t stream) {
  KeyPrep p{};
  p.k = s.k;
  p.q = s.q != s.k ? s.q : nullptr;
  p.k_sb = s.k_sb, p.k_sh = s.k_sh, p.k_st = s.k_st;
  p.q_sb = s.q_sb, p.q_sh = s.q_sh, p.q_st = s.q_st;
  p.hkv = s.hkv, p.hq = Hq, p.T = T, p.D = s.dim;
  p.maxbits = maxbits, p.scale = scale, p.k16 = k16;
  const int64_t nbk = (int64_t)B * s.hkv;
  const int64_t nbx = nbk + (p.q != nullptr ? (int64_t)B * Hq : 0);
  const int64_t nby = std::min<int64_t>((T + kKeyRows - 1) / kKeyRows, 65535);
  if (nbx > INT32_MAX) return hipErrorInvalidValue;
  const dim3 grid((unsigned)nbx, (unsigned)nby), block(kPrepBlock);
  hipLaunchKernelGGL(clear_u32_kernel, dim3(1), dim3(64), 0, stream, maxbits);
  hipLaunchKernelGGL(keys_f16_kernel, grid, block, 0, stream, p, (int)nbk);
  hipLaunchKernelGGL(keys_f16_fixup_kernel, grid, block, 0, stream, p, (int)nbk);
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
