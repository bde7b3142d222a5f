// Fused forward of the autograd boundary (AttnKLAlignFn.forward,
// integration.py:8-45): ONE pass over the key tiles of each query row tile
// produces, per row,
//   lse_s, lse_t            online max / sum of both relations
//                           (the reference runs stage A twice, kernel_A.py:111-154),
//   KL_i                    E_{p_t}[x_t - x_s] - lse_t + lse_s, accumulated online
//                           (equal to sum_j p_t (l_t - l_s) of kernel_B.py:206-213
//                           because sum_j p_t = 1 on every valid row),
//
// It serves the shapes the throughput kernels (hot_kernels.h) do not cover:
// Ds == Dt == 256.  Tile mapping is that of row_kernel: 4 waves x 32 query
// rows; S^T tiles keep one query row per lane (pair), so row statistics are
// in-lane reductions plus one cross-half exchange.
#pragma once

#include "stage_kernels.h"

namespace lard {

template <int DP, bool BF>
__global__ __launch_bounds__(kStageThreads) void fused_fwd_kernel(const FusedArgs f) {
  const RelArgs& a = f.r;
  constexpr int DPS = DP;  // student and teacher share the head dim and dtype on this path
  constexpr int DPT = DP;
  constexpr int BN = 32;
  constexpr int KS = DPS / 16;
  constexpr int KT = DPT / 16;
  constexpr int SS = DPS + 8;
  constexpr int ST = DPT + 8;

  __shared__ __attribute__((aligned(16))) u16 lks[BN * SS];
  __shared__ __attribute__((aligned(16))) u16 lkt[BN * ST];
  __shared__ int lcol[BN];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int T = a.T;
  const int nrb = (T + kStageRows - 1) / kStageRows;
  const int rb = nrb - 1 - (int)blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / a.Hq;
  const int h = bh - b * a.Hq;
  const int i0w = rb * kStageRows + w * 32;
  const int my_i = i0w + l32;
  const bool in_range = my_i < T;
  const bool row_valid = in_range && mask_at(a.mask, a.mask_kind, (int64_t)b * a.mask_sb + my_i);
  u16x8 fq_s[KS];
  u16x8 fq_t[KT];
  {
    const u16* p = a.s.q + (int64_t)b * a.s.q_sb + (int64_t)h * a.s.q_sh + (int64_t)my_i * a.s.q_st;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int d0 = 16 * kk + 8 * half;
      fq_s[kk] = (in_range && d0 < a.s.dim) ? *reinterpret_cast<const u16x8*>(p + d0) : (u16x8)(0);
    }
    const u16* pt = a.t.q + (int64_t)b * a.t.q_sb + (int64_t)h * a.t.q_sh + (int64_t)my_i * a.t.q_st;
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      const int d0 = 16 * kk + 8 * half;
      fq_t[kk] = (in_range && d0 < a.t.dim) ? *reinterpret_cast<const u16x8*>(pt + d0) : (u16x8)(0);
    }
  }

  // Online state (natural-log units; x = rounded dot * sm_scale).
  float m_s = kNegInf, l_s = 0.f;
  float m_t = kNegInf, l_t = 0.f;
  float a_t = 0.f;  // sum_j p_t ((x_t - m_t) - (x_s - m_s)), same scaling as l_t

  const int hs = h / a.s.group;
  const int ht = h / a.t.group;
  const u16* ks_base = a.s.k + (int64_t)b * a.s.k_sb + (int64_t)hs * a.s.k_sh;
  const u16* kt_base = a.t.k + (int64_t)b * a.t.k_sb + (int64_t)ht * a.t.k_sh;

  int nkb = (T + BN - 1) / BN;
  if (a.causal) nkb = min(nkb, (rb * kStageRows + kStageRows - 1) / BN + 1);
  const int wave_last_kb = a.causal ? (i0w + 31) / BN : nkb - 1;

  // Key tiles go through registers: tile kb + 1 is loaded while tile kb is
  // consumed.
  TileRegs<BN, DPS, kStageThreads> rks;
  TileRegs<BN, DPT, kStageThreads> rkt;
  rks.load(ks_base, a.s.k_st, 0, T, a.s.dim, tid);
  rkt.load(kt_base, a.t.k_st, 0, T, a.t.dim, tid);

  for (int kb = 0; kb < nkb; ++kb) {
    const int j0 = kb * BN;
    __syncthreads();
    rks.store(lks, SS, tid);
    rkt.store(lkt, ST, tid);
    if (kb + 1 < nkb) {
      rks.load(ks_base, a.s.k_st, j0 + BN, T, a.s.dim, tid);
      rkt.load(kt_base, a.t.k_st, j0 + BN, T, a.t.dim, tid);
    }
    if (tid < BN) {
      const int j = j0 + tid;
      lcol[tid] = (j < T) && mask_at(a.mask, a.mask_kind, (int64_t)b * a.mask_sb + j);
    }
    __syncthreads();
    if (kb > wave_last_kb) continue;

    f32x16 ss = (f32x16)(0.f);
    f32x16 st = (f32x16)(0.f);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
      ss = mfma32<BF>(*reinterpret_cast<const u16x8*>(lks + l32 * SS + 16 * kk + 8 * half), fq_s[kk], ss);
#pragma unroll
    for (int kk = 0; kk < KT; ++kk)
      st = mfma32<BF>(*reinterpret_cast<const u16x8*>(lkt + l32 * ST + 16 * kk + 8 * half), fq_t[kk], st);

    float xs[16], xt[16];
    bool valid[16];
    float mb_s = kNegInf, mb_t = kNegInf;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int jj = 8 * (r >> 2) + 4 * half + (r & 3);
      valid[r] = row_valid && lcol[jj] && (!a.causal || j0 + jj <= my_i);
      xs[r] = valid[r] ? mul_rn(ss[r], a.s.scale) : kNegInf;
      xt[r] = valid[r] ? mul_rn(st[r], a.t.scale) : kNegInf;
      mb_s = fmaxf(mb_s, xs[r]);
      mb_t = fmaxf(mb_t, xt[r]);
    }
    mb_s = fmaxf(mb_s, xor32(mb_s));
    mb_t = fmaxf(mb_t, xor32(mb_t));
    const float mn_s = fmaxf(m_s, mb_s);
    const float mn_t = fmaxf(m_t, mb_t);
    const float c_s = (m_s == kNegInf) ? 0.f : fast_exp2((m_s - mn_s) * kLog2e);
    const float c_t = (m_t == kNegInf) ? 0.f : fast_exp2((m_t - mn_t) * kLog2e);
    // terms of a_t are relative to the maxima: moving them to the new maxima
    // adds (mn_s - m_s) - (mn_t - m_t) to each (both maxima are finite
    // together: every valid element is valid on both sides)
    const float shift = (m_t == kNegInf) ? 0.f : (mn_s - m_s) - (mn_t - m_t);
    a_t = c_t * fmaf(l_t, shift, a_t);
    m_s = mn_s;
    m_t = mn_t;

    float ps[16], pt[16];
    float sum_s = 0.f, sum_t = 0.f, sum_a = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      ps[r] = valid[r] ? fast_exp2((xs[r] - mn_s) * kLog2e) : 0.f;
      pt[r] = valid[r] ? fast_exp2((xt[r] - mn_t) * kLog2e) : 0.f;
      sum_s += ps[r];
      sum_t += pt[r];
      sum_a += valid[r] ? pt[r] * ((xt[r] - mn_t) - (xs[r] - mn_s)) : 0.f;
    }
    sum_s += xor32(sum_s);
    sum_t += xor32(sum_t);
    sum_a += xor32(sum_a);
    l_s = l_s * c_s + sum_s;
    l_t = l_t * c_t + sum_t;
    a_t += sum_a;
  }

  const bool ok = row_valid && l_s > 0.f && l_t > 0.f;
  const float lse_s = (l_s > 0.f) ? m_s + fast_log2(l_s) * kLn2 : kNegInf;
  const float lse_t = (l_t > 0.f) ? m_t + fast_log2(l_t) * kLn2 : kNegInf;
  const int64_t row_index = (int64_t)bh * T + my_i;
  if (in_range && half == 0) {
    f.lse_s_out[row_index] = row_valid ? lse_s : 0.f;  // kernel_A.py:157-158
    f.lse_t_out[row_index] = row_valid ? lse_t : 0.f;
    // KL = E_pt[(x_t - m_t) - (x_s - m_s)] + ln(l_s / l_t) with lse = m + ln(l):
    // max-relative terms only, so a row dominated by one key loses nothing to
    // cancellation and a one-key row gives exactly 0 (its terms are 0 - 0 and ln 1).
    f.row_out[row_index] = ok ? a_t / l_t + (fast_log2(l_s) - fast_log2(l_t)) * kLn2 : 0.f;
  }
}

// Coverage: Ds == Dt and one dtype for both relations (other shapes run the
// stage kernels).
bool fused_fwd_supported(int ds, int dt, bool same_dtype);
hipError_t launch_fused_fwd(const FusedArgs& f, int dp, bool bf16, hipStream_t stream);

}  // namespace lard
