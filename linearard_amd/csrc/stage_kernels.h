// Reference-semantics stage kernels (stage A, B, C) as two MFMA templates:
//
//   row_kernel<MODE, DPS, DPT>  one workgroup owns 128 query rows of one
//                               (b, h); it streams 32-key column tiles of K
//                               through LDS and keeps Q in registers.
//                               MODE_LSE  -> lse          (kernel_A.py:42-159)
//                               MODE_KL   -> per-row KL   (kernel_B.py:57-218)
//                               MODE_DQ   -> dq           (kernel_C.py:224-239, :256-261)
//   col_kernel<DPS, DPT>        one workgroup owns 128 key columns of one
//                               (b, kv-head g); it streams 32-row query tiles
//                               of every head of the GQA group and
//                               accumulates dk in registers -- no atomics
//                               (kernel_C.py:242-253 uses fp32 atomics).
//
// DPS/DPT are the head dims padded to a multiple of 16 (D=8 runs as 16 with
// zero padding, which adds exact zeros to every dot product).  The second
// GEMM of stage C (dq, dk) reads its transposed operand straight from the
// row-major tile of the first with ds_read_b64_tr_b16 (TrRowTile).
#pragma once

#include "lard_device.h"

namespace lard {

constexpr int kStageThreads = 256;  // 4 waves
constexpr int kStageRows = 128;     // rows (or columns) owned per workgroup

template <int MODE, int DPS, int DPT>
__global__ __launch_bounds__(kStageThreads) void row_kernel(const RelArgs a) {
  constexpr int BN = 32;
  constexpr bool HAS_T = MODE != MODE_LSE;
  constexpr bool HAS_DQ = MODE == MODE_DQ;
  constexpr int KS = DPS / 16;
  constexpr int KT = DPT / 16;
  constexpr int SS = DPS + 8;  // LDS row strides (elements); +8 breaks bank alignment
  constexpr int ST = DPT + 8;
  constexpr int NDB = DPS >= 32 ? DPS / 32 : 1;  // 32-wide d blocks of dq

  __shared__ __attribute__((aligned(16))) u16 lks[BN * SS];
  __shared__ __attribute__((aligned(16))) u16 lkt[HAS_T ? BN * ST : 8];
  __shared__ int lcol[BN];
  __shared__ int lfull;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int T = a.T;
  const int nrb = (T + kStageRows - 1) / kStageRows;
  const int rb = nrb - 1 - (int)blockIdx.x;  // longest causal rows first
  const int bh = blockIdx.y;
  const int b = bh / a.Hq;
  const int h = bh - b * a.Hq;
  const int i0w = rb * kStageRows + w * 32;
  const int my_i = i0w + l32;
  const bool in_range = my_i < T;
  const bool row_valid = in_range && mask_at(a.mask, a.mask_kind, (int64_t)b * a.mask_sb + my_i);
  const bool sbf = a.s.bf16 != 0;
  const bool tbf = a.t.bf16 != 0;

  // MODE_DQ: K^T operand of the second GEMM, read transposed from lks
  TrRowTile<DPS, SS> trk;
  if constexpr (HAS_DQ) trk.init(lane);

  // Query fragments (B operand): lane holds q[i = l32][16kk + 8*half .. +7].
  u16x8 fq_s[KS];
  u16x8 fq_t[HAS_T ? KT : 1];
  {
    const u16* p = a.s.q + (int64_t)b * a.s.q_sb + (int64_t)h * a.s.q_sh + (int64_t)my_i * a.s.q_st;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int d0 = 16 * kk + 8 * half;
      fq_s[kk] = (in_range && d0 < a.s.dim) ? *reinterpret_cast<const u16x8*>(p + d0) : (u16x8)(0);
    }
    if constexpr (HAS_T) {
      const u16* pt = a.t.q + (int64_t)b * a.t.q_sb + (int64_t)h * a.t.q_sh + (int64_t)my_i * a.t.q_st;
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) {
        const int d0 = 16 * kk + 8 * half;
        fq_t[kk] = (in_range && d0 < a.t.dim) ? *reinterpret_cast<const u16x8*>(pt + d0) : (u16x8)(0);
      }
    }
  }

  // Row state.
  bool ok = row_valid;
  float lse_s = 0.f, lse_t = 0.f;  // natural-log LSE, -inf replaced by 0 (kernel_B.py:142-143)
  if constexpr (MODE == MODE_KL || MODE == MODE_DQ) {
    float ls = 0.f, lt = 0.f;
    if (in_range) {
      ls = a.lse_s_in[(int64_t)bh * T + my_i];
      lt = a.lse_t_in[(int64_t)bh * T + my_i];
    }
    ok = ok && (ls != kNegInf) && (lt != kNegInf);
    lse_s = (ls == kNegInf) ? 0.f : ls;
    lse_t = (lt == kNegInf) ? 0.f : lt;
  }
  const bool wave_ok = __all(ok) != 0;
  float run_m = kNegInf, run_r = 0.f;  // MODE_LSE online max / sum
  float kl_acc = 0.f;                  // MODE_KL
  f32x16 dq[HAS_DQ ? NDB : 1];
#pragma unroll
  for (int db = 0; db < (HAS_DQ ? NDB : 1); ++db) dq[db] = (f32x16)(0.f);

  const int hs = h / a.s.group;
  const int ht = h / a.t.group;
  const u16* ks_base = a.s.k + (int64_t)b * a.s.k_sb + (int64_t)hs * a.s.k_sh;
  const u16* kt_base = a.t.k + (int64_t)b * a.t.k_sb + (int64_t)ht * a.t.k_sh;

  int nkb = (T + BN - 1) / BN;
  if (a.causal) nkb = min(nkb, (rb * kStageRows + kStageRows - 1) / BN + 1);
  const int wave_last_kb = a.causal ? (i0w + 31) / BN : nkb - 1;

  // Key tiles go through registers: tile kb + 1 is loaded while tile kb is
  // consumed (except where the registers would not fit: the largest dq
  // variants load each tile right before storing it).
  TileRegs<BN, DPS, kStageThreads> rks;
  TileRegs<BN, HAS_T ? DPT : 16, kStageThreads> rkt;
  constexpr bool kPrefetch = !(HAS_DQ && DPS == 256 && DPT >= 128);
  auto load_tile = [&](int j0) {
    rks.load(ks_base, a.s.k_st, j0, T, a.s.dim, tid);
    if constexpr (HAS_T) rkt.load(kt_base, a.t.k_st, j0, T, a.t.dim, tid);
  };
  if constexpr (kPrefetch) load_tile(0);

  for (int kb = 0; kb < nkb; ++kb) {
    const int j0 = kb * BN;
    __syncthreads();
    if constexpr (!kPrefetch) load_tile(j0);
    rks.store(lks, SS, tid);
    if constexpr (HAS_T) rkt.store(lkt, ST, tid);
    if constexpr (kPrefetch) {
      if (kb + 1 < nkb) load_tile(j0 + BN);
    }
    if (tid < 64) {  // wave 0: key validity, and whether the whole tile is valid
      bool v = true;
      if (tid < BN) {
        const int j = j0 + tid;
        v = (j < T) && mask_at(a.mask, a.mask_kind, (int64_t)b * a.mask_sb + j);
        lcol[tid] = v;
      }
      const int all = __all(v);
      if (tid == 0) lfull = all;
    }
    __syncthreads();
    if (kb > wave_last_kb) continue;

    // S^T[j][i] = K[j] . Q[i]: A = K tile rows (LDS), B = query fragment.
    f32x16 ss = (f32x16)(0.f);
    if (sbf) {
#pragma unroll
      for (int kk = 0; kk < KS; ++kk)
        ss = mfma32<true>(*reinterpret_cast<const u16x8*>(lks + l32 * SS + 16 * kk + 8 * half), fq_s[kk], ss);
    } else {
#pragma unroll
      for (int kk = 0; kk < KS; ++kk)
        ss = mfma32<false>(*reinterpret_cast<const u16x8*>(lks + l32 * SS + 16 * kk + 8 * half), fq_s[kk], ss);
    }
    f32x16 st = (f32x16)(0.f);
    if constexpr (HAS_T) {
      if (tbf) {
#pragma unroll
        for (int kk = 0; kk < KT; ++kk)
          st = mfma32<true>(*reinterpret_cast<const u16x8*>(lkt + l32 * ST + 16 * kk + 8 * half), fq_t[kk], st);
      } else {
#pragma unroll
        for (int kk = 0; kk < KT; ++kk)
          st = mfma32<false>(*reinterpret_cast<const u16x8*>(lkt + l32 * ST + 16 * kk + 8 * half), fq_t[kk], st);
      }
    }

    // Per-element work in two forms: full tiles (every key valid, at or
    // below the diagonal for every row of the wave, every row of the wave
    // valid) skip the per-element validity; the values of the elements both
    // forms compute are identical.
    const bool full = wave_ok && __builtin_amdgcn_readfirstlane(lfull) != 0 && (!a.causal || j0 + BN - 1 <= i0w);
    auto elements = [&](auto full_tag) {
      constexpr bool FULL = decltype(full_tag)::value;
      // Validity of the 16 (i, j) entries this lane holds.
      bool valid[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if constexpr (FULL) {
          valid[r] = true;
        } else {
          const int jj = 8 * (r >> 2) + 4 * half + (r & 3);
          valid[r] = ok && lcol[jj] && (!a.causal || j0 + jj <= my_i);
        }
      }

      if constexpr (MODE == MODE_LSE) {
        float x[16];
        float mb = kNegInf;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          x[r] = valid[r] ? mul_rn(ss[r], a.s.scale) : kNegInf;  // tl.dot(q, k^T) * sm_scale
          mb = fmaxf(mb, x[r]);
        }
        mb = fmaxf(mb, xor32(mb));
        const float mbs = (mb == kNegInf) ? 0.f : mb;
        float rs = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) rs += valid[r] ? fast_exp2((x[r] - mbs) * kLog2e) : 0.f;
        rs += xor32(rs);
        // Online merge (kernel_A.py:152-154) with the empty-block case guarded.
        const float mn = fmaxf(run_m, mb);
        const float f_old = (run_m == kNegInf) ? 0.f : fast_exp2((run_m - mn) * kLog2e);
        const float f_new = (mb == kNegInf) ? 0.f : fast_exp2((mb - mn) * kLog2e);
        run_r = run_r * f_old + rs * f_new;
        run_m = mn;
      } else if constexpr (MODE == MODE_KL) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          if (valid[r]) {
            const float lps = mul_rn(ss[r], a.s.scale) - lse_s;
            const float lpt = mul_rn(st[r], a.t.scale) - lse_t;
            kl_acc += fast_exp2(lpt * kLog2e) * (lpt - lps);
          }
        }
      } else {  // MODE_DQ
        float pd[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          pd[r] = valid[r] ? fast_exp2((mul_rn(ss[r], a.s.scale) - lse_s) * kLog2e) -
                                 fast_exp2((mul_rn(st[r], a.t.scale) - lse_t) * kLog2e)
                           : 0.f;
        }
        u16x8 dv[2];  // dval.to(qs.dtype)  (kernel_C.py:233)
        if constexpr (DPS == 256) {
          // one element at a time: the 8-wide conversions need registers
          // this variant (128 accumulator registers) does not have
#pragma unroll
          for (int r = 0; r < 16; ++r) dv[r >> 3][r & 7] = to_bits(pd[r], sbf);
        } else if (sbf) {
          dv[0] = to_bits8<true>(pd);
          dv[1] = to_bits8<true>(pd + 8);
        } else {
          dv[0] = to_bits8<false>(pd);
          dv[1] = to_bits8<false>(pd + 8);
        }
        // dq^T[d][i] += sum_j K^T[d][j] D^T[j][i]
#pragma unroll
        for (int m = 0; m < 2; ++m) {
#pragma unroll
          for (int db = 0; db < NDB; ++db) {
            const u16x8 aop = trk.read(lks, m, db);
            dq[db] = sbf ? mfma32<true>(aop, dv[m], dq[db]) : mfma32<false>(aop, dv[m], dq[db]);
          }
        }
      }
    };
    if (full)
      elements(Flag<true>{});
    else
      elements(Flag<false>{});
  }

  const int64_t row_index = (int64_t)bh * T + my_i;
  if constexpr (MODE == MODE_LSE) {
    float lse = (run_r > 0.f) ? run_m + fast_log2(run_r) * kLn2 : kNegInf;
    if (!row_valid) lse = 0.f;  // kernel_A.py:157-158
    if (in_range && half == 0) a.lse_out[row_index] = lse;
  } else if constexpr (MODE == MODE_KL) {
    kl_acc += xor32(kl_acc);
    const float v = ok ? kl_acc : 0.f;  // kernel_B.py:216
    if (in_range && half == 0) a.row_out[row_index] = v;
  } else {
    // alpha_s (times dloss when asked), invalid rows zeroed (kernel_C.py:256)
    const float f = ok ? a.s.scale * (a.dscale != nullptr ? *a.dscale : 1.f) : 0.f;
    if (in_range) {
      float* out = a.dq_out + row_index * a.s.dim;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = 32 * db + 8 * g + 4 * half;
          if (d0 < a.s.dim) {
            const f32x4 v = {dq[db][4 * g] * f, dq[db][4 * g + 1] * f, dq[db][4 * g + 2] * f, dq[db][4 * g + 3] * f};
            *reinterpret_cast<f32x4*>(out + d0) = v;
          }
        }
      }
    }
  }
}

template <int DPS, int DPT>
__global__ __launch_bounds__(kStageThreads) void col_kernel(const RelArgs a) {
  constexpr int BM = 32;
  constexpr int KS = DPS / 16;
  constexpr int KT = DPT / 16;
  constexpr int SS = DPS + 8;
  constexpr int ST = DPT + 8;
  constexpr int NDB = DPS >= 32 ? DPS / 32 : 1;

  __shared__ __attribute__((aligned(16))) u16 lqs[BM * SS];
  __shared__ __attribute__((aligned(16))) u16 lqt[BM * ST];
  __shared__ __attribute__((aligned(16))) float llse_s[BM];
  __shared__ __attribute__((aligned(16))) float llse_t[BM];
  __shared__ int lok[BM];
  __shared__ int lfull;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int T = a.T;
  const int cb = blockIdx.x;  // small cb = longest causal columns, launched first
  const int bg = blockIdx.y;
  const int b = bg / a.s.hkv;
  const int g = bg - b * a.s.hkv;
  const int j0w = cb * kStageRows + w * 32;
  const int my_j = j0w + l32;
  const bool in_range = my_j < T;
  const bool col_valid = in_range && mask_at(a.mask, a.mask_kind, (int64_t)b * a.mask_sb + my_j);
  const bool wave_cols_ok = __all(col_valid) != 0;
  const bool sbf = a.s.bf16 != 0;
  const bool tbf = a.t.bf16 != 0;

  // Q^T operand of the second GEMM, read transposed from lqs
  TrRowTile<DPS, SS> trq;
  trq.init(lane);

  // Key fragments (B operand of S[i][j]): lane holds k[j = l32][16kk + 8*half .. +7].
  u16x8 fk_s[KS];
  u16x8 fk_t[KT];
  {
    const u16* p = a.s.k + (int64_t)b * a.s.k_sb + (int64_t)g * a.s.k_sh + (int64_t)my_j * a.s.k_st;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int d0 = 16 * kk + 8 * half;
      fk_s[kk] = (in_range && d0 < a.s.dim) ? *reinterpret_cast<const u16x8*>(p + d0) : (u16x8)(0);
    }
  }
  f32x16 dk[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dk[db] = (f32x16)(0.f);

  const int nib = (T + BM - 1) / BM;
  const int ib_first = a.causal ? (cb * kStageRows) / BM : 0;
  const int wave_first_ib = a.causal ? j0w / BM : 0;
  int loaded_ht = -1;

  for (int hh = 0; hh < a.s.group; ++hh) {
    const int h = g * a.s.group + hh;
    const int ht = h / a.t.group;
    if (ht != loaded_ht) {
      const u16* p = a.t.k + (int64_t)b * a.t.k_sb + (int64_t)ht * a.t.k_sh + (int64_t)my_j * a.t.k_st;
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) {
        const int d0 = 16 * kk + 8 * half;
        fk_t[kk] = (in_range && d0 < a.t.dim) ? *reinterpret_cast<const u16x8*>(p + d0) : (u16x8)(0);
      }
      loaded_ht = ht;
    }
    const int64_t bh = (int64_t)b * a.Hq + h;
    const u16* qs_base = a.s.q + (int64_t)b * a.s.q_sb + (int64_t)h * a.s.q_sh;
    const u16* qt_base = a.t.q + (int64_t)b * a.t.q_sb + (int64_t)h * a.t.q_sh;

    // Query tiles and their rows' validity and LSEs go through registers:
    // tile ib + 1 is loaded while tile ib is consumed (except where the
    // registers would not fit: the largest variants load each tile right
    // before storing it).
    constexpr bool kPrefetch = !(DPS == 256 && DPT >= 128);
    TileRegs<BM, DPS, kStageThreads> rqs;
    TileRegs<BM, DPT, kStageThreads> rqt;
    float nls = 0.f, nlt = 0.f;
    bool nrv = false;
    auto load_tile = [&](int i0) {
      rqs.load(qs_base, a.s.q_st, i0, T, a.s.dim, tid);
      rqt.load(qt_base, a.t.q_st, i0, T, a.t.dim, tid);
      if (tid < BM) {
        const int i = i0 + tid;
        nrv = false;
        nls = nlt = 0.f;
        if (i < T) {
          nrv = mask_at(a.mask, a.mask_kind, (int64_t)b * a.mask_sb + i);
          nls = a.lse_s_in[bh * T + i];
          nlt = a.lse_t_in[bh * T + i];
        }
      }
    };
    if constexpr (kPrefetch) {
      if (ib_first < nib) load_tile(ib_first * BM);
    }

    for (int ib = ib_first; ib < nib; ++ib) {
      const int i0 = ib * BM;
      __syncthreads();
      if constexpr (!kPrefetch) load_tile(i0);
      rqs.store(lqs, SS, tid);
      rqt.store(lqt, ST, tid);
      const float ls = nls, lt = nlt;
      const bool rv = nrv;
      if constexpr (kPrefetch) {
        if (ib + 1 < nib) load_tile(i0 + BM);
      }
      if (tid < 64) {  // wave 0: row validity and LSEs, and whether every row is valid
        bool v = true;
        if (tid < BM) {
          v = rv && (ls != kNegInf) && (lt != kNegInf);
          lok[tid] = v;
          llse_s[tid] = (ls == kNegInf) ? 0.f : ls;
          llse_t[tid] = (lt == kNegInf) ? 0.f : lt;
        }
        const int all = __all(v);
        if (tid == 0) lfull = all;
      }
      __syncthreads();
      if (ib < wave_first_ib) continue;

      // S[i][j] = Q[i] . K[j]: A = query tile rows (LDS), B = key fragment.
      f32x16 ss = (f32x16)(0.f);
      f32x16 st = (f32x16)(0.f);
      if (sbf) {
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
          ss = mfma32<true>(*reinterpret_cast<const u16x8*>(lqs + l32 * SS + 16 * kk + 8 * half), fk_s[kk], ss);
      } else {
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
          ss = mfma32<false>(*reinterpret_cast<const u16x8*>(lqs + l32 * SS + 16 * kk + 8 * half), fk_s[kk], ss);
      }
      if (tbf) {
#pragma unroll
        for (int kk = 0; kk < KT; ++kk)
          st = mfma32<true>(*reinterpret_cast<const u16x8*>(lqt + l32 * ST + 16 * kk + 8 * half), fk_t[kk], st);
      } else {
#pragma unroll
        for (int kk = 0; kk < KT; ++kk)
          st = mfma32<false>(*reinterpret_cast<const u16x8*>(lqt + l32 * ST + 16 * kk + 8 * half), fk_t[kk], st);
      }

      // Per-element work in two forms: full tiles (every row of the tile and
      // every column of the wave valid, the whole tile at or below the
      // diagonal) skip the per-element validity; the values of the elements
      // both forms compute are identical.
      const bool full =
          wave_cols_ok && __builtin_amdgcn_readfirstlane(lfull) != 0 && (!a.causal || j0w + 31 <= i0);
      auto elements = [&](auto full_tag) {
        constexpr bool FULL = decltype(full_tag)::value;
        float pd[16];
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int ii0 = 8 * r4 + 4 * half;
          const f32x4 ls4 = *reinterpret_cast<const f32x4*>(llse_s + ii0);
          const f32x4 lt4 = *reinterpret_cast<const f32x4*>(llse_t + ii0);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * r4 + e;
            const bool v = FULL || (lok[ii0 + e] && col_valid && (!a.causal || my_j <= i0 + ii0 + e));
            pd[r] = v ? fast_exp2((mul_rn(ss[r], a.s.scale) - ls4[e]) * kLog2e) -
                            fast_exp2((mul_rn(st[r], a.t.scale) - lt4[e]) * kLog2e)
                      : 0.f;
          }
        }
        u16x8 dv[2];  // kernel_C.py:233
        if (sbf) {
          dv[0] = to_bits8<true>(pd);
          dv[1] = to_bits8<true>(pd + 8);
        } else {
          dv[0] = to_bits8<false>(pd);
          dv[1] = to_bits8<false>(pd + 8);
        }
        // dk^T[d][j] += sum_i Q^T[d][i] D[i][j]
#pragma unroll
        for (int m = 0; m < 2; ++m) {
#pragma unroll
          for (int db = 0; db < NDB; ++db) {
            const u16x8 aop = trq.read(lqs, m, db);
            dk[db] = sbf ? mfma32<true>(aop, dv[m], dk[db]) : mfma32<false>(aop, dv[m], dk[db]);
          }
        }
      };
      if (full)
        elements(Flag<true>{});
      else
        elements(Flag<false>{});
    }
  }

  if (in_range) {
    const int64_t off = ((int64_t)bg * T + my_j) * a.s.dim;
    float* out = a.dk_out + off;
    const float f = a.s.scale;
    const float mult = a.dscale != nullptr ? *a.dscale : 1.f;  // chain rule (integration.py:63-64)
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int d0 = 32 * db + 8 * gq + 4 * half;
        if (d0 < a.s.dim) {
          f32x4 v = {dk[db][4 * gq] * f, dk[db][4 * gq + 1] * f, dk[db][4 * gq + 2] * f, dk[db][4 * gq + 3] * f};
          if (a.dk_add != nullptr) v += *reinterpret_cast<const f32x4*>(a.dk_add + off + d0);
          if (a.dscale != nullptr) v *= mult;
          *reinterpret_cast<f32x4*>(out + d0) = v;
        }
      }
    }
  }
}

// Launchers (one translation unit per family, see stage_*.hip).
hipError_t launch_row_lse(const RelArgs& a, int dps, hipStream_t stream);
hipError_t launch_row_kl(const RelArgs& a, int dps, int dpt, hipStream_t stream);
hipError_t launch_row_dq(const RelArgs& a, int dps, int dpt, hipStream_t stream);
hipError_t launch_col_dk(const RelArgs& a, int dps, int dpt, hipStream_t stream);
// Loss reduction: out = sum(x[0..n)) through kReduceBlocks double partials.
constexpr int kReduceBlocks = 512;
hipError_t launch_reduce_sum(const float* x, int64_t n, double* partial, float* out, hipStream_t stream);
// x[0..n) *= (*dscale) in place (dscale a device scalar; n a multiple of 4,
// x 16-byte aligned): the chain rule of a gradient computed before dloss.
hipError_t launch_scale_inplace(float* x, int64_t n, const float* dscale, hipStream_t stream);

}  // namespace lard
