// Throughput kernels of the autograd path for Ds == Dt <= 128 and one dtype
// (every shape train.py produces: Llama/Mistral heads are d=128 bf16).
//
//   token_prep_kernel      per token: valid (j < T and mask != 0), one byte.
//   row_prep_kernel        per query row of the backward: -lse * log2(e) for
//                          student and teacher, -inf outside the valid set
//                          (kernel_C.py:155-161), so exp2(x * c + nl) is P.
//   hot_fwd_kernel         forward of AttnKLAlignFn (integration.py:8-45):
//                          per query row both online softmaxes (stage A for
//                          student and teacher) and the KL (stage B), one pass.
//   hot_dq_kernel          backward, row side (kernel_C.py:224-239): per query
//                          row dq = sm_scale_s D K_s, D = P_s - P_t from the
//                          forward's LSEs, cast to the input dtype before the
//                          product exactly like kernel_C.py:232-233, so the
//                          error is relative to D, not to P.  The K operand of
//                          the second GEMM is read transposed from the same
//                          row-major LDS tile as the first (ds_read_b64_tr_b16).
//   hot_bwd_kernel         backward, column side (kernel_C.py:242-253): per key
//                          column dk = sm_scale_s sum_i D_ij q_i, summed over
//                          the GQA group by its owner (no atomics), plus the
//                          row side when q is k, times dloss.
//
// Memory pipeline: K (fwd, dq) / Q (dk) tiles of 64 rows are copied
// HBM->LDS with global_load_lds_dwordx4 (no staging registers) into four LDS
// buffers used as two tile pairs: one pair is consumed while the next lands,
// one barrier per pair.  Every wave issues the same number of copies per
// tile, so "a tile landed" is one s_waitcnt vmcnt(N).  LDS tiles are
// XOR-swizzled by 16-byte chunk so the MFMA operand reads (16 lanes at a
// time, one row each) hit 16 distinct bank groups.
//
// Work order: workgroups are numbered so that each XCD (8 per MI355X, one L2
// each; workgroups are dealt to XCDs round robin) receives a contiguous range
// of (head, tile) work, longest causal tiles first within each head.
#pragma once

#include "fused_kernels.h"

namespace lard {

constexpr int kTile = 64;     // rows of K (fwd, dq) or Q (dk) per LDS tile
constexpr int kWaves = 8;     // waves per workgroup: 8 x 32 rows / columns
constexpr int kRows = kWaves * 32;
constexpr int kXcds = 8;

struct HotArgs {
  RelArgs r;
  int Tp;                        // T rounded up to kTile
  const unsigned char* tok_ok;   // [B][Tp] token validity
  const int* first2;             // [B][2] first and second valid token of each sequence (T if none)
  const float* nl_s;             // backward: [B*Hq][Tp] -lse_s*log2(e), -inf for excluded rows
  const float* nl_t;
  float* lse_s_out;              // fwd: [B, Hq, T]
  float* lse_t_out;
  float* row_out;                // fwd: per-row KL
  float* dq_out;                 // dq: [B, Hq, T, Ds]
  // Fused row-gradient forward only: each side's keys as float16 (the input
  // itself for float16 inputs, a scaled copy for bfloat16 ones) and the
  // device scalar 2^-e they were scaled by (NULL: 1).
  const u16* k16;  // student
  int64_t k16_sb, k16_sh, k16_st;
  const float* k16_scale;
  const u16* k16t;  // teacher
  int64_t k16t_sb, k16t_sh, k16t_st;
  const float* k16t_scale;
};

// LDS byte address of a pointer into a __shared__ array.  Taken where the
// array itself is named (lds_addr(lk[buf][0])), the cast folds to the
// array's constant address plus the index arithmetic, all 32-bit and scalar;
// a generic pointer carried into a helper first costs a 64-bit add and a
// null check per use.
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return (unsigned)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

// 16 bytes per lane HBM -> LDS: lane l copies base + voff (bytes) to LDS
// byte address lds + 16*l.  The base is uniform (an SGPR pair, the "saddr"
// form, so each copy needs one VGPR offset), and so is the LDS destination
// (M0).
// Issued as inline asm on purpose: the compiler cannot prove that later
// ds_reads of OTHER ring buffers do not alias the copies in flight, and for
// the builtin it inserts s_waitcnt vmcnt(0) before every LDS read, which
// serialises the ring.  The kernels order the copies themselves with
// wait_vmcnt<N>() + a barrier; the "memory" clobber keeps the compiler from
// moving LDS accesses across the issue point.  M0 is written here and listed
// as clobbered (the compiler notes that it reserves M0): no compiler-generated
// code in these kernels uses M0 (every M0 write in the kernels' assembly is
// this statement's), so no value of its own is live across a copy.
__device__ __forceinline__ void lds_async16(const void* base, unsigned voff, unsigned lds_chunk0) {
  // readfirstlane is int -> int: both halves go back through unsigned so the
  // low word is zero-extended (a sign-extended low word would corrupt the
  // high word of the address).
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const unsigned lo = static_cast<unsigned>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<unsigned>(b))));
  const unsigned hi =
      static_cast<unsigned>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<unsigned>(b >> 32))));
  const uint64_t sbase = (static_cast<uint64_t>(hi) << 32) | static_cast<uint64_t>(lo);
  const unsigned lds = __builtin_amdgcn_readfirstlane(lds_chunk0);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sbase), "s"(lds)
               : "memory", "m0");
}

// Wait until at most N vector-memory operations of this wave are in flight
// (expcnt / lgkmcnt fields left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate");
  // gfx9 encoding: vmcnt = simm16[15:14]:[3:0], expcnt [6:4], lgkmcnt [11:8]
  __builtin_amdgcn_s_waitcnt(0xF70 | (N & 15) | ((N >> 4) << 14));
}

// Position of workgroup `bid` in a work list of n items after the XCD-aware
// renumbering: XCD x = bid % 8 gets the contiguous range starting at
// x * (n / 8) + min(x, n % 8).
__device__ __forceinline__ int xcd_item(int bid, int n) {
  const int x = bid % kXcds, m = bid / kXcds;
  const int base = n / kXcds, rem = n % kXcds;
  return x * base + min(x, rem) + m;
}

// Swizzled row tile [kTile][DP]: chunk c (8 elements) of row r is stored at
// chunk slot r*CPR + (c ^ swz(r)).  The read patterns that must be free of
// bank conflicts (64 banks x 4 bytes): 16 consecutive rows at one chunk (the
// 16-byte operand reads), and for the transposing reads of the backward,
// aligned blocks of 4 rows x 4 chunks.  For D = 128, swz(r) = 4(r%4) +
// 2((r/4)%2) + (r/8)%2 is a bijection on 16 consecutive rows and sends such
// a block to 16 distinct slots (the plain r%16 sends it to 4 slots).
template <int DP>
__device__ __forceinline__ int swz(int r) {
  if constexpr (DP == 128)
    return 4 * (r & 3) + 2 * ((r >> 2) & 1) + ((r >> 3) & 1);
  else
    return r & (DP / 8 - 1);
}

template <int DP>
__device__ __forceinline__ int row_chunk_off(int r, int c) {  // u16 elements
  constexpr int CPR = DP / 8;
  return (r * CPR + (c ^ swz<DP>(r))) * 8;
}

template <int DP>
__device__ __forceinline__ const u16* row_chunk(const u16* tile, int r, int c) {
  return tile + row_chunk_off<DP>(r, c);
}

// Copies per wave per tile.  They are uniform across waves when the chunk
// count of a tile is a multiple of the wave count (D >= 64); otherwise the
// kernels wait for everything (vmcnt 0) and lose only the look-ahead.
template <int DP, int NW = kWaves>
struct TileCopies {
  static constexpr int kRowInst = kTile * (DP / 8) / 64;  // per row tile
  static constexpr bool kUniform = kRowInst % NW == 0;
  static constexpr int kRowPerWave = kRowInst / NW;
};

// Issue the async copy of rows [row0, row0 + kTile) x [0, DP) of one head
// (src = its row 0, rows row_stride elements apart) into the row tile at LDS
// byte address `tile` (lds_addr of the tile; copy n fills bytes
// [1024 n, 1024 n + 1024) of it).  Rows
// >= T and column chunks >= dim copy clamped, finite data instead of zeros:
// every consumer zeroes or masks their contribution (key rows >= T are
// invalid tokens, query rows >= T have -inf normalisers, padded columns meet
// zero register operands).  The host keeps every offset below 2^31 bytes.
template <int DP, int NW = kWaves>
__device__ __forceinline__ void issue_rows(unsigned tile, const u16* src, int row_stride, int row0, int T, int dim,
                                           int wave, int lane) {
  constexpr int CPR = DP / 8;
  constexpr int NINST = TileCopies<DP>::kRowInst;
  // a compile-time trip count when the copies divide evenly (no branches)
  constexpr int NITER = NINST % NW == 0 ? NINST / NW : (NINST + NW - 1) / NW;
#pragma unroll
  for (int i = 0; i < NITER; ++i) {
    const int n = wave + NW * i;
    if (NINST % NW != 0 && n >= NINST) break;
    const int p = 64 * n + lane;
    const int r = p / CPR;
    int c = (p % CPR) ^ swz<DP>(r);  // logical chunk stored at this slot (XOR is an involution)
    c = c * 8 < dim ? c : 0;
    const int row = min(row0 + r, T - 1);
    lds_async16(src, (unsigned)(row * row_stride + c * 8) * 2u, tile + 1024u * n);
  }
}

// issue_rows with the per-lane byte offsets of a full tile computed once:
// a full tile then costs one uniform base pointer and the copies; the last,
// partial tile (rows clamped to T - 1) goes through issue_rows.
template <int DP, int NW = kWaves>
struct RowCopier {
  static constexpr int CPR = DP / 8;
  static constexpr int NINST = TileCopies<DP, NW>::kRowInst;
  static constexpr int NITER = NINST % NW == 0 ? NINST / NW : (NINST + NW - 1) / NW;
  unsigned voff[NITER];
  __device__ __forceinline__ void init(int row_stride, int dim, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < NITER; ++i) {
      const int p = 64 * (wave + NW * i) + lane;
      const int r = p / CPR;
      int c = (p % CPR) ^ swz<DP>(r);
      c = c * 8 < dim ? c : 0;
      voff[i] = (unsigned)(r * row_stride + c * 8) * 2u;
    }
  }
  __device__ __forceinline__ void issue(unsigned tile, const u16* src, int row_stride, int row0, int T, int dim,
                                        int wave, int lane) const {
    if (row0 + kTile <= T) {
      const u16* base = src + (int64_t)row0 * row_stride;
#pragma unroll
      for (int i = 0; i < NITER; ++i) {
        const int n = wave + NW * i;
        if (NINST % NW != 0 && n >= NINST) break;
        lds_async16(base, voff[i], tile + 1024u * n);
      }
    } else {
      issue_rows<DP, NW>(tile, src, row_stride, row0, T, dim, wave, lane);
    }
  }
};

// One copy per wave: 64 bytes (lanes 0-3, 16 each) of `src` into LDS byte
// address `slot`.
__device__ __forceinline__ void issue_small(unsigned slot, const void* src, int lane) {
  if (lane < 4) lds_async16(src, 16u * lane, slot);
}

// ----------------------------------------------------------------------------
// forward: both online softmaxes and the KL, one pass (2 GEMMs per pair)
//
// Softmax state: each lane keeps its own running maxima for its half of the
// row's keys (lanes l and l+32 share a row), so the loop needs no cross-lane
// exchange; the halves are merged once at the end.  The maxima are lazy (a
// rescale only when a sub-block's sums exceed kLazySum = 2^20, see
// add_block), in raw logit units; a negative scale is handled by flipping
// the sign of q (exact), so the effective scale is positive.  Masked elements
// (causal diagonal, invalid keys) are set to -1e30 in place: with running
// maxima starting at -5e29 their exponentials are exactly 0 and every product
// stays finite.
// ----------------------------------------------------------------------------
constexpr float kMaskedLogit = -1e30f;  // raw logit of a masked element
constexpr float kStartMax = -5e29f;     // running max before the first valid key

// Online-softmax state of one query row for this lane's half of the keys.
// The exponent argument of a logit s is x = fma(s, c2, nm), its log2-domain
// value relative to the stabiliser -nm; the KL term accumulates
// p_t * (x_t - x_s), a difference of max-relative values, so a row dominated
// by one key (logits far above the rest) loses nothing to cancellation, and
// identical relations give exactly 0.
struct SoftRow {
  float m_s, m_t;    // running maxima, raw (sign-corrected) logit units
  float nm_s, nm_t;  // -m * c2 (log2 units)
  float l_s, l_t;    // sums of exp2(x_s), exp2(x_t)
  float acc;         // sum of exp2(x_t) * (x_t - x_s)
};

// Set the invalid elements of a masked sub-block to kMaskedLogit.  Element r
// of this lane is key (first + off(r)), off(r) = 8*(r/4) + r%4; it is valid
// when bit off(r) of `bits` is set and (causal) off(r) <= lim = row - first.
__device__ __forceinline__ void mask_block(f32x16& ss, f32x16& st, unsigned bits, int lim, bool causal) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int off = 8 * (r >> 2) + (r & 3);
    const bool v = ((bits >> off) & 1u) && (!causal || off <= lim);
    ss[r] = v ? ss[r] : kMaskedLogit;
    st[r] = v ? st[r] : kMaskedLogit;
  }
}

// Partial sums of one sub-block against the running maxima.
struct BlockSums {
  float s, t, a;  // sum p_s, sum p_t, sum p_t * (x_t - x_s)   (unnormalised)
};

__device__ __forceinline__ BlockSums block_sums(const f32x16& ss, const f32x16& st, const SoftRow& R, float c2s,
                                                float c2t) {
  float s0 = 0.f, s1 = 0.f, t0 = 0.f, t1 = 0.f, a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int r = 0; r < 16; r += 2) {
    const float xt0 = fmaf(st[r], c2t, R.nm_t), xt1 = fmaf(st[r + 1], c2t, R.nm_t);
    const float xs0 = fmaf(ss[r], c2s, R.nm_s), xs1 = fmaf(ss[r + 1], c2s, R.nm_s);
    const float pt0 = fast_exp2(xt0), pt1 = fast_exp2(xt1);
    s0 += fast_exp2(xs0);
    s1 += fast_exp2(xs1);
    t0 += pt0;
    t1 += pt1;
    a0 = fmaf(pt0, xt0 - xs0, a0);
    a1 = fmaf(pt1, xt1 - xs1, a1);
  }
  return {s0 + s1, t0 + t1, a0 + a1};
}

// Stabiliser -m * c2 of a running maximum m, as a rounded product the
// compiler may not fuse into a later subtraction: two equal maxima must give
// stabilisers whose difference is exactly 0 (a fused fma(-m, c2, -nm) would
// leave the product's rounding error, ~1e21 for the start value kStartMax).
__device__ __forceinline__ float stabiliser(float m, float c2) { return mul_rn(-m, c2); }

// Move a lane's sums from the stabilisers (nm_s, nm_t) to (ns, nt) (log2
// units, ns <= nm_s and nt <= nm_t): every exponent argument x drops by
// nm - n, so the sums scale by exp2(n - nm) and each x_t - x_s term gains
// (nt - nm_t) - (ns - nm_s).  With no term yet (l_t == 0) acc stays 0.
__device__ __forceinline__ void restabilise(float& l_s, float& l_t, float& acc, float nm_s, float nm_t, float ns,
                                            float nt) {
  const float cs = fast_exp2(ns - nm_s), ct = fast_exp2(nt - nm_t);
  acc = ct * fmaf(l_t, (nt - nm_t) - (ns - nm_s), acc);
  l_s *= cs;
  l_t *= ct;
}

// Raise the running maxima to the sub-block's maxima where those are larger,
// rescaling the sums.
__device__ __forceinline__ void raise_max(const f32x16& ss, const f32x16& st, SoftRow& R, float c2s, float c2t) {
  float mb_s = fmaxf(ss[0], ss[1]), mb_t = fmaxf(st[0], st[1]);
#pragma unroll
  for (int r = 2; r < 16; r += 2) {
    mb_s = fmaxf(fmaxf(mb_s, ss[r]), ss[r + 1]);
    mb_t = fmaxf(fmaxf(mb_t, st[r]), st[r + 1]);
  }
  const float ms = fmaxf(mb_s, R.m_s), mt = fmaxf(mb_t, R.m_t);
  const float ns = stabiliser(ms, c2s), nt = stabiliser(mt, c2t);
  restabilise(R.l_s, R.l_t, R.acc, R.nm_s, R.nm_t, ns, nt);
  R.m_s = ms;
  R.m_t = mt;
  R.nm_s = ns;
  R.nm_t = nt;
}

// Lazy maxima, checked on the sums: a lane's sub-block sums stay below
// kLazySum (so every exponential is below it) unless a logit exceeds the
// running max by more than log2(kLazySum) = 20 in log2 units, or the running
// max is still kStartMax (the sums are then +inf).  Only then (a uniform,
// rare branch: in practice the first valid sub-block of a row) are the
// maxima raised and the sub-block recomputed.  Sums kept this way stay below
// 2^20 * T < 2^52: no overflow, and fp32 relative precision throughout (the
// exponentials below the running max lose nothing they would not lose
// against the true max, which is at most 2^20 larger).
constexpr float kLazySum = 1048576.f;  // 2^20

__device__ __forceinline__ void add_block(const f32x16& ss, const f32x16& st, BlockSums bs, SoftRow& R, float c2s,
                                          float c2t) {
  if (__any(!(bs.s <= kLazySum) || !(bs.t <= kLazySum))) {
    raise_max(ss, st, R, c2s, c2t);
    bs = block_sums(ss, st, R, c2s, c2t);
  }
  R.l_s += bs.s;
  R.l_t += bs.t;
  R.acc += bs.a;
}

// S = K Q^T for one 32-key sub-block (rows r0.. of the swizzled student LDS
// tile ks; the teacher tile follows it), both relations: 2 x DP/16 MFMAs.
template <int DP, bool BF>
__device__ __forceinline__ void sub_scores(const u16* ks, int r0, int l32, int half, const u16x8* fq_s,
                                           const u16x8* fq_t, f32x16& ss, f32x16& st) {
  ss = (f32x16)(0.f);
  st = (f32x16)(0.f);
#pragma unroll
  for (int kk = 0; kk < DP / 16; ++kk) {
    const u16* p = row_chunk<DP>(ks, r0 + l32, 2 * kk + half);
    ss = mfma32<BF>(*reinterpret_cast<const u16x8*>(p), fq_s[kk], ss);
    st = mfma32<BF>(*reinterpret_cast<const u16x8*>(p + kTile * DP), fq_t[kk], st);
  }
}

// One pipeline step of the forward: the scores of the next sub-block
// (ns, nt; LDS row `row` of the student tile `ks`, whose teacher tile
// follows it) and the softmax sums of the current one (ss, st),
// interleaved by hand: each k-step's two MFMAs are followed by the VALU work
// of 16/KS of the current sub-block's elements, and scheduling barriers keep
// that order, so the matrix unit and the VALU work at the same time within
// the wave.  LDS operands are read PD k-steps ahead.
//
// PRE_IN: the first k-step's operands were read by the previous step into
// pre (the K/Q chunks of this sub-block); PRE_OUT: the last k-step also reads
// the first k-step's operands of row `pre_row` of the same tile into pre,
// for the next step.
template <int DP, bool BF, int PD = 2, bool PRE_IN = false, bool PRE_OUT = false>
__device__ __forceinline__ BlockSums scores_and_sums(const u16* ks, int row, int half,
                                                     const u16x8* fq_s, const u16x8* fq_t, f32x16& ns, f32x16& nt,
                                                     const f32x16& ss, const f32x16& st, const SoftRow& R, float c2s,
                                                     float c2t, u16x8* pre = nullptr, int pre_row = 0) {
  constexpr int KS = DP / 16, EP = 16 / KS;
  u16x8 os[KS], ot[KS];
  auto load = [&](int kk) {
    const u16* p = row_chunk<DP>(ks, row, 2 * kk + half);
    os[kk] = *reinterpret_cast<const u16x8*>(p);
    ot[kk] = *reinterpret_cast<const u16x8*>(p + kTile * DP);  // same slot of the teacher tile
  };
#pragma unroll
  for (int kk = 0; kk < PD && kk < KS; ++kk) {
    if (PRE_IN && kk == 0) {
      os[0] = pre[0];
      ot[0] = pre[1];
    } else {
      load(kk);
    }
  }
  ns = (f32x16)(0.f);
  nt = (f32x16)(0.f);
  float s0 = 0.f, s1 = 0.f, t0 = 0.f, t1 = 0.f, a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    if (kk + PD < KS) load(kk + PD);
    if (PRE_OUT && kk == KS - 1) {
      const u16* p = row_chunk<DP>(ks, pre_row, half);
      pre[0] = *reinterpret_cast<const u16x8*>(p);
      pre[1] = *reinterpret_cast<const u16x8*>(p + kTile * DP);
    }
    ns = mfma32<BF>(os[kk], fq_s[kk], ns);
    nt = mfma32<BF>(ot[kk], fq_t[kk], nt);
#pragma unroll
    for (int e = 0; e < EP; e += 2) {
      const int r = kk * EP + e;
      // all exponent arguments first, then the four exponentials back to
      // back, then the sums: no fma -> exp -> add dependency at issue
      float xt0 = fmaf(st[r], c2t, R.nm_t), xt1 = fmaf(st[r + 1], c2t, R.nm_t);
      float xs0 = fmaf(ss[r], c2s, R.nm_s), xs1 = fmaf(ss[r + 1], c2s, R.nm_s);
      asm volatile("" : "+v"(xt0), "+v"(xt1), "+v"(xs0), "+v"(xs1));
      const float d0 = xt0 - xs0, d1 = xt1 - xs1;
      const float pt0 = fast_exp2(xt0), pt1 = fast_exp2(xt1);
      const float ps0 = fast_exp2(xs0), ps1 = fast_exp2(xs1);
      s0 += ps0;
      s1 += ps1;
      t0 += pt0;
      t1 += pt1;
      a0 = fmaf(pt0, d0, a0);
      a1 = fmaf(pt1, d1, a1);
    }
    // the empty asm consumes this k-step's sums, so no IR pass can sink their
    // arithmetic past the scheduling barrier
    asm volatile("" : "+v"(s0), "+v"(s1), "+v"(t0), "+v"(t1), "+v"(a0), "+v"(a1));
    __builtin_amdgcn_sched_barrier(0);
  }
  return {s0 + s1, t0 + t1, a0 + a1};
}

template <int DP, bool BF>
__device__ __forceinline__ void hot_fwd_body(const HotArgs& f, int item) {
  const RelArgs& a = f.r;
  using TC = TileCopies<DP>;
  constexpr int KS = DP / 16;
  constexpr int kPerWave = 2 * TC::kRowPerWave + 1;  // K_s rows, K_t rows, token validity
  // Four tile buffers = two pairs: one pair is consumed while the next lands;
  // one barrier per pair (4 sub-blocks).
  constexpr int kBufs = 4;
  static_assert((kBufs & (kBufs - 1)) == 0, "ring indices are masked with kBufs - 1");
  __shared__ __attribute__((aligned(16))) u16 lk[kBufs][2][kTile * DP];  // [buffer][student, teacher]
  __shared__ __attribute__((aligned(16))) unsigned char ltok[kBufs][kWaves][kTile];  // one copy per wave

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches below
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int T = a.T;
  const int nrb = (T + kRows - 1) / kRows;
  const int bh = item / nrb;
  const int rb = nrb - 1 - (item - bh * nrb);  // longest causal rows first
  const int b = bh / a.Hq;
  const int h = bh - b * a.Hq;
  const int row0 = rb * kRows;
  const int my_i = row0 + w * 32 + l32;
  const bool in_range = my_i < T;
  const bool row_valid = in_range && mask_at(a.mask, a.mask_kind, (int64_t)b * a.mask_sb + my_i);
  const int causal = a.causal;
  const int diag_sb = (row0 >> 5) + w;  // this wave's diagonal 32-key sub-block

  // Negative scales: flip the sign of q (exact) so the effective scale is positive.
  const u16 flip_s = a.s.scale < 0.f ? 0x8000 : 0, flip_t = a.t.scale < 0.f ? 0x8000 : 0;
  u16x8 fq_s[KS], fq_t[KS];
  {
    const u16* ps = a.s.q + (int64_t)b * a.s.q_sb + (int64_t)h * a.s.q_sh + (int64_t)my_i * a.s.q_st;
    const u16* pt = a.t.q + (int64_t)b * a.t.q_sb + (int64_t)h * a.t.q_sh + (int64_t)my_i * a.t.q_st;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int d0 = 16 * kk + 8 * half;
      const bool ld = in_range && d0 < a.s.dim;
      fq_s[kk] = ld ? (*reinterpret_cast<const u16x8*>(ps + d0) ^ flip_s) : (u16x8)(0);
      fq_t[kk] = ld ? (*reinterpret_cast<const u16x8*>(pt + d0) ^ flip_t) : (u16x8)(0);
    }
  }

  const float c2s = fabsf(a.s.scale2), c2t = fabsf(a.t.scale2);  // raw logit -> log2 units
  SoftRow R = {kStartMax, kStartMax, stabiliser(kStartMax, c2s), stabiliser(kStartMax, c2t), 0.f, 0.f, 0.f};

  const int hs = h / a.s.group, ht = h / a.t.group;
  const u16* ks_base = a.s.k + (int64_t)b * a.s.k_sb + (int64_t)hs * a.s.k_sh;
  const u16* kt_base = a.t.k + (int64_t)b * a.t.k_sb + (int64_t)ht * a.t.k_sh;
  const unsigned char* tok = f.tok_ok + (int64_t)b * f.Tp;

  const int nkt_all = f.Tp / kTile;
  const int ntiles = causal ? min(nkt_all, (row0 + kRows - 1) / kTile + 1) : nkt_all;
  // causal: the diagonal tiles first, so the running max is set by the
  // dominant self-similarity and rescales are rare
  auto tile_of = [&](int it) { return causal ? ntiles - 1 - it : it; };
  RowCopier<DP> cp_s, cp_t;
  cp_s.init((int)a.s.k_st, a.s.dim, w, lane);
  cp_t.init((int)a.t.k_st, a.t.dim, w, lane);
  auto issue_tile = [&](int it) {
    const int buf = it & (kBufs - 1);
    const int j0 = tile_of(it) * kTile;
    cp_s.issue(lds_addr(lk[buf][0]), ks_base, (int)a.s.k_st, j0, T, a.s.dim, w, lane);
    cp_t.issue(lds_addr(lk[buf][1]), kt_base, (int)a.t.k_st, j0, T, a.t.dim, w, lane);
    issue_small(lds_addr(ltok[buf][w]), tok + j0, lane);
  };

  // Software pipeline over 32-key sub-blocks k = 2*tile + sb: the scores of
  // sub-block k+1 are computed while the softmax sums of sub-block k run.
  // Sub-blocks above the causal diagonal are not skipped but fully masked:
  // every wave then runs the same straight-line steps, and the wave holding
  // the last rows (which has no such sub-block) sets the pace anyway.
  struct Sub {
    f32x16 s, t;
    uint64_t tm;  // token validity of its tile, bit j = key j of the tile
  };
  auto scores = [&](Sub& x, int it, int sb) {
    const int buf = it & (kBufs - 1);
    x.tm = __ballot(ltok[buf][w][lane] != 0);  // read now: the buffer is refilled before its softmax
    sub_scores<DP, BF>(lk[buf][0], 32 * sb, l32, half, fq_s, fq_t, x.s, x.t);
  };
  auto prepare = [&](Sub& x, int it, int sb) {
    const int kt0 = tile_of(it) * kTile;
    const int gsb = (kt0 >> 5) + sb;  // global 32-key sub-block index
    if (x.tm != ~0ull || (causal && gsb >= diag_sb)) {
      const int first = kt0 + 32 * sb + 4 * half;
      mask_block(x.s, x.t, (unsigned)(x.tm >> (32 * sb + 4 * half)), my_i - first, causal);
    }
  };
  // softmax of cur (tile it, half sb) while the scores of nxt (tile it2, half sb2) run.
  // Scoring half 0 of a tile also reads the first operands of its half 1
  // (same tile, no barrier between), which the next step scores.
  u16x8 pre[2];
  auto step = [&](Sub& cur, int it, int sb, Sub& nxt, int it2, int sb2) {
    prepare(cur, it, sb);
    const int buf = it2 & (kBufs - 1);
    nxt.tm = __ballot(ltok[buf][w][lane] != 0);  // read now: the buffer is refilled before its softmax
    BlockSums bs;
    if (sb2 == 0)
      bs = scores_and_sums<DP, BF, 2, false, true>(lk[buf][0], l32, half, fq_s, fq_t, nxt.s, nxt.t, cur.s, cur.t, R,
                                                   c2s, c2t, pre, 32 + l32);
    else
      bs = scores_and_sums<DP, BF, 2, true, false>(lk[buf][0], 32 + l32, half, fq_s, fq_t, nxt.s, nxt.t, cur.s,
                                                   cur.t, R, c2s, c2t, pre);
    add_block(cur.s, cur.t, bs, R, c2s, c2t);
  };
  auto last = [&](Sub& cur, int it, int sb) {
    prepare(cur, it, sb);
    add_block(cur.s, cur.t, block_sums(cur.s, cur.t, R, c2s, c2t), R, c2s, c2t);
  };

  // The register operands loaded above must have landed before the ring
  // starts: the compiler does not count the asm copies, so a wait it placed
  // for these loads inside the loop would be vmcnt(0) and drain the ring.
  wait_vmcnt<0>();
  for (int it = 0; it < 4 && it < ntiles; ++it) issue_tile(it);
  if (TC::kUniform && ntiles >= 4)
    wait_vmcnt<2 * kPerWave>();  // pair 0 landed, pair 1 in flight
  else if (TC::kUniform && ntiles == 3)
    wait_vmcnt<kPerWave>();
  else
    wait_vmcnt<0>();
  __syncthreads();

  // sub-block k = 2 * tile + half; A holds the even ones, B the odd ones
  const int nsub = 2 * ntiles;
  Sub A, B;
  scores(A, 0, 0);
  {  // the first operands of half 1 of tile 0 (see step)
    const u16* p = row_chunk<DP>(lk[0][0], 32 + l32, half);
    pre[0] = *reinterpret_cast<const u16x8*>(p);
    pre[1] = *reinterpret_cast<const u16x8*>(p + kTile * DP);
  }
  for (int k = 0;; k += 2) {
    step(A, k >> 1, 0, B, k >> 1, 1);
    if (k + 2 >= nsub) {
      last(B, k >> 1, 1);
      break;
    }
    if ((k & 3) == 2) {  // sub-block k + 2 starts the next tile pair
      wait_vmcnt<0>();   // which landed (it was issued one pair ago)
      __syncthreads();   // ... in every wave; this pair's buffers are free
      const int p4 = (k >> 1) + 3;
      if (p4 < ntiles) issue_tile(p4);
      step(B, k >> 1, 1, A, (k >> 1) + 1, 0);
      // the second tile one step later: all waves issuing their copies at
      // once would stall on the full memory queue
      if (p4 + 1 < ntiles) issue_tile(p4 + 1);
    } else {
      step(B, k >> 1, 1, A, (k >> 1) + 1, 0);
    }
  }

  // merge the two halves of the row: common maxima (the larger half keeps
  // its stabilisers exactly), sums moved to them
  const float ms = fmaxf(R.m_s, xor32(R.m_s)), mt = fmaxf(R.m_t, xor32(R.m_t));
  const float ns = stabiliser(ms, c2s), nt = stabiliser(mt, c2t);
  restabilise(R.l_s, R.l_t, R.acc, R.nm_s, R.nm_t, ns, nt);
  const float l_s = R.l_s + xor32(R.l_s);
  const float l_t = R.l_t + xor32(R.l_t);
  const float acc = R.acc + xor32(R.acc);
  const bool ok = row_valid && l_s > 0.f && l_t > 0.f;
  const float lg_s = fast_log2(l_s), lg_t = fast_log2(l_t);
  // A valid row with exactly one valid key (the first valid token of a
  // causal row; the only valid token otherwise) has P_s = P_t = 1 there: its
  // KL is exactly 0 and its LSE is the logit itself, rounded once as the
  // reference rounds S = dot * sm_scale (kernel_A.py:147-157, kernel_B.py:206-213).
  const bool one_key = row_valid && (causal ? my_i == f.first2[2 * b] : f.first2[2 * b + 1] >= T);
  const int64_t row_index = (int64_t)bh * T + my_i;
  if (in_range && half == 0) {
    const float ls = one_key ? mul_rn(ms, fabsf(a.s.scale)) : (l_s > 0.f ? (lg_s - ns) * kLn2 : kNegInf);
    const float lt = one_key ? mul_rn(mt, fabsf(a.t.scale)) : (l_t > 0.f ? (lg_t - nt) * kLn2 : kNegInf);
    f.lse_s_out[row_index] = row_valid ? ls : 0.f;
    f.lse_t_out[row_index] = row_valid ? lt : 0.f;
    // KL = E_pt[x_t - x_s] + ln(l_s / l_t): max-relative terms only, no two
    // rounded LSEs or maxima are subtracted
    const float wr = a.weight != nullptr ? *a.weight : 1.f;
    f.row_out[row_index] = ok && !one_key ? (acc / l_t + (lg_s - lg_t)) * kLn2 * wr : 0.f;
  }
}

// ----------------------------------------------------------------------------
// backward helpers
// ----------------------------------------------------------------------------
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// A operand of the second GEMM (m = 32 dims of block db, k-slots = the 16
// rows 16m..16m+15 of 32-row sub-block sb of a row-major swizzled
// [kTile][DP] tile), read with two transposing LDS loads
// (ds_read_b64_tr_b16: in each 16-lane group, lane t receives element t%4 of
// the 8 bytes that lane 4j + t/4 points at, j = 0..3).  Lane l (group
// G = l/16, u = l%16) points at row 16m + 8r + 4(G/2) + u/4, dims
// 32db + 16(G%2) + 4(u%4) .. +3, so lane l receives, for dim 32db + l%32,
// rows 16m + 8r + 4(l/32) + j: the k-slot order (0-3, 8-11, 4-7, 12-15) of
// the accumulator registers that D comes from.  The per-lane part of each
// address is computed once (off[r][db]); the rows 32sb + 16m add a
// compile-time offset.
template <int DP>
struct TrOffsets {
  static constexpr int NDB = DP >= 32 ? DP / 32 : 1;
  unsigned off[2][NDB];  // u16 elements
  __device__ __forceinline__ void init(int lane) {
    const int g = lane >> 4, u = lane & 15;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      int dim = 32 * db + 16 * (g & 1) + 4 * (u & 3);
      if (DP < 32) dim &= DP - 1;
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int row = 8 * r + 4 * (g >> 1) + (u >> 2);  // < 16: the swizzle of rows 16j + row is that of row
        off[r][db] = (unsigned)row_chunk_off<DP>(row, dim >> 3) + (dim & 7);
      }
    }
  }
  __device__ __forceinline__ u16x8 read(const u16* tile, int sb, int m, int db) const {
    const u16* base = tile + (32 * sb + 16 * m) * DP;
    s16x4 v[2];
#pragma unroll
    for (int r = 0; r < 2; ++r)
      v[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)((__attribute__((address_space(3))) u16*)(base + off[r][db])));
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    const s16x8 both = __builtin_shufflevector(v[0], v[1], 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(u16x8, both);
  }
};

// B operand of the second GEMM from 8 D values (k-slots in register order),
// rounded to the input dtype like kernel_C.py:233, two per v_cvt_pk.
template <bool BF>
__device__ __forceinline__ u16x8 pack_d(const float* d) {
  unsigned w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f32x2 x = {d[2 * i], d[2 * i + 1]};
    if constexpr (BF)
      w[i] = __builtin_bit_cast(unsigned, __builtin_convertvector(x, bf16x2));
    else
      w[i] = __builtin_bit_cast(unsigned, __builtin_convertvector(x, f16x2));
  }
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  return __builtin_bit_cast(u16x8, (u32x4){w[0], w[1], w[2], w[3]});
}

// ----------------------------------------------------------------------------
// Phase schedule of the backward kernels
//
// Each wave works through its 32-row (dq) or 32-column (dk) sub-blocks in
// alternating phases: an MFMA phase M(k) (GEMM1 of sub-block k, GEMM2 of
// sub-block k-1) and a VALU phase V(k) (D of sub-block k).  M(k) reads its
// LDS operands several MFMAs ahead; the two waves sharing a SIMD overlap one
// wave's MFMA phase with the other's VALU phase as they drift.
//
// Tile ring: four single-tile buffers.  Tile t is read by M(2t) .. M(2t+2)
// (GEMM2 of sub-block 2t+1 runs in M(2t+2)); V phases read at most the tile
// of their own sub-block.
// ----------------------------------------------------------------------------
template <int kPerWave, bool kUniform>
__device__ __forceinline__ void wait_first_tiles(int ntiles) {  // tile 0 landed, tiles 1 and 2 may be in flight
  if (kUniform && ntiles >= 3)
    wait_vmcnt<2 * kPerWave>();
  else if (kUniform && ntiles == 2)
    wait_vmcnt<kPerWave>();
  else
    wait_vmcnt<0>();
}

// Every wave runs M(0) V(0) M(1) .. freely; the workgroup meets once per
// tile, before M(2t+2): tile t+1 has landed (each wave waits for its own
// copies first), and every wave is past M(2t), the last reader of tile t-1,
// whose buffer then receives tile t+3.  issue_part(t, j) issues part j
// (student rows, teacher rows, side data) of tile t.
template <int kPerWave, bool kUniform, typename MPhase, typename VPhase, typename IssuePart>
__device__ __forceinline__ void free_run(int ntiles, MPhase mphase, VPhase vphase, IssuePart issue_part) {
  for (int t = 0; t < 3 && t < ntiles; ++t)
    for (int j = 0; j < 3; ++j) issue_part(t, j);
  wait_first_tiles<kPerWave, kUniform>(ntiles);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    mphase(2 * t);
    // parts 1 and 2 of tile t+2, one phase after part 0: all waves issuing
    // their copies at once would stall on the full memory queue
    if (t >= 1 && t + 2 < ntiles)
      for (int j = 1; j < 3; ++j) issue_part(t + 2, j);
    vphase(2 * t);
    mphase(2 * t + 1);
    vphase(2 * t + 1);
    if (t + 1 < ntiles) {
      if (kUniform && t + 2 < ntiles)
        wait_vmcnt<kPerWave>();  // tile t+1 landed, tile t+2 in flight
      else
        wait_vmcnt<0>();
      __syncthreads();
      if (t + 3 < ntiles) issue_part(t + 3, 0);
    }
  }
  mphase(2 * ntiles);  // GEMM2 of the last sub-block
}

// One MFMA phase of the backward: GEMM1 of a sub-block (S = A B^T for both
// relations; A: this lane's rows of the student tile t1 at the offsets g1off
// (the teacher tile follows it); B: register operands fb_s, fb_t) and GEMM2
// of the previous sub-block (acc[db] += (rows of tile t2, transposed) x D).  With one wave per SIMD in
// its MFMA phase, nothing hides LDS latency but the wave itself: the operand
// reads run PD MFMAs ahead of their use, and scheduling barriers keep that
// order.
template <int DP, bool BF, int PD = 6>
__device__ __forceinline__ void mfma_phase(const u16* t1, const unsigned* g1off, const u16x8* fb_s, const u16x8* fb_t,
                                           f32x16& ss, f32x16& st, const u16* t2, int sb2, const TrOffsets<DP>& tro,
                                           const u16x8* dop, f32x16* acc) {
  constexpr int KS = DP / 16;
  constexpr int NDB = DP >= 32 ? DP / 32 : 1;
  constexpr int N1 = 2 * KS;       // GEMM1 MFMAs: student / teacher alternating
  constexpr int N = N1 + 2 * NDB;  // then GEMM2: (m, db)
  u16x8 op[N];
  auto load = [&](int i) {
    if (i < N1) {
      op[i] = *reinterpret_cast<const u16x8*>(t1 + g1off[i >> 1] + ((i & 1) ? kTile * DP : 0));
    } else {
      const int j = i - N1;
      op[i] = tro.read(t2, sb2, j / NDB, j % NDB);
    }
  };
  ss = (f32x16)(0.f);
  st = (f32x16)(0.f);
  // while this wave feeds the matrix unit it goes first; the other wave of
  // the SIMD fills the gaps with its VALU phase
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int i = 0; i < PD && i < N; ++i) load(i);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    if (i + PD < N) load(i + PD);
    if (i < N1) {
      if (i & 1)
        st = mfma32<BF>(op[i], fb_t[i >> 1], st);
      else
        ss = mfma32<BF>(op[i], fb_s[i >> 1], ss);
    } else {
      const int j = i - N1;
      acc[j % NDB] = mfma32<BF>(op[i], dop[j / NDB], acc[j % NDB]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  __builtin_amdgcn_s_setprio(0);
}

// ----------------------------------------------------------------------------
// backward, row side: dq = sm_scale_s D K_s, one owner per query row
// ----------------------------------------------------------------------------
template <int DP, bool BF>
__device__ __forceinline__ void hot_dq_body(const HotArgs& f, int item) {
  const RelArgs& a = f.r;
  using TC = TileCopies<DP>;
  constexpr int KS = DP / 16;
  constexpr int NDB = DP >= 32 ? DP / 32 : 1;  // 32-wide dim blocks of dq
  constexpr int kPerWave = 2 * TC::kRowPerWave + 1;
  constexpr int kBufs = 4;
  static_assert((kBufs & (kBufs - 1)) == 0, "ring indices are masked with kBufs - 1");
  __shared__ __attribute__((aligned(16))) u16 lk[kBufs][2][kTile * DP];  // [buffer][student, teacher]
  __shared__ __attribute__((aligned(16))) unsigned char ltok[kBufs][kWaves][kTile];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int T = a.T;
  const int nrb = (T + kRows - 1) / kRows;
  const int bh = item / nrb;
  const int rb = nrb - 1 - (item - bh * nrb);
  const int b = bh / a.Hq;
  const int h = bh - b * a.Hq;
  const int row0 = rb * kRows;
  const int my_i = row0 + w * 32 + l32;
  const bool in_range = my_i < T;
  const int causal = a.causal;
  const int diag_sb = (row0 >> 5) + w;

  // Negative scales: flip the sign of q (exact) so the effective scale is
  // positive and masked logits (kMaskedLogit) give exactly 0.
  const u16 flip_s = a.s.scale < 0.f ? 0x8000 : 0, flip_t = a.t.scale < 0.f ? 0x8000 : 0;
  u16x8 fq_s[KS], fq_t[KS];
  {
    const u16* ps = a.s.q + (int64_t)b * a.s.q_sb + (int64_t)h * a.s.q_sh + (int64_t)my_i * a.s.q_st;
    const u16* pt = a.t.q + (int64_t)b * a.t.q_sb + (int64_t)h * a.t.q_sh + (int64_t)my_i * a.t.q_st;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int d0 = 16 * kk + 8 * half;
      const bool ld = in_range && d0 < a.s.dim;
      fq_s[kk] = ld ? (*reinterpret_cast<const u16x8*>(ps + d0) ^ flip_s) : (u16x8)(0);
      fq_t[kk] = ld ? (*reinterpret_cast<const u16x8*>(pt + d0) ^ flip_t) : (u16x8)(0);
    }
  }
  // Row normalisers in log2 units, -inf outside the valid set (exp2 -> 0).
  const float nls2 = in_range ? f.nl_s[(int64_t)bh * f.Tp + my_i] : kNegInf;
  const float nlt2 = in_range ? f.nl_t[(int64_t)bh * f.Tp + my_i] : kNegInf;
  const bool ok = nls2 != kNegInf;
  const float c2s = fabsf(a.s.scale2), c2t = fabsf(a.t.scale2);
  f32x16 dq[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dq[db] = (f32x16)(0.f);

  const int hs = h / a.s.group, ht = h / a.t.group;
  const u16* ks_base = a.s.k + (int64_t)b * a.s.k_sb + (int64_t)hs * a.s.k_sh;
  const u16* kt_base = a.t.k + (int64_t)b * a.t.k_sb + (int64_t)ht * a.t.k_sh;
  const unsigned char* tok = f.tok_ok + (int64_t)b * f.Tp;

  const int nkt_all = f.Tp / kTile;
  const int ntiles = causal ? min(nkt_all, (row0 + kRows - 1) / kTile + 1) : nkt_all;
  const int nsub = 2 * ntiles;
  RowCopier<DP> cp_s, cp_t;
  cp_s.init((int)a.s.k_st, a.s.dim, w, lane);
  cp_t.init((int)a.t.k_st, a.t.dim, w, lane);
  auto issue_part = [&](int t, int j) {
    const int buf = t & (kBufs - 1);
    const int j0 = t * kTile;
    if (j == 0)
      cp_s.issue(lds_addr(lk[buf][0]), ks_base, (int)a.s.k_st, j0, T, a.s.dim, w, lane);
    else if (j == 1)
      cp_t.issue(lds_addr(lk[buf][1]), kt_base, (int)a.t.k_st, j0, T, a.t.dim, w, lane);
    else
      issue_small(lds_addr(ltok[buf][w]), tok + j0, lane);
  };
  unsigned g1off[KS];  // this lane's row chunks of a tile: row l32 (+ 32 sb), chunk 2kk + half
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) g1off[kk] = (unsigned)row_chunk_off<DP>(l32, 2 * kk + half);
  TrOffsets<DP> tro;
  tro.init(lane);

  // Sub-block k = 2t + sb covers keys 32k .. 32k+31 (tile t, half sb).
  // Sub-blocks above the causal diagonal are fully masked, not skipped (the
  // wave holding the last rows, which has none, sets the pace).
  f32x16 ss, st;     // scores of the sub-block between its M and V phase
  uint64_t tm = 0;   // token validity of that sub-block's tile
  u16x8 dop[2] = {(u16x8)(0), (u16x8)(0)};  // D of the previous sub-block, the B operand of GEMM2
  // M(k): GEMM1 of sub-block k, GEMM2 of sub-block k-1 (dq += D K).  One
  // code path for every k: M(0) multiplies a zero D, M(nsub) recomputes the
  // scores of the last sub-block (still in LDS) and drops them.
  auto mphase = [&](int k) {
    const int k1 = min(k, nsub - 1), k2 = max(k - 1, 0);
    const int buf = (k1 >> 1) & (kBufs - 1);
    tm = __ballot(ltok[buf][w][lane] != 0);
    mfma_phase<DP, BF>(lk[buf][0] + 32 * (k1 & 1) * DP, g1off, fq_s, fq_t, ss, st, lk[(k2 >> 1) & (kBufs - 1)][0], k2 & 1,
                       tro, dop, dq);
  };
  auto vphase = [&](int k) {
    const int sb = k & 1;
    if (tm != ~0ull || (causal && k >= diag_sb)) {
      const int first = 32 * k + 4 * half;
      mask_block(ss, st, (unsigned)(tm >> (32 * sb + 4 * half)), my_i - first, causal);
    }
    float dd[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) dd[r] = fast_exp2(fmaf(ss[r], c2s, nls2)) - fast_exp2(fmaf(st[r], c2t, nlt2));
    dop[0] = pack_d<BF>(dd);  // D cast to the input dtype (kernel_C.py:233)
    dop[1] = pack_d<BF>(dd + 8);
  };

  wait_vmcnt<0>();  // register operands landed before the ring starts
  free_run<kPerWave, TC::kUniform>(ntiles, mphase, vphase, issue_part);

  if (in_range) {
    const float fs =
        ok ? a.s.scale * (a.dscale != nullptr ? *a.dscale * (a.weight != nullptr ? *a.weight : 1.f) : 1.f) : 0.f;
    float* out = f.dq_out + ((int64_t)bh * T + my_i) * a.s.dim;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * db + 8 * g + 4 * half;
        if (d0 < a.s.dim) {
          const f32x4 v = {dq[db][4 * g] * fs, dq[db][4 * g + 1] * fs, dq[db][4 * g + 2] * fs, dq[db][4 * g + 3] * fs};
          *reinterpret_cast<f32x4*>(out + d0) = v;
        }
      }
    }
  }
}


// GEMM1 of one sub-block (S = A B^T for both relations; A: this lane's row
// r0 + l32 of the swizzled student tile, the teacher tile following it; B:
// the register operands fb_s, fb_t), operands read PD MFMAs ahead.
template <int DP, bool BF, int PD = 4>
__device__ __forceinline__ void gemm1(const u16* tile, int r0, int l32, int half, const u16x8* fb_s,
                                      const u16x8* fb_t, f32x16& ss, f32x16& st) {
  constexpr int N = 2 * (DP / 16);  // student / teacher alternating
  u16x8 op[N];
  auto load = [&](int i) {
    op[i] = *reinterpret_cast<const u16x8*>(row_chunk<DP>(tile, r0 + l32, 2 * (i >> 1) + half) +
                                            ((i & 1) ? kTile * DP : 0));
  };
#pragma unroll
  for (int i = 0; i < PD && i < N; ++i) load(i);
  ss = (f32x16)(0.f);
  st = (f32x16)(0.f);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    if (i + PD < N) load(i + PD);
    if (i & 1)
      st = mfma32<BF>(op[i], fb_t[i >> 1], st);
    else
      ss = mfma32<BF>(op[i], fb_s[i >> 1], ss);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// ----------------------------------------------------------------------------
// backward, column side: dk = sm_scale_s sum_{h in group} D^T Q_s
// ----------------------------------------------------------------------------
template <int DP, bool BF>
__device__ __forceinline__ void hot_bwd_body(const HotArgs& f, int item) {
  const RelArgs& a = f.r;
  using TC = TileCopies<DP>;
  constexpr int KS = DP / 16;
  constexpr int NDB = DP >= 32 ? DP / 32 : 1;
  constexpr int kPerWave = 2 * TC::kRowPerWave + 1;
  constexpr int kBufs = 4;
  static_assert((kBufs & (kBufs - 1)) == 0, "ring indices are masked with kBufs - 1");
  __shared__ __attribute__((aligned(16))) u16 lq[kBufs][2][kTile * DP];  // [buffer][student, teacher]
  // per query row of the tile: -lse*log2(e) of student [0, 64) and teacher [64, 128)
  __shared__ __attribute__((aligned(16))) float lnl[kBufs][2 * kTile];
  static_assert(2 * kTile * sizeof(float) == kWaves * 64, "one 64-byte row-data copy per wave");
  static_assert(kWaves == 8 && 2 * kTile * sizeof(float) == 4 * 128, "refills: 4 waves, 128 bytes of row data each");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int T = a.T;
  const int ncb = (T + kRows - 1) / kRows;
  const int bg = item / ncb;
  const int cb = item - bg * ncb;  // small cb = longest causal columns first
  const int b = bg / a.s.hkv;
  const int g = bg - b * a.s.hkv;
  const int j0w = cb * kRows + w * 32;
  const int my_j = j0w + l32;
  const bool in_range = my_j < T;
  const bool col_valid = in_range && mask_at(a.mask, a.mask_kind, (int64_t)b * a.mask_sb + my_j);
  const int causal = a.causal;
  const int diag_sb = j0w >> 5;  // the 32-row sub-block holding this wave's diagonal

  u16x8 fk_s[KS], fk_t[KS];
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

  const float c2s = a.s.scale2, c2t = a.t.scale2;
  const int ntile_all = f.Tp / kTile;
  // Query tiles run from the last one down to this block's diagonal: all
  // workgroups in flight then read the same tile at the same time (one L2
  // fill serves the XCD), instead of each starting at its own diagonal.
  const int ntiles = causal ? ntile_all - (cb * kRows) / kTile : ntile_all;
  auto tile_of = [&](int it) { return ntile_all - 1 - it; };
  RowCopier<DP> cp_s, cp_t;
  cp_s.init((int)a.s.q_st, a.s.dim, w, lane);
  cp_t.init((int)a.t.q_st, a.t.dim, w, lane);
  // Ring refills come from waves 0-3 alone (wave & 3 is the SIMD): with two
  // waves per SIMD the older one wins issue arbitration and reaches each
  // barrier first, so its copy-issue stall overlaps the younger wave's compute
  // instead of stalling both waves of the SIMD.
  RowCopier<DP, 4> cq_s, cq_t;
  cq_s.init((int)a.s.q_st, a.s.dim, w & 3, lane);
  cq_t.init((int)a.t.q_st, a.t.dim, w & 3, lane);
  TrOffsets<DP> tro;
  tro.init(lane);
  int loaded_ht = -1;

  for (int hh = 0; hh < a.s.group; ++hh) {
    const int h = g * a.s.group + hh;
    const int ht = h / a.t.group;
    if (ht != loaded_ht) {
      const u16* p = a.t.k + (int64_t)b * a.t.k_sb + (int64_t)ht * a.t.k_sh + (int64_t)my_j * a.t.k_st;
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const int d0 = 16 * kk + 8 * half;
        fk_t[kk] = (in_range && d0 < a.t.dim) ? *reinterpret_cast<const u16x8*>(p + d0) : (u16x8)(0);
      }
      loaded_ht = ht;
    }
    const int64_t bh = (int64_t)b * a.Hq + h;
    const u16* qs_base = a.s.q + (int64_t)b * a.s.q_sb + (int64_t)h * a.s.q_sh;
    const u16* qt_base = a.t.q + (int64_t)b * a.t.q_sb + (int64_t)h * a.t.q_sh;
    // wave w copies 16 normalisers: student rows 16w.. (w < 4), teacher rows 16(w-4).. (w >= 4)
    const float* nl_src = (w < 4 ? f.nl_s : f.nl_t) + bh * f.Tp + 16 * (w & 3);

    auto issue_tile = [&](int it) {
      const int buf = it & (kBufs - 1);
      const int i0 = tile_of(it) * kTile;
      cp_s.issue(lds_addr(lq[buf][0]), qs_base, (int)a.s.q_st, i0, T, a.s.dim, w, lane);
      cp_t.issue(lds_addr(lq[buf][1]), qt_base, (int)a.t.q_st, i0, T, a.t.dim, w, lane);
      issue_small(lds_addr(&lnl[buf][16 * w]), nl_src + i0, lane);
    };
    // the same tile from waves 0-3 only; wave q = w & 3 copies 32 normalisers:
    // student rows 32q.. (q < 2), teacher rows 32(q-2).. (q >= 2)
    const float* nl_src4 = ((w & 3) < 2 ? f.nl_s : f.nl_t) + bh * f.Tp + 32 * (w & 1);
    auto issue_tile4 = [&](int it) {
      const int buf = it & (kBufs - 1);
      const int i0 = tile_of(it) * kTile;
      cq_s.issue(lds_addr(lq[buf][0]), qs_base, (int)a.s.q_st, i0, T, a.s.dim, w & 3, lane);
      cq_t.issue(lds_addr(lq[buf][1]), qt_base, (int)a.t.q_st, i0, T, a.t.dim, w & 3, lane);
      if (lane < 8) lds_async16(nl_src4 + i0, 16u * lane, lds_addr(&lnl[buf][32 * (w & 3)]));
    };
    auto compute_tile = [&](int it) {
      const int buf = it & (kBufs - 1);
      const int t = tile_of(it);
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        const int gsb = 2 * t + sb;
        if (causal && gsb < diag_sb) continue;
        f32x16 ss, st;
        __builtin_amdgcn_s_setprio(1);  // the MFMA-feeding wave goes first (see mfma_phase)
        gemm1<DP, BF, 4>(lq[buf][0], 32 * sb, l32, half, fk_s, fk_t, ss, st);
        __builtin_amdgcn_s_setprio(0);
        float dd[16];
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int ii0 = 32 * sb + 8 * r4 + 4 * half;
          const f32x4 ls4 = *reinterpret_cast<const f32x4*>(&lnl[buf][ii0]);
          const f32x4 lt4 = *reinterpret_cast<const f32x4*>(&lnl[buf][kTile + ii0]);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            dd[4 * r4 + e] = fast_exp2(fmaf(ss[4 * r4 + e], c2s, ls4[e])) - fast_exp2(fmaf(st[4 * r4 + e], c2t, lt4[e]));
        }
        if (causal && gsb == diag_sb) {
          const int lim = t * kTile + 32 * sb + 4 * half - my_j;  // row(r) - column = off(r) + lim
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int off = 8 * (r >> 2) + (r & 3);
            dd[r] = off + lim >= 0 ? dd[r] : 0.f;
          }
        }
        constexpr int N2 = 2 * NDB, P2 = N2 < 4 ? N2 : 4;
        u16x8 op2[N2];
#pragma unroll
        for (int i = 0; i < P2; ++i) op2[i] = tro.read(lq[buf][0], sb, i / NDB, i % NDB);
        const u16x8 bop[2] = {pack_d<BF>(dd), pack_d<BF>(dd + 8)};  // D cast to the input dtype (kernel_C.py:233)
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int i = 0; i < N2; ++i) {
          if (i + P2 < N2) op2[i + P2] = tro.read(lq[buf][0], sb, (i + P2) / NDB, (i + P2) % NDB);
          dk[i % NDB] = mfma32<BF>(op2[i], bop[i / NDB], dk[i % NDB]);
          __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_setprio(0);
      }
    };

    wait_vmcnt<0>();  // register operands landed before the ring starts
    for (int it = 0; it < 4 && it < ntiles; ++it) issue_tile(it);
    if (TC::kUniform && ntiles >= 4)
      wait_vmcnt<2 * kPerWave>();
    else if (TC::kUniform && ntiles == 3)
      wait_vmcnt<kPerWave>();
    else
      wait_vmcnt<0>();
    __syncthreads();
    for (int p = 0; p < ntiles; p += 2) {
      compute_tile(p);
      if (p + 1 < ntiles) compute_tile(p + 1);
      if (p + 2 < ntiles) {
        wait_vmcnt<0>();
        __syncthreads();
        if (w < 4) {
          if (p + 4 < ntiles) issue_tile4(p + 4);
          if (p + 5 < ntiles) issue_tile4(p + 5);
        }
      }
    }
    __syncthreads();  // every wave is done with the ring before the next head refills it
  }

  if (in_range) {
    const int64_t off = ((int64_t)bg * T + my_j) * a.s.dim;
    float* out = a.dk_out + off;
    const float fs = a.s.scale;
    const float mult = (a.dscale != nullptr ? *a.dscale : 1.f) * (a.weight != nullptr ? *a.weight : 1.f);
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int d0 = 32 * db + 8 * gq + 4 * half;
        if (d0 < a.s.dim) {
          f32x4 v = {dk[db][4 * gq] * fs, dk[db][4 * gq + 1] * fs, dk[db][4 * gq + 2] * fs, dk[db][4 * gq + 3] * fs};
          if (!col_valid) v = (f32x4)(0.f);  // masked key columns get no gradient (kernel_C.py:252-253)
          if (a.dk_add != nullptr) v += *reinterpret_cast<const f32x4*>(a.dk_add + off + d0);
          if (a.dscale != nullptr || a.weight != nullptr) v *= mult;
          *reinterpret_cast<f32x4*>(out + d0) = v;
        }
      }
    }
  }
}

// ----------------------------------------------------------------------------
// launch forms: one relation, or a batch of up to kMaxRelations relations in
// one grid (train.py:369-410 runs Q/Q, K/K and V/V of every layer; their
// head counts differ).  The batch travels in the kernel arguments, so a
// launch needs no device copy of it and stays valid under graph capture.
// ----------------------------------------------------------------------------
constexpr int kMaxRelations = 8;

struct HotBatch {
  int n;                          // relations
  int first[kMaxRelations + 1];   // work items before relation r; first[n] = total
  HotArgs rel[kMaxRelations];
};
// The batch travels by value as the kernel's argument block, whose size HIP
// limits to 4 KiB.
static_assert(sizeof(HotBatch) <= 4096, "HotBatch exceeds the 4 KiB kernel-argument limit");

// work items (workgroups) of one relation: row blocks x B x heads
__host__ __device__ inline int fwd_items(const HotArgs& f) { return (f.r.T + kRows - 1) / kRows * f.r.B * f.r.Hq; }
__host__ __device__ inline int bwd_items(const HotArgs& f) {
  return (f.r.T + kRows - 1) / kRows * f.r.B * f.r.s.hkv;
}

// relation r of batch item g (uniform: a short scalar loop)
__device__ __forceinline__ int batch_relation(const HotBatch& m, int g) {
  int r = 0;
  while (r + 1 < m.n && g >= m.first[r + 1]) ++r;
  return r;
}

template <int DP, bool BF>
__global__ __launch_bounds__(kWaves * 64) void hot_fwd_kernel(const HotArgs f) {
  hot_fwd_body<DP, BF>(f, xcd_item(blockIdx.x, fwd_items(f)));
}
template <int DP, bool BF>
__global__ __launch_bounds__(kWaves * 64) void hot_dq_kernel(const HotArgs f) {
  hot_dq_body<DP, BF>(f, xcd_item(blockIdx.x, fwd_items(f)));
}
template <int DP, bool BF>
__global__ __launch_bounds__(kWaves * 64) void hot_bwd_kernel(const HotArgs f) {
  hot_bwd_body<DP, BF>(f, xcd_item(blockIdx.x, bwd_items(f)));
}
template <int DP, bool BF>
__global__ __launch_bounds__(kWaves * 64) void hot_fwd_batch_kernel(const HotBatch m) {
  const int g = xcd_item(blockIdx.x, m.first[m.n]);
  const int r = batch_relation(m, g);
  hot_fwd_body<DP, BF>(m.rel[r], g - m.first[r]);
}
template <int DP, bool BF>
__global__ __launch_bounds__(kWaves * 64) void hot_dq_batch_kernel(const HotBatch m) {
  const int g = xcd_item(blockIdx.x, m.first[m.n]);
  const int r = batch_relation(m, g);
  hot_dq_body<DP, BF>(m.rel[r], g - m.first[r]);
}
template <int DP, bool BF>
__global__ __launch_bounds__(kWaves * 64) void hot_bwd_batch_kernel(const HotBatch m) {
  const int g = xcd_item(blockIdx.x, m.first[m.n]);
  const int r = batch_relation(m, g);
  hot_bwd_body<DP, BF>(m.rel[r], g - m.first[r]);
}

bool hot_supported(int ds, int dt, bool same_dtype);
hipError_t launch_token_prep(const RelArgs& a, int Tp, unsigned char* tok_ok, int* first2, hipStream_t stream);
hipError_t launch_row_prep(const RelArgs& a, int Tp, const unsigned char* tok_ok, const int* first2, float* nl_s,
                           float* nl_t, hipStream_t stream);
hipError_t launch_hot_fwd(const HotArgs& f, int dp, bool bf16, hipStream_t stream);
hipError_t launch_hot_dq(const HotArgs& f, int dp, bool bf16, hipStream_t stream);
hipError_t launch_hot_bwd(const HotArgs& f, int dp, bool bf16, hipStream_t stream);
// batch: the relations' first[] is filled by the launcher
hipError_t launch_hot_fwd_batch(HotBatch& m, int dp, bool bf16, hipStream_t stream);
hipError_t launch_hot_dq_batch(HotBatch& m, int dp, bool bf16, hipStream_t stream);
hipError_t launch_hot_bwd_batch(HotBatch& m, int dp, bool bf16, hipStream_t stream);

}  // namespace lard
