// Fused forward of the autograd path that also forms the row side of the
// backward (AttnKLAlignFn.forward, integration.py:8-45, plus the dq half of
// kernel_C.py:224-239), for the shapes of the throughput kernels.
//
// Per query row i, one pass over its keys j computes both online softmaxes
// and the KL exactly as hot_fwd_kernel does, and in addition
//   O_s(i) = sum_j p~_s(i,j) k_s[j],   O_t(i) = sum_j p~_t(i,j) k_s[j],
// with p~ = exp2(S * c2 + nm) relative to the row's running stabiliser nm
// (the FlashAttention output accumulation, with the student keys as values
// for both relations).  At the end
//   dq_i = sm_scale_s * (O_s / l_s - O_t / l_t)
//        = sm_scale_s * sum_j (P_s - P_t)_ij k_s[j]          (kernel_C.py:236-239)
// is written as float32 without dloss (autograd supplies it in the backward,
// where the column kernel adds its own term and multiplies once).  The
// backward then runs only the column side: 14 d P MFMA flops per causal
// relation instead of 16 (forward 8, column side 6), and 4 exponentials per
// element instead of 6.
//
// Precision: P_s and P_t enter the products rounded separately (the
// reference rounds their difference D to the input type, kernel_C.py:233),
// so the error is relative to P rather than to D.  The kernel therefore
// runs in float16 whatever the input type: the output products with
// float16 probabilities (11 significant bits against bfloat16's 8, so 2^-12
// relative instead of 2^-9; the lazy maxima keep every probability below
// 2^15, inside float16's range), and both relations' scores from the same
// products as in the input type (a bfloat16 value is a float16 value,
// scaled by a power of two when its tensor holds values of 2^15 or more).
// Both sides go through the same conversion, so identical relations still
// give bitwise identical scores (the float16 and bfloat16 MFMAs need not
// round their sums alike).
//
// Layout: one wave per SIMD (4 waves x 32 query rows per workgroup), since
// the two output accumulators (2 x 4 x 16 float32 per lane at D = 128) do not
// fit two waves per SIMD.  Within the wave, step k interleaves the 16 MFMAs
// of the scores of sub-block k+1 and the 16 MFMAs of the output products of
// sub-block k-1 with the softmax of sub-block k, so the matrix unit and the
// VALU work of one wave overlap.  Running maxima are lazy as in the forward,
// but common to the two lane halves of a row (the product sums over both
// halves' keys), so a rescale exchanges the halves' block maxima once.
//
// Tile ring: four single-tile buffers, one barrier per tile.  Tile t is read
// by steps 2t-1 .. 2t+2 (scores of sub-blocks 2t and 2t+1 in steps 2t-1 and
// 2t, their output products in steps 2t+1 and 2t+2).  The barrier before
// step 2t-1 finds tile t landed and every wave past step 2t-2, the last
// reader of tile t-2, whose buffer then receives tile t+2.
#pragma once

#include <type_traits>

#include "hot_kernels.h"

namespace lard {

constexpr int kWavesQ = 4;            // waves per workgroup (one per SIMD)
constexpr int kRowsQ = kWavesQ * 32;  // query rows per workgroup

// Raise a row's running maxima to the sub-block maxima of both lane halves
// where those are larger; returns the factors (new / old) of the
// exponentials, by which the output accumulators must be scaled.
__device__ __forceinline__ void raise_max_row(const f32x16& ss, const f32x16& st, SoftRow& R, float c2s, float c2t,
                                              float& fs, float& ft) {
  float mb_s = fmaxf(ss[0], ss[1]), mb_t = fmaxf(st[0], st[1]);
#pragma unroll
  for (int r = 2; r < 16; r += 2) {
    mb_s = fmaxf(fmaxf(mb_s, ss[r]), ss[r + 1]);
    mb_t = fmaxf(fmaxf(mb_t, st[r]), st[r + 1]);
  }
  mb_s = fmaxf(mb_s, xor32(mb_s));
  mb_t = fmaxf(mb_t, xor32(mb_t));
  const float ms = fmaxf(mb_s, R.m_s), mt = fmaxf(mb_t, R.m_t);
  const float ns = stabiliser(ms, c2s), nt = stabiliser(mt, c2t);
  fs = fast_exp2(ns - R.nm_s);
  ft = fast_exp2(nt - R.nm_t);
  restabilise(R.l_s, R.l_t, R.acc, R.nm_s, R.nm_t, ns, nt);
  R.m_s = ms;
  R.m_t = mt;
  R.nm_s = ns;
  R.nm_t = nt;
}

// Exponentials of one sub-block against the running stabilisers, their
// sums and the packed operands (the recompute path of a rescale; pairs are
// packed as they are formed, so no array of exponentials stays live).
template <bool BF>
__device__ __forceinline__ BlockSums block_probs_packed(const f32x16& ss, const f32x16& st, const SoftRow& R,
                                                        float c2s, float c2t, unsigned* ws, unsigned* wt);

// Two floats rounded to the operand type, packed into one 32-bit word.
template <bool BF>
__device__ __forceinline__ unsigned pack2(float x, float y) {
  const f32x2 v = {x, y};
  if constexpr (BF)
    return __builtin_bit_cast(unsigned, __builtin_convertvector(v, bf16x2));
  else
    return __builtin_bit_cast(unsigned, __builtin_convertvector(v, f16x2));
}

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

template <bool BF>
__device__ __forceinline__ BlockSums block_probs_packed(const f32x16& ss, const f32x16& st, const SoftRow& R,
                                                        float c2s, float c2t, unsigned* ws, unsigned* wt) {
  float s = 0.f, t = 0.f, acc = 0.f;
#pragma unroll
  for (int r = 0; r < 16; r += 2) {
    const float xt0 = fmaf(st[r], c2t, R.nm_t), xs0 = fmaf(ss[r], c2s, R.nm_s);
    const float xt1 = fmaf(st[r + 1], c2t, R.nm_t), xs1 = fmaf(ss[r + 1], c2s, R.nm_s);
    const float pt0 = fast_exp2(xt0), pt1 = fast_exp2(xt1), ps0 = fast_exp2(xs0), ps1 = fast_exp2(xs1);
    s += ps0 + ps1;
    t += pt0 + pt1;
    acc = fmaf(pt0, xt0 - xs0, acc);
    acc = fmaf(pt1, xt1 - xs1, acc);
    ws[r >> 1] = pack2<BF>(ps0, ps1);
    wt[r >> 1] = pack2<BF>(pt0, pt1);
  }
  return {s, t, acc};
}


// Register classes: the scores live in VGPRs (the softmax reads them), the
// output accumulators and the query operands in AGPRs (only MFMAs touch
// them in the loop), which is what makes the kernel fit one wave's 512
// registers without spills.  The compiler's MFMA selection cannot mix the
// two accumulator classes, so every MFMA of this kernel is issued here as
// inline asm, and the compiler inserts none of the wait states gfx950
// requires around MFMAs it does not see:
//   * VALU write of an operand -> MFMA read: 2 wait states;
//   * MFMA write -> any other access of its result: up to 19 wait states
//     (11 + 1 for these 8-pass MFMAs);
//   * MFMA reading its own previous result as the accumulator (exactly the
//     same registers): none.
// The loop's schedule provides them (operands come from LDS reads or were
// packed a step earlier; a score chain's last MFMA is followed by the rest
// of the step before anything reads the scores), and tests/isa_check.py
// verifies every path of the compiled kernels against these rules; where
// the schedule alone would not be enough (the rescale and the epilogue
// reading the output accumulators) agpr_fence() / agpr_rescale() wait
// explicitly.  No VALU instruction writes an accumulator an MFMA in flight
// reads: the chains start from the constant 0.
template <bool BF>
__device__ __forceinline__ void mfma_first(f32x16& acc, u16x8 a, u16x8 b_agpr) {  // acc = A B
  if constexpr (BF)
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(acc) : "v"(a), "a"(b_agpr));
  else
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(acc) : "v"(a), "a"(b_agpr));
}
template <bool BF>
__device__ __forceinline__ void mfma_next(f32x16& acc, u16x8 a, u16x8 b_agpr) {  // acc += A B
  if constexpr (BF)
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "a"(b_agpr));
  else
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "a"(b_agpr));
}
// Output accumulator blocks live in fixed AGPR ranges: block IDX (student
// blocks 0 .. NDB-1, then the teacher's) in a[16 IDX : 16 IDX + 15].  Every
// access in the loop names its range, so the register allocator keeps each
// block in place across the rescale branch instead of copying all of them
// at the merge.
#define LARD_OACC(IDX, REGS)                                                                               \
  if constexpr (I == IDX) {                                                                                \
    if constexpr (BF)                                                                                      \
      asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+{" REGS "}"(acc) : "v"(a), "v"(b)); \
    else                                                                                                   \
      asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+{" REGS "}"(acc) : "v"(a), "v"(b));  \
  }
template <int I, bool BF>
__device__ __forceinline__ void mfma32_acc(f32x16& acc, u16x8 a, u16x8 b) {  // AGPR block I += A B
  LARD_OACC(0, "a[0:15]")
  LARD_OACC(1, "a[16:31]")
  LARD_OACC(2, "a[32:47]")
  LARD_OACC(3, "a[48:63]")
  LARD_OACC(4, "a[64:79]")
  LARD_OACC(5, "a[80:95]")
  LARD_OACC(6, "a[96:111]")
  LARD_OACC(7, "a[112:127]")
}
#undef LARD_OACC

// Block index known after unrolling: the switch folds to one case.
template <bool BF>
__device__ __forceinline__ void mfma_oacc(int i, f32x16& acc, u16x8 a, u16x8 b) {
  switch (i) {
    case 0: mfma32_acc<0, BF>(acc, a, b); break;
    case 1: mfma32_acc<1, BF>(acc, a, b); break;
    case 2: mfma32_acc<2, BF>(acc, a, b); break;
    case 3: mfma32_acc<3, BF>(acc, a, b); break;
    case 4: mfma32_acc<4, BF>(acc, a, b); break;
    case 5: mfma32_acc<5, BF>(acc, a, b); break;
    case 6: mfma32_acc<6, BF>(acc, a, b); break;
    default: mfma32_acc<7, BF>(acc, a, b); break;
  }
}

// Ties the end of a score chain: every read of the scores comes after this
// point in the instruction stream (the wait states are the schedule's; see
// the rules above).
__device__ __forceinline__ void score_fence(f32x16& s, f32x16& t) {
  asm volatile("" : "+v"(s), "+v"(t));
}

// 24 wait states after the last output MFMA before any other instruction
// reads or writes the accumulators (which the operands tie to this point).
// The teacher blocks follow the student blocks: o_t[db] is block NDB + db.
template <int NDB>
__device__ __forceinline__ void agpr_fence(f32x16* o_s, f32x16* o_t) {
  static_assert(NDB == 1 || NDB == 2 || NDB == 4, "dim blocks");
  if constexpr (NDB == 4)
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+{a[0:15]}"(o_s[0]), "+{a[16:31]}"(o_s[1]), "+{a[32:47]}"(o_s[2]), "+{a[48:63]}"(o_s[3]), "+{a[64:79]}"(o_t[0]), "+{a[80:95]}"(o_t[1]), "+{a[96:111]}"(o_t[2]), "+{a[112:127]}"(o_t[3]));
  else if constexpr (NDB == 2)
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+{a[0:15]}"(o_s[0]), "+{a[16:31]}"(o_s[1]), "+{a[32:47]}"(o_t[0]), "+{a[48:63]}"(o_t[1]));
  else
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+{a[0:15]}"(o_s[0]), "+{a[16:31]}"(o_t[0]));
}

// Zero start of the accumulator blocks, written in their ranges.
#define LARD_Z4(a, b, c, d) \
  "v_accvgpr_write_b32 a" #a ", 0\n\tv_accvgpr_write_b32 a" #b ", 0\n\tv_accvgpr_write_b32 a" #c ", 0\n\tv_accvgpr_write_b32 a" #d ", 0\n\t"
// Rescale of four accumulator registers by the factor operand F (two VGPR
// temporaries, so consecutive registers do not wait on each other).
#define LARD_RS4(a, b, c, d, F)                                                                                     \
  "v_accvgpr_read_b32 %[t0], a" #a "\n\tv_accvgpr_read_b32 %[t1], a" #b "\n\tv_mul_f32 %[t0], %[t0], %[" #F          \
  "]\n\tv_mul_f32 %[t1], %[t1], %[" #F "]\n\tv_accvgpr_write_b32 a" #a ", %[t0]\n\tv_accvgpr_write_b32 a" #b            \
  ", %[t1]\n\tv_accvgpr_read_b32 %[t0], a" #c "\n\tv_accvgpr_read_b32 %[t1], a" #d "\n\tv_mul_f32 %[t0], %[t0], %[" #F \
  "]\n\tv_mul_f32 %[t1], %[t1], %[" #F "]\n\tv_accvgpr_write_b32 a" #c ", %[t0]\n\tv_accvgpr_write_b32 a" #d         \
  ", %[t1]\n\t"

template <int NDB>
__device__ __forceinline__ void agpr_zero(f32x16* o_s, f32x16* o_t) {
  if constexpr (NDB == 4)
    asm volatile(LARD_Z4(0, 1, 2, 3) LARD_Z4(4, 5, 6, 7) LARD_Z4(8, 9, 10, 11) LARD_Z4(12, 13, 14, 15) LARD_Z4(16, 17, 18, 19) LARD_Z4(20, 21, 22, 23) LARD_Z4(24, 25, 26, 27) LARD_Z4(28, 29, 30, 31) LARD_Z4(32, 33, 34, 35) LARD_Z4(36, 37, 38, 39) LARD_Z4(40, 41, 42, 43) LARD_Z4(44, 45, 46, 47) LARD_Z4(48, 49, 50, 51) LARD_Z4(52, 53, 54, 55) LARD_Z4(56, 57, 58, 59) LARD_Z4(60, 61, 62, 63) LARD_Z4(64, 65, 66, 67) LARD_Z4(68, 69, 70, 71) LARD_Z4(72, 73, 74, 75) LARD_Z4(76, 77, 78, 79) LARD_Z4(80, 81, 82, 83) LARD_Z4(84, 85, 86, 87) LARD_Z4(88, 89, 90, 91) LARD_Z4(92, 93, 94, 95) LARD_Z4(96, 97, 98, 99) LARD_Z4(100, 101, 102, 103) LARD_Z4(104, 105, 106, 107) LARD_Z4(108, 109, 110, 111) LARD_Z4(112, 113, 114, 115) LARD_Z4(116, 117, 118, 119) LARD_Z4(120, 121, 122, 123) LARD_Z4(124, 125, 126, 127) : "={a[0:15]}"(o_s[0]), "={a[16:31]}"(o_s[1]), "={a[32:47]}"(o_s[2]), "={a[48:63]}"(o_s[3]), "={a[64:79]}"(o_t[0]), "={a[80:95]}"(o_t[1]), "={a[96:111]}"(o_t[2]), "={a[112:127]}"(o_t[3]));
  else if constexpr (NDB == 2)
    asm volatile(LARD_Z4(0, 1, 2, 3) LARD_Z4(4, 5, 6, 7) LARD_Z4(8, 9, 10, 11) LARD_Z4(12, 13, 14, 15) LARD_Z4(16, 17, 18, 19) LARD_Z4(20, 21, 22, 23) LARD_Z4(24, 25, 26, 27) LARD_Z4(28, 29, 30, 31) LARD_Z4(32, 33, 34, 35) LARD_Z4(36, 37, 38, 39) LARD_Z4(40, 41, 42, 43) LARD_Z4(44, 45, 46, 47) LARD_Z4(48, 49, 50, 51) LARD_Z4(52, 53, 54, 55) LARD_Z4(56, 57, 58, 59) LARD_Z4(60, 61, 62, 63) : "={a[0:15]}"(o_s[0]), "={a[16:31]}"(o_s[1]), "={a[32:47]}"(o_t[0]), "={a[48:63]}"(o_t[1]));
  else
    asm volatile(LARD_Z4(0, 1, 2, 3) LARD_Z4(4, 5, 6, 7) LARD_Z4(8, 9, 10, 11) LARD_Z4(12, 13, 14, 15) LARD_Z4(16, 17, 18, 19) LARD_Z4(20, 21, 22, 23) LARD_Z4(24, 25, 26, 27) LARD_Z4(28, 29, 30, 31) : "={a[0:15]}"(o_s[0]), "={a[16:31]}"(o_t[0]));
}

// Rescale of the accumulators after a raise of the running maxima: student
// blocks by fs, teacher blocks by ft, when `on` (wave-uniform) is nonzero.
// The branch is inside the statement, so the blocks flow through one asm
// statement on every path and never meet at a control-flow merge (where the
// register allocator would copy all of them); the fence before the reads is
// agpr_fence's.
template <int NDB>
__device__ __forceinline__ void agpr_rescale(f32x16* o_s, f32x16* o_t, unsigned on, float fs, float ft) {
  float t0, t1;
  if constexpr (NDB == 4)
    asm volatile("s_cmp_eq_u32 %[on], 0\n\ts_cbranch_scc1 1f\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\t" LARD_RS4(0, 1, 2, 3, fs) LARD_RS4(4, 5, 6, 7, fs) LARD_RS4(8, 9, 10, 11, fs) LARD_RS4(12, 13, 14, 15, fs) LARD_RS4(16, 17, 18, 19, fs) LARD_RS4(20, 21, 22, 23, fs) LARD_RS4(24, 25, 26, 27, fs) LARD_RS4(28, 29, 30, 31, fs) LARD_RS4(32, 33, 34, 35, fs) LARD_RS4(36, 37, 38, 39, fs) LARD_RS4(40, 41, 42, 43, fs) LARD_RS4(44, 45, 46, 47, fs) LARD_RS4(48, 49, 50, 51, fs) LARD_RS4(52, 53, 54, 55, fs) LARD_RS4(56, 57, 58, 59, fs) LARD_RS4(60, 61, 62, 63, fs) LARD_RS4(64, 65, 66, 67, ft) LARD_RS4(68, 69, 70, 71, ft) LARD_RS4(72, 73, 74, 75, ft) LARD_RS4(76, 77, 78, 79, ft) LARD_RS4(80, 81, 82, 83, ft) LARD_RS4(84, 85, 86, 87, ft) LARD_RS4(88, 89, 90, 91, ft) LARD_RS4(92, 93, 94, 95, ft) LARD_RS4(96, 97, 98, 99, ft) LARD_RS4(100, 101, 102, 103, ft) LARD_RS4(104, 105, 106, 107, ft) LARD_RS4(108, 109, 110, 111, ft) LARD_RS4(112, 113, 114, 115, ft) LARD_RS4(116, 117, 118, 119, ft) LARD_RS4(120, 121, 122, 123, ft) LARD_RS4(124, 125, 126, 127, ft) "1:"
                 : "+{a[0:15]}"(o_s[0]), "+{a[16:31]}"(o_s[1]), "+{a[32:47]}"(o_s[2]), "+{a[48:63]}"(o_s[3]), "+{a[64:79]}"(o_t[0]), "+{a[80:95]}"(o_t[1]), "+{a[96:111]}"(o_t[2]), "+{a[112:127]}"(o_t[3]), [t0] "=&v"(t0), [t1] "=&v"(t1)
                 : [on] "s"(on), [fs] "v"(fs), [ft] "v"(ft)
                 : "scc");
  else if constexpr (NDB == 2)
    asm volatile("s_cmp_eq_u32 %[on], 0\n\ts_cbranch_scc1 1f\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\t" LARD_RS4(0, 1, 2, 3, fs) LARD_RS4(4, 5, 6, 7, fs) LARD_RS4(8, 9, 10, 11, fs) LARD_RS4(12, 13, 14, 15, fs) LARD_RS4(16, 17, 18, 19, fs) LARD_RS4(20, 21, 22, 23, fs) LARD_RS4(24, 25, 26, 27, fs) LARD_RS4(28, 29, 30, 31, fs) LARD_RS4(32, 33, 34, 35, ft) LARD_RS4(36, 37, 38, 39, ft) LARD_RS4(40, 41, 42, 43, ft) LARD_RS4(44, 45, 46, 47, ft) LARD_RS4(48, 49, 50, 51, ft) LARD_RS4(52, 53, 54, 55, ft) LARD_RS4(56, 57, 58, 59, ft) LARD_RS4(60, 61, 62, 63, ft) "1:"
                 : "+{a[0:15]}"(o_s[0]), "+{a[16:31]}"(o_s[1]), "+{a[32:47]}"(o_t[0]), "+{a[48:63]}"(o_t[1]), [t0] "=&v"(t0), [t1] "=&v"(t1)
                 : [on] "s"(on), [fs] "v"(fs), [ft] "v"(ft)
                 : "scc");
  else
    asm volatile("s_cmp_eq_u32 %[on], 0\n\ts_cbranch_scc1 1f\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\t" LARD_RS4(0, 1, 2, 3, fs) LARD_RS4(4, 5, 6, 7, fs) LARD_RS4(8, 9, 10, 11, fs) LARD_RS4(12, 13, 14, 15, fs) LARD_RS4(16, 17, 18, 19, ft) LARD_RS4(20, 21, 22, 23, ft) LARD_RS4(24, 25, 26, 27, ft) LARD_RS4(28, 29, 30, 31, ft) "1:"
                 : "+{a[0:15]}"(o_s[0]), "+{a[16:31]}"(o_t[0]), [t0] "=&v"(t0), [t1] "=&v"(t1)
                 : [on] "s"(on), [fs] "v"(fs), [ft] "v"(ft)
                 : "scc");
}
#undef LARD_Z4
#undef LARD_RS4

// Scores of one 32-key sub-block (rows r0.. of the swizzled student tile
// ks; the teacher tile follows it), both relations, fenced.
template <int DP, bool BF>
__device__ __forceinline__ void sub_scores_q(const u16* ks, int r0, int l32, int half, const u16x8* fq_s,
                                             const u16x8* fq_t, f32x16& ss, f32x16& st) {
#pragma unroll
  for (int kk = 0; kk < DP / 16; ++kk) {
    const u16* p = row_chunk<DP>(ks, r0 + l32, 2 * kk + half);
    const u16x8 os = *reinterpret_cast<const u16x8*>(p), ot = *reinterpret_cast<const u16x8*>(p + kTile * DP);
    if (kk == 0) {
      mfma_first<false>(ss, os, fq_s[0]);
      mfma_first<false>(st, ot, fq_t[0]);
    } else {
      mfma_next<false>(ss, os, fq_s[kk]);
      mfma_next<false>(st, ot, fq_t[kk]);
    }
  }
  score_fence(ss, st);
}

// Eight bfloat16 values to float16, times the power of two s (exact while
// the result is a normal float16; tiny values round once, huge ones are
// what s is chosen against).
__device__ __forceinline__ u16x8 bf16_to_f16_scaled(u16x8 x, float s) {
  u16x8 out;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float v = __builtin_bit_cast(float, (unsigned)x[e] << 16) * s;
    out[e] = __builtin_bit_cast(u16, static_cast<_Float16>(v));
  }
  return out;
}

// mask_block with each side's masked logit given (the scores are scaled).
__device__ __forceinline__ void mask_block_q(f32x16& ss, f32x16& st, unsigned bits, int lim, bool causal,
                                             float masked_s, float masked_t) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int off = 8 * (r >> 2) + (r & 3);
    const bool v = ((bits >> off) & 1u) && (!causal || off <= lim);
    ss[r] = v ? ss[r] : masked_s;
    st[r] = v ? st[r] : masked_t;
  }
}


// A 16-byte LDS load at a byte address.
__device__ __forceinline__ u16x8 lds_u16x8(unsigned a) {
  return *(__attribute__((address_space(3))) const u16x8*)(uintptr_t)a;
}
// Transposing operand reads (TrOffsets' pattern) with the swizzle's per-lane
// offsets in XOR form.  The swizzle XORs the chunk index inside a row, so in
// a 256-byte aligned tile the offset of dim block db is the lane's db = 0
// offset with address bits 6-7 flipped by db (one base per 8-row half: for
// D = 128 the two halves swizzle differently), while the 16-row groups and
// sub-blocks add.  Two registers per lane instead of eight, and the constant
// parts fold into the reads' offset field; with the offsets in VGPRs the
// compiler no longer parks them in AGPRs and reads them back every step.
template <int DP>
struct TrXor {
  unsigned base[2];  // bytes
  __device__ __forceinline__ void init(int lane) {
    const int g = lane >> 4, u = lane & 15;
    int dim = 16 * (g & 1) + 4 * (u & 3);
    if (DP < 32) dim &= DP - 1;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int row = 8 * r + 4 * (g >> 1) + (u >> 2);
      base[r] = 2u * ((unsigned)row_chunk_off<DP>(row, dim >> 3) + (dim & 7));
    }
  }
  __device__ __forceinline__ u16x8 read(unsigned tile, int sb, int m, int db) const {
    s16x4 v[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const unsigned a = ((tile + base[r]) ^ (unsigned)(db << 6)) + (unsigned)((32 * sb + 16 * m) * DP * 2);
      v[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(uintptr_t)a);
    }
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    const s16x8 both = __builtin_shufflevector(v[0], v[1], 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(u16x8, both);
  }
};
// Lazy-maximum bound of the fused kernel: every exponential stays below it,
// so the float16 operands (largest finite 65504) never overflow.
constexpr float kLazySumQ = 32768.f;  // 2^15

template <int DP, bool BF>
__device__ __forceinline__ void hot_fwdq_body(const HotArgs& f, int item) {
  const RelArgs& a = f.r;
  using TC = TileCopies<DP, kWavesQ>;
  constexpr int KS = DP / 16;                   // k-steps of the scores
  constexpr int NDB = DP >= 32 ? DP / 32 : 1;   // 32-wide dim blocks of the outputs
  constexpr int NP = 2 * NDB;                   // (k-step, dim block) pairs of the output products
  constexpr int PPK = NP > KS ? NP / KS : 1;    // pairs per score k-step
  constexpr int EP = 16 / KS;                   // softmax elements per score k-step
  static_assert(PPK * KS == NP, "output products must spread evenly over the score k-steps");
  constexpr int kPerWave = 2 * TC::kRowPerWave + 1;  // K_s rows, K_t rows, token validity
  constexpr int kBufs = 4;
  static_assert((kBufs & (kBufs - 1)) == 0, "ring indices are masked with kBufs - 1");
  // [buffer][student, teacher]; 256-byte aligned for the XOR-form operand
  // addresses (g1b, TrXor)
  __shared__ __attribute__((aligned(256))) u16 lk[kBufs][2][kTile * DP];
  static_assert((32 * DP * 2) % 256 == 0, "tiles and sub-blocks start 256-byte aligned");
  __shared__ __attribute__((aligned(16))) unsigned char ltok[kBufs][kWavesQ][kTile];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int T = a.T;
  const int nrb = (T + kRowsQ - 1) / kRowsQ;
  const int bh = item / nrb;
  const int rb = nrb - 1 - (item - bh * nrb);  // longest causal rows first
  const int b = bh / a.Hq;
  const int h = bh - b * a.Hq;
  const int row0 = rb * kRowsQ;
  const int my_i = row0 + w * 32 + l32;
  const bool in_range = my_i < T;
  const bool row_valid = in_range && mask_at(a.mask, a.mask_kind, (int64_t)b * a.mask_sb + my_i);
  const int causal = a.causal;
  const int diag_sb = (row0 >> 5) + w;

  // Negative scales: flip the sign of q (exact) so the effective scale is positive.
  const u16 flip_s = a.s.scale < 0.f ? 0x8000 : 0, flip_t = a.t.scale < 0.f ? 0x8000 : 0;
  // operands in float16 scaled by 2^-e per side (exact: powers of two)
  const float k16s = f.k16_scale != nullptr ? *f.k16_scale : 1.f;
  const float k16t = f.k16t_scale != nullptr ? *f.k16t_scale : 1.f;
  u16x8 fq_s[KS], fq_t[KS];
  {
    const u16* ps = a.s.q + (int64_t)b * a.s.q_sb + (int64_t)h * a.s.q_sh + (int64_t)my_i * a.s.q_st;
    const u16* pt = a.t.q + (int64_t)b * a.t.q_sb + (int64_t)h * a.t.q_sh + (int64_t)my_i * a.t.q_st;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int d0 = 16 * kk + 8 * half;
      const bool ld = in_range && d0 < a.s.dim;
      u16x8 q = ld ? *reinterpret_cast<const u16x8*>(ps + d0) : (u16x8)(0);
      if constexpr (BF) q = bf16_to_f16_scaled(q, k16s);
      fq_s[kk] = q ^ flip_s;
      u16x8 qt = ld ? *reinterpret_cast<const u16x8*>(pt + d0) : (u16x8)(0);
      if constexpr (BF) qt = bf16_to_f16_scaled(qt, k16t);
      fq_t[kk] = qt ^ flip_t;
    }
  }
  // The query operands are read-only for the whole loop: they live in AGPRs
  // (MFMA A/B operands may be AGPRs; see mfma_first), defined there once.
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) asm volatile("" : "+a"(fq_s[kk]), "+a"(fq_t[kk]));

  // scores come out of the MFMA scaled by 2^-2e: c2 absorbs 4^e
  const float inv16 = 1.f / k16s, inv16t = 1.f / k16t;  // 2^e, exact
  const float c2s = fabsf(a.s.scale2) * inv16 * inv16, c2t = fabsf(a.t.scale2) * inv16t * inv16t;
  // the student's masked logit and start maximum in the same scaled units,
  // so every product with c2s equals the unscaled one (and stays finite)
  const float masked_s = kMaskedLogit * k16s * k16s, start_s = kStartMax * k16s * k16s;
  const float masked_t = kMaskedLogit * k16t * k16t, start_t = kStartMax * k16t * k16t;
  SoftRow R = {start_s, start_t, stabiliser(start_s, c2s), stabiliser(start_t, c2t), 0.f, 0.f, 0.f};

  const int hs = h / a.s.group, ht = h / a.t.group;
  const u16* ks_base = f.k16 + (int64_t)b * f.k16_sb + (int64_t)hs * f.k16_sh;
  const u16* kt_base = f.k16t + (int64_t)b * f.k16t_sb + (int64_t)ht * f.k16t_sh;
  const unsigned char* tok = f.tok_ok + (int64_t)b * f.Tp;

  const int nkt_all = f.Tp / kTile;
  const int ntiles = causal ? min(nkt_all, (row0 + kRowsQ - 1) / kTile + 1) : nkt_all;
  const int nsub = 2 * ntiles;
  // causal: the diagonal tiles first, so the running max is set by the
  // dominant self-similarity and rescales are rare
  auto tile_of = [&](int it) { return causal ? ntiles - 1 - it : it; };
  // per-lane copy offsets of a full tile, computed once
  RowCopier<DP, kWavesQ> cp_s, cp_t;
  cp_s.init((int)f.k16_st, a.s.dim, w, lane);
  cp_t.init((int)f.k16t_st, a.t.dim, w, lane);
  auto issue_tile = [&](int it) {
    const int buf = it & (kBufs - 1);
    const int j0 = tile_of(it) * kTile;
    cp_s.issue(lds_addr(lk[buf][0]), ks_base, (int)f.k16_st, j0, T, a.s.dim, w, lane);
    cp_t.issue(lds_addr(lk[buf][1]), kt_base, (int)f.k16t_st, j0, T, a.t.dim, w, lane);
    issue_small(lds_addr(ltok[buf][w]), tok + j0, lane);
  };
  // this lane's row chunk of a sub-block, bytes: row l32, chunk half; chunk
  // 2kk + half is at (tile + g1b) ^ (kk << 5) (the swizzle XORs the chunk)
  const unsigned g1b = 2u * (unsigned)row_chunk_off<DP>(l32, half);
  TrXor<DP> tro;
  tro.init(lane);

  f32x16 o_s[NDB], o_t[NDB];  // O^T: lane l holds row i = l%32, dims 32db + 8(r/4) + 4half + r%4
  agpr_zero<NDB>(o_s, o_t);

  struct Sub {
    f32x16 s, t;
    uint64_t tm;  // token validity of its tile, bit j = key j of the tile
  };
  // processing index k -> tile ring buffer and sub-block half
  auto buf_of = [&](int k) { return (k >> 1) & (kBufs - 1); };
  // Causal: tiles run from the diagonal down, so the tiles that reach this
  // wave's diagonal sub-block are those of the first kmask steps (pair m of
  // steps holds tile ntiles-1-m, whose sub-block 2t+1 reaches diag_sb when
  // t >= diag_sb / 2).  Masking a sub-block of such a tile that lies wholly
  // below the diagonal, with all tokens valid, changes nothing, so one bound
  // per wave replaces the per-step sub-block comparison.
  const int kmask = causal ? 2 * max(ntiles - (diag_sb >> 1), 0) : 0;
  auto prepare = [&](Sub& x, int k) {
    if (x.tm != ~0ull || k < kmask) {
      const int kt0 = tile_of(k >> 1) * kTile;
      const int first = kt0 + 32 * (k & 1) + 4 * half;
      mask_block_q(x.s, x.t, (unsigned)(x.tm >> (32 * (k & 1) + 4 * half)), my_i - first, causal, masked_s, masked_t);
    }
  };

  u16x8 pop_s[2] = {(u16x8)(0), (u16x8)(0)}, pop_t[2] = {(u16x8)(0), (u16x8)(0)};  // packed p~ of sub-block k-1

  // Step k: scores of sub-block k1 into nxt, output products of sub-block
  // k-1 (packed in pop_*), softmax of sub-block k (cur, already scored).
  // First operands of the next step, read at the end of the current one so
  // the next step's first MFMAs need not wait for LDS: the output-product
  // operand (sub-block k, always resident) after every step, the score
  // operands (sub-block k+2) only after odd steps, whose next step scores a
  // tile that landed before the barrier preceding the odd step.
  u16x8 pre_os = (u16x8)(0), pre_ot = (u16x8)(0), pre_oa = (u16x8)(0);
  auto step = [&](Sub& cur, int k, Sub& nxt, int k1, auto pre1_in, auto pre1_out) {
    constexpr bool PRE1_IN = decltype(pre1_in)::value, PRE1_OUT = decltype(pre1_out)::value;
    prepare(cur, k);
    const int b1 = buf_of(k1);
    nxt.tm = __ballot(ltok[b1][w][lane] != 0);
    const u16* t1 = lk[b1][0] + 32 * (k1 & 1) * DP;  // student rows of sub-block k1 (teacher tile follows)
    const int k2 = k > 0 ? k - 1 : 0;
    const u16* t2 = lk[buf_of(k2)][0];
    const int sb2 = k2 & 1;

    constexpr int PD = 1;  // score operands read PD k-steps ahead
    constexpr int PA = 1;  // output-product A operands read PA pairs ahead
    u16x8 os[KS], ot[KS], oa[NP];
    const unsigned ad1 = lds_addr(t1) + g1b, ad2 = lds_addr(t2);
    auto load1 = [&](int kk) {
      const unsigned p = ad1 ^ (unsigned)(kk << 5);
      os[kk] = lds_u16x8(p);
      ot[kk] = lds_u16x8(p + kTile * DP * 2);
    };
    auto load2 = [&](int j) { oa[j] = tro.read(ad2, sb2, j / NDB, j % NDB); };
    static_assert(PD == 1 && PA == 1, "the carried operands are the first k-step's");
    if constexpr (PRE1_IN) {
      os[0] = pre_os;
      ot[0] = pre_ot;
    } else {
      load1(0);
    }
    oa[0] = pre_oa;

    float s0 = 0.f, s1 = 0.f, t0 = 0.f, t1s = 0.f, a0 = 0.f, a1 = 0.f;
    float ps[16], pt[16];
    unsigned ws[8], wt[8];
    // One wave per SIMD issues in order: an MFMA followed directly by the
    // next MFMA would hold the wave until the matrix unit takes it, so every
    // MFMA is followed by one phase of the softmax of NPAIR element pairs
    // (about one MFMA's duration of VALU work), and scheduling barriers keep
    // that order.  Empty asm statements pin each phase's results, so no IR
    // pass moves the arithmetic across the barriers.
    constexpr int NPAIR = EP / 2;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      // operand reads PD / PA ahead, and no further: the memory clobber keeps
      // IR passes from hoisting later reads here (their registers would be
      // live across the whole step)
      asm volatile("" ::: "memory");
      if (kk + PD < KS) load1(kk + PD);
#pragma unroll
      for (int q = 0; q < PPK; ++q) {
        const int j = kk * PPK + q;
        if (j + PA < NP) load2(j + PA);
      }
      if (kk == KS - 1) {  // the next step's first operands
        pre_oa = tro.read(lds_addr(lk[buf_of(k)][0]), k & 1, 0, 0);
        if constexpr (PRE1_OUT) {
          const unsigned p = lds_addr(lk[buf_of(k + 2)][0] + 32 * (k & 1) * DP) + g1b;  // sub-block k+2 has k's half
          pre_os = lds_u16x8(p);
          pre_ot = lds_u16x8(p + kTile * DP * 2);
        }
      }
      float xt[NPAIR][2], xs[NPAIR][2], dd[NPAIR][2];
      // phase 0: student scores; exponent arguments
      if (kk == 0)
        mfma_first<false>(nxt.s, os[0], fq_s[0]);
      else
        mfma_next<false>(nxt.s, os[kk], fq_s[kk]);
#pragma unroll
      for (int p = 0; p < NPAIR; ++p) {
        const int r = kk * EP + 2 * p;
        xt[p][0] = fmaf(cur.t[r], c2t, R.nm_t);
        xt[p][1] = fmaf(cur.t[r + 1], c2t, R.nm_t);
        xs[p][0] = fmaf(cur.s[r], c2s, R.nm_s);
        xs[p][1] = fmaf(cur.s[r + 1], c2s, R.nm_s);
        asm volatile("" : "+v"(xt[p][0]), "+v"(xt[p][1]), "+v"(xs[p][0]), "+v"(xs[p][1]));
      }
      __builtin_amdgcn_sched_barrier(0);
      // phase 1: teacher scores; differences, teacher exponentials
      if (kk == 0)
        mfma_first<false>(nxt.t, ot[0], fq_t[0]);
      else
        mfma_next<false>(nxt.t, ot[kk], fq_t[kk]);
#pragma unroll
      for (int p = 0; p < NPAIR; ++p) {
        const int r = kk * EP + 2 * p;
        dd[p][0] = xt[p][0] - xs[p][0];
        dd[p][1] = xt[p][1] - xs[p][1];
        pt[r] = fast_exp2(xt[p][0]);
        pt[r + 1] = fast_exp2(xt[p][1]);
        asm volatile("" : "+v"(dd[p][0]), "+v"(dd[p][1]), "+v"(pt[r]), "+v"(pt[r + 1]));
      }
      __builtin_amdgcn_sched_barrier(0);
      // phase 2: student output product; student exponentials and sums
      mfma_oacc<false>(kk * PPK % NDB, o_s[kk * PPK % NDB], oa[kk * PPK], pop_s[kk * PPK / NDB]);
#pragma unroll
      for (int p = 0; p < NPAIR; ++p) {
        const int r = kk * EP + 2 * p;
        ps[r] = fast_exp2(xs[p][0]);
        ps[r + 1] = fast_exp2(xs[p][1]);
        s0 += ps[r];
        s1 += ps[r + 1];
        asm volatile("" : "+v"(ps[r]), "+v"(ps[r + 1]), "+v"(s0), "+v"(s1));
      }
      __builtin_amdgcn_sched_barrier(0);
      // phase 3: teacher output product; teacher sums, KL terms, packing
      mfma_oacc<false>(NDB + kk * PPK % NDB, o_t[kk * PPK % NDB], oa[kk * PPK], pop_t[kk * PPK / NDB]);
#pragma unroll
      for (int p = 0; p < NPAIR; ++p) {
        const int r = kk * EP + 2 * p;
        t0 += pt[r];
        t1s += pt[r + 1];
        a0 = fmaf(pt[r], dd[p][0], a0);
        a1 = fmaf(pt[r + 1], dd[p][1], a1);
        ws[r >> 1] = pack2<false>(ps[r], ps[r + 1]);
        wt[r >> 1] = pack2<false>(pt[r], pt[r + 1]);
        asm volatile("" : "+v"(t0), "+v"(t1s), "+v"(a0), "+v"(a1), "+v"(ws[r >> 1]), "+v"(wt[r >> 1]));
      }
      __builtin_amdgcn_sched_barrier(0);
      // the remaining output products of this k-step (D < 32: two per k-step)
#pragma unroll
      for (int q = 1; q < PPK; ++q) {
        const int j = kk * PPK + q;
        mfma_oacc<false>(j % NDB, o_s[j % NDB], oa[j], pop_s[j / NDB]);
        mfma_oacc<false>(NDB + j % NDB, o_t[j % NDB], oa[j], pop_t[j / NDB]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    score_fence(nxt.s, nxt.t);
    BlockSums bs = {s0 + s1, t0 + t1s, a0 + a1};
    // sums are never NaN; +inf raises.  The ballot is wave-uniform: OR-ing its
    // halves gives the rescale its scalar flag without a VALU round trip.
    const uint64_t raise_lanes = __ballot(!(fmaxf(bs.s, bs.t) <= kLazySumQ));
    const bool raise = raise_lanes != 0;
    const unsigned raise_on = (unsigned)raise_lanes | (unsigned)(raise_lanes >> 32);
    float fs = 1.f, ft = 1.f;
    if (raise) {
      raise_max_row(cur.s, cur.t, R, c2s, c2t, fs, ft);
      bs = block_probs_packed<false>(cur.s, cur.t, R, c2s, c2t, ws, wt);
    }
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      pop_s[m] = __builtin_bit_cast(u16x8, (u32x4){ws[4 * m], ws[4 * m + 1], ws[4 * m + 2], ws[4 * m + 3]});
      pop_t[m] = __builtin_bit_cast(u16x8, (u32x4){wt[4 * m], wt[4 * m + 1], wt[4 * m + 2], wt[4 * m + 3]});
    }
    agpr_rescale<NDB>(o_s, o_t, raise_on, fs, ft);
    R.l_s += bs.s;
    R.l_t += bs.t;
    R.acc += bs.a;
  };

  // The register operands loaded above must have landed before the ring
  // starts (the compiler does not count the asm copies).
  wait_vmcnt<0>();
  for (int it = 0; it < 3 && it < ntiles; ++it) issue_tile(it);
  if (TC::kUniform && ntiles >= 3)
    wait_vmcnt<2 * kPerWave>();  // tile 0 landed, tiles 1 and 2 in flight
  else if (TC::kUniform && ntiles == 2)
    wait_vmcnt<kPerWave>();
  else
    wait_vmcnt<0>();
  __syncthreads();

  Sub A, B;
  A.tm = __ballot(ltok[0][w][lane] != 0);
  sub_scores_q<DP, BF>(lk[0][0], 0, l32, half, fq_s, fq_t, A.s, A.t);
  {  // what step 0 would have carried: scores of sub-block 1, products of "sub-block -1" (zero operands)
    const unsigned p = lds_addr(lk[0][0] + 32 * DP) + g1b;
    pre_os = lds_u16x8(p);
    pre_ot = lds_u16x8(p + kTile * DP * 2);
    pre_oa = tro.read(lds_addr(lk[0][0]), 0, 0, 0);
  }
  for (int k = 0; k < nsub; k += 2) {
    step(A, k, B, k + 1, std::true_type{}, std::false_type{});
    // barrier before step 2t-1 = k+1 (t = k/2 + 1): tile t landed, tile t-2 free
    const int t = (k >> 1) + 1;
    if (t < ntiles) {
      if (TC::kUniform && t + 1 < ntiles)
        wait_vmcnt<kPerWave>();  // tile t landed, tile t+1 in flight
      else
        wait_vmcnt<0>();
      __syncthreads();
      if (t + 2 < ntiles) issue_tile(t + 2);
    }
    // the last step recomputes the scores of the last sub-block (still in
    // LDS) and drops them: one code path for every step
    step(B, k + 1, A, min(k + 2, nsub - 1), std::false_type{}, std::true_type{});
  }
  // output products of the last sub-block
  {
    const int k2 = nsub - 1;
    const u16* t2 = lk[buf_of(k2)][0];
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const u16x8 op = tro.read(lds_addr(t2), k2 & 1, j / NDB, j % NDB);
      mfma_oacc<false>(j % NDB, o_s[j % NDB], op, pop_s[j / NDB]);
      mfma_oacc<false>(NDB + j % NDB, o_t[j % NDB], op, pop_t[j / NDB]);
    }
  }
  agpr_fence<NDB>(o_s, o_t);

  // merge the two halves of the row: the stabilisers are common, so the
  // partial sums add
  const float ms = R.m_s, mt = R.m_t, ns = R.nm_s, nt = R.nm_t;
  const float l_s = R.l_s + xor32(R.l_s);
  const float l_t = R.l_t + xor32(R.l_t);
  const float acc = R.acc + xor32(R.acc);
  const bool ok = row_valid && l_s > 0.f && l_t > 0.f;
  const float lg_s = fast_log2(l_s), lg_t = fast_log2(l_t);
  // A valid row with exactly one valid key has P_s = P_t = 1 there: KL 0,
  // LSE the logit itself rounded once (kernel_A.py:147-157,
  // kernel_B.py:206-213), and D = 0, so no row-side gradient.
  const bool one_key = row_valid && (causal ? my_i == f.first2[2 * b] : f.first2[2 * b + 1] >= T);
  const int64_t row_index = (int64_t)bh * T + my_i;
  if (in_range && half == 0) {
    const float ls = one_key ? mul_rn(ms * inv16 * inv16, fabsf(a.s.scale)) : (l_s > 0.f ? (lg_s - ns) * kLn2 : kNegInf);
    const float lt = one_key ? mul_rn(mt * inv16t * inv16t, fabsf(a.t.scale)) : (l_t > 0.f ? (lg_t - nt) * kLn2 : kNegInf);
    f.lse_s_out[row_index] = row_valid ? ls : 0.f;
    f.lse_t_out[row_index] = row_valid ? lt : 0.f;
    const float wr = a.weight != nullptr ? *a.weight : 1.f;
    f.row_out[row_index] = ok && !one_key ? (acc / l_t + (lg_s - lg_t)) * kLn2 * wr : 0.f;
  }
  if (in_range) {
    const bool g_ok = ok && !one_key;
    // the products used the scaled keys: sm_scale_s * 2^e / l
    const float fs = g_ok ? a.s.scale * inv16 / l_s : 0.f;
    const float ft = g_ok ? a.s.scale * inv16 / l_t : 0.f;
    float* out = f.dq_out + row_index * a.s.dim;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * db + 8 * g + 4 * half;
        if (d0 < a.s.dim) {
          f32x4 v;
#pragma unroll
          // two rounded products: equal accumulators and sums give exactly 0
          for (int e = 0; e < 4; ++e) v[e] = mul_rn(o_s[db][4 * g + e], fs) - mul_rn(o_t[db][4 * g + e], ft);
          *reinterpret_cast<f32x4*>(out + d0) = v;
        }
      }
    }
  }
}

__host__ __device__ inline int fwdq_items(const HotArgs& f) { return (f.r.T + kRowsQ - 1) / kRowsQ * f.r.B * f.r.Hq; }

template <int DP, bool BF>
__global__ __launch_bounds__(kWavesQ * 64) void hot_fwdq_kernel(const HotArgs f) {
  hot_fwdq_body<DP, BF>(f, xcd_item(blockIdx.x, fwdq_items(f)));
}
template <int DP, bool BF>
__global__ __launch_bounds__(kWavesQ * 64) void hot_fwdq_batch_kernel(const HotBatch m) {
  const int g = xcd_item(blockIdx.x, m.first[m.n]);
  const int r = batch_relation(m, g);
  hot_fwdq_body<DP, BF>(m.rel[r], g - m.first[r]);
}

hipError_t launch_hot_fwdq(const HotArgs& f, int dp, bool bf16, hipStream_t stream);
// bfloat16 inputs, one side: k16 = float16(k * scale) as a contiguous
// [B, Hkv, T, D] tensor, *scale = the power of two 2^-e chosen against
// max |q|, |k| (device; maxbits is scratch).
hipError_t launch_keys_f16(const SideArgs& s, int B, int Hq, int T, unsigned* maxbits, float* scale, u16* k16,
                           hipStream_t stream);
hipError_t launch_hot_fwdq_batch(HotBatch& m, int dp, bool bf16, hipStream_t stream);

}  // namespace lard
