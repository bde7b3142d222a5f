// Device-side building blocks shared by every attention-relation KL kernel.
//
// Conventions used throughout (gfx950 / CDNA4, wave64):
//   * One MFMA tile is v_mfma_f32_32x32x16_{bf16,f16}: C[32x32] += A[32x16] B[16x32].
//     Lane l supplies A[m = l%32][k-slot 8*(l/32)+e] and B[k-slot 8*(l/32)+e][n = l%32]
//     (e = 0..7).  The k-slot order inside a lane is free as long as A and B use
//     the same one; the kernels exploit that to feed register-resident
//     probability tiles straight into the second GEMM.
//   * The 16 accumulator registers of lane l hold C[m][n] with
//     n = l%32 and m = 8*(r/4) + 4*(l/32) + r%4.
//   * Stage kernels keep logits, maxima and LSE in natural-log units like
//     the reference (scores = dot * sm_scale, kernel_A.py:135), so that
//     S - lse is exactly 0 for a single-entry row; exp(x) is evaluated as
//     v_exp_f32(x * log2(e)).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lard {

typedef unsigned short u16;
typedef u16 u16x8 __attribute__((ext_vector_type(8)));
typedef u16 u16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();

// Kernel modes of the row-owner template.
enum RowMode : int {
  MODE_LSE = 0,  // stage A: one relation's row LSE           (kernel_A.py:42-159)
  MODE_KL = 1,   // stage B: per-row KL given both LSE vectors (kernel_B.py:57-218)
  MODE_DQ = 2,   // stage C row side: dq = a_s D K_s           (kernel_C.py:224-239)
};

// One relation q.k^T of the problem (student or teacher).
struct SideArgs {
  const u16* q;       // [B, Hq, T, D] elements (bf16 or f16 bits; floats when f32)
  const u16* k;       // [B, Hkv, T, D]
  int64_t q_sb, q_sh, q_st;  // element strides (D stride is 1)
  int64_t k_sb, k_sh, k_st;
  int hkv;            // Hkv
  int group;          // Hq / Hkv  (kv head = h / group, kernel_A.py:77)
  int dim;            // D (<= the kernel's padded D)
  int bf16;           // 1: bfloat16, 0: float16
  int f32;            // 1: float32 (q / k point to floats; stage_f32.hip kernels)
  float scale;        // softmax scale (natural)
  float scale2;       // scale * log2(e)
};

struct RelArgs {
  SideArgs s, t;      // student, teacher
  int B, Hq, T;
  int causal;
  const void* mask;   // [B, T] or null
  int mask_kind;      // 0 none, 1 one byte (bool/u8), 2 int32, 3 int64
  int64_t mask_sb;    // batch stride of the mask (T stride is 1)
  const float* lse_s_in;  // [B, Hq, T] contiguous (modes KL, DQ, and the dk kernel)
  const float* lse_t_in;
  float* lse_out;     // [B, Hq, T] (mode LSE)
  float* row_out;     // [B, Hq, T] per-row KL (mode KL)
  float* dq_out;      // [B, Hq, T, Ds] fp32 (mode DQ)
  float* dk_out;      // [B, Hkv_s, T, Ds] fp32 (dk kernel)
  // Optional epilogues used by the autograd backward:
  //   dq_out = scale_s * dq * (*dscale)
  //   dk_out = (scale_s * dk + dk_add) * (*dscale)
  const float* dk_add;  // [B, Hkv_s, T, Ds] or null (self relation: the row-side term dq)
  const float* dscale;  // device scalar or null (autograd's dloss)
  // Throughput kernels only: device scalar or null, the relation's weight in
  // a batched loss (multiplies the per-row KL, and the gradient wherever
  // dscale is applied).
  const float* weight;
  // float32-input kernels only: the double-precision LSEs of both sides,
  // [2][B, Hq, T] (student, then teacher).  The refine pass writes them; the
  // dq / dk passes read them (instead of lse_*_in) when non-null.
  double* lse64_out;
  const double* lse64_in;
};

// Outputs of the fused forward (one pass: both LSEs and the per-row KL).
struct FusedArgs {
  RelArgs r;
  float* lse_s_out;   // [B, Hq, T]
  float* lse_t_out;   // [B, Hq, T]
  float* row_out;     // [B, Hq, T] per-row KL
};

// Compile-time flag passed to generic lambdas that are instantiated twice
// (e.g. per-element work of full and partial tiles).
template <bool V>
struct Flag {
  static constexpr bool value = V;
};

__device__ __forceinline__ bool mask_at(const void* m, int kind, int64_t idx) {
  if (kind == 1) return static_cast<const unsigned char*>(m)[idx] != 0;
  if (kind == 2) return static_cast<const int32_t*>(m)[idx] != 0;
  if (kind == 3) return static_cast<const int64_t*>(m)[idx] != 0;
  return true;
}

template <bool BF>
__device__ __forceinline__ f32x16 mfma32(u16x8 a, u16x8 b, f32x16 c) {
  if constexpr (BF) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// Round-to-nearest-even conversion of one float to the 16-bit input type.
__device__ __forceinline__ u16 to_bits(float x, bool bf) {
  return bf ? __builtin_bit_cast(u16, static_cast<__bf16>(x))
            : __builtin_bit_cast(u16, static_cast<_Float16>(x));
}

// to_bits for 8 floats at once, in element order: the vector conversion lets
// the compiler use the two-lane conversions (v_cvt_pk_bf16_f32) and skip the
// per-element repacking.
typedef float f32x8 __attribute__((ext_vector_type(8)));
template <bool BF>
__device__ __forceinline__ u16x8 to_bits8(const float* x) {
  const f32x8 v = {x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]};
  if constexpr (BF) {
    return __builtin_bit_cast(u16x8, __builtin_convertvector(v, bf16x8));
  } else {
    return __builtin_bit_cast(u16x8, __builtin_convertvector(v, f16x8));
  }
}

// Rounded product that the compiler may not fuse into a following add:
// the reference forms scores = dot * sm_scale as a rounded fp32 value before
// subtracting the LSE (kernel_B.py:190, :206), which makes S - lse exactly 0
// for single-entry rows.  hipcc's default -ffp-contract=fast-honor-pragmas
// honors this pragma.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

// Rows [row0, row0+NROWS) x [0, DP) of a [T, D]-strided 16-bit matrix,
// staged into LDS (row stride lds_stride elements) through registers in two
// steps, so that one tile's global loads are in flight while the previous
// tile is consumed: load() issues the loads (a chunk outside the matrix --
// row >= T or column >= dim -- loads row 0, column 0 instead, which exists
// whenever T > 0, and is remembered as invalid), store() writes the
// registers to LDS later, zeros for the invalid chunks, so the MFMA sees
// exact zero padding.
template <int NROWS, int DP, int NTHREADS>
struct TileRegs {
  static constexpr int CPR = DP / 8;  // 16-byte chunks per row
  static constexpr int NCH = NROWS * CPR;
  static constexpr int N = (NCH + NTHREADS - 1) / NTHREADS;
  u16x8 v[N];
  bool ok[N];

  __device__ __forceinline__ void load(const u16* g, int64_t row_stride, int row0, int T, int dim, int tid) {
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const int c = tid + n * NTHREADS;
      if (NCH % NTHREADS == 0 || c < NCH) {
        const int row = row0 + c / CPR;
        const int dc = (c % CPR) * 8;
        ok[n] = row < T && dc < dim;
        v[n] = *reinterpret_cast<const u16x8*>(g + (ok[n] ? (int64_t)row * row_stride + dc : 0));
      }
    }
  }

  __device__ __forceinline__ void store(u16* lds, int lds_stride, int tid) const {
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const int c = tid + n * NTHREADS;
      if (NCH % NTHREADS == 0 || c < NCH)
        *reinterpret_cast<u16x8*>(lds + (c / CPR) * lds_stride + (c % CPR) * 8) = ok[n] ? v[n] : (u16x8)(0);
    }
  }
};

// A operand of the second GEMM (m = 32 dims of block db, k-slots = rows
// 16kk .. 16kk+15 of a row-major [32][STRIDE] LDS tile), read with two
// transposing LDS loads instead of from a transposed copy.
// ds_read_b64_tr_b16: in each 16-lane group, lane t receives element t%4 of
// the 8 bytes that lane 4j + t/4 points at, j = 0..3.  Lane l (group
// G = l/16, u = l%16) points at row 16kk + 8r + 4(G/2) + u/4, dims
// 32db + 16(G%2) + 4(u%4) .. +3, so lane l receives, for dim 32db + l%32,
// rows 16kk + 8r + 4(l/32) + j (k-slots 4r + j): the order (0-3, 8-11,
// 4-7, 12-15) of the first GEMM's accumulator rows 8(e/4) + 4(l/32) + e%4,
// whose registers 8kk .. 8kk+7 are the B operand.  DP < 32 (one 16-dim
// block) repeats dims 0-15 in accumulator rows 16-31, which are never
// stored.  Addresses: 8-byte aligned (STRIDE a multiple of 4), inside rows
// 0-31 and dims 0..DP-1.
template <int DP, int STRIDE>
struct TrRowTile {
  static_assert(STRIDE % 4 == 0, "8-byte aligned lane addresses");
  static constexpr int NDB = DP >= 32 ? DP / 32 : 1;
  unsigned off[2][NDB];  // u16 elements
  __device__ __forceinline__ void init(int lane) {
    const int g = lane >> 4, u = lane & 15;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      int dim = 32 * db + 16 * (g & 1) + 4 * (u & 3);
      if (DP < 32) dim &= DP - 1;
#pragma unroll
      for (int r = 0; r < 2; ++r) off[r][db] = (unsigned)((8 * r + 4 * (g >> 1) + (u >> 2)) * STRIDE + dim);
    }
  }
  __device__ __forceinline__ u16x8 read(const u16* tile, int kk, int db) const {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    const u16* base = tile + 16 * kk * STRIDE;
    s16x4 v[2];
#pragma unroll
    for (int r = 0; r < 2; ++r)
      v[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)((__attribute__((address_space(3))) u16*)(base + off[r][db])));
    return __builtin_bit_cast(u16x8, __builtin_shufflevector(v[0], v[1], 0, 1, 2, 3, 4, 5, 6, 7));
  }
};

}  // namespace lard
