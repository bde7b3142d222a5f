// float32 inputs: the four stage kernels (LSE, KL, dq, dk) with float32
// products and D = P_s - P_t kept in float32 (the reference's cast of D to
// the input dtype, kernel_C.py:232-233, is the identity for float32).
//
// The reference's kernels accept only fp16/bf16 (kernel_A.py:195-196); this
// path serves float32 callers (the materialised CPU case of the benchmark
// configs runs in float32) with the stage kernels' semantics:
//   lse = log sum_{j in V} exp(S) for a valid row, 0 for an invalid one,
//         -inf for a valid row with no valid column  (kernel_A.py:157-158);
//   KL_i = sum_{j in V} p_t (l_t - l_s) for ok rows    (kernel_B.py:206-217);
//   dq_i = a_s sum_j D_ij k_j, dk_j = a_s sum_{h in group} sum_i D_ij q_i
//         (kernel_C.py:236-253), times dloss and plus dk_add as asked.
// The dot products are summed in double and S = dot * scale is rounded once
// to float32 (so S - lse is exactly 0 for a one-entry row, as in the other
// stage kernels); everything after it (exponentials, sums, log-sum-exp, the
// KL terms, D and the gradient sums) is evaluated in double and rounded once
// on output.  The KL of a near-identical pair is a small difference of
// log-sum-exps: with float32 exponentials and sums its relative error
// reaches 1e-4.  The fused mode (the autograd forward) forms both LSEs and
// the KL in one pass, so the loss does not inherit the float32 rounding of
// the stored LSEs.
//
// Structure: one workgroup of 256 threads owns 32 rows (query rows, or key
// rows for dk) of one (b, head) and walks 32-row tiles of the other side.
// Both sides' tiles sit in LDS as float32 rows padded by 4 floats; thread
// (r = tid / 8, c = tid % 8) forms the scores of row r against columns
// c, c + 8, c + 16, c + 24 with 16-byte LDS reads (conflict-free: the 8
// rows a read touches start 4 banks apart), so a row's 32 scores live in
// 8 consecutive lanes and reduce with three xor shuffles.  The gradient
// products read the D tile from LDS; each thread owns D/8 output dims.
// This path is about exactness, not speed: double FMAs on the VALU (the
// same rate as float32 on gfx950), one or two workgroups per CU.

#include "stage_f32.h"

namespace lard {
namespace {

constexpr int kF32Rows = 32;             // rows per tile (both sides)
constexpr int kModeFused = 3;            // lse_s, lse_t and the per-row KL in one pass
constexpr int kModeRefine = 4;           // lse_s, lse_t in double (for the autograd backward)
constexpr int kF32Threads = 256;
constexpr int kF32MaxDim = 256;

// LDS tiles for head dims up to MAXD (rows padded by 4 floats): the
// launchers pick the smallest of 64 / 128 / 256 that holds both sides, so
// d <= 128 fits two workgroups per CU (76 KB each) instead of one (142 KB).
template <int MAXD>
struct F32Tiles {
  static constexpr int kPitch = MAXD + 4;  // LDS row pitch (floats)
  float a_s[kF32Rows][kPitch];  // owned rows (student)
  float a_t[kF32Rows][kPitch];  // owned rows (teacher)
  float b_s[kF32Rows][kPitch];  // the other side's tile (student)
  float b_t[kF32Rows][kPitch];  // (teacher)
  double d[kF32Rows][kF32Rows + 1];  // D tile, [owned row][other row]
  double lse_s[kF32Rows], lse_t[kF32Rows];
  unsigned char ok[kF32Rows];        // the other side's row flags (dk)
  unsigned char col[kF32Rows];       // the other side's validity (row modes)
};

// Rows row0.. of one head into an LDS tile (zeros past T); dim floats each.
template <int PITCH>
__device__ __forceinline__ void load_rows(float (*dst)[PITCH], const float* base, int64_t row_stride, int row0,
                                          int T, int dim) {
  const int q4 = dim / 4;
  for (int idx = threadIdx.x; idx < kF32Rows * q4; idx += kF32Threads) {
    const int r = idx / q4, c = idx - r * q4;
    const int row = row0 + r;
    f32x4 v = (f32x4)(0.f);
    if (row < T) v = *reinterpret_cast<const f32x4*>(base + (int64_t)row * row_stride + 4 * c);
    *reinterpret_cast<f32x4*>(&dst[r][4 * c]) = v;
  }
}

// S = dot(A[r], B[c + 8 j]) * scale for j = 0..3: exact products of floats
// summed in double.
template <int PITCH>
__device__ __forceinline__ void scores(const float (*A)[PITCH], const float (*B)[PITCH], int r, int c, int dim,
                                       float scale, double (&out)[4]) {
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  for (int d = 0; d < dim; d += 4) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(&A[r][d]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 y = *reinterpret_cast<const f32x4*>(&B[c + 8 * j][d]);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[j] = __builtin_fma((double)x[e], (double)y[e], acc[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) out[j] = acc[j] * (double)scale;
}

// With float32 LSEs from the caller, S is rounded to float32 first, so that
// S - lse is exactly 0 for a one-entry row (the LSE of such a row is its S,
// rounded the same way); with the double LSEs of the refine pass S stays
// double.
__device__ __forceinline__ void match_lse_rounding(double (&x)[4], bool lse_is_f32) {
  if (lse_is_f32) {
#pragma unroll
    for (int q = 0; q < 4; ++q) x[q] = (double)(float)x[q];
  }
}

template <class V>
__device__ __forceinline__ V row8_max(V v) {
  v = fmax(v, __shfl_xor(v, 1, 64));
  v = fmax(v, __shfl_xor(v, 2, 64));
  return fmax(v, __shfl_xor(v, 4, 64));
}

template <class V>
__device__ __forceinline__ V row8_sum(V v) {
  v += __shfl_xor(v, 1, 64);
  v += __shfl_xor(v, 2, 64);
  return v + __shfl_xor(v, 4, 64);
}

constexpr double kNegInfD = -__builtin_inf();

// Online log-sum-exp of one row in double (8 lanes hold 4 values each).
struct OnlineLse {
  double m = kNegInfD, r = 0.0;
  __device__ __forceinline__ void add(const double (&x)[4], const bool (&valid)[4]) {
    double mb = kNegInfD;
#pragma unroll
    for (int q = 0; q < 4; ++q) mb = fmax(mb, valid[q] ? x[q] : kNegInfD);
    mb = row8_max(mb);
    const double mn = fmax(m, mb);
    double rs = 0.0;
    if (mn != kNegInfD) {
#pragma unroll
      for (int q = 0; q < 4; ++q) rs += valid[q] ? exp(x[q] - mn) : 0.0;
    }
    rs = row8_sum(rs);
    r = (m == kNegInfD ? 0.0 : r * exp(m - mn)) + rs;
    m = mn;
  }
  __device__ __forceinline__ double lse() const { return r > 0.0 ? m + log(r) : kNegInfD; }
};

template <class SideT>
__device__ __forceinline__ const float* qptr(const SideT& s, int b, int h) {
  return reinterpret_cast<const float*>(s.q) + (int64_t)b * s.q_sb + (int64_t)h * s.q_sh;
}
template <class SideT>
__device__ __forceinline__ const float* kptr(const SideT& s, int b, int g) {
  return reinterpret_cast<const float*>(s.k) + (int64_t)b * s.k_sb + (int64_t)g * s.k_sh;
}

// ---------------------------------------------------------------------------
// row modes: LSE (stage A), KL (stage B), DQ (stage C row side)
// ---------------------------------------------------------------------------
template <int MODE, int MAXD>
__global__ __launch_bounds__(kF32Threads) void row_f32_kernel(const RelArgs a) {
  __shared__ F32Tiles<MAXD> sh;
  const int tid = threadIdx.x;
  const int r = tid >> 3, c = tid & 7;
  const int T = a.T;
  const int bh = blockIdx.y;
  const int b = bh / a.Hq, h = bh - b * a.Hq;
  const int row0 = blockIdx.x * kF32Rows;
  const int my_i = row0 + r;
  const bool in_range = my_i < T;
  const bool row_valid = in_range && mask_at(a.mask, a.mask_kind, (int64_t)b * a.mask_sb + my_i);
  const int64_t row_index = (int64_t)bh * T + my_i;
  const bool two = MODE != MODE_LSE;

  bool ok = row_valid;
  double lse_s = 0.0, lse_t = 0.0;
  const bool lse_f32 = !(MODE == MODE_DQ && a.lse64_in != nullptr);  // float32 LSEs (or none)
  if constexpr (MODE == MODE_KL || MODE == MODE_DQ) {
    const int64_t rows = (int64_t)a.B * a.Hq * T;
    const double ls = !in_range ? 0.0 : lse_f32 ? (double)a.lse_s_in[row_index] : a.lse64_in[row_index];
    const double lt = !in_range ? 0.0 : lse_f32 ? (double)a.lse_t_in[row_index] : a.lse64_in[rows + row_index];
    ok = ok && (ls != kNegInfD) && (lt != kNegInfD);
    lse_s = (ls == kNegInfD) ? 0.0 : ls;
    lse_t = (lt == kNegInfD) ? 0.0 : lt;
  }

  load_rows(sh.a_s, qptr(a.s, b, h), a.s.q_st, row0, T, a.s.dim);
  if (two) load_rows(sh.a_t, qptr(a.t, b, h), a.t.q_st, row0, T, a.t.dim);

  const float* ks = kptr(a.s, b, h / a.s.group);
  const float* kt = kptr(a.t, b, h / a.t.group);
  const int last = a.causal ? (row0 + kF32Rows < T ? row0 + kF32Rows : T) : T;  // keys < last can be valid

  OnlineLse on_s, on_t;  // LSE and fused modes
  double kl_num = 0.0;   // fused: sum p_t (S_t - S_s) against the teacher's running max
  double kl_acc = 0.0;   // KL mode
  constexpr int kDq = MAXD / 32;  // 4-dim groups per thread of dq (dims 4 (c + 8 m) ..)
  double dq[kDq][4] = {};

  for (int j0 = 0; j0 < last; j0 += kF32Rows) {
    __syncthreads();  // the previous tile is consumed
    load_rows(sh.b_s, ks, a.s.k_st, j0, T, a.s.dim);
    if (two) load_rows(sh.b_t, kt, a.t.k_st, j0, T, a.t.dim);
    if (tid < kF32Rows) {
      const int j = j0 + tid;
      sh.col[tid] = j < T && mask_at(a.mask, a.mask_kind, (int64_t)b * a.mask_sb + j);
    }
    __syncthreads();
    double ss[4], st[4];  // S = dot * scale
    bool valid[4];
    scores(sh.a_s, sh.b_s, r, c, a.s.dim, a.s.scale, ss);
    if (two) scores(sh.a_t, sh.b_t, r, c, a.t.dim, a.t.scale, st);
    if constexpr (MODE == MODE_KL || MODE == MODE_DQ) {
      match_lse_rounding(ss, lse_f32);
      match_lse_rounding(st, lse_f32);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int jj = c + 8 * q, j = j0 + jj;
      valid[q] = ok && sh.col[jj] && (!a.causal || j <= my_i);
    }
    if constexpr (MODE == MODE_LSE) {
      double x[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) x[q] = ss[q];  // tl.dot(q, k^T) * sm_scale
      on_s.add(x, valid);
    } else if constexpr (MODE == kModeRefine) {
      on_s.add(ss, valid);
      on_t.add(st, valid);
    } else if constexpr (MODE == kModeFused) {
      const double (&xs)[4] = ss;
      const double (&xt)[4] = st;
      // the KL numerator sum p_t (S_t - S_s), kept against the teacher's running max
      const double mt_old = on_t.m;
      on_s.add(xs, valid);
      on_t.add(xt, valid);
      if (on_t.m != kNegInfD) {
        double acc = 0.0;
#pragma unroll
        for (int q = 0; q < 4; ++q) acc += valid[q] ? exp(xt[q] - on_t.m) * (xt[q] - xs[q]) : 0.0;
        acc = row8_sum(acc);
        kl_num = (mt_old == kNegInfD ? 0.0 : kl_num * exp(mt_old - on_t.m)) + acc;
      }
    } else if constexpr (MODE == MODE_KL) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (valid[q]) {
          const double lps = ss[q] - lse_s;
          const double lpt = st[q] - lse_t;
          kl_acc += exp(lpt) * (lpt - lps);
        }
      }
    } else {  // MODE_DQ: D tile to LDS, then dq[r][:] += D[r][:] K_s
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const double pd = valid[q] ? exp(ss[q] - lse_s) - exp(st[q] - lse_t) : 0.0;
        sh.d[r][c + 8 * q] = pd;
      }
      __syncthreads();
      for (int jj = 0; jj < kF32Rows; ++jj) {
        const double dv = sh.d[r][jj];
#pragma unroll
        for (int m = 0; m < kDq; ++m) {
          const int d0 = 4 * (c + 8 * m);
          if (d0 < a.s.dim) {
            const f32x4 kv = *reinterpret_cast<const f32x4*>(&sh.b_s[jj][d0]);
#pragma unroll
            for (int e = 0; e < 4; ++e) dq[m][e] = __builtin_fma(dv, (double)kv[e], dq[m][e]);
          }
        }
      }
    }
  }

  if constexpr (MODE == MODE_LSE) {
    float lse = (float)on_s.lse();
    if (!row_valid) lse = 0.f;  // kernel_A.py:157-158
    if (in_range && c == 0) a.lse_out[row_index] = lse;
  } else if constexpr (MODE == kModeRefine) {
    const int64_t rows = (int64_t)a.B * a.Hq * T;
    if (in_range && c == 0) {
      a.lse64_out[row_index] = row_valid ? on_s.lse() : 0.0;
      a.lse64_out[rows + row_index] = row_valid ? on_t.lse() : 0.0;
    }
  } else if constexpr (MODE == kModeFused) {
    // lse as stage A; the KL as stage B on rows whose both LSEs are finite
    const double ls = on_s.lse(), lt = on_t.lse();
    const bool fok = row_valid && ls != kNegInfD && lt != kNegInfD;
    const double kl = fok ? kl_num / on_t.r - lt + ls : 0.0;  // E_pt[S_t - S_s] - lse_t + lse_s
    if (in_range && c == 0) {
      a.lse_out[row_index] = row_valid ? (float)ls : 0.f;
      a.dq_out[row_index] = row_valid ? (float)lt : 0.f;  // the teacher's LSE (see launch_fused_fwd_f32)
      a.row_out[row_index] = (float)kl;
    }
  } else if constexpr (MODE == MODE_KL) {
    kl_acc = row8_sum(kl_acc);
    const float v = ok ? (float)kl_acc : 0.f;  // kernel_B.py:216
    if (in_range && c == 0) a.row_out[row_index] = v;
  } else {
    // alpha_s (times dloss when asked), invalid rows zeroed (kernel_C.py:256)
    const double f = ok ? (double)a.s.scale * (a.dscale != nullptr ? (double)*a.dscale : 1.0) : 0.0;
    if (in_range) {
      float* out = a.dq_out + row_index * a.s.dim;
#pragma unroll
      for (int m = 0; m < kDq; ++m) {
        const int d0 = 4 * (c + 8 * m);
        if (d0 < a.s.dim) {
          const f32x4 v = {(float)(dq[m][0] * f), (float)(dq[m][1] * f), (float)(dq[m][2] * f),
                           (float)(dq[m][3] * f)};
          *reinterpret_cast<f32x4*>(out + d0) = ok ? v : (f32x4)(0.f);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// column side: dk (stage C), one owner per key row and student kv head
// ---------------------------------------------------------------------------
template <int MAXD>
__global__ __launch_bounds__(kF32Threads) void col_f32_kernel(const RelArgs a) {
  __shared__ F32Tiles<MAXD> sh;
  const int tid = threadIdx.x;
  const int r = tid >> 3, c = tid & 7;
  const int T = a.T;
  const int bg = blockIdx.y;
  const int b = bg / a.s.hkv, g = bg - b * a.s.hkv;
  const int j0 = blockIdx.x * kF32Rows;
  const int my_j = j0 + r;
  const bool in_range = my_j < T;
  const bool col_valid = in_range && mask_at(a.mask, a.mask_kind, (int64_t)b * a.mask_sb + my_j);

  const bool lse_f32 = a.lse64_in == nullptr;
  load_rows(sh.a_s, kptr(a.s, b, g), a.s.k_st, j0, T, a.s.dim);
  constexpr int kDk = MAXD / 32;
  double dk[kDk][4] = {};

  int loaded_t = -1;  // teacher kv head whose key rows are in a_t
  for (int h = g * a.s.group; h < (g + 1) * a.s.group; ++h) {
    const int gt = h / a.t.group;
    const int first = a.causal ? j0 : 0;  // query rows below the key block see none of it
    for (int i0 = first - first % kF32Rows; i0 < T; i0 += kF32Rows) {
      __syncthreads();
      if (gt != loaded_t) load_rows(sh.a_t, kptr(a.t, b, gt), a.t.k_st, j0, T, a.t.dim);
      load_rows(sh.b_s, qptr(a.s, b, h), a.s.q_st, i0, T, a.s.dim);
      load_rows(sh.b_t, qptr(a.t, b, h), a.t.q_st, i0, T, a.t.dim);
      if (tid < kF32Rows) {
        const int i = i0 + tid;
        const bool in = i < T;
        const int64_t ri = ((int64_t)b * a.Hq + h) * T + i, rows = (int64_t)a.B * a.Hq * T;
        const bool rv = in && mask_at(a.mask, a.mask_kind, (int64_t)b * a.mask_sb + i);
        const double ls = !in ? 0.0 : lse_f32 ? (double)a.lse_s_in[ri] : a.lse64_in[ri];
        const double lt = !in ? 0.0 : lse_f32 ? (double)a.lse_t_in[ri] : a.lse64_in[rows + ri];
        sh.ok[tid] = rv && (ls != kNegInfD) && (lt != kNegInfD);
        sh.lse_s[tid] = (ls == kNegInfD) ? 0.0 : ls;
        sh.lse_t[tid] = (lt == kNegInfD) ? 0.0 : lt;
      }
      __syncthreads();
      loaded_t = gt;
      double ss[4], st[4];
      scores(sh.a_s, sh.b_s, r, c, a.s.dim, a.s.scale, ss);
      scores(sh.a_t, sh.b_t, r, c, a.t.dim, a.t.scale, st);
      match_lse_rounding(ss, lse_f32);
      match_lse_rounding(st, lse_f32);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int ii = c + 8 * q, i = i0 + ii;
        const bool v = sh.ok[ii] && col_valid && (!a.causal || my_j <= i);
        const double pd = v ? exp(ss[q] - sh.lse_s[ii]) - exp(st[q] - sh.lse_t[ii]) : 0.0;
        sh.d[r][ii] = pd;  // D^T: [key row][query row]
      }
      __syncthreads();
      for (int ii = 0; ii < kF32Rows; ++ii) {
        const double dv = sh.d[r][ii];
#pragma unroll
        for (int m = 0; m < kDk; ++m) {
          const int d0 = 4 * (c + 8 * m);
          if (d0 < a.s.dim) {
            const f32x4 qv = *reinterpret_cast<const f32x4*>(&sh.b_s[ii][d0]);
#pragma unroll
            for (int e = 0; e < 4; ++e) dk[m][e] = __builtin_fma(dv, (double)qv[e], dk[m][e]);
          }
        }
      }
    }
  }

  if (in_range) {
    const double mult = a.dscale != nullptr ? (double)*a.dscale : 1.0;  // chain rule (integration.py:63-64)
    const int64_t off = ((int64_t)b * a.s.hkv + g) * T * a.s.dim + (int64_t)my_j * a.s.dim;
#pragma unroll
    for (int m = 0; m < kDk; ++m) {
      const int d0 = 4 * (c + 8 * m);
      if (d0 < a.s.dim) {
        f32x4 add = (f32x4)(0.f);
        if (a.dk_add != nullptr) add = *reinterpret_cast<const f32x4*>(a.dk_add + off + d0);
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (float)((dk[m][e] * (double)a.s.scale + (double)add[e]) * mult);
        *reinterpret_cast<f32x4*>(a.dk_out + off + d0) = v;
      }
    }
  }
}

dim3 row_grid(const RelArgs& a) { return dim3((a.T + kF32Rows - 1) / kF32Rows, a.B * a.Hq); }

// The smallest tile width of 64 / 128 / 256 that holds both sides' dims.
int tile_dims(const RelArgs& a) {
  const int d = a.s.dim > a.t.dim ? a.s.dim : a.t.dim;
  return d <= 64 ? 64 : d <= 128 ? 128 : kF32MaxDim;
}

template <int MODE>
hipError_t launch_row(const RelArgs& a, hipStream_t stream) {
  switch (tile_dims(a)) {
    case 64: hipLaunchKernelGGL((row_f32_kernel<MODE, 64>), row_grid(a), dim3(kF32Threads), 0, stream, a); break;
    case 128: hipLaunchKernelGGL((row_f32_kernel<MODE, 128>), row_grid(a), dim3(kF32Threads), 0, stream, a); break;
    default: hipLaunchKernelGGL((row_f32_kernel<MODE, kF32MaxDim>), row_grid(a), dim3(kF32Threads), 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_row_lse_f32(const RelArgs& a, hipStream_t stream) { return launch_row<MODE_LSE>(a, stream); }

hipError_t launch_row_kl_f32(const RelArgs& a, hipStream_t stream) { return launch_row<MODE_KL>(a, stream); }

hipError_t launch_fused_fwd_f32(const FusedArgs& f, hipStream_t stream) {
  RelArgs a = f.r;  // the fused mode writes lse_s to lse_out, lse_t to dq_out (as floats), the KL to row_out
  a.lse_out = f.lse_s_out;
  a.dq_out = f.lse_t_out;
  a.row_out = f.row_out;
  return launch_row<kModeFused>(a, stream);
}

hipError_t launch_refine_lse_f32(const RelArgs& a, hipStream_t stream) { return launch_row<kModeRefine>(a, stream); }

hipError_t launch_row_dq_f32(const RelArgs& a, hipStream_t stream) { return launch_row<MODE_DQ>(a, stream); }

hipError_t launch_col_dk_f32(const RelArgs& a, hipStream_t stream) {
  const dim3 grid((a.T + kF32Rows - 1) / kF32Rows, a.B * a.s.hkv);
  switch (tile_dims(a)) {
    case 64: hipLaunchKernelGGL(col_f32_kernel<64>, grid, dim3(kF32Threads), 0, stream, a); break;
    case 128: hipLaunchKernelGGL(col_f32_kernel<128>, grid, dim3(kF32Threads), 0, stream, a); break;
    default: hipLaunchKernelGGL(col_f32_kernel<kF32MaxDim>, grid, dim3(kF32Threads), 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace lard
