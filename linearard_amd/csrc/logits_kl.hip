// Logits KL over the kept positions: the output-alignment term of the
// distillation loss (train.py:412-420).
//
// For every kept position r (row of V vocabulary logits) with the scaled
// logits q = R(x * (1/T)) (R the rounding to the logits dtype, as a tensor
// division by a host scalar computes it):
//
//   lse_x = log sum_v exp(q_x[v])
//   KL_r  = sum_v p_t[v] (l_t[v] - l_s[v]),   l_x = q_x - lse_x, p_t = exp(l_t)
//         = E_{p_t}[q_t - q_s] - lse_t + lse_s
//   loss  = mean_r KL_r
//
// Forward: one pass over both rows.  Each workgroup owns one chunk of one
// row and keeps, per thread, running maxima and the sums
//   z_t = sum e^{q_t - m_t},  a = sum e^{q_t - m_t} (q_t - q_s),  z_s = sum e^{q_s - m_s}
// in base-2 units (one fma and one v_exp_f32 per logit).  The maxima are
// raised lazily: a group of 8 is exponentiated against the current maximum
// and only when its sum exceeds 2^20 is the maximum raised and the group
// redone, so the common path has no per-element max.  The workgroup merges
// its threads in a fixed order and writes one partial per chunk; a one-block
// finish kernel merges the chunks of each row, writes lse_t, lse_s and KL_r
// and sums the rows in a fixed order (deterministic loss).
//
// Backward (autograd of the same lines, both gradients optional):
//   d/dx_s = c (p_s - p_t) / T,   d/dx_t = c p_t (l_t - l_s - KL_r) / T
// with c the upstream gradient of the row (dloss / rows for the mean).  One
// pass reads both rows and writes the gradients in the logits dtype.
//
// Both kernels are HBM-bound: 4 bytes per logit pair read (bf16) forward,
// 6 bytes (read 4, write 2) backward with the student gradient only.

#include "logits_kl_kernels.h"

namespace lard {
namespace {

constexpr float kL2E = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kStartMax = -1e30f;   // running maximum (base-2 units) before the first logit
constexpr float kPadLogit = -3e38f;   // logits past V: exp2 underflows to 0 and q_t - q_s = 0
constexpr float kLazyGroupSum = 1048576.f;
constexpr int kThreads = 256;
constexpr int64_t kStep = kThreads * 8;  // logits per workgroup per group of 8

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

template <int DT>
struct Raw {
  u32x4 w[DT == kLogitsF32 ? 2 : 1];
};

// Streaming (nontemporal) loads: every logit is read once per pass.
template <int DT>
__device__ __forceinline__ Raw<DT> load_raw(const void* row, int64_t v) {
  Raw<DT> r;
  if constexpr (DT == kLogitsF32) {
    const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const float*>(row) + v);
    r.w[0] = __builtin_nontemporal_load(p);
    r.w[1] = __builtin_nontemporal_load(p + 1);
  } else {
    r.w[0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(static_cast<const u16*>(row) + v));
  }
  return r;
}

template <int DT>
__device__ __forceinline__ float round_elem(float x) {  // value after a cast to the logits dtype
  if constexpr (DT == kLogitsBF16)
    return __builtin_bit_cast(float, (unsigned)__builtin_bit_cast(u16, static_cast<__bf16>(x)) << 16);
  else if constexpr (DT == kLogitsF16)
    return (float)static_cast<_Float16>(x);
  else
    return x;
}

template <int DT, bool SCALED>
__device__ __forceinline__ void unpack(const Raw<DT>& r, float inv_temp, float (&x)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (DT == kLogitsF32) {
      // (unsigned) makes the element a value: a bit_cast of the vector-element
      // lvalue itself reads element 0 with this compiler
      x[j] = __builtin_bit_cast(float, (unsigned)r.w[0][j]);
      x[4 + j] = __builtin_bit_cast(float, (unsigned)r.w[1][j]);
    } else if constexpr (DT == kLogitsBF16) {
      x[2 * j] = __builtin_bit_cast(float, r.w[0][j] << 16);
      x[2 * j + 1] = __builtin_bit_cast(float, r.w[0][j] & 0xffff0000u);
    } else {
      x[2 * j] = (float)__builtin_bit_cast(_Float16, (u16)(r.w[0][j] & 0xffffu));
      x[2 * j + 1] = (float)__builtin_bit_cast(_Float16, (u16)(r.w[0][j] >> 16));
    }
  }
  if constexpr (SCALED) {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = round_elem<DT>(x[e] * inv_temp);
  }
}

template <int DT>
__device__ __forceinline__ float load_one(const void* row, int64_t v) {
  if constexpr (DT == kLogitsF32)
    return static_cast<const float*>(row)[v];
  else if constexpr (DT == kLogitsBF16)
    return __builtin_bit_cast(float, (unsigned)static_cast<const u16*>(row)[v] << 16);
  else
    return (float)__builtin_bit_cast(_Float16, static_cast<const u16*>(row)[v]);
}

// Group of 8 that may cross the end v1 of the row: elements at or past v1
// read as `pad` (after the temperature scaling).
template <int DT, bool SCALED>
__device__ __forceinline__ void load_tail(const void* row, int64_t v, int64_t v1, float inv_temp, float pad,
                                          float (&x)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float y = pad;
    if (v + e < v1) {
      y = load_one<DT>(row, v + e);
      if constexpr (SCALED) y = round_elem<DT>(y * inv_temp);
    }
    x[e] = y;
  }
}

template <int DT>
__device__ __forceinline__ void store_one(void* row, int64_t v, float g) {
  if constexpr (DT == kLogitsF32)
    static_cast<float*>(row)[v] = g;
  else
    static_cast<u16*>(row)[v] = to_bits(g, DT == kLogitsBF16);
}

template <int DT>
__device__ __forceinline__ void store8(void* row, int64_t v, int64_t v1, const float (&g)[8]) {
  if (v + 8 <= v1) {
    if constexpr (DT == kLogitsF32) {
      f32x4* p = reinterpret_cast<f32x4*>(static_cast<float*>(row) + v);
      p[0] = (f32x4){g[0], g[1], g[2], g[3]};
      p[1] = (f32x4){g[4], g[5], g[6], g[7]};
    } else {
      u32x4 w;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        w[j] = (unsigned)to_bits(g[2 * j], DT == kLogitsBF16) |
               ((unsigned)to_bits(g[2 * j + 1], DT == kLogitsBF16) << 16);
      *reinterpret_cast<u32x4*>(static_cast<u16*>(row) + v) = w;  // plain stores measured faster than nt
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (v + e < v1) store_one<DT>(row, v + e, g[e]);
  }
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Running state of one thread: maxima in base-2 units, sums relative to them.
struct Acc {
  float mt, zt, a, ms, zs;
};

__device__ __forceinline__ void add_group(Acc& c, const float (&t)[8], const float (&s)[8]) {
  float wt[8], ws[8];
  float sum_t = 0.f, sum_s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    wt[e] = exp2_fast(__builtin_fmaf(t[e], kL2E, -c.mt));
    ws[e] = exp2_fast(__builtin_fmaf(s[e], kL2E, -c.ms));
    sum_t += wt[e];
    sum_s += ws[e];
  }
  if (__builtin_expect(!(sum_t <= kLazyGroupSum && sum_s <= kLazyGroupSum), 0)) {
    // raise the maxima to this group's and redo it (first group, or a jump of > 2^20)
    float mt = c.mt, ms = c.ms;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      mt = fmaxf(mt, t[e] * kL2E);
      ms = fmaxf(ms, s[e] * kL2E);
    }
    const float ft = exp2_fast(c.mt - mt), fs = exp2_fast(c.ms - ms);
    c.zt *= ft;
    c.a *= ft;
    c.zs *= fs;
    c.mt = mt;
    c.ms = ms;
    sum_t = 0.f;
    sum_s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      wt[e] = exp2_fast(__builtin_fmaf(t[e], kL2E, -c.mt));
      ws[e] = exp2_fast(__builtin_fmaf(s[e], kL2E, -c.ms));
      sum_t += wt[e];
      sum_s += ws[e];
    }
  }
  c.zt += sum_t;
  c.zs += sum_s;
#pragma unroll
  for (int e = 0; e < 8; ++e) c.a = __builtin_fmaf(wt[e], t[e] - s[e], c.a);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Fixed-order merge of the 256 threads' states; the result is valid in thread 0.
__device__ __forceinline__ Acc block_merge(Acc c) {
  __shared__ float red[kThreads / 64][4];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float mt = wave_max(c.mt), ms = wave_max(c.ms);
  if (lane == 0) {
    red[w][0] = mt;
    red[w][1] = ms;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) {
    mt = fmaxf(mt, red[i][0]);
    ms = fmaxf(ms, red[i][1]);
  }
  __syncthreads();
  const float ft = exp2_fast(c.mt - mt), fs = exp2_fast(c.ms - ms);
  const float zt = wave_sum(c.zt * ft), a = wave_sum(c.a * ft), zs = wave_sum(c.zs * fs);
  if (lane == 0) {
    red[w][0] = zt;
    red[w][1] = a;
    red[w][2] = zs;
  }
  __syncthreads();
  Acc r{mt, 0.f, 0.f, ms, 0.f};
  if (threadIdx.x == 0) {
#pragma unroll
    for (int i = 0; i < kThreads / 64; ++i) {
      r.zt += red[i][0];
      r.a += red[i][1];
      r.zs += red[i][2];
    }
  }
  return r;
}

struct RowSpan {
  const void* t;
  const void* s;
  int64_t v0, v1;
  int row;
};

template <int DT>
__device__ __forceinline__ RowSpan row_span(const LogitsArgs& a) {
  constexpr int64_t esize = DT == kLogitsF32 ? 4 : 2;
  const int split = (int)(blockIdx.x % (unsigned)a.splits);
  const int row = (int)(blockIdx.x / (unsigned)a.splits);
  const int b = row / a.K, k = row - b * a.K;
  RowSpan r;
  r.t = static_cast<const char*>(a.t) + (b * a.t_sb + k * a.t_sk) * esize;
  r.s = static_cast<const char*>(a.s) + (b * a.s_sb + k * a.s_sk) * esize;
  r.v0 = split * a.chunk;
  r.v1 = r.v0 + a.chunk < a.V ? r.v0 + a.chunk : a.V;
  r.row = row;
  return r;
}


// Groups of 8 per thread in one unit: 16 bytes of each row per group for
// 16-bit types (2 groups), 32 bytes for fp32 (1 group): 4096 logits per
// workgroup, 64 bytes of loads per thread in flight during the compute.
// (62 VGPRs: 8 waves per SIMD; 4 groups per unit measured slower.)
template <int DT>
constexpr int kGroups = DT == kLogitsF32 ? 1 : 2;

template <int DT>
struct Unit {
  Raw<DT> t[kGroups<DT>], s[kGroups<DT>];
};

// Loads every group of a unit.  Groups that do not lie wholly inside the
// chunk load the row's first 8 logits instead (V >= 8) and are never
// visited: the loads stay unconditional, so the compiler's wait counts stay
// exact and the next unit's loads remain in flight during the compute.
template <int DT>
__device__ __forceinline__ void load_unit(Unit<DT>& u, const RowSpan& r, int64_t v) {
#pragma unroll
  for (int g = 0; g < kGroups<DT>; ++g) {
    const int64_t gv = v + g * kStep;
    const int64_t src = gv + 8 <= r.v1 ? gv : 0;
    u.t[g] = load_raw<DT>(r.t, src);
    u.s[g] = load_raw<DT>(r.s, src);
  }
}

template <int DT, bool SCALED, class F>
__device__ __forceinline__ void visit_unit(const Unit<DT>& u, const RowSpan& r, int64_t v, float inv_temp, F& f) {
#pragma unroll
  for (int g = 0; g < kGroups<DT>; ++g) {
    const int64_t gv = v + g * kStep;
    if (gv + 8 <= r.v1) {
      float t[8], s[8];
      unpack<DT, SCALED>(u.t[g], inv_temp, t);
      unpack<DT, SCALED>(u.s[g], inv_temp, s);
      f(gv, t, s, true);
    }
  }
}

// Streams this thread's groups of 8 logits of the chunk through
// f(v, t, s, full), one unit at a time, with the next unit's loads in flight
// while the current one is computed (two register buffers, no copies).  The
// group holding the row's last V % 8 logits (all of them when V < 8) is
// read element by element after the loop, padded with `pad`, and passed
// with full = false.
template <int DT, bool SCALED, class F>
__device__ __forceinline__ void stream_chunk(const RowSpan& r, int64_t V, float inv_temp, float pad, F& f) {
  constexpr int64_t kUnitStep = kGroups<DT> * kStep;
  if (V >= 8) {
    int64_t v = r.v0 + threadIdx.x * 8;
    Unit<DT> a, b;
    load_unit<DT>(a, r, v);
    while (v < r.v1) {
      load_unit<DT>(b, r, v + kUnitStep);
      visit_unit<DT, SCALED>(a, r, v, inv_temp, f);
      v += kUnitStep;
      if (v >= r.v1) break;
      load_unit<DT>(a, r, v + kUnitStep);
      visit_unit<DT, SCALED>(b, r, v, inv_temp, f);
      v += kUnitStep;
    }
  }
  const int64_t gp = V & ~(int64_t)7;
  if (gp < V && gp >= r.v0 && gp < r.v1 && (int)(((gp - r.v0) >> 3) % kThreads) == (int)threadIdx.x) {
    float t[8], s[8];
    load_tail<DT, SCALED>(r.t, gp, r.v1, inv_temp, pad, t);
    load_tail<DT, SCALED>(r.s, gp, r.v1, inv_temp, pad, s);
    f(gp, t, s, false);
  }
}

template <int DT, bool SCALED>
__global__ __launch_bounds__(kThreads) void logits_kl_forward_kernel(const LogitsArgs a) {
  const RowSpan r = row_span<DT>(a);
  Acc c{kStartMax, 0.f, 0.f, kStartMax, 0.f};
  auto f = [&](int64_t, const float (&t)[8], const float (&s)[8], bool) { add_group(c, t, s); };
  stream_chunk<DT, SCALED>(r, a.V, a.inv_temp, kPadLogit, f);
  const Acc m = block_merge(c);
  if (threadIdx.x == 0) {
    float* p = a.part + ((int64_t)r.row * a.splits + (int)(blockIdx.x % (unsigned)a.splits)) * kLogitsPartFloats;
    *reinterpret_cast<f32x4*>(p) = (f32x4){m.mt, m.zt, m.a, m.ms};
    *reinterpret_cast<f32x4*>(p + 4) = (f32x4){m.zs, 0.f, 0.f, 0.f};
  }
}

// One workgroup: merge each row's chunks, write lse_t / lse_s / KL, and the
// mean over the rows (rows summed in a fixed order).
__global__ __launch_bounds__(kThreads) void logits_kl_finish_kernel(const LogitsArgs a) {
  float local = 0.f;
  for (int r = threadIdx.x; r < a.rows; r += kThreads) {
    float kl = 0.f, lse_t = -__builtin_inff(), lse_s = -__builtin_inff();
    if (a.V > 0) {
      const float* p = a.part + (int64_t)r * a.splits * kLogitsPartFloats;
      float mt = kStartMax, ms = kStartMax;
      for (int i = 0; i < a.splits; ++i) {
        mt = fmaxf(mt, p[i * kLogitsPartFloats]);
        ms = fmaxf(ms, p[i * kLogitsPartFloats + 3]);
      }
      float zt = 0.f, at = 0.f, zs = 0.f;
      for (int i = 0; i < a.splits; ++i) {
        const float* q = p + i * kLogitsPartFloats;
        const float ft = exp2_fast(q[0] - mt), fs = exp2_fast(q[3] - ms);
        zt += q[1] * ft;
        at += q[2] * ft;
        zs += q[4] * fs;
      }
      // rounded products: a product fused into the KL's subtraction would
      // treat the two log-sum-exps differently (identical rows must give 0)
      lse_t = mul_rn(mt + __builtin_amdgcn_logf(zt), kLn2);
      lse_s = mul_rn(ms + __builtin_amdgcn_logf(zs), kLn2);
      kl = at / zt - lse_t + lse_s;
    }
    a.lse_t[r] = lse_t;
    a.lse_s[r] = lse_s;
    a.kl[r] = kl;
    local += kl;
  }
  __shared__ float red[kThreads / 64];
  local = wave_sum(local);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = local;
  __syncthreads();
  if (threadIdx.x == 0) {
    float total = 0.f;
#pragma unroll
    for (int i = 0; i < kThreads / 64; ++i) total += red[i];
    a.loss[0] = total / (float)a.rows;  // rows == 0: NaN, the mean of an empty tensor
  }
}

template <int DT, bool SCALED, bool GT, bool GS>
__global__ __launch_bounds__(kThreads) void logits_kl_grad_kernel(const LogitsArgs a) {
  constexpr int64_t esize = DT == kLogitsF32 ? 4 : 2;
  const RowSpan r = row_span<DT>(a);
  const int b = r.row / a.K, k = r.row - b * a.K;
  void* gt = GT ? static_cast<char*>(a.gt) + (b * a.gt_sb + k * a.gt_sk) * esize : nullptr;
  void* gs = GS ? static_cast<char*>(a.gs) + (b * a.gs_sb + k * a.gs_sk) * esize : nullptr;
  const float c = a.dloss[a.dloss_per_row ? r.row : 0] * a.row_scale * a.inv_temp;
  const float lt = a.lse_t[r.row], ls = a.lse_s[r.row];
  const float lt2 = lt * kL2E, ls2 = ls * kL2E;
  const float kl = GT ? a.kl[r.row] : 0.f;

  auto group = [&](int64_t v, const float (&t)[8], const float (&s)[8], bool full) {
    float g_s[8], g_t[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float pt = exp2_fast(__builtin_fmaf(t[e], kL2E, -lt2));
      const float ps = exp2_fast(__builtin_fmaf(s[e], kL2E, -ls2));
      g_s[e] = c * (ps - pt);
      g_t[e] = c * pt * ((t[e] - lt) - (s[e] - ls) - kl);
    }
    if constexpr (GS) store8<DT>(gs, v, full ? v + 8 : r.v1, g_s);
    if constexpr (GT) store8<DT>(gt, v, full ? v + 8 : r.v1, g_t);
  };

  stream_chunk<DT, SCALED>(r, a.V, a.inv_temp, 0.f, group);  // pad values are never stored (store8 stops at v1)
}

template <int DT, bool SCALED>
hipError_t forward_dt(const LogitsArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)((int64_t)a.rows * a.splits)), block(kThreads);
  hipLaunchKernelGGL((logits_kl_forward_kernel<DT, SCALED>), grid, block, 0, st, a);
  return hipGetLastError();
}

template <int DT, bool SCALED>
hipError_t grad_dt(const LogitsArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)((int64_t)a.rows * a.splits)), block(kThreads);
  if (a.gt != nullptr && a.gs != nullptr)
    hipLaunchKernelGGL((logits_kl_grad_kernel<DT, SCALED, true, true>), grid, block, 0, st, a);
  else if (a.gt != nullptr)
    hipLaunchKernelGGL((logits_kl_grad_kernel<DT, SCALED, true, false>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((logits_kl_grad_kernel<DT, SCALED, false, true>), grid, block, 0, st, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_logits_kl_forward(const LogitsArgs& a, int dtype, hipStream_t stream) {
  const bool scaled = a.inv_temp != 1.f;
  switch (dtype) {
    case kLogitsBF16:
      return scaled ? forward_dt<kLogitsBF16, true>(a, stream) : forward_dt<kLogitsBF16, false>(a, stream);
    case kLogitsF16:
      return scaled ? forward_dt<kLogitsF16, true>(a, stream) : forward_dt<kLogitsF16, false>(a, stream);
    default:
      return scaled ? forward_dt<kLogitsF32, true>(a, stream) : forward_dt<kLogitsF32, false>(a, stream);
  }
}

hipError_t launch_logits_kl_finish(const LogitsArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(logits_kl_finish_kernel, dim3(1), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_logits_kl_grad(const LogitsArgs& a, int dtype, hipStream_t stream) {
  const bool scaled = a.inv_temp != 1.f;
  switch (dtype) {
    case kLogitsBF16:
      return scaled ? grad_dt<kLogitsBF16, true>(a, stream) : grad_dt<kLogitsBF16, false>(a, stream);
    case kLogitsF16:
      return scaled ? grad_dt<kLogitsF16, true>(a, stream) : grad_dt<kLogitsF16, false>(a, stream);
    default:
      return scaled ? grad_dt<kLogitsF32, true>(a, stream) : grad_dt<kLogitsF32, false>(a, stream);
  }
}

}  // namespace lard
