// C ABI entry points: argument validation, descriptor packing, dispatch.
//
// Validation restates the preconditions of the reference wrappers
// (kernel_A.py:192-220, kernel_B.py:262-322, kernel_C.py:307-368) as error
// returns, plus the alignment rules of the 16-byte vector loads.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <utility>
#include <vector>
#include <string>

#include "../../include/linearard_amd.h"
#include "hot_fwdq.h"
#include "logits_kl_kernels.h"
#include "rope_kernels.h"
#include "stage_f32.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return LARD_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(LARD_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

bool supported_dim(int64_t d) {
  return d == 8 || d == 16 || d == 32 || d == 64 || d == 128 || d == 256;  // kernel_A.py:18
}

int padded_dim(int64_t d) { return d < 16 ? 16 : (int)d; }

int check_tensor(const lard_tensor4* t, const char* name) {
  if (t == nullptr) return fail(LARD_ERR_INVALID_ARGUMENT, "%s must not be NULL", name);
  if (t->data == nullptr && t->size[0] * t->size[1] * t->size[2] * t->size[3] != 0)
    return fail(LARD_ERR_INVALID_ARGUMENT, "%s data pointer is NULL", name);
  for (int i = 0; i < 4; ++i)
    if (t->size[i] < 0) return fail(LARD_ERR_INVALID_ARGUMENT, "%s has a negative size", name);
  if (t->dtype != LARD_DTYPE_F16 && t->dtype != LARD_DTYPE_BF16 && t->dtype != LARD_DTYPE_F32)
    return fail(LARD_ERR_UNSUPPORTED, "%s dtype supports only fp16/bf16/fp32", name);
  if (t->stride[3] != 1) return fail(LARD_ERR_INVALID_ARGUMENT, "%s last-dim stride must be 1", name);
  const int64_t vec = t->dtype == LARD_DTYPE_F32 ? 4 : 8;  // elements per 16-byte load
  for (int i = 0; i < 3; ++i)
    if (t->stride[i] % vec != 0)
      return fail(LARD_ERR_UNSUPPORTED, "%s strides must be multiples of %d elements", name, (int)vec);
  if (reinterpret_cast<uintptr_t>(t->data) % 16 != 0)
    return fail(LARD_ERR_UNSUPPORTED, "%s data pointer must be 16-byte aligned", name);
  if (t->size[2] > (int64_t)1 << 30) return fail(LARD_ERR_UNSUPPORTED, "%s sequence length too large", name);
  return LARD_OK;
}

// Checks a (q, k) relation pair (kernel_A.py:192-208).
int check_pair(const lard_tensor4* q, const lard_tensor4* k, const char* qn, const char* kn) {
  int rc;
  if ((rc = check_tensor(q, qn)) != LARD_OK) return rc;
  if ((rc = check_tensor(k, kn)) != LARD_OK) return rc;
  if (q->dtype != k->dtype) return fail(LARD_ERR_INVALID_ARGUMENT, "%s/%s dtype must match", qn, kn);
  if (q->size[0] != k->size[0]) return fail(LARD_ERR_INVALID_ARGUMENT, "%s/%s B must match", qn, kn);
  if (q->size[2] != k->size[2]) return fail(LARD_ERR_INVALID_ARGUMENT, "%s/%s T must match", qn, kn);
  if (q->size[3] != k->size[3]) return fail(LARD_ERR_INVALID_ARGUMENT, "%s/%s D must match", qn, kn);
  if (!supported_dim(q->size[3])) return fail(LARD_ERR_UNSUPPORTED, "D is not in the supported set");
  if (k->size[1] <= 0 && q->size[1] > 0) return fail(LARD_ERR_INVALID_ARGUMENT, "%s has no heads", kn);
  if (k->size[1] > 0 && q->size[1] % k->size[1] != 0)
    return fail(LARD_ERR_INVALID_ARGUMENT, "Hq must be divisible by Hkv");
  return LARD_OK;
}

int check_mask(const lard_mask* m, int64_t B, int64_t T) {
  if (m == nullptr || m->kind == LARD_MASK_NONE) return LARD_OK;
  if (m->kind != LARD_MASK_U8 && m->kind != LARD_MASK_I32 && m->kind != LARD_MASK_I64)
    return fail(LARD_ERR_INVALID_ARGUMENT, "attn_mask dtype is invalid");
  if (m->size[0] != B || m->size[1] != T) return fail(LARD_ERR_INVALID_ARGUMENT, "attn_mask shape must be [B,T]");
  if (m->stride[1] != 1 && T > 1) return fail(LARD_ERR_INVALID_ARGUMENT, "attn_mask last-dim stride must be 1");
  if (m->data == nullptr && B * T != 0) return fail(LARD_ERR_INVALID_ARGUMENT, "attn_mask data pointer is NULL");
  return LARD_OK;
}

void fill_side(lard::SideArgs& s, const lard_tensor4* q, const lard_tensor4* k, int64_t Hq, float scale) {
  s.q = static_cast<const lard::u16*>(q->data);
  s.k = static_cast<const lard::u16*>(k->data);
  s.q_sb = q->stride[0];
  s.q_sh = q->stride[1];
  s.q_st = q->stride[2];
  s.k_sb = k->stride[0];
  s.k_sh = k->stride[1];
  s.k_st = k->stride[2];
  s.hkv = (int)k->size[1];
  s.group = (int)(Hq / k->size[1]);
  s.dim = (int)q->size[3];
  s.bf16 = q->dtype == LARD_DTYPE_BF16;
  s.f32 = q->dtype == LARD_DTYPE_F32;
  s.scale = scale;
  s.scale2 = scale * lard::kLog2e;
}

void fill_common(lard::RelArgs& a, int64_t B, int64_t Hq, int64_t T, const lard_mask* m, int causal) {
  a.B = (int)B;
  a.Hq = (int)Hq;
  a.T = (int)T;
  a.causal = causal ? 1 : 0;
  if (m != nullptr && m->kind != LARD_MASK_NONE) {
    a.mask = m->data;
    a.mask_kind = m->kind;
    a.mask_sb = m->stride[0];
  } else {
    a.mask = nullptr;
    a.mask_kind = 0;
    a.mask_sb = 0;
  }
}

int check_grid(int64_t rows) {
  if (rows > 65536) return fail(LARD_ERR_UNSUPPORTED, "B * heads must be <= 65536");
  return LARD_OK;
}

int check_scale(float s, const char* name) {
  if (!std::isfinite(s)) return fail(LARD_ERR_INVALID_ARGUMENT, "%s must be a finite scalar", name);
  return LARD_OK;
}

// Stage B / C share their argument checks (kernel_B.py:262-322).
int check_two_sided(const lard_tensor4* qs, const lard_tensor4* ks, const float* lse_s, const lard_tensor4* qt,
                    const lard_tensor4* kt, const float* lse_t, const lard_mask* mask, float ss, float st) {
  int rc;
  if ((rc = check_pair(qs, ks, "qs", "ks")) != LARD_OK) return rc;
  if ((rc = check_pair(qt, kt, "qt", "kt")) != LARD_OK) return rc;
  if (qs->size[0] != qt->size[0] || qs->size[1] != qt->size[1] || qs->size[2] != qt->size[2])
    return fail(LARD_ERR_INVALID_ARGUMENT, "student/teacher B/Hq/T must align");
  if ((qs->dtype == LARD_DTYPE_F32) != (qt->dtype == LARD_DTYPE_F32))
    return fail(LARD_ERR_UNSUPPORTED, "float32 inputs need float32 on both sides");
  const int64_t n = qs->size[0] * qs->size[1] * qs->size[2];
  if (n > 0 && (lse_s == nullptr || lse_t == nullptr)) return fail(LARD_ERR_INVALID_ARGUMENT, "lse must not be NULL");
  if ((rc = check_mask(mask, qs->size[0], qs->size[2])) != LARD_OK) return rc;
  if ((rc = check_scale(ss, "sm_scale_s")) != LARD_OK) return rc;
  if ((rc = check_scale(st, "sm_scale_t")) != LARD_OK) return rc;
  return check_grid(qs->size[0] * (qs->size[1] > ks->size[1] ? qs->size[1] : ks->size[1]));
}

// The throughput kernels run one flat grid of (T / 256) x B x heads workgroups.
int check_blocks(int64_t B, int64_t heads, int64_t T) {
  if ((T + lard::kRows - 1) / lard::kRows * B * heads > (int64_t)INT32_MAX)
    return fail(LARD_ERR_UNSUPPORTED, "B * heads * T / %d must be < 2^31", lard::kRows);
  return LARD_OK;
}

int64_t padded_len(int64_t T) { return (T + lard::kTile - 1) / lard::kTile * lard::kTile; }

// The throughput kernels address one head of every operand with 32-bit byte
// offsets: (T-1) * row_stride + D elements must stay below 2^30 elements.
// Larger heads run the stage kernels.
bool hot_offsets_ok(std::initializer_list<const lard_tensor4*> ts, int64_t T) {
  constexpr int64_t kMax = (int64_t)1 << 30;
  for (const lard_tensor4* t : ts)
    if ((T - 1) * t->stride[2] + t->size[3] >= kMax) return false;
  return true;
}

// The throughput kernels give masked logits the raw value -1e30 and start
// the forward's running maxima at -5e29; with the scales' magnitudes in
// [1e-6, 1e6] and within a factor 1e6 of each other every masked
// exponential is exactly 0 and every product stays finite.  Other scales
// take the stage kernels.
bool hot_scales_ok(float s, float t) {
  const float as = std::fabs(s), at = std::fabs(t);
  return as >= 1e-6f && at >= 1e-6f && as <= 1e6f && at <= 1e6f && as <= 1e6f * at && at <= 1e6f * as;
}

// The kernels an autograd call (lard_attn_kl_forward / _backward) runs for
// these operands, and in `why` the condition that took it off the
// throughput kernels (empty on them).  Checked operands only.
int attn_kl_path(const lard_tensor4* qs, const lard_tensor4* ks, const lard_tensor4* qt, const lard_tensor4* kt,
                 float sm_scale_s, float sm_scale_t, std::string* why) {
  const int ds = (int)qs->size[3], dt = (int)qt->size[3];
  const bool same = qs->dtype == qt->dtype;
  char buf[160];
  if (qs->dtype == LARD_DTYPE_F32) {
    *why = "float32 inputs run the double-precision kernels";
    return LARD_PATH_FLOAT32;
  }
  if (!lard::hot_supported(ds, dt, same)) {
    if (!same)
      *why = "student and teacher dtypes differ";
    else if (ds != dt)
      snprintf(buf, sizeof(buf), "student head dim %d != teacher head dim %d", ds, dt), *why = buf;
    else
      snprintf(buf, sizeof(buf), "head dim %d > 128", ds), *why = buf;
    return lard::fused_fwd_supported(ds, dt, same) ? LARD_PATH_FUSED_FORWARD : LARD_PATH_STAGE;
  }
  if (!hot_offsets_ok({qs, ks, qt, kt}, qs->size[2])) {
    *why = "a head spans 2^30 elements or more (32-bit offsets)";
    return LARD_PATH_FUSED_FORWARD;
  }
  if (!hot_scales_ok(sm_scale_s, sm_scale_t)) {
    snprintf(buf, sizeof(buf), "scales %g / %g outside [1e-6, 1e6] or more than 1e6 apart", sm_scale_s, sm_scale_t);
    *why = buf;
    return LARD_PATH_FUSED_FORWARD;
  }
  why->clear();
  return LARD_PATH_THROUGHPUT;
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// Carves 256-byte aligned regions out of a caller workspace in a fixed
// order; with a null base it only counts bytes (the *_workspace_bytes calls).
class Carver {
 public:
  explicit Carver(void* base) : base_(static_cast<char*>(base)) {}
  template <class T>
  T* take(int64_t count) {
    T* p = base_ != nullptr ? reinterpret_cast<T*>(base_ + off_) : nullptr;
    off_ += align256((size_t)count * sizeof(T));
    return p;
  }
  size_t bytes() const { return off_; }

 private:
  char* base_;
  size_t off_ = 0;
};

// Loss reduction: per-row KL terms, then double partials.
struct LossWs {
  float* rows;
  double* partial;
};

LossWs loss_layout(void* base, int64_t n, size_t* bytes) {
  Carver c(base);
  LossWs w;
  w.rows = c.take<float>(n);
  w.partial = c.take<double>(lard::kReduceBlocks);
  if (bytes != nullptr) *bytes = c.bytes();
  return w;
}

// Forward of the autograd path: loss regions + token validity + the first
// two valid tokens of each sequence.
struct FwdWs {
  LossWs loss;
  unsigned char* tok_ok;
  int* first2;
};

FwdWs fwd_layout(void* base, int64_t B, int64_t H, int64_t T, size_t* bytes) {
  size_t loss_bytes = 0;
  FwdWs w;
  w.loss = loss_layout(base, B * H * T, &loss_bytes);
  Carver c(base != nullptr ? static_cast<char*>(base) + loss_bytes : nullptr);
  const int64_t Tp = padded_len(T);
  w.tok_ok = c.take<unsigned char>(B * Tp);
  w.first2 = c.take<int>(2 * B);
  if (bytes != nullptr) *bytes = loss_bytes + c.bytes();
  return w;
}

// Forward with the row-side gradient: the forward's regions, then both
// sides' keys as float16 ([B, Hkv_s, T, D] and [B, Hkv_t, T, D]; bfloat16
// inputs), the scratch of their maxima and the powers of two they were
// scaled by.
struct KeysF16 {
  lard::u16* k16;
  unsigned* maxbits;
  float* scale;
};

KeysF16 take_keys(Carver& c, int64_t B, int64_t Hkv, int64_t T, int64_t D) {
  KeysF16 k;
  k.k16 = c.take<lard::u16>(B * Hkv * T * D);
  k.maxbits = c.take<unsigned>(1);
  k.scale = c.take<float>(1);
  return k;
}

struct RowgradWs {
  FwdWs fwd;
  KeysF16 s, t;
};

RowgradWs rowgrad_layout(void* base, int64_t B, int64_t Hq, int64_t Hkv_s, int64_t Hkv_t, int64_t T, int64_t D,
                         size_t* bytes) {
  size_t fwd_bytes = 0;
  RowgradWs w;
  w.fwd = fwd_layout(base, B, Hq, T, &fwd_bytes);
  Carver c(base != nullptr ? static_cast<char*>(base) + fwd_bytes : nullptr);
  w.s = take_keys(c, B, Hkv_s, T, D);
  w.t = take_keys(c, B, Hkv_t, T, D);
  if (bytes != nullptr) *bytes = fwd_bytes + c.bytes();
  return w;
}

// Both sides' float16 keys for the fused row-gradient forward: scaled copies
// for bfloat16 inputs, the tensors themselves for float16 ones.
hipError_t keys_f16(lard::HotArgs& f, bool bf, const KeysF16& ks, const KeysF16& kt, hipStream_t st) {
  if (!bf) {
    f.k16 = f.r.s.k;
    f.k16_sb = f.r.s.k_sb;
    f.k16_sh = f.r.s.k_sh;
    f.k16_st = f.r.s.k_st;
    f.k16_scale = nullptr;
    f.k16t = f.r.t.k;
    f.k16t_sb = f.r.t.k_sb;
    f.k16t_sh = f.r.t.k_sh;
    f.k16t_st = f.r.t.k_st;
    f.k16t_scale = nullptr;
    return hipSuccess;
  }
  const int64_t D = f.r.s.dim, T = f.r.T;
  f.k16 = ks.k16;
  f.k16_st = D;
  f.k16_sh = T * D;
  f.k16_sb = (int64_t)f.r.s.hkv * T * D;
  f.k16_scale = ks.scale;
  f.k16t = kt.k16;
  f.k16t_st = D;
  f.k16t_sh = T * D;
  f.k16t_sb = (int64_t)f.r.t.hkv * T * D;
  f.k16t_scale = kt.scale;
  hipError_t e = lard::launch_keys_f16(f.r.s, f.r.B, f.r.Hq, f.r.T, ks.maxbits, ks.scale, ks.k16, st);
  if (e != hipSuccess) return e;
  return lard::launch_keys_f16(f.r.t, f.r.B, f.r.Hq, f.r.T, kt.maxbits, kt.scale, kt.k16, st);
}

// Backward of the autograd path: token validity, the first two valid tokens
// of each sequence and the log2-domain row normalisers (the size depends on
// B, Hq and T only).
struct BwdWs {
  unsigned char* tok_ok;
  int* first2;
  float* nl_s;
  float* nl_t;
};

BwdWs bwd_layout(void* base, int64_t B, int64_t Hq, int64_t T, size_t* bytes) {
  Carver c(base);
  BwdWs w;
  const int64_t Tp = padded_len(T);
  w.tok_ok = c.take<unsigned char>(B * Tp);
  w.first2 = c.take<int>(2 * B);
  w.nl_s = c.take<float>(B * Hq * Tp);
  w.nl_t = c.take<float>(B * Hq * Tp);
  if (bytes != nullptr) *bytes = c.bytes();
  return w;
}

// Opt-in launch timing (lard_timing_*): event pairs recorded around the
// throughput launches, drained by lard_timing_read.  Events are pooled and
// never destroyed, so a read never races a record on another thread.
struct Timing {
  std::mutex mu;
  bool on = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pending[LARD_KERNEL_COUNT];
  std::vector<hipEvent_t> pool;

  hipEvent_t take() {
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    return hipEventCreate(&e) == hipSuccess ? e : nullptr;
  }
};

Timing& timing() {
  static Timing t;
  return t;
}

// Runs launch() on stream st; brackets it with events when timing is on.
template <class F>
hipError_t timed(int kernel, hipStream_t st, F&& launch) {
  Timing& tm = timing();
  hipEvent_t start = nullptr;
  {
    std::lock_guard<std::mutex> g(tm.mu);
    if (tm.on && (start = tm.take()) != nullptr && hipEventRecord(start, st) != hipSuccess) {
      tm.pool.push_back(start);
      start = nullptr;
    }
  }
  const hipError_t e = launch();
  if (start != nullptr) {
    std::lock_guard<std::mutex> g(tm.mu);
    hipEvent_t stop = tm.take();
    if (stop != nullptr && hipEventRecord(stop, st) == hipSuccess) {
      tm.pending[kernel].emplace_back(start, stop);
    } else {
      tm.pool.push_back(start);
      if (stop != nullptr) tm.pool.push_back(stop);
    }
  }
  return e;
}


// ---- batched relation loss (lard_attn_kl_batched_*) ----

// per-row KL terms of every relation, loss partials, token validity (shared:
// one B and T), row normalisers of every relation
struct BatchWs {
  LossWs loss;
  unsigned char* tok_ok;
  int* first2;
  float* nl_s;
  float* nl_t;
};

int64_t rel_rows(const lard_relation& r) { return r.xs.size[0] * r.xs.size[1] * r.xs.size[2]; }

BatchWs batch_layout(void* base, const lard_relation* rels, int nrel, size_t* bytes) {
  int64_t rows = 0, prows = 0;
  for (int r = 0; r < nrel; ++r) {
    rows += rel_rows(rels[r]);
    prows += rels[r].xs.size[0] * rels[r].xs.size[1] * padded_len(rels[r].xs.size[2]);
  }
  size_t loss_bytes = 0;
  BatchWs w;
  w.loss = loss_layout(base, rows, &loss_bytes);
  Carver c(base != nullptr ? static_cast<char*>(base) + loss_bytes : nullptr);
  w.tok_ok = c.take<unsigned char>(rels[0].xs.size[0] * padded_len(rels[0].xs.size[2]));
  w.first2 = c.take<int>(2 * rels[0].xs.size[0]);
  w.nl_s = c.take<float>(prows);
  w.nl_t = c.take<float>(prows);
  if (bytes != nullptr) *bytes = loss_bytes + c.bytes();
  return w;
}

// A batch the throughput kernels take: self relations sharing B, T, dtype
// and head dim D <= 128, moderate scales.  Everything else is rejected.
int check_batch(const lard_relation* rels, int nrel, const lard_mask* mask, float sm_scale_s, float sm_scale_t) {
  int rc;
  if (rels == nullptr || nrel < 1) return fail(LARD_ERR_INVALID_ARGUMENT, "rels must hold at least one relation");
  const lard_tensor4& x0 = rels[0].xs;
  for (int r = 0; r < nrel; ++r) {
    const lard_tensor4& xs = rels[r].xs;
    const lard_tensor4& xt = rels[r].xt;
    if ((rc = check_pair(&xs, &xs, "xs", "xs")) != LARD_OK) return rc;
    if ((rc = check_pair(&xt, &xt, "xt", "xt")) != LARD_OK) return rc;
    if (xs.size[0] != xt.size[0] || xs.size[1] != xt.size[1] || xs.size[2] != xt.size[2])
      return fail(LARD_ERR_INVALID_ARGUMENT, "relation %d: student/teacher B/H/T must align", r);
    if (xs.size[0] != x0.size[0] || xs.size[2] != x0.size[2])
      return fail(LARD_ERR_INVALID_ARGUMENT, "relation %d: every relation must share B and T", r);
    if (xs.dtype != x0.dtype || xt.dtype != x0.dtype || xs.size[3] != x0.size[3] || xt.size[3] != x0.size[3])
      return fail(LARD_ERR_UNSUPPORTED, "relation %d: batched relations must share the dtype and head dim", r);
    if (xs.dtype == LARD_DTYPE_F32)
      return fail(LARD_ERR_UNSUPPORTED, "relation %d: float32 relations run one by one (stage kernels)", r);
    if (!lard::hot_supported((int)xs.size[3], (int)xt.size[3], true) || !hot_offsets_ok({&xs, &xt}, xs.size[2]))
      return fail(LARD_ERR_UNSUPPORTED, "relation %d: shape outside the batched kernels (D <= 128)", r);
    if (xs.size[1] <= 0) return fail(LARD_ERR_INVALID_ARGUMENT, "relation %d has no heads", r);
    if ((rc = check_blocks(xs.size[0], xs.size[1], xs.size[2])) != LARD_OK) return rc;
  }
  if ((rc = check_mask(mask, x0.size[0], x0.size[2])) != LARD_OK) return rc;
  if ((rc = check_scale(sm_scale_s, "sm_scale_s")) != LARD_OK) return rc;
  if ((rc = check_scale(sm_scale_t, "sm_scale_t")) != LARD_OK) return rc;
  if (!hot_scales_ok(sm_scale_s, sm_scale_t))
    return fail(LARD_ERR_UNSUPPORTED, "scales outside the batched kernels' range");
  return LARD_OK;
}

lard::HotArgs relation_args(const lard_relation& R, const lard_mask* mask, int causal, float sm_scale_s,
                            float sm_scale_t, int Tp, const unsigned char* tok_ok, const int* first2) {
  lard::HotArgs f{};
  const int64_t H = R.xs.size[1];
  fill_side(f.r.s, &R.xs, &R.xs, H, sm_scale_s);
  fill_side(f.r.t, &R.xt, &R.xt, H, sm_scale_t);
  fill_common(f.r, R.xs.size[0], H, R.xs.size[2], mask, causal);
  f.Tp = Tp;
  f.tok_ok = tok_ok;
  f.first2 = first2;
  return f;
}


// ---- logits KL (lard_logits_kl_*) ----

int logits_esize(int32_t dtype) { return dtype == LARD_DTYPE_F32 ? 4 : 2; }

// [B, K, V] logits (or their gradient): vocabulary stride 1, 16-byte aligned
// rows (the kernels read and write 16 bytes at a time).
int check_logits(const lard_logits* x, const char* name) {
  if (x == nullptr) return fail(LARD_ERR_INVALID_ARGUMENT, "%s must not be NULL", name);
  for (int i = 0; i < 3; ++i)
    if (x->size[i] < 0) return fail(LARD_ERR_INVALID_ARGUMENT, "%s has a negative size", name);
  if (x->dtype != LARD_DTYPE_F16 && x->dtype != LARD_DTYPE_BF16 && x->dtype != LARD_DTYPE_F32)
    return fail(LARD_ERR_UNSUPPORTED, "%s dtype supports only fp16/bf16/fp32", name);
  const int64_t n = x->size[0] * x->size[1] * x->size[2];
  if (n == 0) return LARD_OK;
  if (x->data == nullptr) return fail(LARD_ERR_INVALID_ARGUMENT, "%s data pointer is NULL", name);
  if (x->stride[2] != 1 && x->size[2] > 1)
    return fail(LARD_ERR_INVALID_ARGUMENT, "%s vocabulary stride must be 1", name);
  const int64_t vec = 16 / logits_esize(x->dtype);
  if (reinterpret_cast<uintptr_t>(x->data) % 16 != 0 || (x->size[0] > 1 && x->stride[0] % vec != 0) ||
      (x->size[1] > 1 && x->stride[1] % vec != 0))
    return fail(LARD_ERR_UNSUPPORTED, "%s rows must start on 16-byte boundaries", name);
  return LARD_OK;
}

int check_logits_like(const lard_logits* x, const lard_logits* ref, const char* name) {
  int rc;
  if ((rc = check_logits(x, name)) != LARD_OK) return rc;
  if (x->size[0] != ref->size[0] || x->size[1] != ref->size[1] || x->size[2] != ref->size[2])
    return fail(LARD_ERR_INVALID_ARGUMENT, "%s shape must match the teacher logits", name);
  if (x->dtype != ref->dtype) return fail(LARD_ERR_INVALID_ARGUMENT, "%s dtype must match the teacher logits", name);
  return LARD_OK;
}

// 1 / T as a float32 quotient, as a tensor division by a host scalar forms it.
int check_temperature(float temperature, float* inv) {
  if (!std::isfinite(temperature) || temperature == 0.f)
    return fail(LARD_ERR_INVALID_ARGUMENT, "temperature must be finite and nonzero");
  *inv = 1.0f / temperature;
  if (!std::isfinite(*inv)) return fail(LARD_ERR_INVALID_ARGUMENT, "1 / temperature overflows float32");
  return LARD_OK;
}

int logits_common(const lard_logits* t, const lard_logits* s, float temperature, lard::LogitsArgs* a) {
  int rc;
  if ((rc = check_logits(t, "t_logits")) != LARD_OK) return rc;
  if ((rc = check_logits_like(s, t, "s_logits")) != LARD_OK) return rc;
  *a = lard::LogitsArgs{};
  if ((rc = check_temperature(temperature, &a->inv_temp)) != LARD_OK) return rc;
  const int64_t rows = t->size[0] * t->size[1], V = t->size[2];
  if (rows > INT32_MAX) return fail(LARD_ERR_UNSUPPORTED, "B * K must be < 2^31");
  const lard::LogitsSplit sp = lard::logits_split(rows, V);
  if (rows * sp.splits > INT32_MAX) return fail(LARD_ERR_UNSUPPORTED, "logits grid too large");
  a->t = t->data;
  a->s = s->data;
  a->t_sb = t->stride[0];
  a->t_sk = t->stride[1];
  a->s_sb = s->stride[0];
  a->s_sk = s->stride[1];
  a->K = (int)(t->size[1] > 0 ? t->size[1] : 1);
  a->rows = (int)rows;
  a->V = V;
  a->splits = sp.splits;
  a->chunk = sp.chunk;
  return LARD_OK;
}

}  // namespace

extern "C" {

int lard_timing_enable(int on) {
  Timing& tm = timing();
  std::lock_guard<std::mutex> g(tm.mu);
  tm.on = on != 0;
  return ok();
}

int lard_timing_read(int kernel, double* total_ms, int64_t* launches) {
  if (kernel < 0 || kernel >= LARD_KERNEL_COUNT) return fail(LARD_ERR_INVALID_ARGUMENT, "unknown kernel id %d", kernel);
  if (total_ms == nullptr || launches == nullptr)
    return fail(LARD_ERR_INVALID_ARGUMENT, "total_ms / launches must not be NULL");
  Timing& tm = timing();
  std::lock_guard<std::mutex> g(tm.mu);
  double sum = 0.0;
  int64_t n = 0;
  hipError_t err = hipSuccess;
  for (auto& pr : tm.pending[kernel]) {
    float ms = 0.f;
    if (err == hipSuccess) err = hipEventSynchronize(pr.second);
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, pr.first, pr.second);
    sum += ms;
    ++n;
    tm.pool.push_back(pr.first);
    tm.pool.push_back(pr.second);
  }
  tm.pending[kernel].clear();
  *total_ms = sum;
  *launches = n;
  return hip_status(err, "timing read");
}


const char* lard_version(void) { return "linearard_amd 0.1.0 gfx950"; }

const char* lard_last_error(void) { return g_last_error.c_str(); }

int lard_attn_kl_path(const lard_tensor4* qs, const lard_tensor4* ks, const lard_tensor4* qt, const lard_tensor4* kt,
                      float sm_scale_s, float sm_scale_t) {
  int rc;
  if ((rc = check_pair(qs, ks, "qs", "ks")) != LARD_OK) return rc;
  if ((rc = check_pair(qt, kt, "qt", "kt")) != LARD_OK) return rc;
  if (qs->size[0] != qt->size[0] || qs->size[1] != qt->size[1] || qs->size[2] != qt->size[2])
    return fail(LARD_ERR_INVALID_ARGUMENT, "student/teacher B/Hq/T must align");
  if ((qs->dtype == LARD_DTYPE_F32) != (qt->dtype == LARD_DTYPE_F32))
    return fail(LARD_ERR_UNSUPPORTED, "float32 inputs need float32 on both sides");
  if ((rc = check_scale(sm_scale_s, "sm_scale_s")) != LARD_OK) return rc;
  if ((rc = check_scale(sm_scale_t, "sm_scale_t")) != LARD_OK) return rc;
  std::string why;
  const int path = attn_kl_path(qs, ks, qt, kt, sm_scale_s, sm_scale_t, &why);
  g_last_error = why;
  return path;
}

int lard_lse_stats(const lard_tensor4* q, const lard_tensor4* k, const lard_mask* mask, int causal, float sm_scale,
                   float* lse_out, void* stream) {
  int rc;
  if ((rc = check_pair(q, k, "q", "k")) != LARD_OK) return rc;
  if ((rc = check_mask(mask, q->size[0], q->size[2])) != LARD_OK) return rc;
  if ((rc = check_scale(sm_scale, "sm_scale")) != LARD_OK) return rc;
  const int64_t B = q->size[0], Hq = q->size[1], T = q->size[2];
  if (B * Hq * T == 0) return ok();
  if (lse_out == nullptr) return fail(LARD_ERR_INVALID_ARGUMENT, "lse_out must not be NULL");
  if ((rc = check_grid(B * Hq)) != LARD_OK) return rc;
  lard::RelArgs a{};
  fill_side(a.s, q, k, Hq, sm_scale);
  a.t = a.s;
  fill_common(a, B, Hq, T, mask, causal);
  a.lse_out = lse_out;
  return hip_status(lard::launch_row_lse(a, padded_dim(q->size[3]), static_cast<hipStream_t>(stream)),
                    "lse_stats launch");
}

size_t lard_kl_forward_workspace_bytes(int64_t batch, int64_t heads, int64_t seq_len) {
  if (batch <= 0 || heads <= 0 || seq_len <= 0) return 0;
  size_t bytes = 0;
  loss_layout(nullptr, batch * heads * seq_len, &bytes);
  return bytes;
}

int lard_kl_forward(const lard_tensor4* qs, const lard_tensor4* ks, const float* lse_s, const lard_tensor4* qt,
                    const lard_tensor4* kt, const float* lse_t, const lard_mask* mask, int causal, float sm_scale_s,
                    float sm_scale_t, float* loss_out, void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = check_two_sided(qs, ks, lse_s, qt, kt, lse_t, mask, sm_scale_s, sm_scale_t)) != LARD_OK) return rc;
  if (loss_out == nullptr) return fail(LARD_ERR_INVALID_ARGUMENT, "loss_out must not be NULL");
  const int64_t B = qs->size[0], Hq = qs->size[1], T = qs->size[2];
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t n = B * Hq * T;
  if (n > 0) {
    if (workspace == nullptr || workspace_bytes < lard_kl_forward_workspace_bytes(B, Hq, T))
      return fail(LARD_ERR_INVALID_ARGUMENT, "workspace too small: need %zu bytes",
                  lard_kl_forward_workspace_bytes(B, Hq, T));
    lard::RelArgs a{};
    fill_side(a.s, qs, ks, Hq, sm_scale_s);
    fill_side(a.t, qt, kt, Hq, sm_scale_t);
    fill_common(a, B, Hq, T, mask, causal);
    a.lse_s_in = lse_s;
    a.lse_t_in = lse_t;
    const LossWs w = loss_layout(workspace, n, nullptr);
    a.row_out = w.rows;
    if ((rc = hip_status(lard::launch_row_kl(a, padded_dim(qs->size[3]), padded_dim(qt->size[3]), st),
                         "kl_forward launch")) != LARD_OK)
      return rc;
    return hip_status(lard::launch_reduce_sum(w.rows, n, w.partial, loss_out, st), "kl_forward reduce launch");
  }
  return hip_status(lard::launch_reduce_sum(nullptr, 0, nullptr, loss_out, st), "kl_forward reduce launch");
}

int lard_kl_backward(const lard_tensor4* qs, const lard_tensor4* ks, const float* lse_s, const lard_tensor4* qt,
                     const lard_tensor4* kt, const float* lse_t, const lard_mask* mask, int causal, float sm_scale_s,
                     float sm_scale_t, float* dq_out, float* dk_out, void* stream) {
  int rc;
  if ((rc = check_two_sided(qs, ks, lse_s, qt, kt, lse_t, mask, sm_scale_s, sm_scale_t)) != LARD_OK) return rc;
  const int64_t B = qs->size[0], Hq = qs->size[1], T = qs->size[2];
  if (B * Hq * T == 0) return ok();
  if (dq_out == nullptr || dk_out == nullptr) return fail(LARD_ERR_INVALID_ARGUMENT, "dq_out/dk_out must not be NULL");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  lard::RelArgs a{};
  fill_side(a.s, qs, ks, Hq, sm_scale_s);
  fill_side(a.t, qt, kt, Hq, sm_scale_t);
  fill_common(a, B, Hq, T, mask, causal);
  a.lse_s_in = lse_s;
  a.lse_t_in = lse_t;
  a.dq_out = dq_out;
  a.dk_out = dk_out;
  const int dps = padded_dim(qs->size[3]), dpt = padded_dim(qt->size[3]);
  if ((rc = hip_status(timed(LARD_KERNEL_ROW_GRAD, st, [&] { return lard::launch_row_dq(a, dps, dpt, st); }),
                       "kl_backward dq launch")) != LARD_OK)
    return rc;
  return hip_status(timed(LARD_KERNEL_COL_GRAD, st, [&] { return lard::launch_col_dk(a, dps, dpt, st); }),
                    "kl_backward dk launch");
}

size_t lard_attn_kl_forward_workspace_bytes(int64_t batch, int64_t heads, int64_t seq_len) {
  if (batch <= 0 || heads <= 0 || seq_len <= 0) return 0;
  size_t bytes = 0;
  fwd_layout(nullptr, batch, heads, seq_len, &bytes);
  return bytes;
}

}  // extern "C"

namespace {

// The forward of lard_attn_kl_forward.  need_workspace(B, Hq, T) returns the
// workspace to use once the shapes are checked: the caller's (checked
// against its size), or the library's scratch array (lard_attn_kl_forward_noalloc).
template <class NeedWorkspace>
int attn_kl_forward_impl(const lard_tensor4* qs, const lard_tensor4* ks, const lard_tensor4* qt,
                         const lard_tensor4* kt, const lard_mask* mask, int causal, float sm_scale_s,
                         float sm_scale_t, float* lse_s_out, float* lse_t_out, float* loss_out,
                         NeedWorkspace need_workspace, void* stream) {
  int rc;
  if ((rc = check_pair(qs, ks, "qs", "ks")) != LARD_OK) return rc;
  if ((rc = check_pair(qt, kt, "qt", "kt")) != LARD_OK) return rc;
  if (qs->size[0] != qt->size[0] || qs->size[1] != qt->size[1] || qs->size[2] != qt->size[2])
    return fail(LARD_ERR_INVALID_ARGUMENT, "student/teacher B/Hq/T must align");
  if ((qs->dtype == LARD_DTYPE_F32) != (qt->dtype == LARD_DTYPE_F32))
    return fail(LARD_ERR_UNSUPPORTED, "float32 inputs need float32 on both sides");
  if ((rc = check_mask(mask, qs->size[0], qs->size[2])) != LARD_OK) return rc;
  if ((rc = check_scale(sm_scale_s, "sm_scale_s")) != LARD_OK) return rc;
  if ((rc = check_scale(sm_scale_t, "sm_scale_t")) != LARD_OK) return rc;
  if (loss_out == nullptr) return fail(LARD_ERR_INVALID_ARGUMENT, "loss_out must not be NULL");
  const int64_t B = qs->size[0], Hq = qs->size[1], T = qs->size[2];
  const int64_t n = B * Hq * T;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (n > 0) {
    if (lse_s_out == nullptr || lse_t_out == nullptr)
      return fail(LARD_ERR_INVALID_ARGUMENT, "lse outputs must not be NULL");
    if ((rc = check_grid(B * Hq)) != LARD_OK) return rc;
    void* workspace = nullptr;
    if ((rc = need_workspace(B, Hq, T, &workspace)) != LARD_OK) return rc;
    const int ds = (int)qs->size[3], dt = (int)qt->size[3];
    const bool bf = qs->dtype == LARD_DTYPE_BF16;
    const FwdWs w = fwd_layout(workspace, B, Hq, T, nullptr);
    std::string why;
    const int path = attn_kl_path(qs, ks, qt, kt, sm_scale_s, sm_scale_t, &why);
    const bool hot = path == LARD_PATH_THROUGHPUT;
    const bool f32 = path == LARD_PATH_FLOAT32;
    if (hot || path == LARD_PATH_FUSED_FORWARD) {
      lard::HotArgs f{};
      fill_side(f.r.s, qs, ks, Hq, sm_scale_s);
      fill_side(f.r.t, qt, kt, Hq, sm_scale_t);
      fill_common(f.r, B, Hq, T, mask, causal);
      f.lse_s_out = lse_s_out;
      f.lse_t_out = lse_t_out;
      f.row_out = w.loss.rows;
      if (hot) {
        if ((rc = check_blocks(B, Hq, T)) != LARD_OK) return rc;
        f.Tp = (int)padded_len(T);
        f.tok_ok = w.tok_ok;
        f.first2 = w.first2;
        if ((rc = hip_status(lard::launch_token_prep(f.r, f.Tp, w.tok_ok, w.first2, st),
                             "attn_kl_forward token prep launch")) != LARD_OK)
          return rc;
        rc = hip_status(timed(LARD_KERNEL_FORWARD, st, [&] { return lard::launch_hot_fwd(f, padded_dim(ds), bf, st); }),
                        "attn_kl_forward launch");
      } else {
        lard::FusedArgs g{};
        g.r = f.r;
        g.lse_s_out = lse_s_out;
        g.lse_t_out = lse_t_out;
        g.row_out = f.row_out;
        rc = hip_status(timed(LARD_KERNEL_FORWARD, st, [&] { return lard::launch_fused_fwd(g, padded_dim(ds), bf, st); }),
                        "attn_kl_forward fused launch");
      }
      if (rc != LARD_OK) return rc;
    } else if (f32) {
      // float32: both LSEs and the KL in one double-precision pass
      lard::FusedArgs g{};
      fill_side(g.r.s, qs, ks, Hq, sm_scale_s);
      fill_side(g.r.t, qt, kt, Hq, sm_scale_t);
      fill_common(g.r, B, Hq, T, mask, causal);
      g.lse_s_out = lse_s_out;
      g.lse_t_out = lse_t_out;
      g.row_out = w.loss.rows;
      if ((rc = hip_status(timed(LARD_KERNEL_FORWARD, st, [&] { return lard::launch_fused_fwd_f32(g, st); }),
                           "attn_kl_forward float32 launch")) != LARD_OK)
        return rc;
    } else {
      // Stage A twice, then stage B (the reference's own composition).
      if ((rc = lard_lse_stats(qs, ks, mask, causal, sm_scale_s, lse_s_out, stream)) != LARD_OK) return rc;
      if ((rc = lard_lse_stats(qt, kt, mask, causal, sm_scale_t, lse_t_out, stream)) != LARD_OK) return rc;
      lard::RelArgs a{};
      fill_side(a.s, qs, ks, Hq, sm_scale_s);
      fill_side(a.t, qt, kt, Hq, sm_scale_t);
      fill_common(a, B, Hq, T, mask, causal);
      a.lse_s_in = lse_s_out;
      a.lse_t_in = lse_t_out;
      a.row_out = w.loss.rows;
      if ((rc = hip_status(lard::launch_row_kl(a, padded_dim(ds), padded_dim(dt), st), "attn_kl_forward kl launch")) !=
          LARD_OK)
        return rc;
    }
    return hip_status(lard::launch_reduce_sum(w.loss.rows, n, w.loss.partial, loss_out, st),
                      "attn_kl_forward reduce launch");
  }
  return hip_status(lard::launch_reduce_sum(nullptr, 0, nullptr, loss_out, st), "attn_kl_forward reduce launch");
}

// ---- the library's own forward workspace (lard_attn_kl_forward_noalloc) ----

// One array per GPU, held until the process ends.  Host code never uses its
// name as an address: each device's copy is reached through the pointer
// hipGetSymbolAddress returns with that device current.
constexpr size_t kScratchBytes = LARD_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device the work of `stream` runs on (the current device for the null stream).
int stream_device(hipStream_t stream, int* dev) {
  hipError_t e = stream != nullptr ? hipStreamGetDevice(stream, dev) : hipGetDevice(dev);
  if (e != hipSuccess) return fail(LARD_ERR_HIP, "stream device: %s", hipGetErrorString(e));
  if (*dev < 0 || *dev >= kMaxDevices) return fail(LARD_ERR_UNSUPPORTED, "device %d beyond %d", *dev, kMaxDevices);
  return LARD_OK;
}

// This device's copy of `scratch`, looked up once per device with that device current.
int scratch_on(int dev, void** out) {
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur >= 0 && cur != dev) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess) return fail(LARD_ERR_HIP, "scratch address on device %d: %s", dev, hipGetErrorString(e));
    if (p == nullptr) return fail(LARD_ERR_HIP, "scratch address on device %d is NULL", dev);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return LARD_OK;
}

}  // namespace

extern "C" {

int lard_attn_kl_forward(const lard_tensor4* qs, const lard_tensor4* ks, const lard_tensor4* qt,
                         const lard_tensor4* kt, const lard_mask* mask, int causal, float sm_scale_s,
                         float sm_scale_t, float* lse_s_out, float* lse_t_out, float* loss_out, void* workspace,
                         size_t workspace_bytes, void* stream) {
  auto caller_ws = [&](int64_t B, int64_t Hq, int64_t T, void** ws) {
    const size_t need = lard_attn_kl_forward_workspace_bytes(B, Hq, T);
    if (workspace == nullptr || workspace_bytes < need)
      return fail(LARD_ERR_INVALID_ARGUMENT, "workspace too small: need %zu bytes", need);
    *ws = workspace;
    return LARD_OK;
  };
  return attn_kl_forward_impl(qs, ks, qt, kt, mask, causal, sm_scale_s, sm_scale_t, lse_s_out, lse_t_out, loss_out,
                              caller_ws, stream);
}

int lard_attn_kl_forward_noalloc(const lard_tensor4* qs, const lard_tensor4* ks, const lard_tensor4* qt,
                                 const lard_tensor4* kt, const lard_mask* mask, int causal, float sm_scale_s,
                                 float sm_scale_t, float* lse_s_out, float* lse_t_out, float* loss_out, void* stream) {
  auto library_ws = [&](int64_t B, int64_t Hq, int64_t T, void** ws) {
    const size_t need = lard_attn_kl_forward_workspace_bytes(B, Hq, T);
    if (need > kScratchBytes)
      return fail(LARD_ERR_UNSUPPORTED, "forward needs %zu bytes of scratch; the library holds %zu per device "
                                        "(B * Hq * T is too large for the no-allocation entry point)",
                  need, kScratchBytes);
    int dev = -1, rc;
    if ((rc = stream_device(static_cast<hipStream_t>(stream), &dev)) != LARD_OK) return rc;
    return scratch_on(dev, ws);
  };
  return attn_kl_forward_impl(qs, ks, qt, kt, mask, causal, sm_scale_s, sm_scale_t, lse_s_out, lse_t_out, loss_out,
                              library_ws, stream);
}

size_t lard_attn_kl_backward_workspace_bytes(int64_t batch, int64_t heads, int64_t kv_heads, int64_t seq_len,
                                             int64_t head_dim, int self_relation) {
  if (batch <= 0 || heads <= 0 || seq_len <= 0) return 0;
  (void)kv_heads;
  (void)head_dim;
  (void)self_relation;
  size_t bytes = 0;
  bwd_layout(nullptr, batch, heads, seq_len, &bytes);
  // float32 inputs: both sides' LSEs in double (the refine pass)
  const size_t f64 = align256((size_t)(2 * batch * heads * seq_len) * sizeof(double));
  return bytes > f64 ? bytes : f64;
}

int lard_attn_kl_backward(const lard_tensor4* qs, const lard_tensor4* ks, const float* lse_s, const lard_tensor4* qt,
                          const lard_tensor4* kt, const float* lse_t, const lard_mask* mask, int causal,
                          float sm_scale_s, float sm_scale_t, const float* dloss, int self_relation, float* dq_out,
                          float* dk_out, void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = check_two_sided(qs, ks, lse_s, qt, kt, lse_t, mask, sm_scale_s, sm_scale_t)) != LARD_OK) return rc;
  const int64_t B = qs->size[0], Hq = qs->size[1], T = qs->size[2];
  if (B * Hq * T == 0) return ok();
  if (dk_out == nullptr) return fail(LARD_ERR_INVALID_ARGUMENT, "dk_out must not be NULL");
  if (self_relation) {
    if (ks->size[1] != Hq || qs->data != ks->data || qs->stride[0] != ks->stride[0] ||
        qs->stride[1] != ks->stride[1] || qs->stride[2] != ks->stride[2])
      return fail(LARD_ERR_INVALID_ARGUMENT, "self relation needs q and k to be the same tensor");
  } else if (dq_out == nullptr) {
    return fail(LARD_ERR_INVALID_ARGUMENT, "dq_out must not be NULL");
  }
  // Row side first (into dk_out for a self relation), then the column side,
  // which adds the row side in place and applies dloss once.
  float* dq_dst = self_relation ? dk_out : dq_out;
  lard::RelArgs a{};
  fill_side(a.s, qs, ks, Hq, sm_scale_s);
  fill_side(a.t, qt, kt, Hq, sm_scale_t);
  fill_common(a, B, Hq, T, mask, causal);
  a.lse_s_in = lse_s;
  a.lse_t_in = lse_t;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int ds = (int)qs->size[3], dt = (int)qt->size[3];
  std::string why;
  if (attn_kl_path(qs, ks, qt, kt, sm_scale_s, sm_scale_t, &why) == LARD_PATH_THROUGHPUT) {
    const size_t need = lard_attn_kl_backward_workspace_bytes(B, Hq, ks->size[1], T, ds, self_relation);
    if (workspace == nullptr || workspace_bytes < need)
      return fail(LARD_ERR_INVALID_ARGUMENT, "workspace too small: need %zu bytes", need);
    if ((rc = check_blocks(B, Hq, T)) != LARD_OK) return rc;
    const int Tp = (int)padded_len(T);
    const BwdWs w = bwd_layout(workspace, B, Hq, T, nullptr);
    if ((rc = hip_status(lard::launch_token_prep(a, Tp, w.tok_ok, w.first2, st),
                         "attn_kl_backward token prep launch")) != LARD_OK)
      return rc;
    if ((rc = hip_status(lard::launch_row_prep(a, Tp, w.tok_ok, w.first2, w.nl_s, w.nl_t, st),
                         "attn_kl_backward row prep launch")) != LARD_OK)
      return rc;
    lard::HotArgs f{};
    f.r = a;
    f.Tp = Tp;
    f.tok_ok = w.tok_ok;
    f.first2 = w.first2;
    f.nl_s = w.nl_s;
    f.nl_t = w.nl_t;
    f.dq_out = dq_dst;
    f.r.dscale = self_relation ? nullptr : dloss;
    const bool bf = qs->dtype == LARD_DTYPE_BF16;
    if ((rc = hip_status(timed(LARD_KERNEL_ROW_GRAD, st, [&] { return lard::launch_hot_dq(f, padded_dim(ds), bf, st); }),
                         "attn_kl_backward dq launch")) != LARD_OK)
      return rc;
    f.r.dk_out = dk_out;
    f.r.dk_add = self_relation ? dk_out : nullptr;
    f.r.dscale = dloss;
    return hip_status(timed(LARD_KERNEL_COL_GRAD, st, [&] { return lard::launch_hot_bwd(f, padded_dim(ds), bf, st); }),
                      "attn_kl_backward dk launch");
  }
  const int dps = padded_dim(ds), dpt = padded_dim(dt);
  if (qs->dtype == LARD_DTYPE_F32) {
    // float32: refine both LSEs in double first (the stored ones are float32
    // roundings, too coarse for D = P_s - P_t of a near-identical pair)
    const size_t need = lard_attn_kl_backward_workspace_bytes(B, Hq, ks->size[1], T, ds, self_relation);
    if (workspace == nullptr || workspace_bytes < need)
      return fail(LARD_ERR_INVALID_ARGUMENT, "workspace too small: need %zu bytes", need);
    if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
      return fail(LARD_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
    a.lse64_out = static_cast<double*>(workspace);
    if ((rc = hip_status(lard::launch_refine_lse_f32(a, st), "attn_kl_backward float32 lse launch")) != LARD_OK)
      return rc;
    a.lse64_out = nullptr;
    a.lse64_in = static_cast<const double*>(workspace);
  }
  a.dq_out = dq_dst;
  a.dscale = self_relation ? nullptr : dloss;
  if ((rc = hip_status(timed(LARD_KERNEL_ROW_GRAD, st, [&] { return lard::launch_row_dq(a, dps, dpt, st); }),
                       "attn_kl_backward dq launch")) != LARD_OK)
    return rc;
  a.dk_out = dk_out;
  a.dk_add = self_relation ? dk_out : nullptr;
  a.dscale = dloss;
  return hip_status(timed(LARD_KERNEL_COL_GRAD, st, [&] { return lard::launch_col_dk(a, dps, dpt, st); }),
                    "attn_kl_backward dk launch");
}

size_t lard_attn_kl_forward_rowgrad_workspace_bytes(int64_t batch, int64_t heads, int64_t kv_heads,
                                                    int64_t kv_heads_t, int64_t seq_len, int64_t head_dim) {
  if (batch <= 0 || heads <= 0 || kv_heads <= 0 || kv_heads_t <= 0 || seq_len <= 0 || head_dim <= 0) return 0;
  size_t bytes = 0;
  rowgrad_layout(nullptr, batch, heads, kv_heads, kv_heads_t, seq_len, head_dim, &bytes);
  return bytes;
}

int lard_attn_kl_forward_rowgrad(const lard_tensor4* qs, const lard_tensor4* ks, const lard_tensor4* qt,
                                 const lard_tensor4* kt, const lard_mask* mask, int causal, float sm_scale_s,
                                 float sm_scale_t, float* lse_s_out, float* lse_t_out, float* loss_out,
                                 float* dq_row_out, void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = check_pair(qs, ks, "qs", "ks")) != LARD_OK) return rc;
  if ((rc = check_pair(qt, kt, "qt", "kt")) != LARD_OK) return rc;
  if (qs->size[0] != qt->size[0] || qs->size[1] != qt->size[1] || qs->size[2] != qt->size[2])
    return fail(LARD_ERR_INVALID_ARGUMENT, "student/teacher B/Hq/T must align");
  if ((rc = check_mask(mask, qs->size[0], qs->size[2])) != LARD_OK) return rc;
  if ((rc = check_scale(sm_scale_s, "sm_scale_s")) != LARD_OK) return rc;
  if ((rc = check_scale(sm_scale_t, "sm_scale_t")) != LARD_OK) return rc;
  if (loss_out == nullptr) return fail(LARD_ERR_INVALID_ARGUMENT, "loss_out must not be NULL");
  std::string why;
  if (attn_kl_path(qs, ks, qt, kt, sm_scale_s, sm_scale_t, &why) != LARD_PATH_THROUGHPUT)
    return fail(LARD_ERR_UNSUPPORTED, "the row-gradient forward runs on the throughput kernels only (%s)",
                why.c_str());
  const int64_t B = qs->size[0], Hq = qs->size[1], T = qs->size[2];
  const int64_t n = B * Hq * T;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (n == 0)
    return hip_status(lard::launch_reduce_sum(nullptr, 0, nullptr, loss_out, st), "attn_kl_forward reduce launch");
  if (lse_s_out == nullptr || lse_t_out == nullptr || dq_row_out == nullptr)
    return fail(LARD_ERR_INVALID_ARGUMENT, "lse and dq_row outputs must not be NULL");
  if (reinterpret_cast<uintptr_t>(dq_row_out) % 16 != 0)
    return fail(LARD_ERR_INVALID_ARGUMENT, "dq_row_out must be 16-byte aligned");
  if ((rc = check_grid(B * Hq)) != LARD_OK) return rc;
  if ((rc = check_blocks(B, Hq, T)) != LARD_OK) return rc;
  const int64_t Hkv = ks->size[1], Hkv_t = kt->size[1], D = qs->size[3];
  const size_t need = lard_attn_kl_forward_rowgrad_workspace_bytes(B, Hq, Hkv, Hkv_t, T, D);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(LARD_ERR_INVALID_ARGUMENT, "workspace too small: need %zu bytes", need);
  const RowgradWs rw = rowgrad_layout(workspace, B, Hq, Hkv, Hkv_t, T, D, nullptr);
  const FwdWs& w = rw.fwd;
  lard::HotArgs f{};
  fill_side(f.r.s, qs, ks, Hq, sm_scale_s);
  fill_side(f.r.t, qt, kt, Hq, sm_scale_t);
  fill_common(f.r, B, Hq, T, mask, causal);
  f.lse_s_out = lse_s_out;
  f.lse_t_out = lse_t_out;
  f.row_out = w.loss.rows;
  f.dq_out = dq_row_out;
  f.Tp = (int)padded_len(T);
  f.tok_ok = w.tok_ok;
  f.first2 = w.first2;
  if ((rc = hip_status(lard::launch_token_prep(f.r, f.Tp, w.tok_ok, w.first2, st),
                       "attn_kl_forward_rowgrad token prep launch")) != LARD_OK)
    return rc;
  const bool bf = qs->dtype == LARD_DTYPE_BF16;
  if ((rc = hip_status(keys_f16(f, bf, rw.s, rw.t, st),
                       "attn_kl_forward_rowgrad float16 keys launch")) != LARD_OK)
    return rc;
  if ((rc = hip_status(timed(LARD_KERNEL_FORWARD_ROWGRAD, st,
                             [&] { return lard::launch_hot_fwdq(f, padded_dim(qs->size[3]), bf, st); }),
                       "attn_kl_forward_rowgrad launch")) != LARD_OK)
    return rc;
  return hip_status(lard::launch_reduce_sum(w.loss.rows, n, w.loss.partial, loss_out, st),
                    "attn_kl_forward_rowgrad reduce launch");
}

int lard_attn_kl_backward_colgrad(const lard_tensor4* qs, const lard_tensor4* ks, const float* lse_s,
                                  const lard_tensor4* qt, const lard_tensor4* kt, const float* lse_t,
                                  const lard_mask* mask, int causal, float sm_scale_s, float sm_scale_t,
                                  const float* dloss, int self_relation, float* dq_row, float* dk_out,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = check_two_sided(qs, ks, lse_s, qt, kt, lse_t, mask, sm_scale_s, sm_scale_t)) != LARD_OK) return rc;
  const int64_t B = qs->size[0], Hq = qs->size[1], T = qs->size[2];
  if (B * Hq * T == 0) return ok();
  if (dk_out == nullptr || dq_row == nullptr) return fail(LARD_ERR_INVALID_ARGUMENT, "dq_row and dk_out must not be NULL");
  if (self_relation) {
    if (ks->size[1] != Hq || qs->data != ks->data || qs->stride[0] != ks->stride[0] ||
        qs->stride[1] != ks->stride[1] || qs->stride[2] != ks->stride[2])
      return fail(LARD_ERR_INVALID_ARGUMENT, "self relation needs q and k to be the same tensor");
  }
  std::string why;
  if (attn_kl_path(qs, ks, qt, kt, sm_scale_s, sm_scale_t, &why) != LARD_PATH_THROUGHPUT)
    return fail(LARD_ERR_UNSUPPORTED, "the column-gradient backward runs on the throughput kernels only (%s)",
                why.c_str());
  const int ds = (int)qs->size[3];
  const size_t need = lard_attn_kl_backward_workspace_bytes(B, Hq, ks->size[1], T, ds, self_relation);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(LARD_ERR_INVALID_ARGUMENT, "workspace too small: need %zu bytes", need);
  if ((rc = check_blocks(B, Hq, T)) != LARD_OK) return rc;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int Tp = (int)padded_len(T);
  const BwdWs w = bwd_layout(workspace, B, Hq, T, nullptr);
  lard::HotArgs f{};
  fill_side(f.r.s, qs, ks, Hq, sm_scale_s);
  fill_side(f.r.t, qt, kt, Hq, sm_scale_t);
  fill_common(f.r, B, Hq, T, mask, causal);
  f.r.lse_s_in = lse_s;
  f.r.lse_t_in = lse_t;
  if ((rc = hip_status(lard::launch_token_prep(f.r, Tp, w.tok_ok, w.first2, st),
                       "attn_kl_backward_colgrad token prep launch")) != LARD_OK)
    return rc;
  if ((rc = hip_status(lard::launch_row_prep(f.r, Tp, w.tok_ok, w.first2, w.nl_s, w.nl_t, st),
                       "attn_kl_backward_colgrad row prep launch")) != LARD_OK)
    return rc;
  f.Tp = Tp;
  f.tok_ok = w.tok_ok;
  f.first2 = w.first2;
  f.nl_s = w.nl_s;
  f.nl_t = w.nl_t;
  f.r.dk_out = dk_out;
  f.r.dk_add = self_relation ? dq_row : nullptr;
  f.r.dscale = dloss;
  const bool bf = qs->dtype == LARD_DTYPE_BF16;
  if ((rc = hip_status(timed(LARD_KERNEL_COL_GRAD, st, [&] { return lard::launch_hot_bwd(f, padded_dim(ds), bf, st); }),
                       "attn_kl_backward_colgrad dk launch")) != LARD_OK)
    return rc;
  if (self_relation) return ok();
  return hip_status(lard::launch_scale_inplace(dq_row, B * Hq * T * qs->size[3], dloss, st),
                    "attn_kl_backward_colgrad dq scale launch");
}

size_t lard_attn_kl_batched_workspace_bytes(const lard_relation* rels, int nrel) {
  if (rels == nullptr || nrel < 1) return 0;
  size_t bytes = 0;
  batch_layout(nullptr, rels, nrel, &bytes);
  return bytes;
}

}  // extern "C"

namespace {

// The batched workspace, then per relation both sides' float16 keys.
struct BatchRowgradWs {
  BatchWs batch;
  std::vector<KeysF16> s, t;
};

BatchRowgradWs batch_rowgrad_layout(void* base, const lard_relation* rels, int nrel, size_t* bytes) {
  size_t batch_bytes = 0;
  BatchRowgradWs w;
  w.batch = batch_layout(base, rels, nrel, &batch_bytes);
  Carver c(base != nullptr ? static_cast<char*>(base) + batch_bytes : nullptr);
  for (int r = 0; r < nrel; ++r) {
    const lard_tensor4& x = rels[r].xs;
    w.s.push_back(take_keys(c, x.size[0], x.size[1], x.size[2], x.size[3]));
    w.t.push_back(take_keys(c, x.size[0], x.size[1], x.size[2], x.size[3]));
  }
  if (bytes != nullptr) *bytes = batch_bytes + c.bytes();
  return w;
}

}  // namespace

extern "C" {

size_t lard_attn_kl_batched_rowgrad_workspace_bytes(const lard_relation* rels, int nrel) {
  if (rels == nullptr || nrel < 1) return 0;
  size_t bytes = 0;
  batch_rowgrad_layout(nullptr, rels, nrel, &bytes);
  return bytes;
}

int lard_attn_kl_batched_forward(const lard_relation* rels, int nrel, const lard_mask* mask, int causal,
                                 float sm_scale_s, float sm_scale_t, const float* weights, float* loss_out,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = check_batch(rels, nrel, mask, sm_scale_s, sm_scale_t)) != LARD_OK) return rc;
  if (loss_out == nullptr) return fail(LARD_ERR_INVALID_ARGUMENT, "loss_out must not be NULL");
  int64_t rows = 0;
  for (int r = 0; r < nrel; ++r) {
    if (rel_rows(rels[r]) > 0 && (rels[r].lse_s == nullptr || rels[r].lse_t == nullptr))
      return fail(LARD_ERR_INVALID_ARGUMENT, "relation %d: lse outputs must not be NULL", r);
    rows += rel_rows(rels[r]);
  }
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (rows == 0)
    return hip_status(lard::launch_reduce_sum(nullptr, 0, nullptr, loss_out, st), "batched forward reduce launch");
  const size_t need = lard_attn_kl_batched_workspace_bytes(rels, nrel);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(LARD_ERR_INVALID_ARGUMENT, "workspace too small: need %zu bytes", need);
  const BatchWs w = batch_layout(workspace, rels, nrel, nullptr);
  const int Tp = (int)padded_len(rels[0].xs.size[2]);
  const int dp = padded_dim(rels[0].xs.size[3]);
  const bool bf = rels[0].xs.dtype == LARD_DTYPE_BF16;
  {
    const lard::HotArgs f0 = relation_args(rels[0], mask, causal, sm_scale_s, sm_scale_t, Tp, w.tok_ok, w.first2);
    if ((rc = hip_status(lard::launch_token_prep(f0.r, Tp, w.tok_ok, w.first2, st),
                         "batched forward token prep launch")) !=
        LARD_OK)
      return rc;
  }
  int64_t row_off = 0;
  for (int g = 0; g < nrel; g += lard::kMaxRelations) {
    lard::HotBatch m{};
    for (int r = g; r < nrel && r < g + lard::kMaxRelations; ++r) {
      if (rel_rows(rels[r]) == 0) continue;
      lard::HotArgs f = relation_args(rels[r], mask, causal, sm_scale_s, sm_scale_t, Tp, w.tok_ok, w.first2);
      f.lse_s_out = rels[r].lse_s;
      f.lse_t_out = rels[r].lse_t;
      f.row_out = w.loss.rows + row_off;
      f.r.weight = weights != nullptr ? weights + r : nullptr;
      row_off += rel_rows(rels[r]);
      m.rel[m.n++] = f;
    }
    if (m.n == 0) continue;
    if ((rc = hip_status(timed(LARD_KERNEL_FORWARD, st, [&] { return lard::launch_hot_fwd_batch(m, dp, bf, st); }),
                         "batched forward launch")) != LARD_OK)
      return rc;
  }
  return hip_status(lard::launch_reduce_sum(w.loss.rows, rows, w.loss.partial, loss_out, st),
                    "batched forward reduce launch");
}

int lard_attn_kl_batched_backward(const lard_relation* rels, int nrel, const lard_mask* mask, int causal,
                                  float sm_scale_s, float sm_scale_t, const float* weights, const float* dloss,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = check_batch(rels, nrel, mask, sm_scale_s, sm_scale_t)) != LARD_OK) return rc;
  int64_t rows = 0;
  for (int r = 0; r < nrel; ++r) {
    if (rel_rows(rels[r]) > 0 && (rels[r].lse_s == nullptr || rels[r].lse_t == nullptr || rels[r].dxs == nullptr))
      return fail(LARD_ERR_INVALID_ARGUMENT, "relation %d: lse inputs and dxs must not be NULL", r);
    rows += rel_rows(rels[r]);
  }
  if (rows == 0) return ok();
  const size_t need = lard_attn_kl_batched_workspace_bytes(rels, nrel);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(LARD_ERR_INVALID_ARGUMENT, "workspace too small: need %zu bytes", need);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const BatchWs w = batch_layout(workspace, rels, nrel, nullptr);
  const int Tp = (int)padded_len(rels[0].xs.size[2]);
  const int dp = padded_dim(rels[0].xs.size[3]);
  const bool bf = rels[0].xs.dtype == LARD_DTYPE_BF16;
  std::vector<lard::HotArgs> fs((size_t)nrel);
  int64_t nl_off = 0;
  for (int r = 0; r < nrel; ++r) {
    lard::HotArgs& f = fs[(size_t)r];
    f = relation_args(rels[r], mask, causal, sm_scale_s, sm_scale_t, Tp, w.tok_ok, w.first2);
    f.r.lse_s_in = rels[r].lse_s;
    f.r.lse_t_in = rels[r].lse_t;
    float* nl_s = w.nl_s + nl_off;
    float* nl_t = w.nl_t + nl_off;
    f.nl_s = nl_s;
    f.nl_t = nl_t;
    nl_off += rels[r].xs.size[0] * rels[r].xs.size[1] * (int64_t)Tp;
    if (r == 0 && (rc = hip_status(lard::launch_token_prep(f.r, Tp, w.tok_ok, w.first2, st),
                                   "batched backward token prep launch")) != LARD_OK)
      return rc;
    if (rel_rows(rels[r]) > 0 &&
        (rc = hip_status(lard::launch_row_prep(f.r, Tp, w.tok_ok, w.first2, nl_s, nl_t, st),
                                                  "batched backward row prep launch")) != LARD_OK)
      return rc;
  }
  for (int g = 0; g < nrel; g += lard::kMaxRelations) {
    // row side first (into dxs), then the column side, which adds it in place
    // and applies dloss * weight once
    lard::HotBatch mq{}, mk{};
    for (int r = g; r < nrel && r < g + lard::kMaxRelations; ++r) {
      if (rel_rows(rels[r]) == 0) continue;
      lard::HotArgs f = fs[(size_t)r];
      f.dq_out = rels[r].dxs;
      mq.rel[mq.n++] = f;
      f.r.dk_out = rels[r].dxs;
      f.r.dk_add = rels[r].dxs;
      f.r.dscale = dloss;
      f.r.weight = weights != nullptr ? weights + r : nullptr;
      mk.rel[mk.n++] = f;
    }
    if (mq.n == 0) continue;
    if ((rc = hip_status(timed(LARD_KERNEL_ROW_GRAD, st, [&] { return lard::launch_hot_dq_batch(mq, dp, bf, st); }),
                         "batched backward dq launch")) != LARD_OK)
      return rc;
    if ((rc = hip_status(timed(LARD_KERNEL_COL_GRAD, st, [&] { return lard::launch_hot_bwd_batch(mk, dp, bf, st); }),
                         "batched backward dk launch")) != LARD_OK)
      return rc;
  }
  return ok();
}

int lard_attn_kl_batched_forward_rowgrad(const lard_relation* rels, int nrel, const lard_mask* mask, int causal,
                                         float sm_scale_s, float sm_scale_t, const float* weights, float* loss_out,
                                         void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = check_batch(rels, nrel, mask, sm_scale_s, sm_scale_t)) != LARD_OK) return rc;
  if (loss_out == nullptr) return fail(LARD_ERR_INVALID_ARGUMENT, "loss_out must not be NULL");
  int64_t rows = 0;
  for (int r = 0; r < nrel; ++r) {
    if (rel_rows(rels[r]) > 0 && (rels[r].lse_s == nullptr || rels[r].lse_t == nullptr || rels[r].dxs == nullptr))
      return fail(LARD_ERR_INVALID_ARGUMENT, "relation %d: lse outputs and dxs must not be NULL", r);
    if (rels[r].dxs != nullptr && reinterpret_cast<uintptr_t>(rels[r].dxs) % 16 != 0)
      return fail(LARD_ERR_INVALID_ARGUMENT, "relation %d: dxs must be 16-byte aligned", r);
    rows += rel_rows(rels[r]);
  }
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (rows == 0)
    return hip_status(lard::launch_reduce_sum(nullptr, 0, nullptr, loss_out, st), "batched forward reduce launch");
  const size_t need = lard_attn_kl_batched_rowgrad_workspace_bytes(rels, nrel);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(LARD_ERR_INVALID_ARGUMENT, "workspace too small: need %zu bytes", need);
  const BatchRowgradWs rw = batch_rowgrad_layout(workspace, rels, nrel, nullptr);
  const BatchWs& w = rw.batch;
  const int Tp = (int)padded_len(rels[0].xs.size[2]);
  const int dp = padded_dim(rels[0].xs.size[3]);
  const bool bf = rels[0].xs.dtype == LARD_DTYPE_BF16;
  {
    const lard::HotArgs f0 = relation_args(rels[0], mask, causal, sm_scale_s, sm_scale_t, Tp, w.tok_ok, w.first2);
    if ((rc = hip_status(lard::launch_token_prep(f0.r, Tp, w.tok_ok, w.first2, st),
                         "batched forward_rowgrad token prep launch")) != LARD_OK)
      return rc;
  }
  int64_t row_off = 0;
  for (int g = 0; g < nrel; g += lard::kMaxRelations) {
    lard::HotBatch m{};
    for (int r = g; r < nrel && r < g + lard::kMaxRelations; ++r) {
      if (rel_rows(rels[r]) == 0) continue;
      lard::HotArgs f = relation_args(rels[r], mask, causal, sm_scale_s, sm_scale_t, Tp, w.tok_ok, w.first2);
      f.lse_s_out = rels[r].lse_s;
      f.lse_t_out = rels[r].lse_t;
      f.row_out = w.loss.rows + row_off;
      f.dq_out = rels[r].dxs;
      f.r.weight = weights != nullptr ? weights + r : nullptr;
      if ((rc = hip_status(keys_f16(f, bf, rw.s[(size_t)r], rw.t[(size_t)r], st),
                           "batched forward_rowgrad float16 keys launch")) != LARD_OK)
        return rc;
      row_off += rel_rows(rels[r]);
      m.rel[m.n++] = f;
    }
    if (m.n == 0) continue;
    if ((rc = hip_status(timed(LARD_KERNEL_FORWARD_ROWGRAD, st,
                               [&] { return lard::launch_hot_fwdq_batch(m, dp, bf, st); }),
                         "batched forward_rowgrad launch")) != LARD_OK)
      return rc;
  }
  return hip_status(lard::launch_reduce_sum(w.loss.rows, rows, w.loss.partial, loss_out, st),
                    "batched forward_rowgrad reduce launch");
}

int lard_attn_kl_batched_backward_colgrad(const lard_relation* rels, int nrel, const lard_mask* mask, int causal,
                                          float sm_scale_s, float sm_scale_t, const float* weights,
                                          const float* dloss, void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = check_batch(rels, nrel, mask, sm_scale_s, sm_scale_t)) != LARD_OK) return rc;
  int64_t rows = 0;
  for (int r = 0; r < nrel; ++r) {
    if (rel_rows(rels[r]) > 0 && (rels[r].lse_s == nullptr || rels[r].lse_t == nullptr || rels[r].dxs == nullptr))
      return fail(LARD_ERR_INVALID_ARGUMENT, "relation %d: lse inputs and dxs must not be NULL", r);
    rows += rel_rows(rels[r]);
  }
  if (rows == 0) return ok();
  const size_t need = lard_attn_kl_batched_workspace_bytes(rels, nrel);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(LARD_ERR_INVALID_ARGUMENT, "workspace too small: need %zu bytes", need);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const BatchWs w = batch_layout(workspace, rels, nrel, nullptr);
  const int Tp = (int)padded_len(rels[0].xs.size[2]);
  const int dp = padded_dim(rels[0].xs.size[3]);
  const bool bf = rels[0].xs.dtype == LARD_DTYPE_BF16;
  std::vector<lard::HotArgs> fs((size_t)nrel);
  int64_t nl_off = 0;
  for (int r = 0; r < nrel; ++r) {
    lard::HotArgs& f = fs[(size_t)r];
    f = relation_args(rels[r], mask, causal, sm_scale_s, sm_scale_t, Tp, w.tok_ok, w.first2);
    f.r.lse_s_in = rels[r].lse_s;
    f.r.lse_t_in = rels[r].lse_t;
    float* nl_s = w.nl_s + nl_off;
    float* nl_t = w.nl_t + nl_off;
    f.nl_s = nl_s;
    f.nl_t = nl_t;
    nl_off += rels[r].xs.size[0] * rels[r].xs.size[1] * (int64_t)Tp;
    if (r == 0 && (rc = hip_status(lard::launch_token_prep(f.r, Tp, w.tok_ok, w.first2, st),
                                   "batched backward_colgrad token prep launch")) != LARD_OK)
      return rc;
    if (rel_rows(rels[r]) > 0 &&
        (rc = hip_status(lard::launch_row_prep(f.r, Tp, w.tok_ok, w.first2, nl_s, nl_t, st),
                         "batched backward_colgrad row prep launch")) != LARD_OK)
      return rc;
  }
  for (int g = 0; g < nrel; g += lard::kMaxRelations) {
    // the column side adds itself to the row side in place and applies
    // dloss * weight once
    lard::HotBatch mk{};
    for (int r = g; r < nrel && r < g + lard::kMaxRelations; ++r) {
      if (rel_rows(rels[r]) == 0) continue;
      lard::HotArgs f = fs[(size_t)r];
      f.r.dk_out = rels[r].dxs;
      f.r.dk_add = rels[r].dxs;
      f.r.dscale = dloss;
      f.r.weight = weights != nullptr ? weights + r : nullptr;
      mk.rel[mk.n++] = f;
    }
    if (mk.n == 0) continue;
    if ((rc = hip_status(timed(LARD_KERNEL_COL_GRAD, st, [&] { return lard::launch_hot_bwd_batch(mk, dp, bf, st); }),
                         "batched backward_colgrad dk launch")) != LARD_OK)
      return rc;
  }
  return ok();
}

int lard_rope_pair(const lard_tensor4* x, const float* inv_freq_t, const float* inv_freq_s, float att_t, float att_s,
                   const int64_t* position_ids, int64_t pos_stride_b, void* out_t, void* out_s, void* stream) {
  int rc;
  if ((rc = check_tensor(x, "x")) != LARD_OK) return rc;
  if (x->dtype == LARD_DTYPE_F32) return fail(LARD_ERR_UNSUPPORTED, "rope_pair supports only fp16/bf16");
  const int64_t B = x->size[0], H = x->size[1], T = x->size[2], D = x->size[3];
  if (D % 16 != 0) return fail(LARD_ERR_UNSUPPORTED, "rope_pair needs D to be a multiple of 16");
  if (B * H * T == 0) return ok();
  if (inv_freq_t == nullptr || inv_freq_s == nullptr || out_t == nullptr || out_s == nullptr)
    return fail(LARD_ERR_INVALID_ARGUMENT, "inv_freq and outputs must not be NULL");
  if (B * T * (D / 16) > (int64_t)INT32_MAX * 256)
    return fail(LARD_ERR_UNSUPPORTED, "rope_pair grid too large");
  if (!std::isfinite(att_t) || !std::isfinite(att_s))
    return fail(LARD_ERR_INVALID_ARGUMENT, "att_t / att_s must be finite");
  lard::RopeArgs a{};
  a.x = static_cast<const lard::u16*>(x->data);
  a.sb = x->stride[0];
  a.sh = x->stride[1];
  a.st = x->stride[2];
  a.B = (int)B;
  a.H = (int)H;
  a.T = (int)T;
  a.D = (int)D;
  a.inv_freq_t = inv_freq_t;
  a.inv_freq_s = inv_freq_s;
  a.att_t = att_t;
  a.att_s = att_s;
  a.pos = position_ids;
  a.pos_sb = pos_stride_b;
  a.out_t = static_cast<lard::u16*>(out_t);
  a.out_s = static_cast<lard::u16*>(out_s);
  return hip_status(lard::launch_rope_pair(a, x->dtype == LARD_DTYPE_BF16, static_cast<hipStream_t>(stream)),
                    "rope_pair launch");
}

size_t lard_logits_kl_workspace_bytes(int64_t rows, int64_t vocab) {
  if (rows <= 0 || vocab <= 0) return 0;
  return (size_t)rows * lard::logits_split(rows, vocab).splits * lard::kLogitsPartFloats * sizeof(float);
}

int lard_logits_kl_forward(const lard_logits* t_logits, const lard_logits* s_logits, float temperature,
                           float* lse_t, float* lse_s, float* kl_rows, float* loss, void* workspace,
                           size_t workspace_bytes, void* stream) {
  int rc;
  lard::LogitsArgs a;
  if ((rc = logits_common(t_logits, s_logits, temperature, &a)) != LARD_OK) return rc;
  if (loss == nullptr) return fail(LARD_ERR_INVALID_ARGUMENT, "loss must not be NULL");
  if (a.rows > 0 && (lse_t == nullptr || lse_s == nullptr || kl_rows == nullptr))
    return fail(LARD_ERR_INVALID_ARGUMENT, "lse_t / lse_s / kl_rows must not be NULL");
  const size_t need = lard_logits_kl_workspace_bytes(a.rows, a.V);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(LARD_ERR_INVALID_ARGUMENT, "workspace too small: need %zu bytes", need);
  if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
    return fail(LARD_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  a.part = static_cast<float*>(workspace);
  a.lse_t = lse_t;
  a.lse_s = lse_s;
  a.kl = kl_rows;
  a.loss = loss;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (a.rows > 0 && a.V > 0) {
    if ((rc = hip_status(timed(LARD_KERNEL_LOGITS_FORWARD, st,
                               [&] { return lard::launch_logits_kl_forward(a, t_logits->dtype, st); }),
                         "logits_kl forward launch")) != LARD_OK)
      return rc;
  }
  return hip_status(lard::launch_logits_kl_finish(a, st), "logits_kl finish launch");
}

int lard_logits_kl_backward(const lard_logits* t_logits, const lard_logits* s_logits, float temperature,
                            const float* lse_t, const float* lse_s, const float* kl_rows, const float* dloss,
                            int dloss_per_row, float row_scale, const lard_logits* grad_t,
                            const lard_logits* grad_s, void* stream) {
  int rc;
  lard::LogitsArgs a;
  if ((rc = logits_common(t_logits, s_logits, temperature, &a)) != LARD_OK) return rc;
  if (grad_t != nullptr && (rc = check_logits_like(grad_t, t_logits, "grad_t")) != LARD_OK) return rc;
  if (grad_s != nullptr && (rc = check_logits_like(grad_s, t_logits, "grad_s")) != LARD_OK) return rc;
  if (!std::isfinite(row_scale)) return fail(LARD_ERR_INVALID_ARGUMENT, "row_scale must be finite");
  if (a.rows == 0 || a.V == 0 || (grad_t == nullptr && grad_s == nullptr)) return ok();
  if (lse_t == nullptr || lse_s == nullptr || dloss == nullptr)
    return fail(LARD_ERR_INVALID_ARGUMENT, "lse_t / lse_s / dloss must not be NULL");
  if (grad_t != nullptr && kl_rows == nullptr)
    return fail(LARD_ERR_INVALID_ARGUMENT, "kl_rows must not be NULL when grad_t is requested");
  a.lse_t = const_cast<float*>(lse_t);
  a.lse_s = const_cast<float*>(lse_s);
  a.kl = const_cast<float*>(kl_rows);
  a.dloss = dloss;
  a.dloss_per_row = dloss_per_row != 0;
  a.row_scale = row_scale;
  if (grad_t != nullptr) {
    a.gt = const_cast<void*>(grad_t->data);
    a.gt_sb = grad_t->stride[0];
    a.gt_sk = grad_t->stride[1];
  }
  if (grad_s != nullptr) {
    a.gs = const_cast<void*>(grad_s->data);
    a.gs_sb = grad_s->stride[0];
    a.gs_sk = grad_s->stride[1];
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  return hip_status(timed(LARD_KERNEL_LOGITS_GRAD, st, [&] { return lard::launch_logits_kl_grad(a, t_logits->dtype, st); }),
                    "logits_kl backward launch");
}

}  // extern "C"
