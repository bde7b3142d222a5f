// Logits KL over the kept positions (logits_kl.hip): arguments and launchers.
#pragma once

#include "lard_device.h"

namespace lard {

// Element types of the logits (the model dtype).
enum LogitsDtype { kLogitsF16 = 0, kLogitsBF16 = 1, kLogitsF32 = 2 };

// Vocabulary split: a row of V logits is cut into `splits` chunks of
// `chunk` elements (a multiple of 8), one workgroup each.
struct LogitsSplit {
  int splits;
  int64_t chunk;
};

// Splits chosen so the grid has about 2048 workgroups (8 per CU) and every
// chunk holds at least 8192 logits (4 groups of 8 per thread).
inline LogitsSplit logits_split(int64_t rows, int64_t V) {
  int64_t by_blocks = rows > 0 ? (2048 + rows - 1) / rows : 1;
  int64_t by_size = V / 8192;
  int64_t s = by_blocks < by_size ? by_blocks : by_size;
  if (s < 1) s = 1;
  if (s > 64) s = 64;
  int64_t chunk = (V + s - 1) / s;
  chunk = (chunk + 7) / 8 * 8;
  if (chunk < 8) chunk = 8;
  s = (V + chunk - 1) / chunk;
  if (s < 1) s = 1;
  return {(int)s, chunk};
}

constexpr int kLogitsPartFloats = 8;  // per (row, split): max_t, z_t, a, max_s, z_s, pad

struct LogitsArgs {
  const void* t;            // teacher logits [B, K, V] (element strides below, V stride 1)
  const void* s;            // student logits, same shape and dtype
  int64_t t_sb, t_sk, s_sb, s_sk;
  void* gt;                 // teacher gradient (same layout rules), or null
  void* gs;                 // student gradient, or null
  int64_t gt_sb, gt_sk, gs_sb, gs_sk;
  int K;                    // kept positions per batch entry; row r = (r / K, r % K)
  int rows;                 // B * K
  int64_t V;
  int splits;
  int64_t chunk;
  float inv_temp;           // 1 / T as a float32 quotient (logits * (1/T))
  float* part;              // workspace [rows][splits][kLogitsPartFloats]
  float* lse_t;             // [rows] log-sum-exp of the scaled logits
  float* lse_s;
  float* kl;                // [rows] KL(p_t || p_s) per kept position
  float* loss;              // mean over rows
  const float* dloss;       // backward: upstream gradient, one value or one per row
  int dloss_per_row;
  float row_scale;          // 1 / rows for the mean, 1 per row otherwise
};

hipError_t launch_logits_kl_forward(const LogitsArgs& a, int dtype, hipStream_t stream);
hipError_t launch_logits_kl_finish(const LogitsArgs& a, hipStream_t stream);
hipError_t launch_logits_kl_grad(const LogitsArgs& a, int dtype, hipStream_t stream);

}  // namespace lard
