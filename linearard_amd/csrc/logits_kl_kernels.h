// Logits KL over the kept positions (logits_kl.hip): arguments and launchers.
#pragma once

#include "lard_device.h"

namespace lard {

// Element types of the logits (the model dtype).
enum LogitsDtype { kLogitsF16 = 0, kLogitsBF16 = 1, kLogitsF32 = 2 };

// Vocabulary split: a row of V logits is cut into `splits` chunks of
// `chunk` elements, one workgroup each.  Chunks are whole multiples of
// kLogitsUnit logits (two of the kernels' load steps of 4096 logits).
constexpr int64_t kLogitsUnit = 8192;
#ifndef LARD_LOGITS_TARGET_BLOCKS
#define LARD_LOGITS_TARGET_BLOCKS 2048
#endif

struct LogitsSplit {
  int splits;
  int64_t chunk;
};

// Splits chosen so the grid has about LARD_LOGITS_TARGET_BLOCKS workgroups
// (at most one per unit, at most 64 per row).
inline LogitsSplit logits_split(int64_t rows, int64_t V) {
  const int64_t units = V > 0 ? (V + kLogitsUnit - 1) / kLogitsUnit : 1;
  int64_t s = rows > 0 ? (LARD_LOGITS_TARGET_BLOCKS + rows - 1) / rows : 1;
  if (s > units) s = units;
  if (s > 64) s = 64;
  if (s < 1) s = 1;
  const int64_t chunk = (units + s - 1) / s * kLogitsUnit;
  s = V > 0 ? (V + chunk - 1) / chunk : 1;
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
