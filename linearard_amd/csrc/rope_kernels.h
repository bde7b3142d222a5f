// RoPE teacher/student pair producer (rope.hip): arguments and launcher.
#pragma once

#include "lard_device.h"

namespace lard {

struct RopeArgs {
  const u16* x;             // pre-RoPE [B, H, T, D]
  int64_t sb, sh, st;       // element strides (D stride 1)
  int B, H, T, D;
  const float* inv_freq_t;  // [D/2] teacher
  const float* inv_freq_s;  // [D/2] student
  float att_t, att_s;       // cos / sin multipliers (HF's attention_scaling; 1 for most rope types)
  const int64_t* pos;       // [B, T] position ids, or null for 0..T-1
  int64_t pos_sb;
  u16* out_t;               // [B, H, T, D] contiguous
  u16* out_s;
};

hipError_t launch_rope_pair(const RopeArgs& a, bool bf16, hipStream_t stream);

}  // namespace lard
