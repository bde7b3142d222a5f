// float32-input stage kernels (stage_f32.hip): launchers.  The bf16/fp16
// stage launchers forward to these when a RelArgs side is float32.
#pragma once

#include "lard_device.h"

namespace lard {

hipError_t launch_row_lse_f32(const RelArgs& a, hipStream_t stream);
hipError_t launch_row_kl_f32(const RelArgs& a, hipStream_t stream);
hipError_t launch_row_dq_f32(const RelArgs& a, hipStream_t stream);
// both LSEs in double into a.lse64_out (the autograd backward's first pass)
hipError_t launch_refine_lse_f32(const RelArgs& a, hipStream_t stream);
// lse_s, lse_t and the per-row KL in one pass (the autograd forward)
hipError_t launch_fused_fwd_f32(const FusedArgs& f, hipStream_t stream);
hipError_t launch_col_dk_f32(const RelArgs& a, hipStream_t stream);

}  // namespace lard
