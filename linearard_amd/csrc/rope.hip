// RoPE teacher/student pair producer: the step before the attention KL.
//
// The reference's relations are taken after each model's rotary embedding:
// the teacher with its native RoPE, the student with a scaled one (linear
// scaling, factor 4 or 8, scripts/train_linearard_*.sh:9), both in HF LLaMA's
// rotate_half layout.  From one pre-RoPE tensor x [B, H, T, D] this kernel
// writes both rotated tensors, contiguous [B, H, T, D], with HF's arithmetic:
//
//   angle = pos * inv_freq[i]                  (float32, one rounding)
//   c, s  = cos(angle) * att, sin(angle) * att rounded to the input dtype
//           (att: HF's attention_scaling of the rope type, a float32 product;
//           1 for default / linear / dynamic / llama3, which changes nothing)
//   out[i]       = R(R(x[i] * c) + R(-x[i + D/2] * s))       i < D/2
//   out[i + D/2] = R(R(x[i + D/2] * c) + R(x[i] * s))
//
// with R the rounding to the input dtype after every operation (the bf16
// tensor arithmetic of q * cos + rotate_half(q) * sin).  One thread owns one
// token and 8 frequency pairs and loops over the heads, so every cos / sin
// is evaluated once per token and shared by all heads; the kernel is then
// bound by HBM (read x once, write two tensors).

#include "rope_kernels.h"

namespace lard {

template <bool BF>
__device__ __forceinline__ float bits_to_float(u16 v) {
  if constexpr (BF)
    return __builtin_bit_cast(float, (unsigned)v << 16);
  else
    return (float)__builtin_bit_cast(_Float16, v);
}

template <bool BF>
__device__ __forceinline__ float round_to_input(float x) {  // value after a cast to the input dtype
  return bits_to_float<BF>(to_bits(x, BF));
}

// A rounded product kept as its own value: the empty asm stops the compiler
// from narrowing the fp16 arithmetic and fusing the product into the next
// add (an fp16 fma rounds once where the tensor arithmetic rounds twice).
template <bool BF>
__device__ __forceinline__ float rounded_product(float x, float y) {
  float p = round_to_input<BF>(x * y);
  asm volatile("" : "+v"(p));
  return p;
}

template <bool BF>
__global__ __launch_bounds__(256) void rope_pair_kernel(const RopeArgs a) {
  const int chunks = a.D / 16;  // 8 frequency pairs per thread
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (int64_t)a.B * a.T * chunks) return;
  const int c = (int)(gid % chunks);
  const int64_t bt = gid / chunks;
  const int t = (int)(bt % a.T);
  const int b = (int)(bt / a.T);
  const float p = a.pos != nullptr ? (float)a.pos[(int64_t)b * a.pos_sb + t] : (float)t;
  float ct[8], sn_t[8], cs[8], sn_s[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float at = p * a.inv_freq_t[8 * c + e];
    const float as = p * a.inv_freq_s[8 * c + e];
    ct[e] = round_to_input<BF>(cosf(at) * a.att_t);
    sn_t[e] = round_to_input<BF>(sinf(at) * a.att_t);
    cs[e] = round_to_input<BF>(cosf(as) * a.att_s);
    sn_s[e] = round_to_input<BF>(sinf(as) * a.att_s);
  }
  const int half = a.D / 2;
  const u16* xb = a.x + (int64_t)b * a.sb + (int64_t)t * a.st + 8 * c;
  const int64_t ob = (((int64_t)b * a.H) * a.T + t) * a.D + 8 * c;  // head 0, this token and chunk
  const int64_t oh = (int64_t)a.T * a.D;                            // output head stride
#pragma unroll 4
  for (int h = 0; h < a.H; ++h) {
    const u16x8 v1 = *reinterpret_cast<const u16x8*>(xb + (int64_t)h * a.sh);
    const u16x8 v2 = *reinterpret_cast<const u16x8*>(xb + (int64_t)h * a.sh + half);
    u16x8 t1, t2, s1, s2;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x1 = bits_to_float<BF>(v1[e]), x2 = bits_to_float<BF>(v2[e]);
      t1[e] = to_bits(rounded_product<BF>(x1, ct[e]) + rounded_product<BF>(-x2, sn_t[e]), BF);
      t2[e] = to_bits(rounded_product<BF>(x2, ct[e]) + rounded_product<BF>(x1, sn_t[e]), BF);
      s1[e] = to_bits(rounded_product<BF>(x1, cs[e]) + rounded_product<BF>(-x2, sn_s[e]), BF);
      s2[e] = to_bits(rounded_product<BF>(x2, cs[e]) + rounded_product<BF>(x1, sn_s[e]), BF);
    }
    // Streaming stores: the two outputs (twice the input) exceed the 256 MB
    // last-level cache at long contexts; write-allocated lines would be
    // written back during the next launch (measured 188 us vs 145 us per
    // back-to-back launch at B=1, H=32, n=32768, d=128).
    const int64_t o = ob + h * oh;
    __builtin_nontemporal_store(t1, reinterpret_cast<u16x8*>(a.out_t + o));
    __builtin_nontemporal_store(t2, reinterpret_cast<u16x8*>(a.out_t + o + half));
    __builtin_nontemporal_store(s1, reinterpret_cast<u16x8*>(a.out_s + o));
    __builtin_nontemporal_store(s2, reinterpret_cast<u16x8*>(a.out_s + o + half));
  }
}

hipError_t launch_rope_pair(const RopeArgs& a, bool bf16, hipStream_t stream) {
  const int64_t threads = (int64_t)a.B * a.T * (a.D / 16);
  const dim3 grid((unsigned)((threads + 255) / 256)), block(256);
  if (bf16)
    hipLaunchKernelGGL(rope_pair_kernel<true>, grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL(rope_pair_kernel<false>, grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace lard
