/*
 * linearard_amd.h -- C ABI of the MI355X (gfx950) attention-relation KL library.
 *
 * This is the drop-in boundary for LinearARD's linear-memory attention KL
 * (reference: kernels/attention_KL/).  Each entry point replaces one
 * reference interface; the citation is on the declaration.  The library is
 * `linearard_amd/liblinearard_amd.so`.
 *
 * Conventions
 *   - Every tensor argument is a device pointer the caller owns.  The
 *     library never allocates or frees device memory; scratch space is
 *     passed in by the caller, sized by the matching *_workspace_bytes().
 *   - q/k tensors are [B, H, T, D] with element strides; stride[3] must be 1,
 *     the data pointer 16-byte aligned and strides[0..2] multiples of 8
 *     elements (4 for float32; every contiguous tensor with D in
 *     {8,16,32,64,128,256} qualifies).
 *   - Outputs (lse, dq, dk, dx) are contiguous float32 of the stated shape.
 *   - GQA: kv head of query head h is h / (Hq / Hkv)   (kernel_A.py:77).
 *   - All work is enqueued on `stream` (a hipStream_t) and is asynchronous;
 *     no entry point synchronises the host.  Calls are reentrant; the only
 *     library state is the thread-local error string.
 *   - Return value: LARD_OK (0) or a negative LARD_ERR_* code; the message
 *     is available from lard_last_error() on the calling thread.
 */
#ifndef LINEARARD_AMD_H
#define LINEARARD_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LARD_OK 0
#define LARD_ERR_INVALID_ARGUMENT (-1)
#define LARD_ERR_UNSUPPORTED (-2)
#define LARD_ERR_HIP (-3)

/* element type of q / k (kernel_A.py:195-196 accepts fp16 and bf16 only) */
#define LARD_DTYPE_F16 0
#define LARD_DTYPE_BF16 1
/* float32 (an extension): q / k of the stage and single-relation entry points
 * (float32 products, D not rounded; both sides float32, strides multiples of
 * 4 elements), and logits (lard_logits_kl_*).  The batched relation entry
 * points and lard_rope_pair take fp16/bf16 only. */
#define LARD_DTYPE_F32 2

/* attention-mask element type, [B, T], nonzero = valid token (kernel_A.py:218) */
#define LARD_MASK_NONE 0
#define LARD_MASK_U8 1 /* torch.bool or torch.uint8 */
#define LARD_MASK_I32 2
#define LARD_MASK_I64 3

typedef struct lard_tensor4 {
  const void* data;  /* device pointer */
  int64_t size[4];   /* B, H, T, D */
  int64_t stride[4]; /* element strides, stride[3] == 1 */
  int32_t dtype;     /* LARD_DTYPE_* */
} lard_tensor4;

/* [B, K, V] logits of the K kept positions (logits_to_keep, train.py:343) */
typedef struct lard_logits {
  const void* data;  /* device pointer */
  int64_t size[3];   /* B, K, V */
  int64_t stride[3]; /* element strides, stride[2] == 1 */
  int32_t dtype;     /* LARD_DTYPE_F16 / BF16 / F32 */
} lard_logits;

typedef struct lard_mask {
  const void* data;  /* device pointer, ignored when kind == LARD_MASK_NONE */
  int32_t kind;      /* LARD_MASK_* */
  int64_t size[2];   /* B, T */
  int64_t stride[2]; /* element strides, stride[1] == 1 */
} lard_mask;

/* Library version string, e.g. "linearard_amd 0.1.0 gfx950". */
const char* lard_version(void);

/* Message of the last failed call on this thread ("" after a success). */
const char* lard_last_error(void);

/*
 * Stage A -- replaces lse_stats_triton(q, k, attn_mask, causal, sm_scale)
 * (kernel_A.py:190-265).  Writes lse[B, Hq, T] (float32, contiguous):
 * log sum_j exp(sm_scale q_i.k_j) over the valid set, 0 for masked rows.
 * `mask` may be NULL (no padding).
 */
int lard_lse_stats(const lard_tensor4* q, const lard_tensor4* k, const lard_mask* mask,
                   int causal, float sm_scale, float* lse_out, void* stream);

/* Workspace needed by lard_kl_forward for B x Hq x T rows (bytes): the
 * per-row KL terms and the partials of the fixed-order loss sum. */
size_t lard_kl_forward_workspace_bytes(int64_t batch, int64_t heads, int64_t seq_len);

/*
 * Stage B -- replaces kl_forward_triton(qs, ks, lse_s, qt, kt, lse_t,
 * attn_mask, causal, sm_scale_s, sm_scale_t)  (kernel_B.py:249-391).
 * Writes the 0-d float32 SUM over rows of sum_j p_t (log p_t - log p_s) to
 * loss_out[0].  lse_s / lse_t are contiguous float32 [B, Hq, T].  The sum is
 * deterministic (fixed-order reduction; the reference uses atomics).
 */
int lard_kl_forward(const lard_tensor4* qs, const lard_tensor4* ks, const float* lse_s,
                    const lard_tensor4* qt, const lard_tensor4* kt, const float* lse_t,
                    const lard_mask* mask, int causal, float sm_scale_s, float sm_scale_t,
                    float* loss_out, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Stage C -- replaces kl_backward_triton(...)  (kernel_C.py:293-449).
 * Writes dq[B, Hq, T, Ds] and dk[B, Hkv_s, T, Ds] (float32, contiguous,
 * every element written): D = p_s - p_t cast to the student dtype,
 * dq = sm_scale_s D K_s, dk = sm_scale_s sum_{h in group} D^T Q_s.
 * dk is accumulated by one owner per key tile (no atomics).
 */
int lard_kl_backward(const lard_tensor4* qs, const lard_tensor4* ks, const float* lse_s,
                     const lard_tensor4* qt, const lard_tensor4* kt, const float* lse_t,
                     const lard_mask* mask, int causal, float sm_scale_s, float sm_scale_t,
                     float* dq_out, float* dk_out, void* stream);

/* Kernels of the autograd calls (lard_attn_kl_forward / _backward), by operands. */
#define LARD_PATH_THROUGHPUT 0     /* the throughput kernels: one-pass forward (with the row-side gradient), column backward */
#define LARD_PATH_FUSED_FORWARD 1  /* one-pass forward, stage-kernel backward (several times slower) */
#define LARD_PATH_STAGE 2          /* stage kernels only: the reference's composition (about 4x slower) */
#define LARD_PATH_FLOAT32 3        /* float32 inputs: the double-precision kernels */

/*
 * Which kernels lard_attn_kl_forward / lard_attn_kl_backward run for these
 * operands: a LARD_PATH_* value (>= 0), or the negative error that
 * lard_attn_kl_forward would return for invalid operands (q/k pairs that do
 * not match, student and teacher B/Hq/T that differ, float32 on one side
 * only, scales that are not finite).  After a non-throughput answer,
 * lard_last_error() names the condition (head dims differ or exceed 128,
 * dtypes differ, a head of 2^30 elements or more, scales outside
 * [1e-6, 1e6] or more than 1e6 apart, float32); it is empty for LARD_PATH_THROUGHPUT.  No counterpart in the
 * reference (one Triton path, kernel_A.py / kernel_B.py / kernel_C.py); it
 * lets a caller see the slower paths the reference does not have.
 */
int lard_attn_kl_path(const lard_tensor4* qs, const lard_tensor4* ks, const lard_tensor4* qt, const lard_tensor4* kt,
                      float sm_scale_s, float sm_scale_t);

/* Workspace needed by lard_attn_kl_forward (bytes): the per-row KL terms,
 * the loss-sum partials and one validity byte per token. */
size_t lard_attn_kl_forward_workspace_bytes(int64_t batch, int64_t heads, int64_t seq_len);

/*
 * Autograd forward -- replaces AttnKLAlignFn.forward (integration.py:8-45):
 * stage A for both relations followed by stage B, in one pass over the key
 * tiles when Ds == Dt and both relations share a dtype (the stage kernels
 * otherwise).  Writes lse_s_out / lse_t_out [B, Hq, T] (as stage A; the
 * backward's input) and loss_out[0] (as stage B, a deterministic sum).
 */
int lard_attn_kl_forward(const lard_tensor4* qs, const lard_tensor4* ks, const lard_tensor4* qt,
                         const lard_tensor4* kt, const lard_mask* mask, int causal, float sm_scale_s,
                         float sm_scale_t, float* lse_s_out, float* lse_t_out, float* loss_out,
                         void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of the library's own forward workspace on each GPU (16 MiB), held
 * from the first lard_attn_kl_forward_noalloc call on that GPU until the
 * process ends. */
#define LARD_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)

/*
 * lard_attn_kl_forward without a workspace argument and without any device
 * allocation: no counterpart in the reference.  It is for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, outputs and results as
 * lard_attn_kl_forward; the workspace is a library array of
 * LARD_NOALLOC_SCRATCH_BYTES per GPU, so lard_attn_kl_forward_workspace_bytes(B,
 * Hq, T) must not exceed it (about 4M rows B * Hq * T; cfg4's 1M rows fit),
 * else LARD_ERR_UNSUPPORTED.  Every call on one GPU uses that GPU's array:
 * calls that overlap on one GPU (other streams, other host threads) race;
 * calls ordered on one stream do not.  Nothing in the array needs clearing:
 * each call writes every byte it reads.
 */
int lard_attn_kl_forward_noalloc(const lard_tensor4* qs, const lard_tensor4* ks, const lard_tensor4* qt,
                                 const lard_tensor4* kt, const lard_mask* mask, int causal, float sm_scale_s,
                                 float sm_scale_t, float* lse_s_out, float* lse_t_out, float* loss_out,
                                 void* stream);

/* Workspace needed by lard_attn_kl_backward (bytes): one validity byte per
 * token and two log2-domain row normalisers per query row.  kv_heads,
 * head_dim and self_relation do not change the size; they are kept so the
 * call describes the whole problem. */
size_t lard_attn_kl_backward_workspace_bytes(int64_t batch, int64_t heads, int64_t kv_heads, int64_t seq_len,
                                             int64_t head_dim, int self_relation);

/*
 * Autograd backward -- replaces AttnKLAlignFn.backward (integration.py:48-67):
 * stage C from the forward's LSE vectors followed by the chain rule with
 * dloss (a device float32 scalar, or NULL for 1).  Writes
 *   dq_out[B, Hq, T, Ds]    = dloss * sm_scale_s D K_s
 *   dk_out[B, Hkv_s, T, Ds] = dloss * sm_scale_s sum_{h in group} D^T Q_s
 * with D = P_s - P_t cast to the student dtype (kernel_C.py:232-233).  With
 * self_relation != 0 (q and k are the same tensor, the train.py call) the
 * sum dq + dk -- the whole gradient of that tensor -- goes to dk_out and
 * dq_out is not used.  Both sides have one owning workgroup per row / key
 * tile: no atomics, bitwise deterministic.
 */
int lard_attn_kl_backward(const lard_tensor4* qs, const lard_tensor4* ks, const float* lse_s,
                          const lard_tensor4* qt, const lard_tensor4* kt, const float* lse_t,
                          const lard_mask* mask, int causal, float sm_scale_s, float sm_scale_t,
                          const float* dloss, int self_relation, float* dq_out, float* dk_out,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * Autograd forward with the row side of the backward -- AttnKLAlignFn.forward
 * (integration.py:8-45) for a caller that will run the backward: the same
 * outputs as lard_attn_kl_forward (same workspace) plus
 *   dq_row_out[B, Hq, T, Ds] = sm_scale_s sum_j (P_s - P_t)_ij k_s[j]
 * (float32, 16-byte aligned; the row-side product of kernel_C.py:224-239
 * without dloss), from the same pass over the keys: the output products
 * P_s K_s and P_t K_s accumulate next to the online softmaxes, with P_s and
 * P_t rounded separately to float16 (the reference rounds their difference
 * to the input type, kernel_C.py:233) and both relations' scores from
 * float16 operands (bfloat16 inputs are converted into the workspace, each
 * side scaled by a power of two when it holds values of 2^15 or more; the
 * products are those of the input values).  Workspace:
 * lard_attn_kl_forward_rowgrad_workspace_bytes.  lard_attn_kl_backward_colgrad then runs only
 * the column side.  Throughput shapes only (lard_attn_kl_path ==
 * LARD_PATH_THROUGHPUT), else LARD_ERR_UNSUPPORTED.  No counterpart in the
 * reference, which recomputes both relations in the backward.
 */
/* Workspace needed by lard_attn_kl_forward_rowgrad (bytes): the forward's,
 * plus both sides' keys as float16 ([B, kv_heads, T, D] student,
 * [B, kv_heads_t, T, D] teacher; bfloat16 inputs are converted) and four
 * scalars. */
size_t lard_attn_kl_forward_rowgrad_workspace_bytes(int64_t batch, int64_t heads, int64_t kv_heads,
                                                    int64_t kv_heads_t, int64_t seq_len, int64_t head_dim);

int lard_attn_kl_forward_rowgrad(const lard_tensor4* qs, const lard_tensor4* ks, const lard_tensor4* qt,
                                 const lard_tensor4* kt, const lard_mask* mask, int causal, float sm_scale_s,
                                 float sm_scale_t, float* lse_s_out, float* lse_t_out, float* loss_out,
                                 float* dq_row_out, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Autograd backward after lard_attn_kl_forward_rowgrad --
 * AttnKLAlignFn.backward (integration.py:48-67) with the row side already
 * formed: runs the column side (kernel_C.py:242-253, D cast to the student
 * dtype) and the chain rule with dloss (device scalar, NULL for 1).
 *   self_relation != 0: dk_out = dloss (dq_row + sm_scale_s sum_h D^T Q_s),
 *                       the whole gradient of the tensor (dk_out may be dq_row);
 *   otherwise:          dq_row *= dloss in place (it is then dq), and
 *                       dk_out = dloss sm_scale_s sum_{h in group} D^T Q_s.
 * Workspace as lard_attn_kl_backward_workspace_bytes.  Throughput shapes
 * only, else LARD_ERR_UNSUPPORTED.
 */
int lard_attn_kl_backward_colgrad(const lard_tensor4* qs, const lard_tensor4* ks, const float* lse_s,
                                  const lard_tensor4* qt, const lard_tensor4* kt, const float* lse_t,
                                  const lard_mask* mask, int causal, float sm_scale_s, float sm_scale_t,
                                  const float* dloss, int self_relation, float* dq_row, float* dk_out,
                                  void* workspace, size_t workspace_bytes, void* stream);

/*
 * One self relation of a batched relation loss: the student tensor xs is
 * both q and k, the teacher tensor xt likewise -- the call
 * attn_kl_align(x_s, x_s, x_t, x_t) of train.py:380-402.  lse_s / lse_t
 * [B, H, T] float32 are written by the batched forward and read by the
 * batched backward; dxs [B, H, T, D] float32 receives the gradient of xs.
 */
typedef struct lard_relation {
  lard_tensor4 xs;
  lard_tensor4 xt;
  float* lse_s;
  float* lse_t;
  float* dxs;
} lard_relation;

/* Workspace of lard_attn_kl_batched_forward and _backward (bytes, the same
 * for both): per-row KL terms of every relation, the loss-sum partials, one
 * validity byte per token and two row normalisers per query row. */
size_t lard_attn_kl_batched_workspace_bytes(const lard_relation* rels, int nrel);

/*
 * Batched forward -- replaces the caller's loop of attn_kl_align calls over
 * layers and Q/K/V relations (train.py:369-410) with one launch per
 * 8 relations (head counts may differ, as Q/Q 32 vs K/K 8 heads):
 *   loss_out[0] = sum_r weights[r] * KL_r,
 * KL_r the relation's loss as lard_attn_kl_forward computes it (a sum over
 * rows), weights a device float32 [nrel] array or NULL (all 1), the whole
 * sum one deterministic reduction.  All relations share B, T, the dtype and
 * the head dim (Ds == Dt <= 128); scales must lie in [1e-6, 1e6] within a
 * factor 1e6 of each other.  Other batches are LARD_ERR_UNSUPPORTED and go
 * relation by relation through lard_attn_kl_forward.
 */
int lard_attn_kl_batched_forward(const lard_relation* rels, int nrel, const lard_mask* mask, int causal,
                                 float sm_scale_s, float sm_scale_t, const float* weights, float* loss_out,
                                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * Batched backward -- AttnKLAlignFn.backward (integration.py:48-67) of every
 * relation of the batched forward, from the LSE vectors it wrote:
 *   rels[r].dxs = dloss * weights[r] * dKL_r / dxs
 * (dloss a device float32 scalar or NULL for 1), each the whole gradient of
 * xs (row and column side summed), bitwise deterministic.
 */
int lard_attn_kl_batched_backward(const lard_relation* rels, int nrel, const lard_mask* mask, int causal,
                                  float sm_scale_s, float sm_scale_t, const float* weights, const float* dloss,
                                  void* workspace, size_t workspace_bytes, void* stream);

/*
 * Batched forward with the row side of the backward: lard_attn_kl_batched_forward
 * (train.py:369-410) whose relations also receive, in rels[r].dxs, the row
 * side of their gradient as lard_attn_kl_forward_rowgrad forms it (no
 * weight, no dloss).  Workspace: lard_attn_kl_batched_rowgrad_workspace_bytes.
 * Pair with lard_attn_kl_batched_backward_colgrad (which takes the smaller
 * lard_attn_kl_batched_workspace_bytes).
 */
/* Workspace of lard_attn_kl_batched_forward_rowgrad (bytes): the batched
 * workspace plus each relation's keys (both sides) as float16. */
size_t lard_attn_kl_batched_rowgrad_workspace_bytes(const lard_relation* rels, int nrel);

int lard_attn_kl_batched_forward_rowgrad(const lard_relation* rels, int nrel, const lard_mask* mask, int causal,
                                         float sm_scale_s, float sm_scale_t, const float* weights, float* loss_out,
                                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * Batched backward after lard_attn_kl_batched_forward_rowgrad
 * (integration.py:48-67 of every relation): adds the column side to the row
 * side in rels[r].dxs and applies the chain rule once,
 *   rels[r].dxs = dloss * weights[r] * dKL_r / dxs,
 * the same result as lard_attn_kl_batched_backward.
 */
int lard_attn_kl_batched_backward_colgrad(const lard_relation* rels, int nrel, const lard_mask* mask, int causal,
                                          float sm_scale_s, float sm_scale_t, const float* weights,
                                          const float* dloss, void* workspace, size_t workspace_bytes, void* stream);

/*
 * RoPE pair producer -- the step before the path: each model's rotary
 * embedding of the captured q / k (HF LLaMA apply_rotary_pos_emb, rotate_half
 * layout), the teacher with its native frequencies and the student with the
 * scaled ones of --student-rope-scaling (train.py:206-213; linear, factor 4
 * or 8 in scripts/train_linearard_*.sh:9).  From the pre-RoPE x [B, H, T, D]
 * (any element strides with stride[3] == 1, so a [B, T, H, D] tensor's
 * permuted view needs no copy; D a multiple of 16) writes out_t and out_s,
 * contiguous [B, H, T, D] of x's dtype:
 *   out[i]       = R(R(x[i] c_i) + R(-x[i+D/2] s_i)),
 *   out[i + D/2] = R(R(x[i+D/2] c_i) + R(x[i] s_i)),
 * c_i, s_i = R(cos / sin of pos * inv_freq[i], times att) (the angle one
 * float32 product, then the float32 product with att), R the rounding to x's
 * dtype after every operation.  inv_freq_t / inv_freq_s: device float32
 * [D/2], any HF rope type's frequencies (default, linear, dynamic NTK, yarn,
 * longrope, llama3, or another base); att_t / att_s: that type's
 * attention_scaling (1 unless yarn / longrope); position_ids: device int64
 * [B, T] with batch stride pos_stride_b, or NULL for 0..T-1.
 */
int lard_rope_pair(const lard_tensor4* x, const float* inv_freq_t, const float* inv_freq_s, float att_t, float att_s,
                   const int64_t* position_ids, int64_t pos_stride_b, void* out_t, void* out_s, void* stream);

/*
 * Logits KL -- replaces the output-alignment lines of the distillation step
 * (train.py:412-419):
 *   t_logp = log_softmax(t_logits / T); s_logp = log_softmax(s_logits / T)
 *   kl_per_tok = (t_logp.exp() * (t_logp - s_logp)).sum(-1); logits_kl = kl_per_tok.mean()
 * over the [B, K, V] logits of the K kept positions (train.py:343-358).
 * t_logits / s_logits: same shape and dtype (fp16, bf16 or fp32), V stride 1,
 * rows on 16-byte boundaries (data 16-byte aligned, B and K strides multiples
 * of 8 elements for 16-bit types, 4 for fp32).  The scaled logits are
 * q = R(x * (1/T)) with 1/T a float32 quotient and R the rounding to the
 * dtype (a tensor division by a host scalar); everything after that is
 * float32.  Writes lse_t, lse_s (log-sum-exp of q) and kl_rows (KL of each
 * kept position), float32 [B*K] contiguous, and the mean into *loss (NaN
 * for B*K == 0, the mean of an empty tensor; rows of V == 0 give KL 0).
 * Deterministic: fixed reduction orders.  workspace: at least
 * lard_logits_kl_workspace_bytes(B*K, V) bytes, 16-byte aligned.
 */
size_t lard_logits_kl_workspace_bytes(int64_t rows, int64_t vocab);
int lard_logits_kl_forward(const lard_logits* t_logits, const lard_logits* s_logits, float temperature,
                           float* lse_t, float* lse_s, float* kl_rows, float* loss, void* workspace,
                           size_t workspace_bytes, void* stream);

/*
 * Logits KL backward -- autograd of the same lines (train.py:424 backward):
 *   grad_s = c (p_s - p_t) / T,  grad_t = c p_t (l_t - l_s - KL) / T
 * with p_x = exp(q_x - lse_x), l_x = q_x - lse_x and c = dloss[r] * row_scale
 * (dloss_per_row != 0: one upstream value per row, as for kl_per_tok) or
 * dloss[0] * row_scale (the mean: row_scale = 1 / (B*K)).  grad_t / grad_s:
 * [B, K, V] of the logits' dtype with the same layout rules, or NULL to skip
 * (the reference's teacher runs under no_grad, train.py:337); written in the
 * logits dtype (one rounding of the float32 value).  kl_rows is read only
 * for grad_t.
 */
int lard_logits_kl_backward(const lard_logits* t_logits, const lard_logits* s_logits, float temperature,
                            const float* lse_t, const float* lse_s, const float* kl_rows, const float* dloss,
                            int dloss_per_row, float row_scale, const lard_logits* grad_t,
                            const lard_logits* grad_s, void* stream);

/* Kernel ids of the timing hook. */
#define LARD_KERNEL_FORWARD 0  /* one-pass forward: both LSEs and the per-row KL */
#define LARD_KERNEL_ROW_GRAD 1 /* backward, row side: dq (kernel_C.py:224-239) */
#define LARD_KERNEL_COL_GRAD 2 /* backward, column side: dk (kernel_C.py:242-253) */
#define LARD_KERNEL_LOGITS_FORWARD 3 /* logits KL forward pass (lard_logits_kl_forward) */
#define LARD_KERNEL_LOGITS_GRAD 4    /* logits KL gradient pass (lard_logits_kl_backward) */
#define LARD_KERNEL_FORWARD_ROWGRAD 5 /* forward with the row-side gradient (lard_attn_kl_*forward_rowgrad) */
#define LARD_KERNEL_COUNT 6

/*
 * Timing hook for measurement harnesses -- no counterpart in the reference
 * (its kernels are timed from outside).  While enabled, every launch of the
 * kernels above by lard_attn_kl_forward / lard_attn_kl_backward /
 * lard_kl_backward / lard_attn_kl_batched_* / lard_logits_kl_* is bracketed
 * by two HIP events recorded on its launch stream.  lard_timing_read() waits for the recorded
 * events and returns the summed elapsed milliseconds and the launch count of
 * one kernel since its last read, then clears them.  Off by default.  While enabled, launches
 * cannot be captured into a HIP graph and calls from several host threads
 * serialise briefly on one lock.
 */
int lard_timing_enable(int on);
int lard_timing_read(int kernel, double* total_ms, int64_t* launches);

#ifdef __cplusplus
}
#endif

#endif /* LINEARARD_AMD_H */
