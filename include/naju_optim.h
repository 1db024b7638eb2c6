/*
 * naju_optim.h -- C ABI of the MI355X (gfx950) optimizer step of the Naju LM
 * training loop: the reference's
 *
 *   nn.utils.clip_grad_norm_(model.parameters(), grad_clip)
 *   opt.step()          # opt = torch.optim.AdamW(...)
 *
 * (/root/reference/evals/lm/train.py:79-80, 165-166; the gate-aware param
 * groups of /root/reference/naju/optim.py:30-52) over float32 parameters, in
 * two multi-tensor passes: one over the gradients for the global L2 norm,
 * one that applies the clipped AdamW update to every tensor.
 *
 * The tensors of a call are described by a table in device memory:
 * naju_adamw_tensor entries, and for every chunk of NAJU_OPTIM_CHUNK
 * elements the index of the tensor it belongs to. A tensor of numel
 * elements owns ceil(numel / NAJU_OPTIM_CHUNK) consecutive chunks starting at
 * its first_chunk; n_chunks counts them all. One workgroup serves one chunk.
 *
 * Update (torch.optim.AdamW, amsgrad = False, maximize = False, in the
 * operation order of its default multi-tensor path), per element, in
 * float32, with c the clip coefficient (1 without clipping):
 *
 *   g  = grad * c
 *   p *= decay                                   decay = 1 - lr * weight_decay
 *   m += one_minus_beta1 * (g - m)
 *   v  = v * beta2 + one_minus_beta2 * g * g
 *   p -= step_size * (m / (sqrt(v) / bias_correction2_sqrt + eps))
 *
 * with step_size = lr / (1 - beta1^t) and bias_correction2_sqrt =
 * sqrt(1 - beta2^t) at step t, every constant formed in double precision by
 * the caller and rounded once to float32 (as torch forms them in Python).
 *
 * Every call is asynchronous on `stream`, never synchronises the host and is
 * deterministic (fixed-order sums); errors are reported as in naju_scan.h,
 * with the message in naju_optim_last_error(). No reference counterpart as
 * an ABI: the reference runs these as torch's own kernels.
 */
#ifndef NAJU_OPTIM_H
#define NAJU_OPTIM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NAJU_OPTIM_CHUNK 8192     /* elements per chunk (one workgroup) */
#define NAJU_OPTIM_MAX_GROUPS 16  /* hyper-parameter sets per naju_adamw_step call */

/* One float32 tensor and its optimizer state (all numel elements, dense).
 * grad may be read-only; param, exp_avg and exp_avg_sq are updated in place.
 * 16-byte aligned pointers take the vector path, others an element loop. */
typedef struct naju_adamw_tensor {
  float* param;
  float* grad;
  float* exp_avg;
  float* exp_avg_sq;
  int64_t numel;
  int64_t first_chunk;
  int32_t group; /* index into the groups of naju_adamw_step */
  int32_t reserved;
} naju_adamw_tensor;

/* The constants of one param group at the current step (see above). */
typedef struct naju_adamw_group {
  float decay;
  float beta1;
  float one_minus_beta1;
  float beta2;
  float one_minus_beta2;
  float step_size;
  float bias_correction2_sqrt;
  float eps;
} naju_adamw_group;

/* One float32 tensor of naju_cast_multi: numel elements from src (NULL:
 * zeros) to element dst_offset of the destination; chunks as for
 * naju_adamw_tensor. */
typedef struct naju_cast_tensor {
  const float* src;
  int64_t dst_offset;
  int64_t numel;
  int64_t first_chunk;
} naju_cast_tensor;

/* Message of the last failed call of this thread ("" after a success). */
const char* naju_optim_last_error(void);

/* Bytes of workspace naju_grad_norm needs for n_chunks chunks. */
size_t naju_grad_norm_workspace_bytes(int64_t n_chunks);

/* norm[0] = sqrt(sum of grad^2 over every tensor of the table), as
 * clip_grad_norm_'s total_norm (norm_type 2); coef[0] = min(1, max_norm /
 * (norm + 1e-6)), its clip_coef_clamped (coef may be NULL). Per-chunk sums
 * in float32, their total in float64, in chunk order. tensors and
 * chunk_tensor are device pointers; norm and coef device float32. */
int naju_grad_norm(const naju_adamw_tensor* tensors, const int32_t* chunk_tensor, int n_tensors, int64_t n_chunks,
                   float max_norm, float* norm, float* coef, void* workspace, size_t workspace_bytes, void* stream);

/* The AdamW update above on every tensor of the table. groups is a HOST
 * array of n_groups (<= NAJU_OPTIM_MAX_GROUPS) entries, passed to the kernel
 * by value; grad_coef a device float32 (the coef of naju_grad_norm) or NULL. */
int naju_adamw_step(const naju_adamw_tensor* tensors, const int32_t* chunk_tensor, int n_tensors, int64_t n_chunks,
                    const naju_adamw_group* groups, int n_groups, const float* grad_coef, void* stream);

/* Every tensor of the table rounded to dst_dtype (NAJU_DTYPE_BF16 or
 * NAJU_DTYPE_F16; round to nearest even) into one destination buffer at its
 * dst_offset, in one launch: the 16-bit weight copies that autocast makes
 * one cast kernel each (and the concatenation of weights that share a
 * GEMM, when their offsets are consecutive). Bitwise torch's .to(dtype) for
 * finite and infinite values. table and chunk_tensor are device pointers; a
 * chunk is moved as float4 when src is 16-byte and its destination 8-byte
 * aligned. No reference counterpart (torch's autocast casts per tensor). */
int naju_cast_multi(const naju_cast_tensor* tensors, const int32_t* chunk_tensor, int n_tensors, int64_t n_chunks,
                    void* dst, int dst_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NAJU_OPTIM_H */
