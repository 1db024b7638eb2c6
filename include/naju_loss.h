/*
 * naju_loss.h -- C ABI of the MI355X (gfx950) cross-entropy of the Naju LM
 * training step: the reference's
 *
 *   loss = nn.functional.cross_entropy(logits.reshape(-1, V), y.reshape(-1))
 *
 * under bf16 autocast (/root/reference/evals/lm/train.py:70-74), which
 * evaluates it in float32 on the upcast logits with the defaults
 * ignore_index = -100 and reduction = "mean":
 *
 *   loss = sum_{r valid} ( logsumexp_c x[r,c] - x[r, target[r]] ) / #valid,
 *   valid = target[r] != ignore_index.
 *
 * Layouts: x (logits) [n_rows, n_cols] with x_ld >= n_cols elements between
 * rows, dtype F32, BF16 or F16 (codes of naju_scan.h); target [n_rows] int64;
 * lse [n_rows] float32; loss and scale one float32 each: the mean loss and
 * 1 / #valid (the scale of every valid row's gradient). Arithmetic is
 * float32, the final mean is summed in float64 in a fixed order, so both
 * calls are deterministic. A target outside [0, n_cols) that is not
 * ignore_index gives that row a NaN loss (and NaN gradients) instead of a
 * device fault; no valid row gives a NaN loss, as torch does.
 *
 * Every call is asynchronous on `stream`, allocates nothing and never
 * synchronises the host; errors are reported as in naju_scan.h, with the
 * message in naju_loss_last_error().
 */
#ifndef NAJU_LOSS_H
#define NAJU_LOSS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message of the last failed call of this thread ("" after a success). */
const char* naju_loss_last_error(void);

/* Bytes of workspace naju_xent_fwd needs (per-row losses); no zero-fill. */
size_t naju_xent_workspace_bytes(int64_t n_rows);

/* Forward: lse[r] = logsumexp of row r, loss and scale as above. One pass over the
 * logits. Replaces the float32 upcast, log_softmax and nll_loss forward that
 * cross_entropy runs under autocast (evals/lm/train.py:74). */
int naju_xent_fwd(const void* x, int64_t x_ld, const int64_t* target, int64_t n_rows, int64_t n_cols, int x_dtype,
                  int64_t ignore_index, float* lse, float* loss, float* scale, void* workspace,
                  size_t workspace_bytes, void* stream);

/* Backward: dx[r,c] = dloss[0] * scale[0] * (exp(x[r,c] - lse[r]) - [c == target[r]])
 * for valid rows, 0 for ignored rows; dx [n_rows, n_cols] with dx_ld >= n_cols,
 * in dx_dtype. dloss is the device float32 gradient of the loss. One pass over
 * the logits; the autograd of the same cross_entropy call, including the cast
 * of the gradient back to the logits' dtype. */
int naju_xent_bwd(const void* x, int64_t x_ld, const int64_t* target, int64_t n_rows, int64_t n_cols, int x_dtype,
                  int64_t ignore_index, const float* lse, const float* scale, const float* dloss, void* dx,
                  int64_t dx_ld, int dx_dtype, void* stream);

/* Forward and gradient in one pass over the logits, for a caller that will
 * take the gradient (autograd's loss.backward()): naju_xent_fwd's outputs,
 * and dx written as naju_xent_bwd writes it for dloss = 1. Each row is read
 * twice by its workgroup (the second time mostly from the caches) instead of
 * a second full pass in the backward. No reference counterpart (the
 * reference's loss is torch's, forward then backward). */
int naju_xent_fwd_grad(const void* x, int64_t x_ld, const int64_t* target, int64_t n_rows, int64_t n_cols,
                       int x_dtype, int64_t ignore_index, float* lse, float* loss, float* scale, void* dx,
                       int64_t dx_ld, int dx_dtype, void* workspace, size_t workspace_bytes, void* stream);

/* The backward after naju_xent_fwd_grad: when dloss[0] is 1 the dx that call
 * wrote is the gradient and nothing is done (each workgroup reads dloss and
 * returns); otherwise dx is rewritten as naju_xent_bwd writes it. */
int naju_xent_bwd_if_scaled(const void* x, int64_t x_ld, const int64_t* target, int64_t n_rows, int64_t n_cols,
                            int x_dtype, int64_t ignore_index, const float* lse, const float* scale,
                            const float* dloss, void* dx, int64_t dx_ld, int dx_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NAJU_LOSS_H */
