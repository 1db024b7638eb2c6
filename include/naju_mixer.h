/*
 * naju_mixer.h -- C ABI of the MI355X (gfx950) kernels around the Naju scan
 * inside the mixer: the depthwise causal convolutions of the content branch
 * and of the gate logits (reference /root/reference/naju/mixer.py:75-76,
 * 97-99, 106-110, 115), the readout epilogue after the scan
 * (mixer.py:123-124), and the blocks' RMSNorm (mixer.py:51-58).
 *
 *   y[b,t,c] = act( add[b,t,c] + bias[c] + sum_{j<K} w[c,j] * x[b, t-(K-1)+j, c] )
 *
 * with x taken as 0 before t = 0 (causal), act = identity or SiLU, and add and
 * bias optional (NULL). This is one nn.Conv1d(C, C, K, groups=C,
 * padding=K-1) followed by the slice [..., :T] (mixer.py:115 for the content
 * branch, with SiLU; mixer.py:106-110 for a gate logit, where add is the gate
 * projection and bias the gate bias).
 *
 * Layouts: y, dy, dx : [batch, T, C] row-major (C fastest);
 *          x : [batch, T, C] with C fastest and x_ld >= C elements between
 *              consecutive timesteps (x_ld = C when contiguous; 2C for one half
 *              of the in_proj output [x, z] without a copy);
 *          add : the same with add_ld >= C (one slice of a fused projection
 *              output goes in without a copy);
 *          w, dw : [C, K] float32 (the Conv1d weight [C, 1, K]);
 *          bias, dbias : [C] float32.
 * dtype codes are those of naju_scan.h (F32, BF16, F16). Arithmetic is
 * float32. Every call is asynchronous on `stream`, allocates nothing and never
 * synchronises the host; errors are reported as in naju_scan.h, with the
 * message in naju_mixer_last_error().
 */
#ifndef NAJU_MIXER_H
#define NAJU_MIXER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message of the last failed call of this thread ("" after a success). */
const char* naju_mixer_last_error(void);

/* Forward: y = act(add + bias + causal_dwconv(x, w)). act: 0 = identity,
 * 1 = SiLU (then add must be NULL). K <= 8. Replaces the Conv1d calls of
 * naju/mixer.py:109 and :115 (plus the bias add of :110). */
int naju_dwconv_fwd(const void* x, int64_t x_ld, const float* w, const float* bias, const void* add, int64_t add_ld,
                    void* y, int64_t batch, int64_t T, int64_t C, int K, int act, int x_dtype, int add_dtype,
                    int y_dtype, void* stream);

/* Bytes of workspace naju_dwconv_bwd needs (per-block partial sums of dw and
 * dbias); no zero-fill needed. */
size_t naju_dwconv_workspace_bytes(int64_t batch, int64_t T, int64_t C, int K);

/* Backward of naju_dwconv_fwd: dx (dx_ld >= C elements between rows), dw
 * and dbias (each nullable to skip it) from dy. With act = 1 the
 * pre-activation is recomputed from x. The gradient of add is dy itself;
 * dadd (act = 0 only, nullable) receives it in dadd_dtype with dadd_ld
 * elements between rows, so that it lands in place in a wider gradient
 * buffer (one slice of a fused projection's gradient). act may carry
 * NAJU_DWCONV_ACCUM_DX: dx then receives dx + (the gradient), rounded once
 * to dx_dtype, so that x's gradient from several consumers collects in one
 * buffer without separate additions (no reference counterpart: autograd
 * adds them there). Deterministic (fixed-order sums). The autograd of the
 * reference's Conv1d + slice. */
#define NAJU_DWCONV_ACCUM_DX 2
int naju_dwconv_bwd(const void* x, int64_t x_ld, const float* w, const float* bias, const void* dy, void* dx,
                    int64_t dx_ld, float* dw, float* dbias, void* dadd, int64_t dadd_ld, int64_t batch, int64_t T,
                    int64_t C, int K, int act, int x_dtype, int dy_dtype, int dx_dtype, int dadd_dtype,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Readout epilogue of the mixer (naju/mixer.py:123-124), one pass:
 *
 *   y[r,c] = (cx[r,c] * scale + Dv[c] * h[r,c]) * SiLU(z[r,c])
 *
 * over rows r < n_rows (= batch * T) and channels c < C. cx, h, y are
 * [n_rows, C] contiguous; z has z_ld >= C elements between rows (the second
 * half of the in_proj output [x, z] goes in without a copy); Dv is [C] f32. */
int naju_readout_fwd(const void* cx, const void* h, const void* z, int64_t z_ld, const float* Dv, float scale,
                     void* y, int64_t n_rows, int64_t C, int cx_dtype, int h_dtype, int z_dtype, int y_dtype,
                     void* stream);

/* Bytes of workspace naju_readout_bwd needs for the dD partial sums. */
size_t naju_readout_workspace_bytes(int64_t n_rows, int64_t C);

/* Backward of naju_readout_fwd: dcx, dh ([n_rows, C] contiguous), dz
 * (dz_ld >= C elements between rows, so that it can land in place in the
 * in_proj output's gradient), in the given dtypes, and dD [C] f32 (summed
 * over rows in a fixed order), each nullable to skip it. */
int naju_readout_bwd(const void* cx, const void* h, const void* z, int64_t z_ld, const float* Dv, float scale,
                     const void* dy, void* dcx, void* dh, void* dz, int64_t dz_ld, float* dD, int64_t n_rows,
                     int64_t C, int cx_dtype, int h_dtype, int z_dtype, int dy_dtype, int dcx_dtype, int dh_dtype,
                     int dz_dtype, void* workspace, size_t workspace_bytes, void* stream);

/* RMSNorm of the residual blocks and of the LM's final norm
 * (naju/mixer.py:51-58):
 *
 *   y[r,c] = (w[c] * x[r,c]) * rstd[r],  rstd[r] = 1 / sqrt(mean_c x[r,c]^2 + eps)
 *
 * x, y [n_rows, d] contiguous, w [d] f32, rstd [n_rows] f32 (saved for the
 * backward). y may take another dtype than x: under autocast the consumer is
 * a bf16 GEMM, and writing y in bf16 gives it the same values as the cast
 * autocast would make. Served: x f32 or bf16, d a multiple of 4 up to 4096,
 * 16-byte aligned pointers; anything else returns NAJU_ERR_UNSUPPORTED. */
int naju_rmsnorm_fwd(const void* x, const float* w, float eps, void* y, float* rstd, int64_t n_rows, int64_t d,
                     int x_dtype, int y_dtype, void* stream);

/* Bytes of workspace naju_rmsnorm_bwd needs for the dw partial sums. */
size_t naju_rmsnorm_workspace_bytes(int64_t n_rows, int64_t d);

/* Backward of naju_rmsnorm_fwd: dx [n_rows, d] in x's dtype and dw [d] f32
 * (summed over rows in a fixed order; nullable to skip it) from dy. */
int naju_rmsnorm_bwd(const void* x, const float* w, const float* rstd, const void* dy, void* dx, float* dw,
                     int64_t n_rows, int64_t d, int x_dtype, int dy_dtype, int dx_dtype, void* workspace,
                     size_t workspace_bytes, void* stream);

/* naju_rmsnorm_bwd with dx = dres + (the norm's gradient), dres [n_rows, d]
 * in x's dtype (nullable; not dx itself): the pre-norm block's residual
 * stream feeds both the norm and the residual add (naju/mixer.py:138-144),
 * and this adds the two gradients in the norm's pass instead of a separate
 * addition. No reference counterpart (autograd adds them there). */
int naju_rmsnorm_bwd_add(const void* x, const float* w, const float* rstd, const void* dy, const void* dres,
                         void* dx, float* dw, int64_t n_rows, int64_t d, int x_dtype, int dy_dtype, int dx_dtype,
                         void* workspace, size_t workspace_bytes, void* stream);

/* The pre-norm block's residual add with dropout, u + Dropout(p)(mix)
 * (naju/mixer.py:131-144: NajuBlock's self.drop and residual), in one pass:
 * out = u + (keep_i ? (mix_i / (1 - p) rounded to mix_dtype) : 0), n
 * elements, u and out float32, mix in mix_dtype. keep_i is a pure function
 * of (*seed, i) (a SplitMix64 draw per pair of elements, kept with
 * probability 1 - p), so the backward draws the same mask again and no mask
 * is stored; seed is a device pointer (the caller draws it from its own
 * generator, e.g. torch's, without a host synchronisation) and may be NULL
 * when p = 0. */
int naju_residual_dropout_fwd(const float* u, const void* mix, const int64_t* seed, float p, float* out, int64_t n,
                              int mix_dtype, void* stream);

/* Backward of the dropout in naju_residual_dropout_fwd with the same seed
 * and p: dmix = keep_i ? g_i / (1 - p) : 0 (rounded once to mix_dtype) from
 * the float32 gradient g of out (which is also u's gradient, unchanged). */
int naju_dropout_bwd(const float* g, const int64_t* seed, float p, void* dmix, int64_t n, int mix_dtype,
                     void* stream);

/* The mixer's two gate convolutions over one input in one pass (x read
 * once): y0 = add0 + bias0 + conv(x, w0) and y1 = add1 + bias1 + conv(x, w1),
 * each as naju_dwconv_fwd with act = 0. Served for K = 4, C and the row
 * strides (x_ld, add_ld) multiples of 8, 16-byte aligned pointers, add in x's
 * dtype, y in x's dtype or float32 (else NAJU_ERR_UNSUPPORTED, and the
 * caller makes the two single calls). Both adds share add_ld (slices of one
 * projection output); bias0 / bias1 may be NULL. */
int naju_dwconv_pair_fwd(const void* x, int64_t x_ld, const float* w0, const float* bias0, const void* add0,
                         const float* w1, const float* bias1, const void* add1, int64_t add_ld, void* y0, void* y1,
                         int64_t batch, int64_t T, int64_t C, int K, int x_dtype, int y_dtype, void* stream);

/* Bytes of workspace naju_dwconv_pair_bwd needs (both weights' partial
 * sums); no zero-fill needed. */
size_t naju_dwconv_pair_workspace_bytes(int64_t batch, int64_t T, int64_t C, int K);

/* Backward of naju_dwconv_pair_fwd: dx = conv0^T(dy0) + conv1^T(dy1) (x's
 * gradient from both, rounded once to x's dtype; with accumulate != 0 dx
 * receives dx + that sum), dw0 / dbias0 / dw1 / dbias1 (each nullable; fixed
 * order, deterministic), and the adds' gradients dy0, dy1 written in x's
 * dtype into dadd0 / dadd1 (nullable, row stride dadd_ld). dy0, dy1 are
 * [batch, T, C] in x's dtype or float32 with rows dy_ld apart (a multiple
 * of 8: they may be the slices naju_scan_bwd_ex wrote into the projection's
 * gradient buffer, whose adds' gradients then need no dadd). Same shapes
 * served as the forward. No reference counterpart as one call: the
 * reference's two Conv1d modules and autograd's sum of their input
 * gradients (naju/mixer.py:108-110). */
int naju_dwconv_pair_bwd(const void* x, int64_t x_ld, const float* w0, const float* w1, const void* dy0,
                         const void* dy1, int64_t dy_ld, void* dx, int64_t dx_ld, float* dw0, float* dbias0, float* dw1,
                         float* dbias1, void* dadd0, void* dadd1, int64_t dadd_ld, int64_t batch, int64_t T,
                         int64_t C, int K, int accumulate, int x_dtype, int dy_dtype, void* workspace,
                         size_t workspace_bytes, void* stream);

/* out[i] = sum over s < n_parts of parts[s * n + i], added in s order, all
 * float32 (1 <= n_parts <= 16): the split-K weight gradient's sum of its
 * token parts (naju_amd/linear.py). No reference counterpart: the reference
 * forms the weight gradient as one GEMM. */
int naju_sum_parts(const float* parts, int n_parts, int64_t n, float* out, void* stream);

/* dw[id] += the rows dy[order[q]] of every q with sorted_ids[q] == id, for
 * the n ids sorted with a stable sort (sorted_ids = ids[order]); dy is
 * [n_ids_before_sorting, d] float32, dw [V, d] float32, both row-major; ids
 * outside [0, V) are skipped. Each row of dw gets its rows added in sorted
 * order, one workgroup per run of equal ids: deterministic. The embedding's
 * backward (nn.Embedding without padding_idx, max_norm or
 * scale_grad_by_freq) added in place into a gradient already there (a tied
 * LM head's). Reference counterpart: torch's embedding backward under
 * naju/lm.py:13-33's tied weights, which autograd then adds to the head's. */
int naju_embedding_bwd_add(const int64_t* sorted_ids, const int64_t* order, const float* dy, int64_t n, int64_t d,
                           float* dw, int64_t V, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NAJU_MIXER_H */
