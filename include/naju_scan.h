/*
 * naju_scan.h -- C ABI of the MI355X (gfx950) Naju gated state-space scan.
 *
 * Recurrence (per batch b, channel d, state n), the contract of
 * /root/reference/naju/scan.py:3-19:
 *   f_t = sigmoid(f_logit_t)          i_t = sigmoid(i_logit_t)
 *   x_t[n] = f_t * x_{t-1}[n] + i_t * B_t[n] * u_t        x_{-1} = h0 (or 0)
 *   y_t    = sum_n C_t[n] * x_t[n] + D_skip * u_t
 *
 * Tensor layouts (row-major, contiguous, last index fastest), scan.py:7-11:
 *   u, f_logit, i_logit, y, dy, du, dfl, dil : [batch, T, D]
 *   B, C, dB, dC                             : [batch, T, N]
 *   D_skip, dD                               : [D]        (float32)
 *   h0, hT, dh0                              : [batch, D, N] (float32)
 *   ckpt                                     : naju_scan_ckpt_elems() floats
 * All pointers are device pointers. Every call is asynchronous on `stream`
 * (a hipStream_t; NULL = the default stream), allocates nothing and never
 * synchronises the host.
 *
 * Shape limits: batch, T, D <= 2^30; 1 <= N <= 128; N > 1 needs D < 2^25
 * (NAJU_ERR_UNSUPPORTED otherwise).
 *
 * dtype codes: the u-stream dtype covers u, y, dy and du; the gate dtype
 * covers f_logit, i_logit, dfl and dil; the bc dtype covers B, C, dB and dC.
 * Supported: u in {F32, BF16, F16}; gate and bc each either F32 or equal to
 * the u dtype. Arithmetic and the state are float32 throughout.
 * flags (bit set, 0 = defaults):
 *   NAJU_FLAG_OUT_F32 (1): y, du, dfl, dil, dB and dC are all float32 instead
 *     of their inputs' dtypes (y and du: u dtype; dfl, dil: gate dtype; dB,
 *     dC: bc dtype). bf16 storage rounding alone is up to 2^-8 relative, so
 *     this is the form in which the kernels' own accuracy is measured.
 *   NAJU_FLAG_DETERMINISTIC (2): run-to-run bitwise identical results. At
 *     N = 1 each chunk then takes its carry from its immediate predecessor's
 *     inclusive carry only (a fixed composition order; the carries travel
 *     along the chunks one hop at a time, which is slower). Without it, a
 *     chunk composes whichever predecessors' maps are ready first, so N = 1
 *     results repeat to float32 rounding only. N > 1 is always bitwise
 *     deterministic.
 *   NAJU_CKPT_ROWS(r) (bits 8-15): the forward's checkpoint interval for
 *     N > 1, r rows (32, 64 or 128; 0 = the default). The checkpoint holds
 *     the state every r rows (batch*ceil(T/r)*D*N floats).
 *     The default is 16 rows for 9 <= N <= 64 (the state entering every
 *     sub-block of the matrix-core backward) and 32 rows otherwise; a longer
 *     interval is the memory-light mode of the reference's recompute backend
 *     (naju/cuda/__init__.py:9-12, CK = 32 in naju/cuda/naju_cuda.cu:25):
 *     the forward's time segments always start at multiples of 128 rows
 *     (so the checkpoint holds every state a recompute starts from, and
 *     nothing else), and the backward first recomputes the state at every
 *     16-row sub-block from it into its workspace (one forward-like pass
 *     over u, f_logit, i_logit and B), so the memory held between forward
 *     and backward shrinks r/16-fold at the cost of that pass. Every output
 *     is bitwise the one of the default interval.
 *     Served for 9 <= N <= 64 by naju_scan_fwd and naju_scan_fwd_noalloc;
 *     other N accept only their default (NAJU_ERR_UNSUPPORTED otherwise).
 *     The backward must be given the forward's flags value for these bits,
 *     and the size queries below have _ex forms that take it.
 *
 * Workspace: naju_scan_workspace_bytes() bytes of device memory that MUST be
 * zero-filled once before its first use; every call leaves it reusable
 * (its counters return to zero), so one zeroed workspace serves any number of
 * stream-ordered calls. Calls that overlap in time (different streams) need
 * different workspaces.
 *
 * HIP graphs: the calls issue kernel launches only (no allocation, memset or
 * host synchronisation), so they can be recorded by stream capture. At N = 1
 * a call made while `stream` is capturing also records a one-thread kernel
 * that advances a device-side epoch in the workspace, and the scan kernels
 * take their cross-workgroup hand-off tags from it, so each replay is
 * independent of the previous one (eager calls use host-side tags).
 *
 * Return codes: 0 on success, a negative NAJU_ERR_* otherwise, with a message
 * in naju_scan_last_error() (thread-local). Argument checks run on the host,
 * before any device work, so they are testable without a GPU.
 */
#ifndef NAJU_SCAN_H
#define NAJU_SCAN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NAJU_DTYPE_F32 0
#define NAJU_DTYPE_BF16 1
#define NAJU_DTYPE_F16 2

#define NAJU_FLAG_OUT_F32 1
#define NAJU_FLAG_DETERMINISTIC 2
#define NAJU_CKPT_SHIFT 8
#define NAJU_CKPT_MASK (0xFF << NAJU_CKPT_SHIFT)
#define NAJU_CKPT_ROWS(r) ((((r) / 16) & 0xFF) << NAJU_CKPT_SHIFT)

#define NAJU_OK 0
#define NAJU_ERR_INVALID -1     /* bad pointer, shape or dtype code        */
#define NAJU_ERR_UNSUPPORTED -2 /* valid request this build does not serve */
#define NAJU_ERR_WORKSPACE -3   /* workspace missing or too small          */
#define NAJU_ERR_LAUNCH -4      /* the HIP runtime rejected a launch       */

/* Library version, (major << 16) | minor. */
int naju_scan_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* naju_scan_last_error(void);

/* Number of float32 values of the forward's state checkpoint, which the
 * backward consumes. Depends only on the shape and the dtype codes. Replaces
 * the ckpt tensor of reference naju/cuda/naju_cuda.cu:241-259 (there
 * [B,D,ceil(T/32),N]). */
int64_t naju_scan_ckpt_elems(int64_t batch, int64_t T, int64_t D, int64_t N,
                             int x_dtype, int gate_dtype, int bc_dtype);

/* Bytes of workspace needed by naju_scan_fwd / naju_scan_bwd at this shape
 * (the same figure serves both). */
size_t naju_scan_workspace_bytes(int64_t batch, int64_t T, int64_t D,
                                 int64_t N, int x_dtype, int gate_dtype,
                                 int bc_dtype);

/* The two size queries for the flags value given to naju_scan_fwd /
 * naju_scan_bwd (only its NAJU_CKPT_ROWS bits matter; flags = 0 gives the
 * figures above). A longer checkpoint interval gives a smaller checkpoint
 * and, for the backward's recomputed states, a larger workspace. No
 * counterpart in the reference, whose interval is a compile-time constant.
 * Both return -1 / 0 (with naju_scan_last_error) for an interval the shape
 * does not serve. */
int64_t naju_scan_ckpt_elems_ex(int64_t batch, int64_t T, int64_t D,
                                int64_t N, int x_dtype, int gate_dtype,
                                int bc_dtype, int flags);
size_t naju_scan_workspace_bytes_ex(int64_t batch, int64_t T, int64_t D,
                                    int64_t N, int x_dtype, int gate_dtype,
                                    int bc_dtype, int flags);

/* Forward scan. Replaces the forward of every reference backend: the
 * sequential loop of naju/scan.py:79-93, _ChunkScanTriton.forward
 * (naju/chunk_triton.py:148-181), _AffineChunkScan.forward
 * (naju/chunk_affine_triton.py:257-288) and naju_fwd / naju_fwd_chunked
 * (naju/cuda/naju_cuda.cu:241-259, :211-238).
 *   h0   : optional initial state (NULL = zeros, the reference behaviour)
 *   y    : output, u dtype (float32 with NAJU_FLAG_OUT_F32)
 *   ckpt : optional (NULL under no_grad); state checkpoint for the backward
 *   hT   : optional final state x_{T-1}
 */
int naju_scan_fwd(const void* u, const void* f_logit, const void* i_logit,
                  const void* B, const void* C, const float* D_skip,
                  const float* h0, void* y, float* ckpt, float* hT,
                  int64_t batch, int64_t T, int64_t D, int64_t N, int x_dtype,
                  int gate_dtype, int bc_dtype, int flags, void* workspace,
                  size_t workspace_bytes, void* stream);

/* Fused backward scan. Replaces naju_bwd (naju/cuda/naju_cuda.cu:261-286),
 * naju_chunk_backward (naju/chunk_bwd_triton.py:187-243) and the affine
 * backward (naju/chunk_affine_triton.py:290-342): one reverse pass yields
 *   du, dfl, dil [batch,T,D]  (gradients of u, f_logit, i_logit)
 *   dB, dC       [batch,T,N]  (reduced over D, deterministic order)
 *   dD           [D] float32  (reduced over batch and T)
 *   dh0          [batch,D,N] float32 (gradient of h0)
 * Every gradient pointer may be NULL to skip it. ckpt must come from
 * naju_scan_fwd with the same inputs, shape and dtype codes.
 */
int naju_scan_bwd(const void* u, const void* f_logit, const void* i_logit,
                  const void* B, const void* C, const float* D_skip,
                  const float* ckpt, const void* dy, void* du, void* dfl,
                  void* dil, void* dB, void* dC, float* dD, float* dh0,
                  int64_t batch, int64_t T, int64_t D, int64_t N, int x_dtype,
                  int gate_dtype, int bc_dtype, int flags, void* workspace,
                  size_t workspace_bytes, void* stream);

/* naju_scan_fwd / naju_scan_bwd with B and C read from rows bc_ld elements
 * apart (and dB, dC written to rows dbc_ld apart) instead of N: the mixer's
 * B and C are column slices of one projection output [batch, T, width], so
 * the scan reads them, and writes their gradients, in place. Served on the
 * matrix-core path (9 <= N <= 64) with bc_ld, dbc_ld multiples of 4 and
 * pointers aligned to four elements; elsewhere a stride other than N returns
 * NAJU_ERR_UNSUPPORTED. Every output is bitwise the contiguous call's. No
 * reference counterpart (the reference's backends take contiguous B, C). */
int naju_scan_fwd_strided(const void* u, const void* f_logit, const void* i_logit, const void* B, const void* C,
                          const float* D_skip, const float* h0, void* y, float* ckpt, float* hT, int64_t batch,
                          int64_t T, int64_t D, int64_t N, int64_t bc_ld, int x_dtype, int gate_dtype, int bc_dtype,
                          int flags, void* workspace, size_t workspace_bytes, void* stream);
int naju_scan_bwd_strided(const void* u, const void* f_logit, const void* i_logit, const void* B, const void* C,
                          const float* D_skip, const float* ckpt, const void* dy, void* du, void* dfl, void* dil,
                          void* dB, void* dC, float* dD, float* dh0, int64_t batch, int64_t T, int64_t D, int64_t N,
                          int64_t bc_ld, int64_t dbc_ld, int x_dtype, int gate_dtype, int bc_dtype, int flags,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Output layout options of naju_scan_bwd_ex (initialise with
 * NAJU_SCAN_BWD_LAYOUT_INIT, then set what differs from naju_scan_bwd; a
 * stride <= 0 means the contiguous one):
 *   bc_ld, dbc_ld  as bc_ld / dbc_ld of naju_scan_bwd_strided;
 *   dg_ld          elements between rows of dfl and dil (D when <= 0);
 *   dg_dtype       element type of dfl and dil (NAJU_DTYPE_*), or -1 for
 *                  naju_scan_bwd's (the gates' type, or float32 with
 *                  NAJU_FLAG_OUT_F32);
 *   dfl_sum, dil_sum  [D] float32: dfl and dil summed over batch and time,
 *                  from the float32 values before any rounding to dg_dtype
 *                  (a bias added to the gate logits gets this gradient);
 *                  NULL: not formed.
 * Everything but the defaults is served on the matrix-core path
 * (9 <= N <= 64) only, with strides that are multiples of 4 and pointers
 * aligned to four elements; otherwise NAJU_ERR_UNSUPPORTED. */
typedef struct naju_scan_bwd_layout {
  int64_t bc_ld;
  int64_t dbc_ld;
  int64_t dg_ld;
  int32_t dg_dtype;
  int32_t reserved;
  float* dfl_sum;
  float* dil_sum;
} naju_scan_bwd_layout;

#define NAJU_SCAN_BWD_LAYOUT_INIT {0, 0, 0, -1, 0, NULL, NULL}

/* naju_scan_bwd with the output layout above (layout NULL: naju_scan_bwd
 * itself). The mixer's gate logits are a projection slice plus a
 * convolution plus a bias: their gradient goes into the projection's
 * gradient buffer in its 16-bit type (row stride of that buffer), and the
 * bias gradient comes from the float32 sums, so neither needs a pass of its
 * own. No reference counterpart (the reference's backends return contiguous
 * gradients in the inputs' types). */
int naju_scan_bwd_ex(const void* u, const void* f_logit, const void* i_logit, const void* B, const void* C,
                     const float* D_skip, const float* ckpt, const void* dy, void* du, void* dfl, void* dil,
                     void* dB, void* dC, float* dD, float* dh0, int64_t batch, int64_t T, int64_t D, int64_t N,
                     int x_dtype, int gate_dtype, int bc_dtype, int flags, const naju_scan_bwd_layout* layout,
                     void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free forward: naju_scan_fwd with the caller's workspace
 * replaced by a static device array of NAJU_NOALLOC_SCRATCH_BYTES per GPU
 * (each GPU the library runs on holds it until the process ends; its
 * address is looked up once per device, at the first call there). No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory -- code under HIP-graph capture, tight serving loops,
 * harnesses that forbid hipMalloc. It calls no hipMalloc / hipFree. The
 * caller still passes every input and output (ckpt and hT optional, as in
 * naju_scan_fwd). Shapes whose forward needs more scratch than the maximum
 * (at N = 1 about 0.375 bytes per element of batch*T*D, i.e. up to about
 * 83 M elements; N > 1 uses fewer time segments to fit) are rejected with
 * NAJU_ERR_WORKSPACE. Every call on one GPU shares that GPU's array: calls
 * that overlap in time on one GPU (different streams, threads) race. */
#define NAJU_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int naju_scan_fwd_noalloc(const void* u, const void* f_logit,
                          const void* i_logit, const void* B, const void* C,
                          const float* D_skip, const float* h0, void* y,
                          float* ckpt, float* hT, int64_t batch, int64_t T,
                          int64_t D, int64_t N, int x_dtype, int gate_dtype,
                          int bc_dtype, int flags, void* stream);

/* Reads the workspace's device-side status word (synchronises `stream`)
 * and, when it is nonzero, clears it and rewinds the workspace's ticket
 * counters, so the workspace is usable again.
 * 0 = healthy; 1 = a carry hand-off between workgroups exceeded its
 * bounded wait and the affected outputs were set to NaN; 2 = a ticket
 * counter held a value out of range (a workspace that was not zero-filled
 * before first use), and the affected workgroups wrote NaN outputs. No
 * counterpart in the reference (its kernels have no cross-workgroup waits).
 * Only the N = 1 kernels hand carries between workgroups, so only N = 1
 * calls can set a nonzero status. Test hook: the environment variable
 * NAJU_DEBUG_SPIN_LIMIT, read at every call, lowers the bound on a hand-off's
 * idle polling rounds (default about a second of polling); 0 makes every
 * hand-off give up at once, so status 1 can be produced while every kernel
 * exits normally. */
int naju_scan_workspace_status(const void* workspace, void* stream,
                               uint32_t* status);

/* naju_scan_workspace_status for the static scratch of
 * naju_scan_fwd_noalloc on the current HIP device (synchronises `stream`):
 * reads its status word and, when it is nonzero, clears it and rewinds the
 * scratch's ticket counters, so later naju_scan_fwd_noalloc calls on this
 * device start clean. Status 0 before the first naju_scan_fwd_noalloc call
 * on the device. No counterpart in the reference; it is the recovery path
 * of callers that cannot allocate (they never hold a workspace pointer). */
int naju_scan_noalloc_status(void* stream, uint32_t* status);

#ifdef __cplusplus
}
#endif

#endif /* NAJU_SCAN_H */
