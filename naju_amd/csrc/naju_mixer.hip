// naju_mixer.hip -- depthwise causal convolutions of the Naju mixer on
// MI355X (gfx950), behind the C ABI of include/naju_mixer.h.
//
//   y[b,t,c] = act( add[b,t,c] + bias[c] + sum_{j<K} w[c,j] x[b, t-(K-1)+j, c] )
//
// The reference runs these as nn.Conv1d(groups=C, padding=K-1) plus a slice
// on a transposed copy (/root/reference/naju/mixer.py:108-109, 115), which
// on this stack is an im2col-style library convolution. Here one thread owns
// one channel of one batch row over a block of kRows timesteps, walks them in
// order and keeps the last K-1 inputs in registers, so every element of x is
// read once per block (plus a K-1 row halo) and the [B, T, C] layout is used
// as it is. The backward walks its block in reverse with a window of the
// next K-1 output gradients, recomputing the pre-activation from x when the
// activation is SiLU, and writes per-block partial sums of dw and dbias that
// a second kernel folds in block order (deterministic).
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "naju_mixer.h"
#include "naju_scan.h"

namespace {

typedef __bf16 bf16_t;
typedef _Float16 f16_t;

constexpr int kMaxK = 8;
constexpr int kRows = 64;     // timesteps per block
constexpr int kThreads = 256; // channels per block

__device__ __forceinline__ float ldv(const void* p, int dt, int64_t i) {
  if (dt == NAJU_DTYPE_F32) return ((const float*)p)[i];
  if (dt == NAJU_DTYPE_BF16) return (float)((const bf16_t*)p)[i];
  return (float)((const f16_t*)p)[i];
}
__device__ __forceinline__ void stv(void* p, int dt, int64_t i, float v) {
  if (dt == NAJU_DTYPE_F32)
    ((float*)p)[i] = v;
  else if (dt == NAJU_DTYPE_BF16)
    ((bf16_t*)p)[i] = (bf16_t)v;
  else
    ((f16_t*)p)[i] = (f16_t)v;
}

__device__ __forceinline__ float silu(float z) { return z / (1.f + __expf(-z)); }

// grid: (ceil(C / kThreads), ceil(T / kRows), batch)
template <int K, bool SILU>
__global__ __launch_bounds__(kThreads) void dwconv_fwd_kernel(const void* x, int64_t ldx, const float* w,
                                                             const float* bias, const void* add, void* y, int64_t T,
                                                             int64_t C, int x_dt, int add_dt, int y_dt) {
  const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (c >= C) return;
  const int64_t b = blockIdx.z;
  const int64_t t0 = (int64_t)blockIdx.y * kRows;
  const int64_t t1 = t0 + kRows < T ? t0 + kRows : T;
  float wr[K];
#pragma unroll
  for (int j = 0; j < K; ++j) wr[j] = w[c * K + j];
  const float bc = bias ? bias[c] : 0.f;
  const int64_t base = b * T * C + c, xbase = b * T * ldx + c;
  // window: xw[j] = x[t - (K-1) + j] for j < K-1, entering row t0
  float xw[K > 1 ? K - 1 : 1];
#pragma unroll
  for (int j = 0; j < K - 1; ++j) {
    const int64_t t = t0 - (K - 1) + j;
    xw[j] = t >= 0 ? ldv(x, x_dt, xbase + t * ldx) : 0.f;
  }
#pragma unroll 4
  for (int64_t t = t0; t < t1; ++t) {
    const float xt = ldv(x, x_dt, xbase + t * ldx);
    float acc = fmaf(wr[K - 1], xt, bc);
#pragma unroll
    for (int j = 0; j < K - 1; ++j) acc = fmaf(wr[j], xw[j], acc);
#pragma unroll
    for (int j = 0; j + 1 < K - 1; ++j) xw[j] = xw[j + 1];
    if (K > 1) xw[K - 2] = xt;
    if (add) acc += ldv(add, add_dt, base + t * C);
    stv(y, y_dt, base + t * C, SILU ? silu(acc) : acc);
  }
}

// grid as the forward. part: [batch * ceil(T / kRows)][C][K + 1] (dw, dbias).
template <int K, bool SILU>
__global__ __launch_bounds__(kThreads) void dwconv_bwd_kernel(const void* x, int64_t ldx, const float* w,
                                                             const float* bias, const void* dy, void* dx, float* part,
                                                             int64_t T, int64_t C, int x_dt, int dy_dt, int dx_dt) {
  const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (c >= C) return;
  const int64_t b = blockIdx.z;
  const int64_t t0 = (int64_t)blockIdx.y * kRows;
  const int64_t t1 = t0 + kRows < T ? t0 + kRows : T;
  float wr[K];
#pragma unroll
  for (int j = 0; j < K; ++j) wr[j] = w[c * K + j];
  const float bc = bias ? bias[c] : 0.f;
  const int64_t base = b * T * C + c, xbase = b * T * ldx + c;
  // Walk t downwards from the last row whose output gradient reaches this
  // block (t1 - 1 + K - 1) to t0. Windows entering row t:
  //   gz[j] = dz[t + 1 + j]          (j < K-1; 0 past T)
  //   xv[j] = x[t - (K-1) + j]       (j < K;   0 before 0)
  const int64_t tstart = (t1 - 1 + (K - 1)) < (T - 1) ? (t1 - 1 + (K - 1)) : (T - 1);
  float gz[K > 1 ? K - 1 : 1], xv[K];
#pragma unroll
  for (int j = 0; j < K - 1; ++j) gz[j] = 0.f;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const int64_t t = tstart - (K - 1) + j;
    xv[j] = t >= 0 ? ldv(x, x_dt, xbase + t * ldx) : 0.f;
  }
  float dw[K], db = 0.f;
#pragma unroll
  for (int j = 0; j < K; ++j) dw[j] = 0.f;
#pragma unroll 2
  for (int64_t t = tstart; t >= t0; --t) {
    float dz = ldv(dy, dy_dt, base + t * C);
    if (SILU) {
      float z = bc;
#pragma unroll
      for (int j = 0; j < K; ++j) z = fmaf(wr[j], xv[j], z);
      const float sg = 1.f / (1.f + __expf(-z));
      dz *= sg * fmaf(z, 1.f - sg, 1.f);  // d silu / dz = s (1 + z (1 - s))
    }
    if (t < t1) {
      // dx[t] = sum_j w[j] dz[t + (K-1) - j]
      float g = wr[K - 1] * dz;
#pragma unroll
      for (int j = 0; j < K - 1; ++j) g = fmaf(wr[j], gz[K - 2 - j], g);
      if (dx) stv(dx, dx_dt, base + t * C, g);
#pragma unroll
      for (int j = 0; j < K; ++j) dw[j] = fmaf(dz, xv[j], dw[j]);
      db += dz;
    }
    // shift the windows down by one row
#pragma unroll
    for (int j = K - 2; j > 0; --j) gz[j] = gz[j - 1];
    if (K > 1) gz[0] = dz;
#pragma unroll
    for (int j = K - 1; j > 0; --j) xv[j] = xv[j - 1];
    const int64_t tn = t - K;  // x[(t-1) - (K-1)]
    xv[0] = (tn >= 0 && t - 1 >= t0) ? ldv(x, x_dt, xbase + tn * ldx) : 0.f;
  }
  if (part) {
    float* pp = part + (((int64_t)b * gridDim.y + blockIdx.y) * C + c) * (K + 1);
#pragma unroll
    for (int j = 0; j < K; ++j) pp[j] = dw[j];
    pp[K] = db;
  }
}

// dw[c, j] / dbias[c] = sum over the partials of all blocks, in block order.
__global__ void dwconv_fold_kernel(const float* part, int64_t nblk, int64_t C, int K, float* dw, float* dbias) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // c * (K+1) + j
  if (i >= C * (K + 1)) return;
  float s = 0.f;
#pragma unroll 8
  for (int64_t q = 0; q < nblk; ++q) s += part[q * C * (K + 1) + i];
  const int64_t c = i / (K + 1), j = i - c * (K + 1);
  if (j < K) {
    if (dw) dw[c * K + j] = s;
  } else if (dbias) {
    dbias[c] = s;
  }
}

// ---------------------------------------------------------- readout epilogue
//
// y = (cx * scale + Dv * h) * SiLU(z), one thread per channel over a block of
// kRows rows (grid: channel blocks x row blocks). The backward writes dcx,
// dh, dz and a per-row-block partial of dD = sum_r dy * SiLU(z) * h, folded
// in block order by dwconv_fold_kernel (K = 0).
__global__ __launch_bounds__(kThreads) void readout_fwd_kernel(const void* cx, const void* h, const void* z,
                                                              int64_t z_ld, const float* Dv, float scale, void* y,
                                                              int64_t n_rows, int64_t C, int cx_dt, int h_dt,
                                                              int z_dt, int y_dt) {
  const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (c >= C) return;
  const int64_t r0 = (int64_t)blockIdx.y * kRows;
  const int64_t r1 = r0 + kRows < n_rows ? r0 + kRows : n_rows;
  const float dv = Dv[c];
#pragma unroll 4
  for (int64_t r = r0; r < r1; ++r) {
    const int64_t o = r * C + c;
    const float zz = ldv(z, z_dt, r * z_ld + c);
    const float a = fmaf(ldv(cx, cx_dt, o), scale, dv * ldv(h, h_dt, o));
    stv(y, y_dt, o, a * silu(zz));
  }
}

__global__ __launch_bounds__(kThreads) void readout_bwd_kernel(const void* cx, const void* h, const void* z,
                                                              int64_t z_ld, const float* Dv, float scale,
                                                              const void* dy, void* dcx, void* dh, void* dz,
                                                              float* part, int64_t n_rows, int64_t C, int cx_dt,
                                                              int h_dt, int z_dt, int dy_dt, int dcx_dt, int dh_dt,
                                                              int dz_dt) {
  const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (c >= C) return;
  const int64_t r0 = (int64_t)blockIdx.y * kRows;
  const int64_t r1 = r0 + kRows < n_rows ? r0 + kRows : n_rows;
  const float dv = Dv[c];
  float dd = 0.f;
#pragma unroll 4
  for (int64_t r = r0; r < r1; ++r) {
    const int64_t o = r * C + c;
    const float zz = ldv(z, z_dt, r * z_ld + c);
    const float hh = ldv(h, h_dt, o);
    const float g = ldv(dy, dy_dt, o);
    const float sg = 1.f / (1.f + __expf(-zz));
    const float gs = g * (zz * sg);  // dy * SiLU(z)
    if (dcx) stv(dcx, dcx_dt, o, gs * scale);
    if (dh) stv(dh, dh_dt, o, gs * dv);
    dd = fmaf(gs, hh, dd);
    if (dz) {
      const float a = fmaf(ldv(cx, cx_dt, o), scale, dv * hh);
      stv(dz, dz_dt, o, g * a * sg * fmaf(zz, 1.f - sg, 1.f));
    }
  }
  if (part) part[(int64_t)blockIdx.y * C + c] = dd;
}

thread_local char g_err[256] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

bool dt_ok(int dt) { return dt == NAJU_DTYPE_F32 || dt == NAJU_DTYPE_BF16 || dt == NAJU_DTYPE_F16; }

int check(int64_t batch, int64_t T, int64_t C, int K, int act, int64_t x_ld) {
  if (batch < 0 || T < 0 || C < 0) return fail(NAJU_ERR_INVALID, "negative shape");
  if (x_ld < C) return fail(NAJU_ERR_INVALID, "x_ld (%lld) must be >= C (%lld)", (long long)x_ld, (long long)C);
  if (K < 1 || K > kMaxK) return fail(NAJU_ERR_UNSUPPORTED, "kernel size K must be in [1, %d], got %d", kMaxK, K);
  if (act != 0 && act != 1) return fail(NAJU_ERR_INVALID, "act must be 0 (identity) or 1 (SiLU)");
  if (batch > 65535 || (T + kRows - 1) / kRows > 65535 || C > (1ll << 30))
    return fail(NAJU_ERR_UNSUPPORTED, "shape too large (batch <= 65535, T <= %d)", 65535 * kRows);
  return NAJU_OK;
}

typedef void (*fwd_t)(const void*, int64_t, const float*, const float*, const void*, void*, int64_t, int64_t, int,
                      int, int);
typedef void (*bwd_t)(const void*, int64_t, const float*, const float*, const void*, void*, float*, int64_t, int64_t,
                      int, int, int);

template <int K>
fwd_t pick_fwd_k(bool silu) {
  return silu ? dwconv_fwd_kernel<K, true> : dwconv_fwd_kernel<K, false>;
}
fwd_t pick_fwd(int K, bool silu) {
  switch (K) {
    case 1: return pick_fwd_k<1>(silu);
    case 2: return pick_fwd_k<2>(silu);
    case 3: return pick_fwd_k<3>(silu);
    case 4: return pick_fwd_k<4>(silu);
    case 5: return pick_fwd_k<5>(silu);
    case 6: return pick_fwd_k<6>(silu);
    case 7: return pick_fwd_k<7>(silu);
    default: return pick_fwd_k<8>(silu);
  }
}
template <int K>
bwd_t pick_bwd_k(bool silu) {
  return silu ? dwconv_bwd_kernel<K, true> : dwconv_bwd_kernel<K, false>;
}
bwd_t pick_bwd(int K, bool silu) {
  switch (K) {
    case 1: return pick_bwd_k<1>(silu);
    case 2: return pick_bwd_k<2>(silu);
    case 3: return pick_bwd_k<3>(silu);
    case 4: return pick_bwd_k<4>(silu);
    case 5: return pick_bwd_k<5>(silu);
    case 6: return pick_bwd_k<6>(silu);
    case 7: return pick_bwd_k<7>(silu);
    default: return pick_bwd_k<8>(silu);
  }
}

int64_t n_tblocks(int64_t T) { return (T + kRows - 1) / kRows; }

}  // namespace

extern "C" {

const char* naju_mixer_last_error(void) { return g_err; }

int naju_dwconv_fwd(const void* x, int64_t x_ld, const float* w, const float* bias, const void* add, void* y,
                    int64_t batch, int64_t T, int64_t C, int K, int act, int x_dtype, int add_dtype, int y_dtype,
                    void* stream) {
  g_err[0] = 0;
  int rc = check(batch, T, C, K, act, x_ld);
  if (rc) return rc;
  if (!dt_ok(x_dtype) || !dt_ok(y_dtype) || (add && !dt_ok(add_dtype)))
    return fail(NAJU_ERR_INVALID, "unknown dtype code");
  if (act == 1 && add) return fail(NAJU_ERR_UNSUPPORTED, "add must be NULL with act = SiLU");
  if (batch == 0 || T == 0 || C == 0) return NAJU_OK;
  if (!x || !w || !y) return fail(NAJU_ERR_INVALID, "null pointer (x, w and y are required)");
  const dim3 grid((unsigned)((C + kThreads - 1) / kThreads), (unsigned)n_tblocks(T), (unsigned)batch);
  hipLaunchKernelGGL(pick_fwd(K, act == 1), grid, dim3(kThreads), 0, (hipStream_t)stream, x, x_ld, w, bias, add, y,
                     T, C, x_dtype, add_dtype, y_dtype);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return NAJU_OK;
}

size_t naju_dwconv_workspace_bytes(int64_t batch, int64_t T, int64_t C, int K) {
  if (check(batch, T, C, K, 0, C) != NAJU_OK) return 0;
  return (size_t)batch * n_tblocks(T) * C * (K + 1) * sizeof(float) + 256;
}

int naju_dwconv_bwd(const void* x, int64_t x_ld, const float* w, const float* bias, const void* dy, void* dx,
                    float* dw, float* dbias, int64_t batch, int64_t T, int64_t C, int K, int act, int x_dtype,
                    int dy_dtype, int dx_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  int rc = check(batch, T, C, K, act, x_ld);
  if (rc) return rc;
  if (!dt_ok(x_dtype) || !dt_ok(dy_dtype) || !dt_ok(dx_dtype)) return fail(NAJU_ERR_INVALID, "unknown dtype code");
  hipStream_t st = (hipStream_t)stream;
  if (C == 0) return NAJU_OK;
  if (batch == 0 || T == 0) {
    // empty sums: the fold over zero blocks writes the zeros (a kernel, not a
    // memset, so that the call can be captured into a graph)
    if (dw || dbias) {
      const int64_t n = C * (K + 1);
      hipLaunchKernelGGL(dwconv_fold_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, nullptr,
                         (int64_t)0, C, K, dw, dbias);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
    }
    return NAJU_OK;
  }
  if (!x || !w || !dy) return fail(NAJU_ERR_INVALID, "null pointer (x, w and dy are required)");
  const bool sums = dw || dbias;
  const size_t need = naju_dwconv_workspace_bytes(batch, T, C, K);
  if (sums && (!workspace || workspace_bytes < need))
    return fail(NAJU_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need,
                workspace ? workspace_bytes : (size_t)0);
  const dim3 grid((unsigned)((C + kThreads - 1) / kThreads), (unsigned)n_tblocks(T), (unsigned)batch);
  float* part = sums ? (float*)workspace : nullptr;
  hipLaunchKernelGGL(pick_bwd(K, act == 1), grid, dim3(kThreads), 0, st, x, x_ld, w, bias, dy, dx, part, T, C,
                     x_dtype, dy_dtype, dx_dtype);
  if (sums) {
    const int64_t n = C * (K + 1);
    hipLaunchKernelGGL(dwconv_fold_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, part,
                       batch * n_tblocks(T), C, K, dw, dbias);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return NAJU_OK;
}

int naju_readout_fwd(const void* cx, const void* h, const void* z, int64_t z_ld, const float* Dv, float scale,
                     void* y, int64_t n_rows, int64_t C, int cx_dtype, int h_dtype, int z_dtype, int y_dtype,
                     void* stream) {
  g_err[0] = 0;
  if (n_rows < 0 || C < 0) return fail(NAJU_ERR_INVALID, "negative shape");
  if (z_ld < C) return fail(NAJU_ERR_INVALID, "z_ld (%lld) must be >= C (%lld)", (long long)z_ld, (long long)C);
  if (!dt_ok(cx_dtype) || !dt_ok(h_dtype) || !dt_ok(z_dtype) || !dt_ok(y_dtype))
    return fail(NAJU_ERR_INVALID, "unknown dtype code");
  if ((n_rows + kRows - 1) / kRows > 65535 || C > (1ll << 30))
    return fail(NAJU_ERR_UNSUPPORTED, "shape too large (at most %d rows)", 65535 * kRows);
  if (n_rows == 0 || C == 0) return NAJU_OK;
  if (!cx || !h || !z || !Dv || !y) return fail(NAJU_ERR_INVALID, "null pointer (cx, h, z, Dv and y are required)");
  const dim3 grid((unsigned)((C + kThreads - 1) / kThreads), (unsigned)((n_rows + kRows - 1) / kRows));
  hipLaunchKernelGGL(readout_fwd_kernel, grid, dim3(kThreads), 0, (hipStream_t)stream, cx, h, z, z_ld, Dv, scale, y,
                     n_rows, C, cx_dtype, h_dtype, z_dtype, y_dtype);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return NAJU_OK;
}

size_t naju_readout_workspace_bytes(int64_t n_rows, int64_t C) {
  if (n_rows < 0 || C < 0) return 0;
  return (size_t)((n_rows + kRows - 1) / kRows) * C * sizeof(float) + 256;
}

int naju_readout_bwd(const void* cx, const void* h, const void* z, int64_t z_ld, const float* Dv, float scale,
                     const void* dy, void* dcx, void* dh, void* dz, float* dD, int64_t n_rows, int64_t C,
                     int cx_dtype, int h_dtype, int z_dtype, int dy_dtype, int dcx_dtype, int dh_dtype, int dz_dtype,
                     void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  if (n_rows < 0 || C < 0) return fail(NAJU_ERR_INVALID, "negative shape");
  if (z_ld < C) return fail(NAJU_ERR_INVALID, "z_ld (%lld) must be >= C (%lld)", (long long)z_ld, (long long)C);
  if (!dt_ok(cx_dtype) || !dt_ok(h_dtype) || !dt_ok(z_dtype) || !dt_ok(dy_dtype) || !dt_ok(dcx_dtype) ||
      !dt_ok(dh_dtype) || !dt_ok(dz_dtype))
    return fail(NAJU_ERR_INVALID, "unknown dtype code");
  if ((n_rows + kRows - 1) / kRows > 65535 || C > (1ll << 30))
    return fail(NAJU_ERR_UNSUPPORTED, "shape too large (at most %d rows)", 65535 * kRows);
  hipStream_t st = (hipStream_t)stream;
  if (C == 0) return NAJU_OK;
  const int64_t nblk = (n_rows + kRows - 1) / kRows;
  if (n_rows == 0) {
    if (dD) {
      hipLaunchKernelGGL(dwconv_fold_kernel, dim3((unsigned)((C + 255) / 256)), dim3(256), 0, st, nullptr,
                         (int64_t)0, C, 0, nullptr, dD);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
    }
    return NAJU_OK;
  }
  if (!h || !z || !Dv || !dy) return fail(NAJU_ERR_INVALID, "null pointer (h, z, Dv and dy are required)");
  if (dz && !cx) return fail(NAJU_ERR_INVALID, "cx is required for dz");
  const size_t need = naju_readout_workspace_bytes(n_rows, C);
  if (dD && (!workspace || workspace_bytes < need))
    return fail(NAJU_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need,
                workspace ? workspace_bytes : (size_t)0);
  float* part = dD ? (float*)workspace : nullptr;
  const dim3 grid((unsigned)((C + kThreads - 1) / kThreads), (unsigned)nblk);
  hipLaunchKernelGGL(readout_bwd_kernel, grid, dim3(kThreads), 0, st, cx, h, z, z_ld, Dv, scale, dy, dcx, dh, dz,
                     part, n_rows, C, cx_dtype, h_dtype, z_dtype, dy_dtype, dcx_dtype, dh_dtype, dz_dtype);
  if (dD)
    hipLaunchKernelGGL(dwconv_fold_kernel, dim3((unsigned)((C + 255) / 256)), dim3(256), 0, st, part, nblk, C, 0,
                       nullptr, dD);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return NAJU_OK;
}

}  // extern "C"
