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
// a second kernel folds in a fixed order (deterministic). The K = 4 kernels
// (the mixer's) load every row a thread needs before using the first, so a
// wave waits for memory once per block rather than once per row.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <initializer_list>
#include <type_traits>

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

// sigmoid with the hardware reciprocal (v_rcp_f32, 1 ulp) in place of an
// IEEE divide, whose expansion made the SiLU kernels instruction-bound
__device__ __forceinline__ float sigmoid_f(float z) { return __builtin_amdgcn_rcpf(1.f + __expf(-z)); }
__device__ __forceinline__ float silu(float z) { return z * sigmoid_f(z); }

// grid: (ceil(C / kThreads), ceil(T / kRows), batch)
template <int K, bool SILU>
__global__ __launch_bounds__(kThreads) void dwconv_fwd_kernel(const void* x, int64_t ldx, const float* w,
                                                             const float* bias, const void* add, int64_t ld_add,
                                                             void* y, int64_t T, int64_t C, int x_dt, int add_dt,
                                                             int y_dt) {
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
    if constexpr (K > 1) xw[K - 2] = xt;
    if (add) acc += ldv(add, add_dt, (b * T + t) * ld_add + c);
    stv(y, y_dt, base + t * C, SILU ? silu(acc) : acc);
  }
}

// grid as the forward. part: [batch * ceil(T / kRows)][C][K + 1] (dw, dbias).
template <int K, bool SILU>
__global__ __launch_bounds__(kThreads) void dwconv_bwd_kernel(const void* x, int64_t ldx, const float* w,
                                                             const float* bias, const void* dy, void* dx,
                                                             int64_t ld_dx, void* dadd, int64_t ld_dadd, float* part,
                                                             int64_t T, int64_t C, int x_dt, int dy_dt, int dx_dt,
                                                             int dadd_dt, int acc) {
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
      const float sg = sigmoid_f(z);
      dz *= sg * fmaf(z, 1.f - sg, 1.f);  // d silu / dz = s (1 + z (1 - s))
    }
    if (t < t1) {
      // dx[t] = sum_j w[j] dz[t + (K-1) - j]
      float g = wr[K - 1] * dz;
#pragma unroll
      for (int j = 0; j < K - 1; ++j) g = fmaf(wr[j], gz[K - 2 - j], g);
      if (dx) {
        const int64_t o = (b * T + t) * ld_dx + c;
        stv(dx, dx_dt, o, acc ? ldv(dx, dx_dt, o) + g : g);
      }
      if (dadd) stv(dadd, dadd_dt, (b * T + t) * ld_dadd + c, dz);
#pragma unroll
      for (int j = 0; j < K; ++j) dw[j] = fmaf(dz, xv[j], dw[j]);
      db += dz;
    }
    // shift the windows down by one row
#pragma unroll
    for (int j = K - 2; j > 0; --j) gz[j] = gz[j - 1];
    if constexpr (K > 1) gz[0] = dz;
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

// ---------------------------------------------------------- readout epilogue
//
// y = (cx * scale + Dv * h) * SiLU(z), one thread per channel over a block of
// kRows rows (grid: channel blocks x row blocks). The backward writes dcx,
// dh, dz and a per-row-block partial of dD = sum_r dy * SiLU(z) * h, folded
// in a fixed order by fold_cols_kernel (K = 0).
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
                                                              int64_t dz_ld, float* part, int64_t n_rows, int64_t C,
                                                              int cx_dt,
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
    const float sg = sigmoid_f(zz);
    const float gs = g * (zz * sg);  // dy * SiLU(z)
    if (dcx) stv(dcx, dcx_dt, o, gs * scale);
    if (dh) stv(dh, dh_dt, o, gs * dv);
    dd = fmaf(gs, hh, dd);
    if (dz) {
      const float a = fmaf(ldv(cx, cx_dt, o), scale, dv * hh);
      stv(dz, dz_dt, r * dz_ld + c, g * a * sg * fmaf(zz, 1.f - sg, 1.f));
    }
  }
  if (part) part[(int64_t)blockIdx.y * C + c] = dd;
}

// ------------------------------------------------ vector fast paths (K = 4)
//
// The same operations on several channels per thread with 8- or 16-byte
// accesses (the readout: kRV channels, kVRows or kVRowsR rows per thread,
// one wave per block; the convolutions: kCV channels, below). Used when C and the row
// strides are multiples of 8 and the pointers 16-byte aligned; the scalar
// kernels above serve every other case.
constexpr int kVec = 8;
constexpr int kVRows = 16;
constexpr int kVRowsB = 32;  // rows per block of the vector conv backward (one dw / dbias partial row each)

template <typename T>
__device__ __forceinline__ void ld8(const T* p, float (&o)[kVec]) {
  typedef T v8 __attribute__((ext_vector_type(8)));
  const v8 v = *(const v8*)p;
#pragma unroll
  for (int j = 0; j < kVec; ++j) o[j] = (float)v[j];
}
template <typename T>
__device__ __forceinline__ void st8(T* p, const float (&x)[kVec]) {
  typedef T v8 __attribute__((ext_vector_type(8)));
  v8 v;
#pragma unroll
  for (int j = 0; j < kVec; ++j) v[j] = (T)x[j];
  *(v8*)p = v;
}
__device__ __forceinline__ void ld8f(const float* p, float (&o)[kVec]) {
  const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
  o[0] = a.x, o[1] = a.y, o[2] = a.z, o[3] = a.w, o[4] = b.x, o[5] = b.y, o[6] = b.z, o[7] = b.w;
}

// The K = 4 vector kernels: kCV channels per thread (8- or 16-byte
// accesses), every row a thread needs loaded before the first is used, so a
// wave waits for memory once per block instead of once per row.
constexpr int kCV = 4;    // channels per thread
constexpr int kCRF = 16;  // forward: rows per thread (one wave per workgroup)
constexpr int kCRB = 8;  // backward: rows per wave
constexpr int kCWB = 4;  // backward: waves per workgroup, one block of kCWB * kCRB rows
static_assert(kCWB * kCRB == kVRowsB, "one partial row per kVRowsB rows");

template <typename T>
using cvec_t = T __attribute__((ext_vector_type(kCV)));

template <typename T, int V>
using pvec_t = T __attribute__((ext_vector_type(V)));

#ifndef NAJU_CONV_BWD_V
#define NAJU_CONV_BWD_V 2
#endif
constexpr int kBV = NAJU_CONV_BWD_V;  // single convolution backward: channels per thread
#ifndef NAJU_CONV_FWD_V
#define NAJU_CONV_FWD_V 2
#endif
constexpr int kFV4 = NAJU_CONV_FWD_V;  // forward kernels (single and pair): channels per thread

template <typename T>
__device__ __forceinline__ cvec_t<T> ldc(const T* p) {
  return *(const cvec_t<T>*)p;
}
template <typename T, int V>
__device__ __forceinline__ void stc(T* p, const float (&x)[V]) {
  typedef T v_t __attribute__((ext_vector_type(V)));
  v_t v;
#pragma unroll
  for (int j = 0; j < V; ++j) v[j] = (T)x[j];
  *(v_t*)p = v;
}

// grid: (ceil(C / (64 * kCV)), ceil(T / kCRF), batch), 64 threads: rows
// t0 .. t0 + kCRF - 1 of kCV channels; x rows t0-3 .. and the add rows are
// loaded first (rows outside [0, T) from a clamped row, then zeroed or
// skipped).
template <typename TX, typename TY, bool SILU, bool ADD>
__global__ __launch_bounds__(64) void dwconv4_fwd_vec(const TX* __restrict__ x, int64_t ldx,
                                                      const float* __restrict__ w, const float* __restrict__ bias,
                                                      const TX* __restrict__ add, int64_t ld_add,
                                                      TY* __restrict__ y, int64_t T, int64_t C) {
  constexpr int K = 4, V = kFV4, R = kCRF;
  const int64_t c0 = ((int64_t)blockIdx.x * 64 + threadIdx.x) * V;
  if (c0 >= C) return;
  const int64_t b = blockIdx.z;
  const int64_t t0 = (int64_t)blockIdx.y * R;
  const TX* xb = x + b * T * ldx + c0;
  pvec_t<TX, V> xr[R + K - 1], ar[R];
#pragma unroll
  for (int i = 0; i < R + K - 1; ++i) {
    int64_t t = t0 - (K - 1) + i;
    t = t < 0 ? 0 : (t < T ? t : T - 1);
    xr[i] = *(const pvec_t<TX, V>*)(xb + t * ldx);
  }
  if (ADD) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t t = t0 + r < T ? t0 + r : T - 1;
      ar[r] = *(const pvec_t<TX, V>*)(add + (b * T + t) * ld_add + c0);
    }
  }
  float wr[V][K], bc[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const float4 q = *(const float4*)(w + (c0 + j) * K);
    wr[j][0] = q.x, wr[j][1] = q.y, wr[j][2] = q.z, wr[j][3] = q.w;
    bc[j] = bias ? bias[c0 + j] : 0.f;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t t = t0 + r;
    if (t >= T) break;
    float acc[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      float a = fmaf(wr[j][K - 1], (float)xr[r + K - 1][j], bc[j]);
#pragma unroll
      for (int k = 0; k < K - 1; ++k)
        if (t - (K - 1) + k >= 0) a = fmaf(wr[j][k], (float)xr[r + k][j], a);
      if (ADD) a += (float)ar[r][j];
      acc[j] = SILU ? silu(a) : a;
    }
    stc(y + (b * T + t) * C + c0, acc);
  }
}

// Backward of dwconv4_fwd_vec without add; part [batch * nTB][C][K+1].
// grid: (ceil(C / (64 * kCV)), ceil(T / (kCWB * kCRB)), batch), kCWB waves:
// wave w takes rows tw = t0 + w * kCRB .. + kCRB - 1 and loads dy rows
// tw .. tw + kCRB + 2, x rows tw - 3 .. (tw + kCRB + 2 with SiLU, whose
// derivative needs the pre-activation of those rows) and, when adding, the
// dx rows, all before the first is used. The waves' dw / dbias sums are
// added in wave order through LDS into the block's partial row.
template <typename TX, typename TDY, bool SILU>
__global__ __launch_bounds__(64 * kCWB) void dwconv4_bwd_vec(const TX* __restrict__ x, int64_t ldx,
                                                             const float* __restrict__ w,
                                                             const float* __restrict__ bias,
                                                             const TDY* __restrict__ dy, TX* __restrict__ dx,
                                                             int64_t ld_dx, TX* __restrict__ dadd, int64_t ld_dadd,
                                                             float* __restrict__ part, int64_t T, int64_t C, int acc) {
  constexpr int K = 4, V = kBV, R = kCRB;
  constexpr int NZ = R + K - 1;                 // dz rows tw .. tw + R + 2
  constexpr int NX = SILU ? R + 2 * (K - 1) : R + K - 1;  // x rows tw - 3 ..
  __shared__ float s_red[kCWB][(K + 1) * V][64];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t c0 = ((int64_t)blockIdx.x * 64 + lane) * V;
  const bool cok = c0 < C;
  const int64_t cc = cok ? c0 : 0;  // in-bounds channel for the loads of idle lanes
  const int64_t b = blockIdx.z;
  const int64_t tw = (int64_t)blockIdx.y * (kCWB * R) + wv * R;
  const TX* xb = x + b * T * ldx + cc;
  pvec_t<TDY, V> gr[NZ];
  pvec_t<TX, V> xr[NX], dr[R];
#pragma unroll
  for (int i = 0; i < NZ; ++i) {
    const int64_t t = tw + i < T ? tw + i : T - 1;
    gr[i] = *(const pvec_t<TDY, V>*)(dy + (b * T + t) * C + cc);
  }
#pragma unroll
  for (int i = 0; i < NX; ++i) {
    int64_t t = tw - (K - 1) + i;
    t = t < 0 ? 0 : (t < T ? t : T - 1);
    xr[i] = *(const pvec_t<TX, V>*)(xb + t * ldx);
  }
  if (dx && acc) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t t = tw + r < T ? tw + r : T - 1;
      dr[r] = *(const pvec_t<TX, V>*)(dx + (b * T + t) * ld_dx + cc);
    }
  }
  float wr[V][K], bc[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const float4 q = *(const float4*)(w + (cc + j) * K);
    wr[j][0] = q.x, wr[j][1] = q.y, wr[j][2] = q.z, wr[j][3] = q.w;
    bc[j] = bias ? bias[cc + j] : 0.f;
  }
  // x row i as floats, zero outside [0, T)
  auto xv = [&](int i, int j) -> float {
    const int64_t t = tw - (K - 1) + i;
    return (t >= 0 && t < T) ? (float)xr[i][j] : 0.f;
  };
  // dz of rows tw + i (zero at and beyond T)
  float dz[NZ][V];
#pragma unroll
  for (int i = 0; i < NZ; ++i) {
    const bool tv = tw + i < T;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      float g = tv ? (float)gr[i][j] : 0.f;
      if (SILU) {
        float z = bc[j];
#pragma unroll
        for (int k = 0; k < K; ++k) z = fmaf(wr[j][k], xv(i + k, j), z);
        const float sg = sigmoid_f(z);
        g *= sg * fmaf(z, 1.f - sg, 1.f);
      }
      dz[i][j] = g;
    }
  }
  float dw[V][K], db[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    db[j] = 0.f;
#pragma unroll
    for (int k = 0; k < K; ++k) dw[j][k] = 0.f;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t t = tw + r;
    if (t >= T) break;
    float g[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      float a = wr[j][K - 1] * dz[r][j];
#pragma unroll
      for (int k = 0; k < K - 1; ++k) a = fmaf(wr[j][k], dz[r + K - 1 - k][j], a);
      g[j] = a;
#pragma unroll
      for (int k = 0; k < K; ++k) dw[j][k] = fmaf(dz[r][j], xv(r + k, j), dw[j][k]);
      db[j] += dz[r][j];
    }
    if (cok) {
      if (dx) {
        if (acc) {
#pragma unroll
          for (int j = 0; j < V; ++j) g[j] += (float)dr[r][j];
        }
        stc(dx + (b * T + t) * ld_dx + c0, g);
      }
      if (!SILU && dadd) stc(dadd + (b * T + t) * ld_dadd + c0, dz[r]);
    }
  }
  if (part) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
#pragma unroll
      for (int k = 0; k < K; ++k) s_red[wv][j * (K + 1) + k][lane] = dw[j][k];
      s_red[wv][j * (K + 1) + K][lane] = db[j];
    }
    __syncthreads();
    // wave w sums entries e = w, w + kCWB, ... over the waves in wave order
    float* pp = part + (((int64_t)b * gridDim.y + blockIdx.y) * C + c0) * (K + 1);
    for (int e = wv; e < (K + 1) * V; e += kCWB) {
      float s = 0.f;
#pragma unroll
      for (int u = 0; u < kCWB; ++u) s += s_red[u][e][lane];
      if (cok) pp[e] = s;
    }
  }
}

// ---- the two gate convolutions of a mixer over one input (K = 4, add, no
// activation): y0 = add0 + b0 + conv(x, w0) and y1 = add1 + b1 + conv(x, w1)
// in one pass, x read once. The forward takes the layout of
// dwconv4_fwd_vec; the backward that of dwconv4_bwd_vec with kPW waves of
// kPR rows, x's gradient conv0^T(dy0) + conv1^T(dy1) formed (and added to
// dx) with one rounding, and each weight's partial row in its own part
// array.
constexpr int kPR = 8;  // backward rows per wave
constexpr int kPW = 4;  // backward waves per workgroup
#ifndef NAJU_PAIR_BWD_V
#define NAJU_PAIR_BWD_V 2
#endif
constexpr int kPV = NAJU_PAIR_BWD_V;  // backward channels per thread

static_assert(kPW * kPR == kVRowsB, "one partial row per kVRowsB rows");

template <typename TX, typename TY>
__global__ __launch_bounds__(64) void dwconv4_pair_fwd_vec(const TX* __restrict__ x, int64_t ldx,
                                                           const float* __restrict__ w0,
                                                           const float* __restrict__ b0,
                                                           const float* __restrict__ w1,
                                                           const float* __restrict__ b1,
                                                           const TX* __restrict__ add0, const TX* __restrict__ add1,
                                                           int64_t ld_add, TY* __restrict__ y0, TY* __restrict__ y1,
                                                           int64_t T, int64_t C) {
  constexpr int K = 4, V = kFV4, R = kCRF;
  const int64_t c0 = ((int64_t)blockIdx.x * 64 + threadIdx.x) * V;
  if (c0 >= C) return;
  const int64_t b = blockIdx.z;
  const int64_t t0 = (int64_t)blockIdx.y * R;
  const TX* xb = x + b * T * ldx + c0;
  pvec_t<TX, V> xr[R + K - 1], a0[R], a1[R];
#pragma unroll
  for (int i = 0; i < R + K - 1; ++i) {
    int64_t t = t0 - (K - 1) + i;
    t = t < 0 ? 0 : (t < T ? t : T - 1);
    xr[i] = *(const pvec_t<TX, V>*)(xb + t * ldx);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t t = t0 + r < T ? t0 + r : T - 1;
    a0[r] = *(const pvec_t<TX, V>*)(add0 + (b * T + t) * ld_add + c0);
    a1[r] = *(const pvec_t<TX, V>*)(add1 + (b * T + t) * ld_add + c0);
  }
  float wr0[V][K], wr1[V][K], bc0[V], bc1[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const float4 q0 = *(const float4*)(w0 + (c0 + j) * K);
    const float4 q1 = *(const float4*)(w1 + (c0 + j) * K);
    wr0[j][0] = q0.x, wr0[j][1] = q0.y, wr0[j][2] = q0.z, wr0[j][3] = q0.w;
    wr1[j][0] = q1.x, wr1[j][1] = q1.y, wr1[j][2] = q1.z, wr1[j][3] = q1.w;
    bc0[j] = b0 ? b0[c0 + j] : 0.f;
    bc1[j] = b1 ? b1[c0 + j] : 0.f;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t t = t0 + r;
    if (t >= T) break;
    float o0[V], o1[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float xt = (float)xr[r + K - 1][j];
      float s0 = fmaf(wr0[j][K - 1], xt, bc0[j]), s1 = fmaf(wr1[j][K - 1], xt, bc1[j]);
#pragma unroll
      for (int k = 0; k < K - 1; ++k)
        if (t - (K - 1) + k >= 0) {
          const float xv = (float)xr[r + k][j];
          s0 = fmaf(wr0[j][k], xv, s0);
          s1 = fmaf(wr1[j][k], xv, s1);
        }
      o0[j] = s0 + (float)a0[r][j];
      o1[j] = s1 + (float)a1[r][j];
    }
    stc(y0 + (b * T + t) * C + c0, o0);
    stc(y1 + (b * T + t) * C + c0, o1);
  }
}

template <typename TX, typename TDY>
__global__ __launch_bounds__(64 * kPW) void dwconv4_pair_bwd_vec(const TX* __restrict__ x, int64_t ldx,
                                                                 const float* __restrict__ w0,
                                                                 const float* __restrict__ w1,
                                                                 const TDY* __restrict__ dy0,
                                                                 const TDY* __restrict__ dy1, int64_t ldy,
                                                                 TX* __restrict__ dx, int64_t ld_dx,
                                                                 TX* __restrict__ dadd0, TX* __restrict__ dadd1,
                                                                 int64_t ld_dadd, float* __restrict__ part0,
                                                                 float* __restrict__ part1, int64_t T, int64_t C,
                                                                 int acc) {
  constexpr int K = 4, V = kPV, R = kPR;
  constexpr int NZ = R + K - 1;  // dy rows tw .. tw + R + 2
  constexpr int NX = R + K - 1;  // x rows tw - 3 .. tw + R - 1
  __shared__ float s_red[kPW][(K + 1) * V][64];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t c0 = ((int64_t)blockIdx.x * 64 + lane) * V;
  const bool cok = c0 < C;
  const int64_t cc = cok ? c0 : 0;
  const int64_t b = blockIdx.z;
  const int64_t tw = (int64_t)blockIdx.y * (kPW * R) + wv * R;
  const TX* xb = x + b * T * ldx + cc;
  pvec_t<TDY, V> g0[NZ], g1[NZ];
  pvec_t<TX, V> xr[NX], dr[R];
#pragma unroll
  for (int i = 0; i < NZ; ++i) {
    const int64_t t = tw + i < T ? tw + i : T - 1;
    g0[i] = *(const pvec_t<TDY, V>*)(dy0 + (b * T + t) * ldy + cc);
    g1[i] = *(const pvec_t<TDY, V>*)(dy1 + (b * T + t) * ldy + cc);
  }
#pragma unroll
  for (int i = 0; i < NX; ++i) {
    int64_t t = tw - (K - 1) + i;
    t = t < 0 ? 0 : (t < T ? t : T - 1);
    xr[i] = *(const pvec_t<TX, V>*)(xb + t * ldx);
  }
  if (dx && acc) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t t = tw + r < T ? tw + r : T - 1;
      dr[r] = *(const pvec_t<TX, V>*)(dx + (b * T + t) * ld_dx + cc);
    }
  }
  float wr0[V][K], wr1[V][K];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const float4 q0 = *(const float4*)(w0 + (cc + j) * K);
    const float4 q1 = *(const float4*)(w1 + (cc + j) * K);
    wr0[j][0] = q0.x, wr0[j][1] = q0.y, wr0[j][2] = q0.z, wr0[j][3] = q0.w;
    wr1[j][0] = q1.x, wr1[j][1] = q1.y, wr1[j][2] = q1.z, wr1[j][3] = q1.w;
  }
  // dy of rows tw + i (zero at and beyond T), x of row tw - 3 + i (zero
  // outside [0, T))
  auto d0 = [&](int i, int j) -> float { return tw + i < T ? (float)g0[i][j] : 0.f; };
  auto d1 = [&](int i, int j) -> float { return tw + i < T ? (float)g1[i][j] : 0.f; };
  auto xv = [&](int i, int j) -> float {
    const int64_t t = tw - (K - 1) + i;
    return (t >= 0 && t < T) ? (float)xr[i][j] : 0.f;
  };
  float dw0[V][K], dw1[V][K], db0[V], db1[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    db0[j] = db1[j] = 0.f;
#pragma unroll
    for (int k = 0; k < K; ++k) dw0[j][k] = dw1[j][k] = 0.f;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t t = tw + r;
    if (t >= T) break;
    float g[V], e0[V], e1[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      float a0 = wr0[j][K - 1] * d0(r, j), a1 = wr1[j][K - 1] * d1(r, j);
#pragma unroll
      for (int k = 0; k < K - 1; ++k) {
        a0 = fmaf(wr0[j][k], d0(r + K - 1 - k, j), a0);
        a1 = fmaf(wr1[j][k], d1(r + K - 1 - k, j), a1);
      }
      g[j] = a0 + a1;
#pragma unroll
      for (int k = 0; k < K; ++k) {
        dw0[j][k] = fmaf(d0(r, j), xv(r + k, j), dw0[j][k]);
        dw1[j][k] = fmaf(d1(r, j), xv(r + k, j), dw1[j][k]);
      }
      db0[j] += d0(r, j);
      db1[j] += d1(r, j);
      e0[j] = d0(r, j);
      e1[j] = d1(r, j);
    }
    if (cok) {
      if (dx) {
        if (acc) {
#pragma unroll
          for (int j = 0; j < V; ++j) g[j] += (float)dr[r][j];
        }
        stc(dx + (b * T + t) * ld_dx + c0, g);
      }
      if (dadd0) stc(dadd0 + (b * T + t) * ld_dadd + c0, e0);
      if (dadd1) stc(dadd1 + (b * T + t) * ld_dadd + c0, e1);
    }
  }
  // the waves' sums in wave order, one weight after the other through the
  // same LDS
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    float* part = q == 0 ? part0 : part1;
    if (!part) continue;
#pragma unroll
    for (int j = 0; j < V; ++j) {
#pragma unroll
      for (int k = 0; k < K; ++k) s_red[wv][j * (K + 1) + k][lane] = q == 0 ? dw0[j][k] : dw1[j][k];
      s_red[wv][j * (K + 1) + K][lane] = q == 0 ? db0[j] : db1[j];
    }
    __syncthreads();
    float* pp = part + (((int64_t)b * gridDim.y + blockIdx.y) * C + c0) * (K + 1);
    for (int e = wv; e < (K + 1) * V; e += kPW) {
      float s = 0.f;
#pragma unroll
      for (int u = 0; u < kPW; ++u) s += s_red[u][e][lane];
      if (cok) pp[e] = s;
    }
    __syncthreads();
  }
}


// grid: (ceil(C / (64 * kRV)), ceil(n_rows / kVRows)) (kVRowsR in the
// backward), 64 threads
// Rows of a readout block are taken kRB at a time: in a whole batch every
// load of the kRB rows is issued before the first is used, so a wave waits
// for memory once per kRB rows (the block's last, partial batch goes row by
// row).
constexpr int kRB = 8;
// rows per block of the readout backward (its dD partial rows: one per block)
constexpr int kVRowsR = 32;
static_assert(kVRows % kRB == 0 && kVRowsR % kRB == 0 && kVRowsR >= kVRows, "whole row batches per block");

#ifndef NAJU_READOUT_V
#define NAJU_READOUT_V 4
#endif
constexpr int kRV = NAJU_READOUT_V;  // readout: channels per thread

template <typename T>
using rvec_t = T __attribute__((ext_vector_type(kRV)));

template <typename T>
__device__ __forceinline__ rvec_t<T> ldrv(const T* p) {
  return *(const rvec_t<T>*)p;
}

// An empty asm that takes v's registers as in-out operands: every load
// feeding v is complete there, and nothing that uses v moves above it.
template <typename T>
__device__ __forceinline__ void pinv(rvec_t<T>& v) {
  static_assert(sizeof(rvec_t<T>) % 4 == 0, "whole registers");
  uint32_t w[sizeof(rvec_t<T>) / 4];
  __builtin_memcpy(w, &v, sizeof(w));
#pragma unroll
  for (int i = 0; i < (int)(sizeof(w) / 4); ++i) asm volatile("" : "+v"(w[i]));
  __builtin_memcpy(&v, w, sizeof(w));
}

template <typename T>
__global__ __launch_bounds__(64) void readout_fwd_vec(const T* __restrict__ cx, const T* __restrict__ h,
                                                      const T* __restrict__ z, int64_t z_ld,
                                                      const float* __restrict__ Dv, float scale, T* __restrict__ y,
                                                      int64_t n_rows, int64_t C) {
  const int64_t c0 = ((int64_t)blockIdx.x * 64 + threadIdx.x) * kRV;
  if (c0 >= C) return;
  const int64_t r0 = (int64_t)blockIdx.y * kVRows;
  float dv[kRV];
#pragma unroll
  for (int j = 0; j < kRV; ++j) dv[j] = Dv[c0 + j];
  auto one = [&](const rvec_t<T>& xa, const rvec_t<T>& xh, const rvec_t<T>& xz, int64_t row) {
    float a[kRV];
#pragma unroll
    for (int j = 0; j < kRV; ++j) a[j] = fmaf((float)xa[j], scale, dv[j] * (float)xh[j]) * silu((float)xz[j]);
    stc(y + row * C + c0, a);
  };
  for (int rb = 0; rb < kVRows; rb += kRB) {
    const int64_t b0 = r0 + rb;
    if (b0 + kRB <= n_rows) {
      // a whole batch: straight-line loads, then the rows
      rvec_t<T> xa[kRB], xh[kRB], xz[kRB];
#pragma unroll
      for (int r = 0; r < kRB; ++r) {
        xa[r] = ldrv(cx + (b0 + r) * C + c0);
        xh[r] = ldrv(h + (b0 + r) * C + c0);
        xz[r] = ldrv(z + (b0 + r) * z_ld + c0);
      }
      // (keeps the compiler from sinking the loads into the rows' code)
#pragma unroll
      for (int r = 0; r < kRB; ++r) pinv(xa[r]), pinv(xh[r]), pinv(xz[r]);
#pragma unroll
      for (int r = 0; r < kRB; ++r) one(xa[r], xh[r], xz[r], b0 + r);
    } else {
      for (int64_t row = b0; row < n_rows; ++row)
        one(ldrv(cx + row * C + c0), ldrv(h + row * C + c0), ldrv(z + row * z_ld + c0), row);
      break;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(64) void readout_bwd_vec(const T* __restrict__ cx, const T* __restrict__ h,
                                                      const T* __restrict__ z, int64_t z_ld,
                                                      const float* __restrict__ Dv, float scale,
                                                      const T* __restrict__ dy, T* __restrict__ dcx,
                                                      T* __restrict__ dh, T* __restrict__ dz, int64_t dz_ld,
                                                      float* __restrict__ part, int64_t n_rows, int64_t C) {
  const int64_t c0 = ((int64_t)blockIdx.x * 64 + threadIdx.x) * kRV;
  if (c0 >= C) return;
  const int64_t r0 = (int64_t)blockIdx.y * kVRowsR;
  float dv[kRV], dd[kRV];
#pragma unroll
  for (int j = 0; j < kRV; ++j) dv[j] = Dv[c0 + j];
#pragma unroll
  for (int j = 0; j < kRV; ++j) dd[j] = 0.f;
  auto one = [&](const rvec_t<T>& xc, const rvec_t<T>& xh, const rvec_t<T>& xz, const rvec_t<T>& xg, int64_t row) {
    float o0[kRV], o1[kRV], o2[kRV];
#pragma unroll
    for (int j = 0; j < kRV; ++j) {
      const float zz = (float)xz[j], g = (float)xg[j], hh = (float)xh[j];
      const float sg = sigmoid_f(zz);
      const float gs = g * (zz * sg);
      o0[j] = gs * scale;
      o1[j] = gs * dv[j];
      dd[j] = fmaf(gs, hh, dd[j]);
      const float a = fmaf((float)xc[j], scale, dv[j] * hh);
      o2[j] = g * a * sg * fmaf(zz, 1.f - sg, 1.f);
    }
    if (dcx) stc(dcx + row * C + c0, o0);
    if (dh) stc(dh + row * C + c0, o1);
    if (dz) stc(dz + row * dz_ld + c0, o2);
  };
  for (int rb = 0; rb < kVRowsR; rb += kRB) {
    const int64_t b0 = r0 + rb;
    if (b0 + kRB <= n_rows) {
      // a whole batch: straight-line loads, then the rows
      rvec_t<T> xc[kRB], xh[kRB], xz[kRB], xg[kRB];
#pragma unroll
      for (int r = 0; r < kRB; ++r) {
        xc[r] = ldrv(cx + (b0 + r) * C + c0);
        xh[r] = ldrv(h + (b0 + r) * C + c0);
        xz[r] = ldrv(z + (b0 + r) * z_ld + c0);
        xg[r] = ldrv(dy + (b0 + r) * C + c0);
      }
#pragma unroll
      for (int r = 0; r < kRB; ++r) one(xc[r], xh[r], xz[r], xg[r], b0 + r);
    } else {
      for (int64_t row = b0; row < n_rows; ++row)
        one(ldrv(cx + row * C + c0), ldrv(h + row * C + c0), ldrv(z + row * z_ld + c0), ldrv(dy + row * C + c0),
            row);
      break;
    }
  }
  if (part) {
    float* pp = part + (int64_t)blockIdx.y * C + c0;
#pragma unroll
    for (int q = 0; q < kRV; q += 4) *(float4*)(pp + q) = make_float4(dd[q], dd[q + 1], dd[q + 2], dd[q + 3]);
  }
}

// out[i] (i < ncol) = sum over q < nblk of part[q * ncol + i], in a fixed
// order: each of 16 waves sums every 16th block of a 64-column slice, then
// wave 0 adds the 16 partial sums in wave order. The dw / dbias columns of
// the conv partials ([C][K+1]) go to dw (j < K) and dbias (j == K); with
// K = 0 every column is a dbias (the readout's dD).
__global__ __launch_bounds__(1024) void fold_cols_kernel(const float* __restrict__ part0, int64_t nblk, int64_t C,
                                                         int K, float* __restrict__ dw0, float* __restrict__ dbias0,
                                                         const float* __restrict__ part1, float* __restrict__ dw1,
                                                         float* __restrict__ dbias1) {
  // blockIdx.y selects one of two partial arrays of the same shape (the gate
  // pair's two weights in one launch)
  const bool second = blockIdx.y != 0;
  const float* __restrict__ part = second ? part1 : part0;
  float* __restrict__ dw = second ? dw1 : dw0;
  float* __restrict__ dbias = second ? dbias1 : dbias0;
  __shared__ float s[16][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t ncol = C * (K + 1);
  const int64_t i = (int64_t)blockIdx.x * 64 + lane;
  float acc = 0.f;
  if (i < ncol) {
    // kU blocks per round, all loaded (from an in-bounds block past the
    // end) before the first is added; added in block order
    constexpr int kU = 16;
    for (int64_t q0 = wv; q0 < nblk; q0 += 16 * kU) {
      float v[kU];
#pragma unroll
      for (int k = 0; k < kU; ++k) {
        const int64_t q = q0 + 16 * k;
        v[k] = part[(q < nblk ? q : q0) * ncol + i];
      }
#pragma unroll
      for (int k = 0; k < kU; ++k) asm volatile("" : "+v"(v[k]));
#pragma unroll
      for (int k = 0; k < kU; ++k) {
        const float t = acc + v[k];
        acc = q0 + 16 * k < nblk ? t : acc;
      }
    }
  }
  s[wv][lane] = acc;
  __syncthreads();
  if (wv == 0 && i < ncol) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < 16; ++w) t += s[w][lane];
    const int64_t c = i / (K + 1), j = i - c * (K + 1);
    if (j < K) {
      if (dw) dw[c * K + j] = t;
    } else if (dbias) {
      dbias[c] = t;
    }
  }
}

// out = sum of the n_parts rows of parts [n_parts][n], in row order. The
// vector kernel (S parts, n % 4 == 0, 16-byte aligned pointers) gives a
// thread four consecutive entries and loads them from all S parts before
// adding; other cases take one entry per thread.
constexpr int kMaxParts = 16;
template <int S>
__global__ __launch_bounds__(256) void sum_parts_vec(const float4* __restrict__ parts, int64_t n4,
                                                     float4* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= n4) return;
  float4 v[S];
#pragma unroll
  for (int q = 0; q < S; ++q) v[q] = parts[(int64_t)q * n4 + t];
  float4 a = v[0];
#pragma unroll
  for (int q = 1; q < S; ++q) a.x += v[q].x, a.y += v[q].y, a.z += v[q].z, a.w += v[q].w;
  out[t] = a;
}

__global__ __launch_bounds__(256) void sum_parts_any(const float* __restrict__ parts, int n_parts, int64_t n,
                                                     float* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= n) return;
  float a = parts[t];
  for (int q = 1; q < n_parts; ++q) a += parts[(int64_t)q * n + t];
  out[t] = a;
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

thread_local char g_err[256] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

bool dt_ok(int dt) { return dt == NAJU_DTYPE_F32 || dt == NAJU_DTYPE_BF16 || dt == NAJU_DTYPE_F16; }

// act: 0 (identity) or 1 (SiLU); the backward also takes
// NAJU_DWCONV_ACCUM_DX in it (acc_ok).
int check(int64_t batch, int64_t T, int64_t C, int K, int act, int64_t x_ld, bool acc_ok = false) {
  if (batch < 0 || T < 0 || C < 0) return fail(NAJU_ERR_INVALID, "negative shape");
  if (x_ld < C) return fail(NAJU_ERR_INVALID, "x_ld (%lld) must be >= C (%lld)", (long long)x_ld, (long long)C);
  if (K < 1 || K > kMaxK) return fail(NAJU_ERR_UNSUPPORTED, "kernel size K must be in [1, %d], got %d", kMaxK, K);
  const int a = acc_ok ? (act & ~NAJU_DWCONV_ACCUM_DX) : act;
  if (a != 0 && a != 1)
    return fail(NAJU_ERR_INVALID, acc_ok ? "act must be 0 (identity) or 1 (SiLU), optionally | NAJU_DWCONV_ACCUM_DX"
                                         : "act must be 0 (identity) or 1 (SiLU)");
  if (batch > 65535 || (T + kRows - 1) / kRows > 65535 || C > (1ll << 30))
    return fail(NAJU_ERR_UNSUPPORTED, "shape too large (batch <= 65535, T <= %d)", 65535 * kRows);
  return NAJU_OK;
}

typedef void (*fwd_t)(const void*, int64_t, const float*, const float*, const void*, int64_t, void*, int64_t, int64_t,
                      int, int, int);
typedef void (*bwd_t)(const void*, int64_t, const float*, const float*, const void*, void*, int64_t, void*, int64_t,
                      float*, int64_t, int64_t, int, int, int, int, int);

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

typedef void (*dwf_vec_t)(const void*, int64_t, const float*, const float*, const void*, int64_t, void*, int64_t,
                          int64_t);
typedef void (*dwb_vec_t)(const void*, int64_t, const float*, const float*, const void*, void*, int64_t, void*,
                          int64_t, float*, int64_t, int64_t, int);

template <typename TX>
dwf_vec_t dwf_vec_for(int y_dt, bool silu, bool add) {
  if (y_dt == NAJU_DTYPE_F32) {
    if (silu) return (dwf_vec_t)dwconv4_fwd_vec<TX, float, true, false>;
    return add ? (dwf_vec_t)dwconv4_fwd_vec<TX, float, false, true> : (dwf_vec_t)dwconv4_fwd_vec<TX, float, false, false>;
  }
  if (silu) return (dwf_vec_t)dwconv4_fwd_vec<TX, TX, true, false>;
  return add ? (dwf_vec_t)dwconv4_fwd_vec<TX, TX, false, true> : (dwf_vec_t)dwconv4_fwd_vec<TX, TX, false, false>;
}

// The K = 4 vector kernel for these arguments, or nullptr (scalar path):
// x and add in one dtype, y in that dtype or float32, C, x_ld and add_ld
// multiples of 8, 16-byte aligned pointers, T / kCRF blocks within the
// grid limit.
dwf_vec_t pick_fwd_vec(const void* x, int64_t x_ld, const float* w, const float* bias, const void* add,
                       int64_t add_ld, void* y, int64_t T, int64_t C, int K, int act, int x_dt, int add_dt,
                       int y_dt) {
  if (K != 4 || C % kVec || x_ld % kVec || (add && add_ld % kVec) || (T + kCRF - 1) / kCRF > 65535)
    return nullptr;
  if (!al16(x) || !al16(w) || !al16(y) || (bias && !al16(bias)) || (add && !al16(add))) return nullptr;
  if (add && add_dt != x_dt) return nullptr;
  if (y_dt != x_dt && y_dt != NAJU_DTYPE_F32) return nullptr;
  const bool silu = act == 1, has_add = add != nullptr;
  if (x_dt == NAJU_DTYPE_BF16) return dwf_vec_for<bf16_t>(y_dt, silu, has_add);
  if (x_dt == NAJU_DTYPE_F16) return dwf_vec_for<f16_t>(y_dt, silu, has_add);
  return dwf_vec_for<float>(y_dt, silu, has_add);
}

template <typename TX>
dwb_vec_t dwb_vec_for(int dy_dt, bool silu) {
  if (dy_dt == NAJU_DTYPE_F32 && !std::is_same<TX, float>::value)
    return silu ? (dwb_vec_t)dwconv4_bwd_vec<TX, float, true> : (dwb_vec_t)dwconv4_bwd_vec<TX, float, false>;
  return silu ? (dwb_vec_t)dwconv4_bwd_vec<TX, TX, true> : (dwb_vec_t)dwconv4_bwd_vec<TX, TX, false>;
}

dwb_vec_t pick_bwd_vec(const void* x, int64_t x_ld, const float* w, const float* bias, const void* dy, void* dx,
                       int64_t dx_ld, const void* dadd, int64_t dadd_ld, int64_t T, int64_t C, int K, int act,
                       int x_dt, int dy_dt, int dx_dt, int dadd_dt) {
  // act: the activation only (the accumulate bit is taken off by the caller)
  if (K != 4 || C % kVec || x_ld % kVec || dx_ld % kVec || (dadd && dadd_ld % kVec) ||
      (T + kVRowsB - 1) / kVRowsB > 65535)
    return nullptr;
  if (!al16(x) || !al16(w) || !al16(dy) || (bias && !al16(bias)) || (dx && !al16(dx)) || (dadd && !al16(dadd)))
    return nullptr;
  if (dx_dt != x_dt || (dadd && dadd_dt != x_dt) || (dy_dt != x_dt && dy_dt != NAJU_DTYPE_F32)) return nullptr;
  if (x_dt == NAJU_DTYPE_BF16) return dwb_vec_for<bf16_t>(dy_dt, act == 1);
  if (x_dt == NAJU_DTYPE_F16) return dwb_vec_for<f16_t>(dy_dt, act == 1);
  return dwb_vec_for<float>(dy_dt, act == 1);
}

// Readout vector path: every [n_rows, C] stream in one dtype.
bool readout_vec_ok(int64_t n_rows, int64_t C, int64_t z_ld, std::initializer_list<const void*> ptrs,
                    std::initializer_list<int> dts, int64_t dz_ld = 0) {
  if (C % kVec || z_ld % kVec || dz_ld % kVec || (n_rows + kVRows - 1) / kVRows > 65535) return false;
  for (const void* p : ptrs)
    if (p && !al16(p)) return false;
  int first = -1;
  for (int d : dts) {
    if (first < 0) first = d;
    if (d != first) return false;
  }
  return true;
}

// Folds part0 into dw0 / dbias0 and, when part1 is given, part1 into dw1 /
// dbias1 in the same launch.
int launch_fold(const float* part, int64_t nblk, int64_t C, int K, float* dw, float* dbias, hipStream_t st,
                const float* part1 = nullptr, float* dw1 = nullptr, float* dbias1 = nullptr) {
  const int64_t ncol = C * (K + 1);
  hipLaunchKernelGGL(fold_cols_kernel, dim3((unsigned)((ncol + 63) / 64), part1 ? 2u : 1u), dim3(1024), 0, st, part,
                     nblk, C, K, dw, dbias, part1, dw1, dbias1);
  return hipGetLastError() == hipSuccess ? NAJU_OK : fail(NAJU_ERR_LAUNCH, "fold launch failed");
}


// ------------------------------------------------------------------ RMSNorm
//
//   y[r,c] = (w[c] * x[r,c]) * rstd[r],  rstd[r] = 1 / sqrt(mean_c x[r,c]^2 + eps)
//
// (reference RMSNorm, /root/reference/naju/mixer.py:51-58, same order of the
// two products). One wave per row: lane l holds the columns 4(l + 64g) ..
// +3 for g < G (G * 256 >= d), so the row is read once into registers and
// written once; each wave does RPW rows with all their loads issued first.
// The backward,
//   dx = rstd * (w * dy) - x * rstd^3 * sum_c(w * dy * x) / d,
//   dw = sum_r (dy * rstd) * x,
// keeps each wave's dw terms in registers, adds the waves of a workgroup in
// order and leaves one row of partial sums per workgroup, which
// fold_cols_kernel adds in workgroup order (deterministic).
constexpr int kNormWaves = 4;

template <typename T>
__device__ __forceinline__ void ld4(const T* p, float (&o)[4]) {
  typedef T v_t __attribute__((ext_vector_type(4)));
  const v_t v = *reinterpret_cast<const v_t*>(p);
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = (float)v[e];
}
template <typename T>
__device__ __forceinline__ void st4(T* p, const float (&o)[4]) {
  typedef T v_t __attribute__((ext_vector_type(4)));
  v_t v;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = (T)o[e];
  *reinterpret_cast<v_t*>(p) = v;
}

__device__ __forceinline__ float wave_allsum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

template <int G>
constexpr int norm_rpw() {
  return G <= 4 ? 4 : (G <= 8 ? 2 : 1);
}

// grid: ceil(n_rows / (kNormWaves * RPW)) workgroups of 64 * kNormWaves.
template <typename TX, typename TY, int G>
__global__ __launch_bounds__(64 * kNormWaves) void rmsnorm_fwd_vec(const TX* __restrict__ x,
                                                                   const float* __restrict__ w, float eps,
                                                                   TY* __restrict__ y, float* __restrict__ rstd,
                                                                   int64_t n_rows, int64_t d) {
  constexpr int RPW = norm_rpw<G>();
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t r0 = ((int64_t)blockIdx.x * kNormWaves + wv) * RPW;
  float wr[G][4], xv[RPW][G][4];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int64_t c = ((int64_t)g * 64 + lane) * 4;
    if (c < d) {
      ld4(w + c, wr[g]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) wr[g][e] = 0.f;
    }
  }
#pragma unroll
  for (int i = 0; i < RPW; ++i)
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t c = ((int64_t)g * 64 + lane) * 4;
      if (r0 + i < n_rows && c < d) {
        ld4(x + (r0 + i) * d + c, xv[i][g]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[i][g][e] = 0.f;
      }
    }
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int64_t r = r0 + i;
    float ss = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) ss = fmaf(xv[i][g][e], xv[i][g][e], ss);
    const float rs = rsqrtf(wave_allsum(ss) / (float)d + eps);
    if (r >= n_rows) continue;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t c = ((int64_t)g * 64 + lane) * 4;
      if (c < d) {
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = (wr[g][e] * xv[i][g][e]) * rs;
        st4(y + r * d + c, o);
      }
    }
    if (lane == 0) rstd[r] = rs;
  }
}

template <typename TX, typename TDY, int G>
__global__ __launch_bounds__(64 * kNormWaves) void rmsnorm_bwd_vec(const TX* __restrict__ x,
                                                                   const float* __restrict__ w,
                                                                   const float* __restrict__ rstd,
                                                                   const TDY* __restrict__ dy, TX* __restrict__ dx,
                                                                   const TX* __restrict__ dres,
                                                                   float* __restrict__ part, int64_t n_rows,
                                                                   int64_t d) {
  constexpr int RPW = norm_rpw<G>();
  __shared__ float s_acc[kNormWaves][G * 256];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t r0 = ((int64_t)blockIdx.x * kNormWaves + wv) * RPW;
  float wr[G][4], acc[G][4], xv[RPW][G][4], gv[RPW][G][4], qv[RPW][G][4], rs[RPW];
  // Every load is unconditional, from a clamped in-bounds row and column
  // (d % 4 == 0, so column d - 4 exists), and lanes or rows outside the
  // matrix take zeros afterwards: loads behind per-lane branches were each
  // waited for at the end of their branch.
  const int64_t rlast = n_rows - 1;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int64_t c = ((int64_t)g * 64 + lane) * 4;
    const int64_t cc = c < d ? c : d - 4;
    ld4(w + cc, wr[g]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[g][e] = 0.f;
      wr[g][e] = c < d ? wr[g][e] : 0.f;
    }
  }
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int64_t rr = r0 + i < n_rows ? r0 + i : rlast;
    rs[i] = rstd[rr];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t c = ((int64_t)g * 64 + lane) * 4;
      const int64_t cc = c < d ? c : d - 4;
      ld4(x + rr * d + cc, xv[i][g]);
      ld4(dy + rr * d + cc, gv[i][g]);
    }
  }
  if (dres) {
    // the residual gradient with the other loads, before any is used
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int64_t rr = r0 + i < n_rows ? r0 + i : rlast;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int64_t c = ((int64_t)g * 64 + lane) * 4;
        ld4(dres + rr * d + (c < d ? c : d - 4), qv[i][g]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const bool rv = r0 + i < n_rows;
    rs[i] = rv ? rs[i] : 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const bool ok = rv && ((int64_t)g * 64 + lane) * 4 < d;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xv[i][g][e] = ok ? xv[i][g][e] : 0.f;
        gv[i][g][e] = ok ? gv[i][g][e] : 0.f;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int64_t r = r0 + i;
    float s = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s = fmaf(wr[g][e] * gv[i][g][e], xv[i][g][e], s);
        acc[g][e] = fmaf(gv[i][g][e] * rs[i], xv[i][g][e], acc[g][e]);
      }
    const float k = rs[i] * rs[i] * rs[i] * wave_allsum(s) / (float)d;
    if (r >= n_rows) continue;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t c = ((int64_t)g * 64 + lane) * 4;
      if (c < d) {
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = fmaf(wr[g][e] * gv[i][g][e], rs[i], -xv[i][g][e] * k);
        if (dres) {
          // dx = dres + the norm's gradient (the residual stream's other use)
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] += qv[i][g][e];
        }
        st4(dx + r * d + c, o);
      }
    }
  }
  if (!part) return;
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 4; ++e) s_acc[wv][(g * 64 + lane) * 4 + e] = acc[g][e];
  __syncthreads();
  for (int64_t c = threadIdx.x; c < d; c += 64 * kNormWaves) {
    float t = 0.f;
#pragma unroll
    for (int q = 0; q < kNormWaves; ++q) t += s_acc[q][c];
    part[(int64_t)blockIdx.x * d + c] = t;
  }
}

constexpr int kNormGs[] = {1, 2, 3, 4, 8, 16};

int norm_g(int64_t d) {
  for (int g : kNormGs)
    if ((int64_t)g * 256 >= d) return g;
  return 0;
}

int64_t norm_blocks(int64_t n_rows, int G) {
  const int64_t per = (int64_t)kNormWaves * (G <= 4 ? 4 : (G <= 8 ? 2 : 1));
  return (n_rows + per - 1) / per;
}

template <typename TX, typename TY>
void norm_fwd_launch(int G, dim3 grid, hipStream_t st, const void* x, const float* w, float eps, void* y, float* rstd,
                     int64_t n, int64_t d) {
  const dim3 blk(64 * kNormWaves);
#define NAJU_NORM_F(GG)                                                                                          \
  case GG:                                                                                                      \
    hipLaunchKernelGGL((rmsnorm_fwd_vec<TX, TY, GG>), grid, blk, 0, st, (const TX*)x, w, eps, (TY*)y, rstd, n, d); \
    break;
  switch (G) {
    NAJU_NORM_F(1)
    NAJU_NORM_F(2)
    NAJU_NORM_F(3)
    NAJU_NORM_F(4)
    NAJU_NORM_F(8)
    NAJU_NORM_F(16)
  }
#undef NAJU_NORM_F
}

template <typename TX, typename TDY>
void norm_bwd_launch(int G, dim3 grid, hipStream_t st, const void* x, const float* w, const float* rstd,
                     const void* dy, void* dx, const void* dres, float* part, int64_t n, int64_t d) {
  const dim3 blk(64 * kNormWaves);
#define NAJU_NORM_B(GG)                                                                                          \
  case GG:                                                                                                      \
    hipLaunchKernelGGL((rmsnorm_bwd_vec<TX, TDY, GG>), grid, blk, 0, st, (const TX*)x, w, rstd, (const TDY*)dy,  \
                       (TX*)dx, (const TX*)dres, part, n, d);                                                    \
    break;
  switch (G) {
    NAJU_NORM_B(1)
    NAJU_NORM_B(2)
    NAJU_NORM_B(3)
    NAJU_NORM_B(4)
    NAJU_NORM_B(8)
    NAJU_NORM_B(16)
  }
#undef NAJU_NORM_B
}

template <typename TX>
bool norm_fwd_dt(int y_dt, int G, dim3 grid, hipStream_t st, const void* x, const float* w, float eps, void* y,
                 float* rstd, int64_t n, int64_t d) {
  if (y_dt == NAJU_DTYPE_F32)
    norm_fwd_launch<TX, float>(G, grid, st, x, w, eps, y, rstd, n, d);
  else if (y_dt == NAJU_DTYPE_BF16)
    norm_fwd_launch<TX, bf16_t>(G, grid, st, x, w, eps, y, rstd, n, d);
  else
    norm_fwd_launch<TX, f16_t>(G, grid, st, x, w, eps, y, rstd, n, d);
  return true;
}

template <typename TX>
bool norm_bwd_dt(int dy_dt, int G, dim3 grid, hipStream_t st, const void* x, const float* w, const float* rstd,
                 const void* dy, void* dx, const void* dres, float* part, int64_t n, int64_t d) {
  if (dy_dt == NAJU_DTYPE_F32)
    norm_bwd_launch<TX, float>(G, grid, st, x, w, rstd, dy, dx, dres, part, n, d);
  else if (dy_dt == NAJU_DTYPE_BF16)
    norm_bwd_launch<TX, bf16_t>(G, grid, st, x, w, rstd, dy, dx, dres, part, n, d);
  else
    norm_bwd_launch<TX, f16_t>(G, grid, st, x, w, rstd, dy, dx, dres, part, n, d);
  return true;
}

// Host-side checks shared by both directions; 0 or an error code.
int norm_check(int64_t n_rows, int64_t d, int x_dt, std::initializer_list<int> dts,
               std::initializer_list<const void*> ptrs) {
  if (n_rows < 0 || d < 0) return fail(NAJU_ERR_INVALID, "negative shape");
  if (!dt_ok(x_dt)) return fail(NAJU_ERR_INVALID, "unknown dtype code");
  for (int dt : dts)
    if (!dt_ok(dt)) return fail(NAJU_ERR_INVALID, "unknown dtype code");
  if (x_dt == NAJU_DTYPE_F16) return fail(NAJU_ERR_UNSUPPORTED, "float16 x is not served (float32 or bfloat16)");
  if (d % 4 != 0 || d > 16 * 256)
    return fail(NAJU_ERR_UNSUPPORTED, "d must be a multiple of 4 and at most 4096 (got %lld)", (long long)d);
  if (n_rows > (int64_t)0x7fffffff) return fail(NAJU_ERR_UNSUPPORTED, "too many rows");
  for (const void* p : ptrs)
    if (p && ((uintptr_t)p % 16) != 0)
      return fail(NAJU_ERR_UNSUPPORTED, "pointers must be 16-byte aligned");
  return NAJU_OK;
}


// ------------------------------------------------- residual add with dropout
//
// The pre-norm block's u + Dropout(mix) (reference naju/mixer.py:131-144) in
// one pass, and the dropout's backward in one pass. The keep decision of
// element i is a pure function of (seed, i), drawn again by the backward,
// so no mask is stored: a SplitMix64 output (Steele, Lea and Flood, "Fast
// splittable pseudorandom number generators", OOPSLA 2014) of the 64-bit
// word seed + (i / 2 + 1) * 0x9E3779B97F4A7C15, whose upper and lower
// 32-bit halves decide elements 2m and 2m + 1: kept when the half is at or
// above p * 2^32. Kept elements are scaled by 1 / (1 - p) and rounded to
// mix's dtype first, as the reference's Dropout output is.
struct DropKeep {
  uint32_t thr;  // keep when the 32-bit draw is >= thr
  float scale;   // 1 / (1 - p)
};

DropKeep drop_keep(float p) {
  DropKeep k;
  const double t = (double)p * 4294967296.0;
  k.thr = t >= 4294967295.0 ? 0xffffffffu : (uint32_t)t;
  k.scale = 1.f / (1.f - p);
  return k;
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// keep bits of elements 2m and 2m + 1 (bit 0: element 2m)
__device__ __forceinline__ uint32_t drop_pair(uint64_t seed, int64_t m, uint32_t thr) {
  const uint64_t z = splitmix64(seed + (uint64_t)(m + 1) * 0x9E3779B97F4A7C15ull);
  return ((uint32_t)z >= thr ? 1u : 0u) | ((uint32_t)(z >> 32) >= thr ? 2u : 0u);
}

template <typename TM>
__device__ __forceinline__ float drop_val(float v, bool keep, float scale) {
  return keep ? (float)(TM)(v * scale) : 0.f;
}

// out = u + dropout(mix); VEC: 8 elements per thread (n % 8 == 0, 16-byte
// aligned), else one. seed == nullptr: p = 0, every element kept.
template <typename TM, bool VEC>
__global__ __launch_bounds__(256) void residual_dropout_kernel(const float* __restrict__ u,
                                                               const TM* __restrict__ mix,
                                                               const int64_t* __restrict__ seed, DropKeep dk,
                                                               float* __restrict__ out, int64_t n) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const uint64_t s = seed ? (uint64_t)seed[0] : 0ull;
  if constexpr (VEC) {
    const int64_t i0 = t * kVec;
    if (i0 >= n) return;
    float uv[kVec], mv[kVec];
    ld8f(u + i0, uv);
    ld8(mix + i0, mv);
    uint32_t keep = 0xffu;
    if (seed) {
      keep = 0u;
#pragma unroll
      for (int q = 0; q < kVec / 2; ++q) keep |= drop_pair(s, i0 / 2 + q, dk.thr) << (2 * q);
    }
#pragma unroll
    for (int j = 0; j < kVec; ++j) uv[j] += seed ? drop_val<TM>(mv[j], (keep >> j) & 1u, dk.scale) : mv[j];
    *(float4*)(out + i0) = make_float4(uv[0], uv[1], uv[2], uv[3]);
    *(float4*)(out + i0 + 4) = make_float4(uv[4], uv[5], uv[6], uv[7]);
  } else {
    if (t >= n) return;
    const float mv = (float)mix[t];
    float o = u[t];
    if (seed) {
      const bool keep = (drop_pair(s, t / 2, dk.thr) >> (t & 1)) & 1u;
      o += drop_val<TM>(mv, keep, dk.scale);
    } else {
      o += mv;
    }
    out[t] = o;
  }
}

// dmix = dropout'(g): g * scale where kept, 0 where dropped, rounded once to
// mix's dtype.
template <typename TM, bool VEC>
__global__ __launch_bounds__(256) void dropout_bwd_kernel(const float* __restrict__ g,
                                                          const int64_t* __restrict__ seed, DropKeep dk,
                                                          TM* __restrict__ dmix, int64_t n) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const uint64_t s = seed ? (uint64_t)seed[0] : 0ull;
  if constexpr (VEC) {
    const int64_t i0 = t * kVec;
    if (i0 >= n) return;
    float gv[kVec];
    ld8f(g + i0, gv);
    if (seed) {
      uint32_t keep = 0u;
#pragma unroll
      for (int q = 0; q < kVec / 2; ++q) keep |= drop_pair(s, i0 / 2 + q, dk.thr) << (2 * q);
#pragma unroll
      for (int j = 0; j < kVec; ++j) gv[j] = ((keep >> j) & 1u) ? gv[j] * dk.scale : 0.f;
    }
    st8(dmix + i0, gv);
  } else {
    if (t >= n) return;
    float v = g[t];
    if (seed) v = ((drop_pair(s, t / 2, dk.thr) >> (t & 1)) & 1u) ? v * dk.scale : 0.f;
    dmix[t] = (TM)v;
  }
}

typedef void (*resdrop_t)(const float*, const void*, const int64_t*, DropKeep, float*, int64_t);
typedef void (*dropbwd_t)(const float*, const int64_t*, DropKeep, void*, int64_t);

}  // namespace

namespace {

// Embedding gradient added into dW [V, d] (float32): workgroup p serves the
// run of equal ids that starts at position p of the sorted ids (the other
// workgroups return at once) and adds the dy rows of that run, in sorted
// order (a stable sort keeps the original order of equal ids), to the row
// dW[id]: dW[id] + dy[r1] + dy[r2] + ..., a fixed order. Threads take
// columns 4 at a time.
__global__ __launch_bounds__(256) void embed_bwd_add_kernel(const int64_t* __restrict__ sorted,
                                                            const int64_t* __restrict__ order,
                                                            const float* __restrict__ dy, int64_t n, int64_t d,
                                                            float* __restrict__ dw, int64_t V) {
  const int64_t p = blockIdx.x;
  const int64_t id = sorted[p];
  if ((p > 0 && sorted[p - 1] == id) || id < 0 || id >= V) return;
  int64_t end = p + 1;
  while (end < n && sorted[end] == id) ++end;
  float* __restrict__ row = dw + id * d;
  const bool vec = d % 4 == 0 && ((uintptr_t)dw & 15) == 0 && ((uintptr_t)dy & 15) == 0;
  if (vec) {
    for (int64_t c = 4 * (int64_t)threadIdx.x; c < d; c += 4 * 256) {
      float4 acc = *(const float4*)(row + c);
      for (int64_t q = p; q < end; ++q) {
        const float4 v = *(const float4*)(dy + order[q] * d + c);
        acc.x += v.x, acc.y += v.y, acc.z += v.z, acc.w += v.w;
      }
      *(float4*)(row + c) = acc;
    }
  } else {
    for (int64_t c = threadIdx.x; c < d; c += 256) {
      float acc = row[c];
      for (int64_t q = p; q < end; ++q) acc += dy[order[q] * d + c];
      row[c] = acc;
    }
  }
}

}  // namespace

extern "C" {

const char* naju_mixer_last_error(void) { return g_err; }

int naju_dwconv_fwd(const void* x, int64_t x_ld, const float* w, const float* bias, const void* add, int64_t add_ld,
                    void* y, int64_t batch, int64_t T, int64_t C, int K, int act, int x_dtype, int add_dtype,
                    int y_dtype, void* stream) {
  g_err[0] = 0;
  int rc = check(batch, T, C, K, act, x_ld);
  if (rc) return rc;
  if (add && add_ld < C)
    return fail(NAJU_ERR_INVALID, "add_ld (%lld) must be >= C (%lld)", (long long)add_ld, (long long)C);
  if (!dt_ok(x_dtype) || !dt_ok(y_dtype) || (add && !dt_ok(add_dtype)))
    return fail(NAJU_ERR_INVALID, "unknown dtype code");
  if (act == 1 && add) return fail(NAJU_ERR_UNSUPPORTED, "add must be NULL with act = SiLU");
  if (batch == 0 || T == 0 || C == 0) return NAJU_OK;
  if (!x || !w || !y) return fail(NAJU_ERR_INVALID, "null pointer (x, w and y are required)");
  if (dwf_vec_t kv = pick_fwd_vec(x, x_ld, w, bias, add, add_ld, y, T, C, K, act, x_dtype, add_dtype, y_dtype)) {
    const dim3 grid((unsigned)((C + 64 * kFV4 - 1) / (64 * kFV4)), (unsigned)((T + kCRF - 1) / kCRF),
                    (unsigned)batch);
    hipLaunchKernelGGL(kv, grid, dim3(64), 0, (hipStream_t)stream, x, x_ld, w, bias, add, add_ld, y, T, C);
  } else {
    const dim3 grid((unsigned)((C + kThreads - 1) / kThreads), (unsigned)n_tblocks(T), (unsigned)batch);
    hipLaunchKernelGGL(pick_fwd(K, act == 1), grid, dim3(kThreads), 0, (hipStream_t)stream, x, x_ld, w, bias, add,
                       add_ld, y, T, C, x_dtype, add_dtype, y_dtype);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return NAJU_OK;
}

size_t naju_dwconv_workspace_bytes(int64_t batch, int64_t T, int64_t C, int K) {
  if (check(batch, T, C, K, 0, C) != NAJU_OK) return 0;
  // partial rows: one per block of the scalar (kRows) or vector (kVRowsB) backward
  const int64_t rows = kVRowsB < kRows ? kVRowsB : kRows;
  return (size_t)batch * ((T + rows - 1) / rows) * C * (K + 1) * sizeof(float) + 256;
}

int naju_dwconv_bwd(const void* x, int64_t x_ld, const float* w, const float* bias, const void* dy, void* dx,
                    int64_t dx_ld, float* dw, float* dbias, void* dadd, int64_t dadd_ld, int64_t batch, int64_t T,
                    int64_t C, int K, int act, int x_dtype, int dy_dtype, int dx_dtype, int dadd_dtype,
                    void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  int rc = check(batch, T, C, K, act, x_ld, true);
  if (rc) return rc;
  const int acc = (act & NAJU_DWCONV_ACCUM_DX) ? 1 : 0;
  act &= ~NAJU_DWCONV_ACCUM_DX;
  if (!dt_ok(x_dtype) || !dt_ok(dy_dtype) || !dt_ok(dx_dtype) || (dadd && !dt_ok(dadd_dtype)))
    return fail(NAJU_ERR_INVALID, "unknown dtype code");
  if (dx && dx_ld < C) return fail(NAJU_ERR_INVALID, "dx_ld (%lld) must be >= C (%lld)", (long long)dx_ld, (long long)C);
  if (dadd && dadd_ld < C)
    return fail(NAJU_ERR_INVALID, "dadd_ld (%lld) must be >= C (%lld)", (long long)dadd_ld, (long long)C);
  if (dadd && act == 1) return fail(NAJU_ERR_UNSUPPORTED, "dadd must be NULL with act = SiLU");
  hipStream_t st = (hipStream_t)stream;
  if (C == 0) return NAJU_OK;
  if (batch == 0 || T == 0) {
    // empty sums: the fold over zero blocks writes the zeros (a kernel, not a
    // memset, so that the call can be captured into a graph)
    if (dw || dbias) return launch_fold(nullptr, 0, C, K, dw, dbias, st);
    return NAJU_OK;
  }
  if (!x || !w || !dy) return fail(NAJU_ERR_INVALID, "null pointer (x, w and dy are required)");
  const bool sums = dw || dbias;
  const size_t need = naju_dwconv_workspace_bytes(batch, T, C, K);
  if (sums && (!workspace || workspace_bytes < need))
    return fail(NAJU_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need,
                workspace ? workspace_bytes : (size_t)0);
  float* part = sums ? (float*)workspace : nullptr;
  int64_t nblk;
  if (dwb_vec_t kv = pick_bwd_vec(x, x_ld, w, bias, dy, dx, dx_ld, dadd, dadd_ld, T, C, K, act, x_dtype, dy_dtype,
                                  dx_dtype, dadd_dtype)) {
    const int64_t ntb = (T + kVRowsB - 1) / kVRowsB;
    const dim3 grid((unsigned)((C + 64 * kBV - 1) / (64 * kBV)), (unsigned)ntb, (unsigned)batch);
    hipLaunchKernelGGL(kv, grid, dim3(64 * kCWB), 0, st, x, x_ld, w, bias, dy, dx, dx_ld, dadd, dadd_ld, part, T, C, acc);
    nblk = batch * ntb;
  } else {
    const dim3 grid((unsigned)((C + kThreads - 1) / kThreads), (unsigned)n_tblocks(T), (unsigned)batch);
    hipLaunchKernelGGL(pick_bwd(K, act == 1), grid, dim3(kThreads), 0, st, x, x_ld, w, bias, dy, dx, dx_ld, dadd,
                       dadd_ld, part, T, C, x_dtype, dy_dtype, dx_dtype, dadd_dtype, acc);
    nblk = batch * n_tblocks(T);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  if (sums) return launch_fold(part, nblk, C, K, dw, dbias, st);
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
  if (readout_vec_ok(n_rows, C, z_ld, {cx, h, z, Dv, y}, {cx_dtype, h_dtype, z_dtype, y_dtype})) {
    const dim3 grid((unsigned)((C + 64 * kRV - 1) / (64 * kRV)), (unsigned)((n_rows + kVRows - 1) / kVRows));
    hipStream_t st = (hipStream_t)stream;
    if (cx_dtype == NAJU_DTYPE_BF16)
      hipLaunchKernelGGL(readout_fwd_vec<bf16_t>, grid, dim3(64), 0, st, (const bf16_t*)cx, (const bf16_t*)h,
                         (const bf16_t*)z, z_ld, Dv, scale, (bf16_t*)y, n_rows, C);
    else if (cx_dtype == NAJU_DTYPE_F16)
      hipLaunchKernelGGL(readout_fwd_vec<f16_t>, grid, dim3(64), 0, st, (const f16_t*)cx, (const f16_t*)h,
                         (const f16_t*)z, z_ld, Dv, scale, (f16_t*)y, n_rows, C);
    else
      hipLaunchKernelGGL(readout_fwd_vec<float>, grid, dim3(64), 0, st, (const float*)cx, (const float*)h,
                         (const float*)z, z_ld, Dv, scale, (float*)y, n_rows, C);
  } else {
    const dim3 grid((unsigned)((C + kThreads - 1) / kThreads), (unsigned)((n_rows + kRows - 1) / kRows));
    hipLaunchKernelGGL(readout_fwd_kernel, grid, dim3(kThreads), 0, (hipStream_t)stream, cx, h, z, z_ld, Dv, scale,
                       y, n_rows, C, cx_dtype, h_dtype, z_dtype, y_dtype);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return NAJU_OK;
}

size_t naju_readout_workspace_bytes(int64_t n_rows, int64_t C) {
  if (n_rows < 0 || C < 0) return 0;
  return (size_t)((n_rows + kVRows - 1) / kVRows) * C * sizeof(float) + 256;
}

int naju_readout_bwd(const void* cx, const void* h, const void* z, int64_t z_ld, const float* Dv, float scale,
                     const void* dy, void* dcx, void* dh, void* dz, int64_t dz_ld, float* dD, int64_t n_rows,
                     int64_t C, int cx_dtype, int h_dtype, int z_dtype, int dy_dtype, int dcx_dtype, int dh_dtype,
                     int dz_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  if (n_rows < 0 || C < 0) return fail(NAJU_ERR_INVALID, "negative shape");
  if (z_ld < C) return fail(NAJU_ERR_INVALID, "z_ld (%lld) must be >= C (%lld)", (long long)z_ld, (long long)C);
  if (dz && dz_ld < C)
    return fail(NAJU_ERR_INVALID, "dz_ld (%lld) must be >= C (%lld)", (long long)dz_ld, (long long)C);
  if (!dt_ok(cx_dtype) || !dt_ok(h_dtype) || !dt_ok(z_dtype) || !dt_ok(dy_dtype) || !dt_ok(dcx_dtype) ||
      !dt_ok(dh_dtype) || !dt_ok(dz_dtype))
    return fail(NAJU_ERR_INVALID, "unknown dtype code");
  if ((n_rows + kRows - 1) / kRows > 65535 || C > (1ll << 30))
    return fail(NAJU_ERR_UNSUPPORTED, "shape too large (at most %d rows)", 65535 * kRows);
  hipStream_t st = (hipStream_t)stream;
  if (C == 0) return NAJU_OK;
  if (n_rows == 0) {
    if (dD) return launch_fold(nullptr, 0, C, 0, nullptr, dD, st);
    return NAJU_OK;
  }
  if (!h || !z || !Dv || !dy) return fail(NAJU_ERR_INVALID, "null pointer (h, z, Dv and dy are required)");
  if (dz && !cx) return fail(NAJU_ERR_INVALID, "cx is required for dz");
  const size_t need = naju_readout_workspace_bytes(n_rows, C);
  if (dD && (!workspace || workspace_bytes < need))
    return fail(NAJU_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need,
                workspace ? workspace_bytes : (size_t)0);
  float* part = dD ? (float*)workspace : nullptr;
  int64_t nblk;
  if (readout_vec_ok(n_rows, C, z_ld, {cx, h, z, Dv, dy, dcx, dh, dz},
                     {h_dtype, z_dtype, dy_dtype, cx ? cx_dtype : h_dtype, dcx ? dcx_dtype : h_dtype,
                      dh ? dh_dtype : h_dtype, dz ? dz_dtype : h_dtype},
                     dz ? dz_ld : 0)) {
    nblk = (n_rows + kVRowsR - 1) / kVRowsR;
    const dim3 grid((unsigned)((C + 64 * kRV - 1) / (64 * kRV)), (unsigned)nblk);
    if (h_dtype == NAJU_DTYPE_BF16)
      hipLaunchKernelGGL(readout_bwd_vec<bf16_t>, grid, dim3(64), 0, st, (const bf16_t*)cx, (const bf16_t*)h,
                         (const bf16_t*)z, z_ld, Dv, scale, (const bf16_t*)dy, (bf16_t*)dcx, (bf16_t*)dh, (bf16_t*)dz,
                         dz_ld, part, n_rows, C);
    else if (h_dtype == NAJU_DTYPE_F16)
      hipLaunchKernelGGL(readout_bwd_vec<f16_t>, grid, dim3(64), 0, st, (const f16_t*)cx, (const f16_t*)h,
                         (const f16_t*)z, z_ld, Dv, scale, (const f16_t*)dy, (f16_t*)dcx, (f16_t*)dh, (f16_t*)dz,
                         dz_ld, part, n_rows, C);
    else
      hipLaunchKernelGGL(readout_bwd_vec<float>, grid, dim3(64), 0, st, (const float*)cx, (const float*)h,
                         (const float*)z, z_ld, Dv, scale, (const float*)dy, (float*)dcx, (float*)dh, (float*)dz,
                         dz_ld, part, n_rows, C);
  } else {
    nblk = (n_rows + kRows - 1) / kRows;
    const dim3 grid((unsigned)((C + kThreads - 1) / kThreads), (unsigned)nblk);
    hipLaunchKernelGGL(readout_bwd_kernel, grid, dim3(kThreads), 0, st, cx, h, z, z_ld, Dv, scale, dy, dcx, dh, dz,
                       dz_ld, part, n_rows, C, cx_dtype, h_dtype, z_dtype, dy_dtype, dcx_dtype, dh_dtype, dz_dtype);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  if (dD) return launch_fold(part, nblk, C, 0, nullptr, dD, st);
  return NAJU_OK;
}


int naju_rmsnorm_fwd(const void* x, const float* w, float eps, void* y, float* rstd, int64_t n_rows, int64_t d,
                     int x_dtype, int y_dtype, void* stream) {
  g_err[0] = 0;
  int rc = norm_check(n_rows, d, x_dtype, {y_dtype}, {x, w, y, rstd});
  if (rc) return rc;
  if (n_rows == 0 || d == 0) return NAJU_OK;
  if (!x || !w || !y || !rstd) return fail(NAJU_ERR_INVALID, "null pointer (x, w, y and rstd are required)");
  const int G = norm_g(d);
  const dim3 grid((unsigned)norm_blocks(n_rows, G));
  hipStream_t st = (hipStream_t)stream;
  if (x_dtype == NAJU_DTYPE_F32)
    norm_fwd_dt<float>(y_dtype, G, grid, st, x, w, eps, y, rstd, n_rows, d);
  else
    norm_fwd_dt<bf16_t>(y_dtype, G, grid, st, x, w, eps, y, rstd, n_rows, d);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return NAJU_OK;
}

size_t naju_rmsnorm_workspace_bytes(int64_t n_rows, int64_t d) {
  if (n_rows < 0 || d < 0) return 0;
  const int G = norm_g(d);
  return (size_t)norm_blocks(n_rows, G ? G : 16) * (size_t)d * sizeof(float) + 256;
}

int naju_rmsnorm_bwd(const void* x, const float* w, const float* rstd, const void* dy, void* dx, float* dw,
                     int64_t n_rows, int64_t d, int x_dtype, int dy_dtype, int dx_dtype, void* workspace,
                     size_t workspace_bytes, void* stream) {
  return naju_rmsnorm_bwd_add(x, w, rstd, dy, nullptr, dx, dw, n_rows, d, x_dtype, dy_dtype, dx_dtype, workspace,
                              workspace_bytes, stream);
}

int naju_rmsnorm_bwd_add(const void* x, const float* w, const float* rstd, const void* dy, const void* dres,
                         void* dx, float* dw, int64_t n_rows, int64_t d, int x_dtype, int dy_dtype, int dx_dtype,
                         void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  int rc = norm_check(n_rows, d, x_dtype, {dy_dtype, dx_dtype}, {x, w, dy, dx, dres, workspace});
  if (rc) return rc;
  if (dx_dtype != x_dtype) return fail(NAJU_ERR_UNSUPPORTED, "dx must have x's dtype");
  if (d == 0) return NAJU_OK;
  hipStream_t st = (hipStream_t)stream;
  if (n_rows == 0) {
    if (dw) return launch_fold(nullptr, 0, d, 0, nullptr, dw, st);
    return NAJU_OK;
  }
  if (!x || !w || !rstd || !dy || !dx)
    return fail(NAJU_ERR_INVALID, "null pointer (x, w, rstd, dy and dx are required)");
  if (dres && dres == dx) return fail(NAJU_ERR_INVALID, "dres must not be dx");
  const size_t need = naju_rmsnorm_workspace_bytes(n_rows, d);
  if (dw && (!workspace || workspace_bytes < need))
    return fail(NAJU_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need,
                workspace ? workspace_bytes : (size_t)0);
  const int G = norm_g(d);
  const int64_t nblk = norm_blocks(n_rows, G);
  float* part = dw ? (float*)workspace : nullptr;
  if (x_dtype == NAJU_DTYPE_F32)
    norm_bwd_dt<float>(dy_dtype, G, dim3((unsigned)nblk), st, x, w, rstd, dy, dx, dres, part, n_rows, d);
  else
    norm_bwd_dt<bf16_t>(dy_dtype, G, dim3((unsigned)nblk), st, x, w, rstd, dy, dx, dres, part, n_rows, d);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  if (dw) return launch_fold(part, nblk, d, 0, nullptr, dw, st);
  return NAJU_OK;
}

int naju_residual_dropout_fwd(const float* u, const void* mix, const int64_t* seed, float p, float* out, int64_t n,
                              int mix_dtype, void* stream) {
  g_err[0] = 0;
  if (n < 0) return fail(NAJU_ERR_INVALID, "negative size");
  if (!dt_ok(mix_dtype)) return fail(NAJU_ERR_INVALID, "unknown dtype code");
  if (!(p >= 0.f && p < 1.f)) return fail(NAJU_ERR_INVALID, "p must be in [0, 1)");
  if (n == 0) return NAJU_OK;
  if (!u || !mix || !out || (p > 0.f && !seed))
    return fail(NAJU_ERR_INVALID, "null pointer (u, mix and out are required; seed when p > 0)");
  const DropKeep dk = drop_keep(p);
  hipStream_t st = (hipStream_t)stream;
  const bool vec = n % kVec == 0 && al16(u) && al16(mix) && al16(out);
  const int64_t units = vec ? n / kVec : n;
  const dim3 grid((unsigned)((units + 255) / 256));
  if (grid.x == 0 || (units + 255) / 256 > 0x7fffffffll) return fail(NAJU_ERR_UNSUPPORTED, "too many elements");
  resdrop_t k;
  if (mix_dtype == NAJU_DTYPE_F32)
    k = vec ? (resdrop_t)residual_dropout_kernel<float, true> : (resdrop_t)residual_dropout_kernel<float, false>;
  else if (mix_dtype == NAJU_DTYPE_BF16)
    k = vec ? (resdrop_t)residual_dropout_kernel<bf16_t, true> : (resdrop_t)residual_dropout_kernel<bf16_t, false>;
  else
    k = vec ? (resdrop_t)residual_dropout_kernel<f16_t, true> : (resdrop_t)residual_dropout_kernel<f16_t, false>;
  hipLaunchKernelGGL(k, grid, dim3(256), 0, st, u, mix, p > 0.f ? seed : nullptr, dk, out, n);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? NAJU_OK : fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
}

int naju_dropout_bwd(const float* g, const int64_t* seed, float p, void* dmix, int64_t n, int mix_dtype,
                     void* stream) {
  g_err[0] = 0;
  if (n < 0) return fail(NAJU_ERR_INVALID, "negative size");
  if (!dt_ok(mix_dtype)) return fail(NAJU_ERR_INVALID, "unknown dtype code");
  if (!(p >= 0.f && p < 1.f)) return fail(NAJU_ERR_INVALID, "p must be in [0, 1)");
  if (n == 0) return NAJU_OK;
  if (!g || !dmix || (p > 0.f && !seed))
    return fail(NAJU_ERR_INVALID, "null pointer (g and dmix are required; seed when p > 0)");
  const DropKeep dk = drop_keep(p);
  hipStream_t st = (hipStream_t)stream;
  const bool vec = n % kVec == 0 && al16(g) && al16(dmix);
  const int64_t units = vec ? n / kVec : n;
  const dim3 grid((unsigned)((units + 255) / 256));
  if ((units + 255) / 256 > 0x7fffffffll) return fail(NAJU_ERR_UNSUPPORTED, "too many elements");
  dropbwd_t k;
  if (mix_dtype == NAJU_DTYPE_F32)
    k = vec ? (dropbwd_t)dropout_bwd_kernel<float, true> : (dropbwd_t)dropout_bwd_kernel<float, false>;
  else if (mix_dtype == NAJU_DTYPE_BF16)
    k = vec ? (dropbwd_t)dropout_bwd_kernel<bf16_t, true> : (dropbwd_t)dropout_bwd_kernel<bf16_t, false>;
  else
    k = vec ? (dropbwd_t)dropout_bwd_kernel<f16_t, true> : (dropbwd_t)dropout_bwd_kernel<f16_t, false>;
  hipLaunchKernelGGL(k, grid, dim3(256), 0, st, g, p > 0.f ? seed : nullptr, dk, dmix, n);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? NAJU_OK : fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
}

int naju_sum_parts(const float* parts, int n_parts, int64_t n, float* out, void* stream) {
  g_err[0] = 0;
  if (n < 0) return fail(NAJU_ERR_INVALID, "negative size");
  if (n_parts < 1 || n_parts > kMaxParts) return fail(NAJU_ERR_INVALID, "n_parts must be in [1, %d]", kMaxParts);
  if (n == 0) return NAJU_OK;
  if (!parts || !out) return fail(NAJU_ERR_INVALID, "null pointer");
  if ((n + 255) / 256 > 0x7fffffff) return fail(NAJU_ERR_UNSUPPORTED, "too many entries (%lld)", (long long)n);
  hipStream_t st = (hipStream_t)stream;
  const int64_t n4 = n / 4;
  const dim3 g4((unsigned)((n4 + 255) / 256));
  const bool vec = n % 4 == 0 && al16(parts) && al16(out);
  const float4* p4 = (const float4*)parts;
  float4* o4 = (float4*)out;
  if (vec && n_parts == 2) {
    hipLaunchKernelGGL(sum_parts_vec<2>, g4, dim3(256), 0, st, p4, n4, o4);
  } else if (vec && n_parts == 4) {
    hipLaunchKernelGGL(sum_parts_vec<4>, g4, dim3(256), 0, st, p4, n4, o4);
  } else if (vec && n_parts == 8) {
    hipLaunchKernelGGL(sum_parts_vec<8>, g4, dim3(256), 0, st, p4, n4, o4);
  } else if (vec && n_parts == 16) {
    hipLaunchKernelGGL(sum_parts_vec<16>, g4, dim3(256), 0, st, p4, n4, o4);
  } else {
    hipLaunchKernelGGL(sum_parts_any, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, parts, n_parts, n, out);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return NAJU_OK;
}

int naju_embedding_bwd_add(const int64_t* sorted_ids, const int64_t* order, const float* dy, int64_t n, int64_t d,
                           float* dw, int64_t V, void* stream) {
  g_err[0] = 0;
  if (n < 0 || d < 0 || V < 0) return fail(NAJU_ERR_INVALID, "negative size");
  if (n == 0 || d == 0) return NAJU_OK;
  if (!sorted_ids || !order || !dy || !dw) return fail(NAJU_ERR_INVALID, "null pointer");
  if (n > 0x7fffffff) return fail(NAJU_ERR_UNSUPPORTED, "too many ids (%lld)", (long long)n);
  hipLaunchKernelGGL(embed_bwd_add_kernel, dim3((unsigned)n), dim3(256), 0, (hipStream_t)stream, sorted_ids, order,
                     dy, n, d, dw, V);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return NAJU_OK;
}

}  // extern "C"

// ---- the gate pair (dwconv4_pair_*): host side
namespace {
bool pair_ok(int64_t T, int64_t C, int K, std::initializer_list<int64_t> lds, std::initializer_list<const void*> ptrs) {
  if (K != 4 || C % kVec || (T + kCRF - 1) / kCRF > 65535 || (T + kVRowsB - 1) / kVRowsB > 65535) return false;
  for (int64_t ld : lds)
    if (ld % kVec) return false;
  for (const void* p : ptrs)
    if (p && !al16(p)) return false;
  return true;
}

template <typename TX, typename TY>
void pair_fwd_launch(dim3 grid, hipStream_t st, const void* x, int64_t x_ld, const float* w0, const float* b0,
                     const float* w1, const float* b1, const void* add0, const void* add1, int64_t add_ld, void* y0,
                     void* y1, int64_t T, int64_t C) {
  hipLaunchKernelGGL((dwconv4_pair_fwd_vec<TX, TY>), grid, dim3(64), 0, st, (const TX*)x, x_ld, w0, b0, w1, b1,
                     (const TX*)add0, (const TX*)add1, add_ld, (TY*)y0, (TY*)y1, T, C);
}

template <typename TX>
void pair_fwd_dt(int y_dt, dim3 grid, hipStream_t st, const void* x, int64_t x_ld, const float* w0, const float* b0,
                 const float* w1, const float* b1, const void* add0, const void* add1, int64_t add_ld, void* y0,
                 void* y1, int64_t T, int64_t C) {
  if (y_dt == NAJU_DTYPE_F32)
    pair_fwd_launch<TX, float>(grid, st, x, x_ld, w0, b0, w1, b1, add0, add1, add_ld, y0, y1, T, C);
  else
    pair_fwd_launch<TX, TX>(grid, st, x, x_ld, w0, b0, w1, b1, add0, add1, add_ld, y0, y1, T, C);
}

template <typename TX, typename TDY>
void pair_bwd_launch(dim3 grid, hipStream_t st, const void* x, int64_t x_ld, const float* w0, const float* w1,
                     const void* dy0, const void* dy1, int64_t dy_ld, void* dx, int64_t dx_ld, void* dadd0,
                     void* dadd1, int64_t dadd_ld, float* part0, float* part1, int64_t T, int64_t C, int acc) {
  hipLaunchKernelGGL((dwconv4_pair_bwd_vec<TX, TDY>), grid, dim3(64 * kPW), 0, st, (const TX*)x, x_ld, w0, w1,
                     (const TDY*)dy0, (const TDY*)dy1, dy_ld, (TX*)dx, dx_ld, (TX*)dadd0, (TX*)dadd1, dadd_ld, part0,
                     part1, T, C, acc);
}

template <typename TX>
void pair_bwd_dt(int dy_dt, dim3 grid, hipStream_t st, const void* x, int64_t x_ld, const float* w0,
                 const float* w1, const void* dy0, const void* dy1, int64_t dy_ld, void* dx, int64_t dx_ld,
                 void* dadd0, void* dadd1, int64_t dadd_ld, float* part0, float* part1, int64_t T, int64_t C,
                 int acc) {
  if (dy_dt == NAJU_DTYPE_F32 && !std::is_same<TX, float>::value)
    pair_bwd_launch<TX, float>(grid, st, x, x_ld, w0, w1, dy0, dy1, dy_ld, dx, dx_ld, dadd0, dadd1, dadd_ld, part0,
                               part1, T, C, acc);
  else
    pair_bwd_launch<TX, TX>(grid, st, x, x_ld, w0, w1, dy0, dy1, dy_ld, dx, dx_ld, dadd0, dadd1, dadd_ld, part0,
                            part1, T, C, acc);
}
}  // namespace

extern "C" {

int naju_dwconv_pair_fwd(const void* x, int64_t x_ld, const float* w0, const float* bias0, const void* add0,
                         const float* w1, const float* bias1, const void* add1, int64_t add_ld, void* y0, void* y1,
                         int64_t batch, int64_t T, int64_t C, int K, int x_dtype, int y_dtype, void* stream) {
  g_err[0] = 0;
  int rc = check(batch, T, C, K, 0, x_ld);
  if (rc) return rc;
  if (add_ld < C) return fail(NAJU_ERR_INVALID, "add_ld (%lld) must be >= C (%lld)", (long long)add_ld, (long long)C);
  if (!dt_ok(x_dtype) || !dt_ok(y_dtype)) return fail(NAJU_ERR_INVALID, "unknown dtype code");
  if (y_dtype != x_dtype && y_dtype != NAJU_DTYPE_F32)
    return fail(NAJU_ERR_UNSUPPORTED, "y must have x's dtype or float32");
  if (batch == 0 || T == 0 || C == 0) return NAJU_OK;
  if (!x || !w0 || !w1 || !add0 || !add1 || !y0 || !y1)
    return fail(NAJU_ERR_INVALID, "null pointer (x, both weights, adds and outputs are required)");
  if (!pair_ok(T, C, K, {x_ld, add_ld}, {x, w0, w1, bias0, bias1, add0, add1, y0, y1}))
    return fail(NAJU_ERR_UNSUPPORTED,
                "the pair kernels need K = 4, C and the row strides multiples of 8 and 16-byte aligned pointers");
  const dim3 grid((unsigned)((C + 64 * kFV4 - 1) / (64 * kFV4)), (unsigned)((T + kCRF - 1) / kCRF), (unsigned)batch);
  hipStream_t st = (hipStream_t)stream;
  if (x_dtype == NAJU_DTYPE_BF16)
    pair_fwd_dt<bf16_t>(y_dtype, grid, st, x, x_ld, w0, bias0, w1, bias1, add0, add1, add_ld, y0, y1, T, C);
  else if (x_dtype == NAJU_DTYPE_F16)
    pair_fwd_dt<f16_t>(y_dtype, grid, st, x, x_ld, w0, bias0, w1, bias1, add0, add1, add_ld, y0, y1, T, C);
  else
    pair_fwd_dt<float>(y_dtype, grid, st, x, x_ld, w0, bias0, w1, bias1, add0, add1, add_ld, y0, y1, T, C);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return NAJU_OK;
}

size_t naju_dwconv_pair_workspace_bytes(int64_t batch, int64_t T, int64_t C, int K) {
  const size_t one = naju_dwconv_workspace_bytes(batch, T, C, K);
  return one ? 2 * one : 0;
}

int naju_dwconv_pair_bwd(const void* x, int64_t x_ld, const float* w0, const float* w1, const void* dy0,
                         const void* dy1, int64_t dy_ld, void* dx, int64_t dx_ld, float* dw0, float* dbias0, float* dw1,
                         float* dbias1, void* dadd0, void* dadd1, int64_t dadd_ld, int64_t batch, int64_t T,
                         int64_t C, int K, int accumulate, int x_dtype, int dy_dtype, void* workspace,
                         size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  int rc = check(batch, T, C, K, 0, x_ld);
  if (rc) return rc;
  if (dx && dx_ld < C) return fail(NAJU_ERR_INVALID, "dx_ld (%lld) must be >= C (%lld)", (long long)dx_ld, (long long)C);
  if ((dadd0 || dadd1) && dadd_ld < C)
    return fail(NAJU_ERR_INVALID, "dadd_ld (%lld) must be >= C (%lld)", (long long)dadd_ld, (long long)C);
  if (dy_ld < C) return fail(NAJU_ERR_INVALID, "dy_ld (%lld) must be >= C (%lld)", (long long)dy_ld, (long long)C);
  if (!dt_ok(x_dtype) || !dt_ok(dy_dtype)) return fail(NAJU_ERR_INVALID, "unknown dtype code");
  if (dy_dtype != x_dtype && dy_dtype != NAJU_DTYPE_F32)
    return fail(NAJU_ERR_UNSUPPORTED, "dy must have x's dtype or float32");
  hipStream_t st = (hipStream_t)stream;
  if (C == 0) return NAJU_OK;
  const bool sums = dw0 || dbias0 || dw1 || dbias1;
  if (batch == 0 || T == 0) {
    // empty sums: the folds over zero blocks write the zeros
    if (dw0 || dbias0) {
      if ((rc = launch_fold(nullptr, 0, C, K, dw0, dbias0, st))) return rc;
    }
    if (dw1 || dbias1) return launch_fold(nullptr, 0, C, K, dw1, dbias1, st);
    return NAJU_OK;
  }
  if (!x || !w0 || !w1 || !dy0 || !dy1) return fail(NAJU_ERR_INVALID, "null pointer (x, weights and dy are required)");
  if (!pair_ok(T, C, K, {x_ld, dy_ld, dx ? dx_ld : C, (dadd0 || dadd1) ? dadd_ld : C},
               {x, w0, w1, dy0, dy1, dx, dadd0, dadd1}))
    return fail(NAJU_ERR_UNSUPPORTED,
                "the pair kernels need K = 4, C and the row strides multiples of 8 and 16-byte aligned pointers");
  const size_t one = naju_dwconv_workspace_bytes(batch, T, C, K);
  if (sums && (!workspace || workspace_bytes < 2 * one))
    return fail(NAJU_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", 2 * one,
                workspace ? workspace_bytes : (size_t)0);
  // the second part array starts 16-byte aligned (one = rows * C * (K+1) floats + 256, C % 8 == 0)
  float* part0 = (dw0 || dbias0) ? (float*)workspace : nullptr;
  float* part1 = (dw1 || dbias1) ? (float*)((char*)workspace + one) : nullptr;
  const int64_t ntb = (T + kVRowsB - 1) / kVRowsB;
  const dim3 grid((unsigned)((C + 64 * kPV - 1) / (64 * kPV)), (unsigned)ntb, (unsigned)batch);
  const int acc = accumulate ? 1 : 0;
  if (x_dtype == NAJU_DTYPE_BF16)
    pair_bwd_dt<bf16_t>(dy_dtype, grid, st, x, x_ld, w0, w1, dy0, dy1, dy_ld, dx, dx_ld, dadd0, dadd1, dadd_ld,
                        part0, part1, T, C, acc);
  else if (x_dtype == NAJU_DTYPE_F16)
    pair_bwd_dt<f16_t>(dy_dtype, grid, st, x, x_ld, w0, w1, dy0, dy1, dy_ld, dx, dx_ld, dadd0, dadd1, dadd_ld,
                       part0, part1, T, C, acc);
  else
    pair_bwd_dt<float>(dy_dtype, grid, st, x, x_ld, w0, w1, dy0, dy1, dy_ld, dx, dx_ld, dadd0, dadd1, dadd_ld,
                       part0, part1, T, C, acc);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  const int64_t nblk = batch * ntb;
  if (part0 && part1) return launch_fold(part0, nblk, C, K, dw0, dbias0, st, part1, dw1, dbias1);
  if (part0) return launch_fold(part0, nblk, C, K, dw0, dbias0, st);
  if (part1) return launch_fold(part1, nblk, C, K, dw1, dbias1, st);
  return NAJU_OK;
}

}  // extern "C"
