// naju_loss.hip -- cross-entropy of the Naju LM training step on MI355X
// (gfx950), behind the C ABI of include/naju_loss.h.
//
// The reference computes nn.functional.cross_entropy on the logits under bf16
// autocast (/root/reference/evals/lm/train.py:74): torch upcasts the bf16
// logits to a float32 copy, runs log_softmax (one read, one float32 write),
// nll_loss, and in the backward the softmax gradient in float32 plus a cast
// back to bf16 -- about five passes over an n_rows x V tensor that is 1.6 GB
// in bf16 at the LM configuration (16384 x 50257). Here the forward is one
// read of the logits in their own dtype (an online max / sum-of-exponentials
// per row, then a fixed-order mean), and the backward one read plus one write
// in the logits' dtype, with the loss gradient taken from device memory.
//
// One workgroup per row: lanes stream 16-byte vectors (8 bf16 / 4 fp32) of
// the row, with the row's unaligned head and tail (rows of an odd width start
// at any 2-byte boundary) handled element by element.
#include <hip/hip_runtime.h>

#include <type_traits>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "naju_loss.h"
#include "naju_scan.h"

namespace {

typedef __bf16 bf16_t;
typedef _Float16 f16_t;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kUnroll = 4;  // 16-byte vectors per lane in flight
constexpr float kLog2e = 1.4426950408889634f;

template <typename T>
__device__ __forceinline__ float tof(T v) {
  return (float)v;
}
template <typename T>
__device__ __forceinline__ T fromf(float v) {
  return (T)v;
}

__device__ __forceinline__ float exp2_(float x) { return __builtin_amdgcn_exp2f(x); }

// (m, s): the running maximum and sum_i exp(v_i - m) of a set of values.
// Empty sets are (-inf, 0). Merging is symmetric in its two operands.
__device__ __forceinline__ void ms_merge(float& m, float& s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  s = s * exp2_((m - mn) * kLog2e) + s2 * exp2_((m2 - mn) * kLog2e);
  m = mn;
}

template <int N>
__device__ __forceinline__ void ms_add(float& m, float& s, const float (&v)[N]) {
  float mm = v[0];
#pragma unroll
  for (int i = 1; i < N; ++i) mm = fmaxf(mm, v[i]);
  const float mn = fmaxf(m, mm);
  if (mn == -INFINITY) return;
  float acc = s * exp2_((m - mn) * kLog2e);
#pragma unroll
  for (int i = 0; i < N; ++i) acc += exp2_((v[i] - mn) * kLog2e);
  s = acc;
  m = mn;
}

// Elements of a row before its first 16-byte boundary (at most n).
template <typename T>
__device__ __forceinline__ int64_t head_elems(const T* p, int64_t n) {
  constexpr int E = 16 / sizeof(T);
  const int mis = (int)(((uintptr_t)p & 15) / sizeof(T));
  const int64_t h = (E - mis) % E;
  return h < n ? h : n;
}

// Forward of row blockIdx.x by the workgroup: lse, the row's loss and
// validity; the lse also into *s_l (LDS, visible after a barrier).
template <typename T>
__device__ __forceinline__ void xent_row_fwd(const T* __restrict__ x, int64_t ld, const int64_t* __restrict__ target,
                                             int64_t n_cols, int64_t ignore, float* __restrict__ lse,
                                             float* __restrict__ row_loss, float* __restrict__ row_valid,
                                             float* s_l) {
  constexpr int E = 16 / sizeof(T);
  typedef T vec_t __attribute__((ext_vector_type(E)));
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const T* p = x + r * ld;
  const int64_t head = head_elems(p, n_cols);
  const int64_t nvec = (n_cols - head) / E;
  const int64_t tail0 = head + nvec * E;

  float m = -INFINITY, s = 0.f;
  if (tid < head) {
    const float v[1] = {tof(p[tid])};
    ms_add(m, s, v);
  }
  if (tail0 + tid < n_cols) {
    const float v[1] = {tof(p[tail0 + tid])};
    ms_add(m, s, v);
  }
  const vec_t* q = reinterpret_cast<const vec_t*>(p + head);
  int64_t i = tid;
  for (; i + (kUnroll - 1) * kThreads < nvec; i += kUnroll * kThreads) {
    vec_t a[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) a[u] = q[i + u * kThreads];
    float v[kUnroll * E];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int e = 0; e < E; ++e) v[u * E + e] = tof(a[u][e]);
    ms_add(m, s, v);
  }
  for (; i < nvec; i += kThreads) {
    const vec_t a = q[i];
    float v[E];
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = tof(a[e]);
    ms_add(m, s, v);
  }

  // workgroup-wide merge: butterfly within each wave, then the waves in order
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ms_merge(m, s, __shfl_xor(m, off, 64), __shfl_xor(s, off, 64));
  __shared__ float sm[kWaves], ss[kWaves];
  const int lane = tid & 63, wv = tid >> 6;
  if (lane == 0) {
    sm[wv] = m;
    ss[wv] = s;
  }
  __syncthreads();
  if (tid == 0) {
    float M = sm[0], S = ss[0];
    for (int w = 1; w < kWaves; ++w) ms_merge(M, S, sm[w], ss[w]);
    const float l = M + logf(S);
    lse[r] = l;
    *s_l = l;
    const int64_t t = target[r];
    float loss = 0.f, valid = 0.f;
    if (t != ignore) {
      valid = 1.f;
      loss = (t >= 0 && t < n_cols) ? l - tof(p[t]) : __builtin_nanf("");
    }
    row_loss[r] = loss;
    row_valid[r] = valid;
  }
}

// grid: n_rows workgroups of kThreads.
template <typename T>
__global__ __launch_bounds__(kThreads) void xent_fwd_kernel(const T* __restrict__ x, int64_t ld,
                                                            const int64_t* __restrict__ target, int64_t n_cols,
                                                            int64_t ignore, float* __restrict__ lse,
                                                            float* __restrict__ row_loss,
                                                            float* __restrict__ row_valid) {
  __shared__ float s_l;
  xent_row_fwd<T>(x, ld, target, n_cols, ignore, lse, row_loss, row_valid, &s_l);
}

// One workgroup: loss = sum(row_loss) / sum(row_valid), scale = 1 / count,
// summed in float64 in a fixed order.
__global__ __launch_bounds__(1024) void xent_mean_kernel(const float* __restrict__ row_loss,
                                                         const float* __restrict__ row_valid, int64_t n,
                                                         float* __restrict__ loss, float* __restrict__ scale) {
  __shared__ double sa[1024], sc[1024];
  const int t = threadIdx.x;
  double a = 0.0, c = 0.0;
  for (int64_t i = t; i < n; i += 1024) {
    a += row_loss[i];
    c += row_valid[i];
  }
  sa[t] = a;
  sc[t] = c;
  __syncthreads();
  for (int w = 512; w >= 1; w >>= 1) {
    if (t < w) {
      sa[t] += sa[t + w];
      sc[t] += sc[t + w];
    }
    __syncthreads();
  }
  if (t == 0) {
    loss[0] = (float)(sa[0] / sc[0]);  // 0 / 0 = NaN when no row is valid
    scale[0] = sc[0] > 0.0 ? (float)(1.0 / sc[0]) : 0.f;
  }
}

// Row r of the gradient: dx[c] = g * (exp(x[c] - lse) - [c == t]), 0 for an
// ignored row (t == ignore); g is NaN for a target outside [0, n_cols).
template <typename T, typename TD>
__device__ __forceinline__ void grad_row(const T* __restrict__ p, TD* __restrict__ d, int64_t t, int64_t n_cols,
                                         int64_t ignore, float g, float l, int tid) {
  if (t == ignore) {
    for (int64_t c = tid; c < n_cols; c += kThreads) d[c] = fromf<TD>(0.f);
    return;
  }
  auto grad = [&](float v, int64_t c) {
    const float e = exp2_((v - l) * kLog2e) * g;
    return c == t ? e - g : e;
  };

  constexpr int E = 16 / sizeof(T);
  const int64_t head = head_elems(p, n_cols);
  const bool vec = sizeof(T) == sizeof(TD) && head == head_elems(reinterpret_cast<const T*>(d), n_cols);
  if (!vec) {
    for (int64_t c = tid; c < n_cols; c += kThreads) d[c] = fromf<TD>(grad(tof(p[c]), c));
    return;
  }
  typedef T vec_t __attribute__((ext_vector_type(E)));
  typedef TD dvec_t __attribute__((ext_vector_type(E)));
  const int64_t nvec = (n_cols - head) / E;
  const int64_t tail0 = head + nvec * E;
  if (tid < head) d[tid] = fromf<TD>(grad(tof(p[tid]), tid));
  if (tail0 + tid < n_cols) d[tail0 + tid] = fromf<TD>(grad(tof(p[tail0 + tid]), tail0 + tid));
  const vec_t* q = reinterpret_cast<const vec_t*>(p + head);
  dvec_t* o = reinterpret_cast<dvec_t*>(d + head);
  int64_t i = tid;
  for (; i + (kUnroll - 1) * kThreads < nvec; i += kUnroll * kThreads) {
    vec_t a[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) a[u] = q[i + u * kThreads];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t c0 = head + (i + u * kThreads) * E;
      dvec_t w;
#pragma unroll
      for (int e = 0; e < E; ++e) w[e] = fromf<TD>(grad(tof(a[u][e]), c0 + e));
      o[i + u * kThreads] = w;
    }
  }
  for (; i < nvec; i += kThreads) {
    const vec_t a = q[i];
    const int64_t c0 = head + i * E;
    dvec_t w;
#pragma unroll
    for (int e = 0; e < E; ++e) w[e] = fromf<TD>(grad(tof(a[e]), c0 + e));
    o[i] = w;
  }
}

// grid: n_rows workgroups of kThreads. g = dloss * scale. With if_scaled
// (the forward already wrote dx for dloss = 1) a workgroup returns at once
// when dloss is 1.
template <typename T, typename TD>
__global__ __launch_bounds__(kThreads) void xent_bwd_kernel(const T* __restrict__ x, int64_t ld,
                                                            const int64_t* __restrict__ target, int64_t n_cols,
                                                            int64_t ignore, const float* __restrict__ lse,
                                                            const float* __restrict__ scale,
                                                            const float* __restrict__ dloss, TD* __restrict__ dx,
                                                            int64_t dld, int if_scaled) {
  if (if_scaled && dloss[0] == 1.f) return;
  const int64_t r = blockIdx.x;
  const int64_t t = target[r];
  const float g = (t >= 0 && t < n_cols) ? dloss[0] * scale[0] : __builtin_nanf("");
  grad_row<T, TD>(x + r * ld, dx + r * dld, t, n_cols, ignore, g, t == ignore ? 0.f : lse[r], threadIdx.x);
}

// One workgroup: scale = 1 / (number of rows with target != ignore), the
// count summed in float64 in a fixed order (the value xent_mean_kernel gives).
__global__ __launch_bounds__(1024) void xent_count_kernel(const int64_t* __restrict__ target, int64_t n,
                                                          int64_t ignore, float* __restrict__ scale) {
  __shared__ double sc[1024];
  const int t = threadIdx.x;
  double c = 0.0;
  for (int64_t i = t; i < n; i += 1024) c += target[i] != ignore ? 1.0 : 0.0;
  sc[t] = c;
  __syncthreads();
  for (int w = 512; w >= 1; w >>= 1) {
    if (t < w) sc[t] += sc[t + w];
    __syncthreads();
  }
  if (t == 0) scale[0] = sc[0] > 0.0 ? (float)(1.0 / sc[0]) : 0.f;
}

// grid: n_rows workgroups of kThreads: the forward of row r (as
// xent_fwd_kernel), then its gradient for dloss = 1 (as xent_bwd_kernel),
// the row read a second time (from the caches when it is still there).
template <typename T, typename TD>
__global__ __launch_bounds__(kThreads) void xent_fwd_grad_kernel(const T* __restrict__ x, int64_t ld,
                                                                 const int64_t* __restrict__ target, int64_t n_cols,
                                                                 int64_t ignore, float* __restrict__ lse,
                                                                 float* __restrict__ row_loss,
                                                                 float* __restrict__ row_valid,
                                                                 const float* __restrict__ scale,
                                                                 TD* __restrict__ dx, int64_t dld) {
  __shared__ float s_l;
  xent_row_fwd<T>(x, ld, target, n_cols, ignore, lse, row_loss, row_valid, &s_l);
  __syncthreads();
  const int64_t r = blockIdx.x;
  const int64_t t = target[r];
  const float g = (t >= 0 && t < n_cols) ? 1.f * scale[0] : __builtin_nanf("");
  grad_row<T, TD>(x + r * ld, dx + r * dld, t, n_cols, ignore, g, s_l, threadIdx.x);
}

// ---------------------------------------------- whole rows held in registers
//
// One workgroup of kRT threads per row for rows of kRegMin .. kRT * NV * E
// classes: every 16-byte vector of the row is loaded once into registers
// (NV per thread, all issued before the first is used), the row's maximum
// and then its sum of exp(x - max) are formed from the registers, and with
// GRAD the gradient for dloss = 1 is written from them too, so the row is
// read from memory once instead of twice. The row's few elements before its
// first 16-byte boundary and after its last whole vector are single loads.
// Sums in a fixed order (per thread in vector order, the wave's lanes by
// butterfly, the waves in wave order), so results repeat bitwise; the
// forward-only and the forward-with-gradient forms run the same reduction,
// so their lse (and with it the backward's gradient) agree bitwise.
constexpr int kRT = 1024;
constexpr int kRW = kRT / 64;
constexpr int64_t kRegMin = 2048;

// Element e of a 16-byte vector of T held as four raw 32-bit words.
template <typename T>
__device__ __forceinline__ float elem(const uint32_t (&w)[4], int e) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(w[e]);
  } else if constexpr (std::is_same<T, bf16_t>::value) {
    const uint32_t u = w[e >> 1];
    return __uint_as_float((e & 1) ? (u & 0xffff0000u) : (u << 16));
  } else {
    const uint16_t h = (uint16_t)((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xffffu));
    return (float)__builtin_bit_cast(f16_t, h);
  }
}

// GRAD: the forward only, or with the gradient stored as vectors (dx rows of
// T's size and the logits' alignment) or element by element.
constexpr int kRegFwd = 0, kRegGradVec = 1, kRegGradElem = 2;

template <typename T, typename TD, int NV, int GRAD>
__global__ __launch_bounds__(kRT) __attribute__((amdgpu_waves_per_eu(8))) void xent_row_reg_kernel(
    const T* __restrict__ x, int64_t ld, const int64_t* __restrict__ target, int64_t n_cols64, int64_t ignore,
    float* __restrict__ lse, float* __restrict__ row_loss, float* __restrict__ row_valid,
    const float* __restrict__ scale, TD* __restrict__ dx, int64_t dld) {
  constexpr int E = 16 / sizeof(T);
  __shared__ float s_red[kRW];
  __shared__ float s_bc[2];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6;
  // 32-bit column indices: rows of at most kRT * NV * E elements
  const int n_cols = (int)n_cols64;
  const T* p = x + r * ld;
  const int head = (int)head_elems(p, n_cols64);
  const int nvec = (n_cols - head) / E;
  const int tail0 = head + nvec * E;
  const uint4* q = reinterpret_cast<const uint4*>(p + head);
  // the row as loaded (raw words, four per vector), converted where used:
  // floats kept from one pass to the next would double the registers and
  // leave room for one workgroup per compute unit
  uint32_t a[NV][4];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = tid + k * kRT;
    const uint4 v = q[i < nvec ? i : (nvec > 0 ? nvec - 1 : 0)];
    a[k][0] = v.x, a[k][1] = v.y, a[k][2] = v.z, a[k][3] = v.w;
  }
  // keeps the compiler from carrying converted values across the passes
  auto fence = [&]() {
#pragma unroll
    for (int k = 0; k < NV; ++k) asm volatile("" : "+v"(a[k][0]), "+v"(a[k][1]), "+v"(a[k][2]), "+v"(a[k][3]));
  };
  const float hv = tid < head ? tof(p[tid]) : -INFINITY;
  const float tv = tail0 + tid < n_cols ? tof(p[tail0 + tid]) : -INFINITY;
  auto valid = [&](int k) { return tid + k * kRT < nvec; };

  // the row's maximum
  float m = fmaxf(hv, tv);
#pragma unroll
  for (int k = 0; k < NV; ++k)
    if (valid(k))
#pragma unroll
      for (int e = 0; e < E; ++e) m = fmaxf(m, elem<T>(a[k], e));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if (lane == 0) s_red[wv] = m;
  __syncthreads();
  if (tid == 0) {
    float M = s_red[0];
    for (int w = 1; w < kRW; ++w) M = fmaxf(M, s_red[w]);
    s_bc[0] = M;
  }
  __syncthreads();
  const float M = s_bc[0];
  fence();

  // sum of exp(x - max); an all -inf row sums to 0 (lse -inf)
  float sum = 0.f;
  if (M != -INFINITY) {
    auto ex = [&](float v) { return exp2_((v - M) * kLog2e); };
    if (tid < head) sum += ex(hv);
#pragma unroll
    for (int k = 0; k < NV; ++k)
      if (valid(k))
#pragma unroll
        for (int e = 0; e < E; ++e) sum += ex(elem<T>(a[k], e));
    if (tail0 + tid < n_cols) sum += ex(tv);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
  if (lane == 0) s_red[wv] = sum;  // thread 0 read the maxima before the last barrier
  __syncthreads();
  const int64_t t = target[r];
  if (tid == 0) {
    float S = s_red[0];
    for (int w = 1; w < kRW; ++w) S += s_red[w];
    const float l = M + logf(S);
    lse[r] = l;
    s_bc[1] = l;
    float loss = 0.f, vld = 0.f;
    if (t != ignore) {
      vld = 1.f;
      loss = (t >= 0 && t < n_cols64) ? l - tof(p[t]) : __builtin_nanf("");
    }
    row_loss[r] = loss;
    row_valid[r] = vld;
  }
  if constexpr (GRAD != kRegFwd) {
    fence();
    __syncthreads();
    const float l = s_bc[1];
    TD* d = dx + r * dld;
    // as grad_row: g * exp(x - lse), minus g at the target; an ignored row's
    // gradient is 0 (selected, so that no branch splits the passes)
    const bool ign = t == ignore;
    const bool tin = t >= 0 && t < n_cols64;
    const float g = tin ? 1.f * scale[0] : __builtin_nanf("");
    const int t32 = tin ? (int)t : -1;  // the target's column (none: -1)
    auto grad = [&](float v, int c) {
      const float e = exp2_((v - l) * kLog2e) * g;
      return ign ? 0.f : (c == t32 ? e - g : e);
    };
    if (tid < head) d[tid] = fromf<TD>(grad(hv, tid));
    if (tail0 + tid < n_cols) d[tail0 + tid] = fromf<TD>(grad(tv, tail0 + tid));
    typedef TD dvec_t __attribute__((ext_vector_type(E)));
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      if (!valid(k)) continue;
      const int i = tid + k * kRT;
      const int c0 = head + i * E;
      if constexpr (GRAD == kRegGradVec) {
        dvec_t w;
#pragma unroll
        for (int e = 0; e < E; ++e) w[e] = fromf<TD>(grad(elem<T>(a[k], e), c0 + e));
        reinterpret_cast<dvec_t*>(d + head)[i] = w;
        // the later vectors' work stays after this store (computed ahead,
        // their results would need registers of their own)
#pragma unroll
        for (int kk = k + 1; kk < NV; ++kk)
          asm volatile("" : "+v"(a[kk][0]), "+v"(a[kk][1]), "+v"(a[kk][2]), "+v"(a[kk][3]));
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) d[c0 + e] = fromf<TD>(grad(elem<T>(a[k], e), c0 + e));
      }
    }
  }
}

// Vectors per thread of the register kernel for rows of n_cols elements of
// `size` bytes, or 0 when the row takes the two-pass kernels.
int reg_nv(int64_t n_cols, int size) {
  const int64_t e = 16 / size;
  if (n_cols < kRegMin) return 0;
  for (int nv : {2, 4, 7})
    if (n_cols <= kRT * nv * e) return nv;
  return 0;
}

template <typename T, typename TD, int GRAD>
void launch_reg(int nv, const void* x, int64_t ld, const int64_t* tgt, int64_t rows, int64_t cols, int64_t ignore,
                float* lse, float* rl, float* rv, const float* scale, void* dx, int64_t dld, hipStream_t st) {
  const dim3 g((unsigned)rows), b(kRT);
  if (nv == 2)
    xent_row_reg_kernel<T, TD, 2, GRAD><<<g, b, 0, st>>>((const T*)x, ld, tgt, cols, ignore, lse, rl, rv, scale,
                                                         (TD*)dx, dld);
  else if (nv == 4)
    xent_row_reg_kernel<T, TD, 4, GRAD><<<g, b, 0, st>>>((const T*)x, ld, tgt, cols, ignore, lse, rl, rv, scale,
                                                         (TD*)dx, dld);
  else
    xent_row_reg_kernel<T, TD, 7, GRAD><<<g, b, 0, st>>>((const T*)x, ld, tgt, cols, ignore, lse, rl, rv, scale,
                                                         (TD*)dx, dld);
}

// Whether every row of dx starts at the same offset from a 16-byte boundary
// as the same row of x (then the register kernel stores the gradient as
// vectors): same element size, same base offset, row strides congruent.
bool rows_match(const void* x, int64_t ld, int x_size, const void* dx, int64_t dld, int dx_size) {
  if (x_size != dx_size) return false;
  const int64_t e = 16 / x_size;
  return ((uintptr_t)x & 15) == ((uintptr_t)dx & 15) && (ld - dld) % e == 0;
}

// ------------------------------------------------------------------ host side

thread_local char g_err[256] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

bool dt_ok(int dt) { return dt == NAJU_DTYPE_F32 || dt == NAJU_DTYPE_BF16 || dt == NAJU_DTYPE_F16; }

size_t ws_bytes(int64_t n_rows) { return n_rows < 0 ? 0 : (size_t)n_rows * 2 * sizeof(float) + 256; }

int check_shape(int64_t x_ld, int64_t n_rows, int64_t n_cols, int x_dtype) {
  if (n_rows < 0 || n_cols < 0) return fail(NAJU_ERR_INVALID, "negative shape");
  if (x_ld < n_cols) return fail(NAJU_ERR_INVALID, "x_ld (%lld) must be >= n_cols (%lld)", (long long)x_ld,
                                 (long long)n_cols);
  if (!dt_ok(x_dtype)) return fail(NAJU_ERR_INVALID, "unknown dtype code");
  if (n_rows > 0x7fffffff) return fail(NAJU_ERR_UNSUPPORTED, "at most 2^31-1 rows");
  return NAJU_OK;
}

int launched() {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return NAJU_OK;
}

template <typename T>
void launch_fwd(const void* x, int64_t ld, const int64_t* tgt, int64_t rows, int64_t cols, int64_t ignore,
                float* lse, float* rl, float* rv, hipStream_t st) {
  if (const int nv = reg_nv(cols, sizeof(T))) {
    launch_reg<T, T, kRegFwd>(nv, x, ld, tgt, rows, cols, ignore, lse, rl, rv, nullptr, nullptr, 0, st);
    return;
  }
  xent_fwd_kernel<T><<<dim3((unsigned)rows), dim3(kThreads), 0, st>>>((const T*)x, ld, tgt, cols, ignore, lse, rl,
                                                                      rv);
}

template <typename T, typename TD>
void launch_bwd(const void* x, int64_t ld, const int64_t* tgt, int64_t rows, int64_t cols, int64_t ignore,
                const float* lse, const float* scale, const float* dloss, void* dx, int64_t dld, int if_scaled,
                hipStream_t st) {
  xent_bwd_kernel<T, TD><<<dim3((unsigned)rows), dim3(kThreads), 0, st>>>((const T*)x, ld, tgt, cols, ignore, lse,
                                                                          scale, dloss, (TD*)dx, dld, if_scaled);
}

template <typename T>
void launch_bwd_dt(int dx_dt, const void* x, int64_t ld, const int64_t* tgt, int64_t rows, int64_t cols,
                   int64_t ignore, const float* lse, const float* scale, const float* dloss, void* dx, int64_t dld,
                   int if_scaled, hipStream_t st) {
  if (dx_dt == NAJU_DTYPE_F32)
    launch_bwd<T, float>(x, ld, tgt, rows, cols, ignore, lse, scale, dloss, dx, dld, if_scaled, st);
  else if (dx_dt == NAJU_DTYPE_BF16)
    launch_bwd<T, bf16_t>(x, ld, tgt, rows, cols, ignore, lse, scale, dloss, dx, dld, if_scaled, st);
  else
    launch_bwd<T, f16_t>(x, ld, tgt, rows, cols, ignore, lse, scale, dloss, dx, dld, if_scaled, st);
}

template <typename T, typename TD>
void launch_fwd_grad(const void* x, int64_t ld, const int64_t* tgt, int64_t rows, int64_t cols, int64_t ignore,
                     float* lse, float* rl, float* rv, const float* scale, void* dx, int64_t dld, hipStream_t st) {
  if (const int nv = reg_nv(cols, sizeof(T))) {
    if (rows_match(x, ld, sizeof(T), dx, dld, sizeof(TD)))
      launch_reg<T, TD, kRegGradVec>(nv, x, ld, tgt, rows, cols, ignore, lse, rl, rv, scale, dx, dld, st);
    else
      launch_reg<T, TD, kRegGradElem>(nv, x, ld, tgt, rows, cols, ignore, lse, rl, rv, scale, dx, dld, st);
    return;
  }
  xent_fwd_grad_kernel<T, TD><<<dim3((unsigned)rows), dim3(kThreads), 0, st>>>((const T*)x, ld, tgt, cols, ignore,
                                                                               lse, rl, rv, scale, (TD*)dx, dld);
}

template <typename T>
void launch_fwd_grad_dt(int dx_dt, const void* x, int64_t ld, const int64_t* tgt, int64_t rows, int64_t cols,
                        int64_t ignore, float* lse, float* rl, float* rv, const float* scale, void* dx, int64_t dld,
                        hipStream_t st) {
  if (dx_dt == NAJU_DTYPE_F32)
    launch_fwd_grad<T, float>(x, ld, tgt, rows, cols, ignore, lse, rl, rv, scale, dx, dld, st);
  else if (dx_dt == NAJU_DTYPE_BF16)
    launch_fwd_grad<T, bf16_t>(x, ld, tgt, rows, cols, ignore, lse, rl, rv, scale, dx, dld, st);
  else
    launch_fwd_grad<T, f16_t>(x, ld, tgt, rows, cols, ignore, lse, rl, rv, scale, dx, dld, st);
}

}  // namespace

extern "C" {

const char* naju_loss_last_error(void) { return g_err; }

size_t naju_xent_workspace_bytes(int64_t n_rows) { return ws_bytes(n_rows); }

int naju_xent_fwd(const void* x, int64_t x_ld, const int64_t* target, int64_t n_rows, int64_t n_cols, int x_dtype,
                  int64_t ignore_index, float* lse, float* loss, float* scale, void* workspace,
                  size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  int rc = check_shape(x_ld, n_rows, n_cols, x_dtype);
  if (rc) return rc;
  if (!loss || !scale) return fail(NAJU_ERR_INVALID, "null pointer (loss and scale are required)");
  if (n_rows > 0 && (!x || !target || !lse)) return fail(NAJU_ERR_INVALID, "null pointer (x, target and lse)");
  if (n_rows > 0 && n_cols == 0) return fail(NAJU_ERR_INVALID, "n_cols must be positive when there are rows");
  if (!workspace || workspace_bytes < ws_bytes(n_rows))
    return fail(NAJU_ERR_WORKSPACE, "workspace of %zu bytes needed", ws_bytes(n_rows));
  hipStream_t st = (hipStream_t)stream;
  float* rl = (float*)workspace;
  float* rv = rl + n_rows;
  if (n_rows > 0) {
    if (x_dtype == NAJU_DTYPE_F32)
      launch_fwd<float>(x, x_ld, target, n_rows, n_cols, ignore_index, lse, rl, rv, st);
    else if (x_dtype == NAJU_DTYPE_BF16)
      launch_fwd<bf16_t>(x, x_ld, target, n_rows, n_cols, ignore_index, lse, rl, rv, st);
    else
      launch_fwd<f16_t>(x, x_ld, target, n_rows, n_cols, ignore_index, lse, rl, rv, st);
    if ((rc = launched())) return rc;
  }
  xent_mean_kernel<<<1, 1024, 0, st>>>(rl, rv, n_rows, loss, scale);
  return launched();
}

namespace {
int xent_bwd_impl(const void* x, int64_t x_ld, const int64_t* target, int64_t n_rows, int64_t n_cols, int x_dtype,
                  int64_t ignore_index, const float* lse, const float* scale, const float* dloss, void* dx,
                  int64_t dx_ld, int dx_dtype, int if_scaled, void* stream) {
  g_err[0] = 0;
  int rc = check_shape(x_ld, n_rows, n_cols, x_dtype);
  if (rc) return rc;
  if (dx_ld < n_cols) return fail(NAJU_ERR_INVALID, "dx_ld (%lld) must be >= n_cols (%lld)", (long long)dx_ld,
                                  (long long)n_cols);
  if (!dt_ok(dx_dtype)) return fail(NAJU_ERR_INVALID, "unknown dtype code");
  if (n_rows == 0 || n_cols == 0) return NAJU_OK;
  if (!x || !target || !lse || !scale || !dloss || !dx)
    return fail(NAJU_ERR_INVALID, "null pointer (x, target, lse, scale, dloss and dx are required)");
  hipStream_t st = (hipStream_t)stream;
  if (x_dtype == NAJU_DTYPE_F32)
    launch_bwd_dt<float>(dx_dtype, x, x_ld, target, n_rows, n_cols, ignore_index, lse, scale, dloss, dx, dx_ld,
                         if_scaled, st);
  else if (x_dtype == NAJU_DTYPE_BF16)
    launch_bwd_dt<bf16_t>(dx_dtype, x, x_ld, target, n_rows, n_cols, ignore_index, lse, scale, dloss, dx, dx_ld,
                          if_scaled, st);
  else
    launch_bwd_dt<f16_t>(dx_dtype, x, x_ld, target, n_rows, n_cols, ignore_index, lse, scale, dloss, dx, dx_ld,
                         if_scaled, st);
  return launched();
}
}  // namespace

int naju_xent_bwd(const void* x, int64_t x_ld, const int64_t* target, int64_t n_rows, int64_t n_cols, int x_dtype,
                  int64_t ignore_index, const float* lse, const float* scale, const float* dloss, void* dx,
                  int64_t dx_ld, int dx_dtype, void* stream) {
  return xent_bwd_impl(x, x_ld, target, n_rows, n_cols, x_dtype, ignore_index, lse, scale, dloss, dx, dx_ld, dx_dtype,
                       0, stream);
}

int naju_xent_fwd_grad(const void* x, int64_t x_ld, const int64_t* target, int64_t n_rows, int64_t n_cols,
                       int x_dtype, int64_t ignore_index, float* lse, float* loss, float* scale, void* dx,
                       int64_t dx_ld, int dx_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  int rc = check_shape(x_ld, n_rows, n_cols, x_dtype);
  if (rc) return rc;
  if (dx_ld < n_cols) return fail(NAJU_ERR_INVALID, "dx_ld (%lld) must be >= n_cols (%lld)", (long long)dx_ld,
                                  (long long)n_cols);
  if (!dt_ok(dx_dtype)) return fail(NAJU_ERR_INVALID, "unknown dtype code");
  if (!loss || !scale) return fail(NAJU_ERR_INVALID, "null pointer (loss and scale are required)");
  if (n_rows > 0 && (!x || !target || !lse || !dx))
    return fail(NAJU_ERR_INVALID, "null pointer (x, target, lse and dx)");
  if (n_rows > 0 && n_cols == 0) return fail(NAJU_ERR_INVALID, "n_cols must be positive when there are rows");
  if (!workspace || workspace_bytes < ws_bytes(n_rows))
    return fail(NAJU_ERR_WORKSPACE, "workspace of %zu bytes needed", ws_bytes(n_rows));
  hipStream_t st = (hipStream_t)stream;
  float* rl = (float*)workspace;
  float* rv = rl + n_rows;
  // the gradient's scale first (the count of valid rows), then the rows
  xent_count_kernel<<<1, 1024, 0, st>>>(target, n_rows, ignore_index, scale);
  if ((rc = launched())) return rc;
  if (n_rows > 0) {
    if (x_dtype == NAJU_DTYPE_F32)
      launch_fwd_grad_dt<float>(dx_dtype, x, x_ld, target, n_rows, n_cols, ignore_index, lse, rl, rv, scale, dx,
                                dx_ld, st);
    else if (x_dtype == NAJU_DTYPE_BF16)
      launch_fwd_grad_dt<bf16_t>(dx_dtype, x, x_ld, target, n_rows, n_cols, ignore_index, lse, rl, rv, scale, dx,
                                 dx_ld, st);
    else
      launch_fwd_grad_dt<f16_t>(dx_dtype, x, x_ld, target, n_rows, n_cols, ignore_index, lse, rl, rv, scale, dx,
                                dx_ld, st);
    if ((rc = launched())) return rc;
  }
  xent_mean_kernel<<<1, 1024, 0, st>>>(rl, rv, n_rows, loss, scale);
  return launched();
}

int naju_xent_bwd_if_scaled(const void* x, int64_t x_ld, const int64_t* target, int64_t n_rows, int64_t n_cols,
                            int x_dtype, int64_t ignore_index, const float* lse, const float* scale,
                            const float* dloss, void* dx, int64_t dx_ld, int dx_dtype, void* stream) {
  return xent_bwd_impl(x, x_ld, target, n_rows, n_cols, x_dtype, ignore_index, lse, scale, dloss, dx, dx_ld, dx_dtype,
                       1, stream);
}

}  // extern "C"
