// naju_optim.hip -- the optimizer step of the Naju LM training loop on
// MI355X (gfx950), behind the C ABI of include/naju_optim.h: the global
// gradient norm of clip_grad_norm_ and the clipped AdamW update
// (/root/reference/evals/lm/train.py:79-80, 165-166) as multi-tensor passes.
//
// Every parameter tensor is cut into chunks of NAJU_OPTIM_CHUNK elements and
// one workgroup serves one chunk, finding its tensor through the chunk ->
// tensor map, so a launch covers any mix of tensor sizes with no per-tensor
// launches. A full chunk with 16-byte aligned tensors is moved as float4:
// each thread issues the loads of four float4 of every array before the
// first is used (two such batches per chunk). The update reads param, grad
// and both moments once and writes param and the moments once: 28 bytes per
// element, HBM-bound; the norm pass reads the gradient once (4 bytes).
// The clip coefficient stays on the device: the update reads it, so
// clipping costs no pass over the gradients of its own and no host sync.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "naju_optim.h"
#include "naju_scan.h"

namespace {

constexpr int kThreads = 256;
constexpr int kChunk = NAJU_OPTIM_CHUNK;
constexpr int kVec4 = kChunk / (4 * kThreads);  // float4 of each array per thread in a full chunk
constexpr int kBatch = 4;                       // float4 of each array in flight per thread
static_assert(kVec4 % kBatch == 0, "whole batches per chunk");

struct GroupArgs {
  naju_adamw_group g[NAJU_OPTIM_MAX_GROUPS];
};

__device__ __forceinline__ bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// One element of the update (torch.optim.AdamW, amsgrad = False, in the
// order of its multi-tensor path: mul_, lerp_, mul_ + addcmul_, addcdiv_).
__device__ __forceinline__ void adamw1(float& p, float g, float& m, float& v, const naju_adamw_group& h) {
  p *= h.decay;
  m += h.one_minus_beta1 * (g - m);
  v = v * h.beta2 + h.one_minus_beta2 * g * g;
  const float denom = sqrtf(v) / h.bias_correction2_sqrt + h.eps;
  p -= h.step_size * (m / denom);
}

__device__ __forceinline__ void adamw4(float4& p, const float4& g, float4& m, float4& v, const naju_adamw_group& h,
                                       float c) {
  adamw1(p.x, g.x * c, m.x, v.x, h);
  adamw1(p.y, g.y * c, m.y, v.y, h);
  adamw1(p.z, g.z * c, m.z, v.z, h);
  adamw1(p.w, g.w * c, m.w, v.w, h);
}

// The tensor of chunk c and the chunk's element range in it; false (the
// chunk is skipped) when the table does not place c inside that tensor.
template <typename Rec>
__device__ __forceinline__ bool chunk_of(const Rec* __restrict__ tab, const int32_t* __restrict__ chunk_tensor,
                                         int n_tensors, int64_t c, Rec& t, int64_t& off, int& n) {
  int ti = chunk_tensor[c];
  ti = ti < 0 ? 0 : (ti < n_tensors ? ti : n_tensors - 1);
  t = tab[ti];
  off = (c - t.first_chunk) * kChunk;
  if (off < 0 || off >= t.numel) return false;
  const int64_t rem = t.numel - off;
  n = rem < kChunk ? (int)rem : kChunk;
  return true;
}

__global__ __launch_bounds__(kThreads) void adamw_kernel(const naju_adamw_tensor* __restrict__ tab,
                                                         const int32_t* __restrict__ chunk_tensor, int n_tensors,
                                                         GroupArgs ga, const float* __restrict__ coefp) {
  naju_adamw_tensor t;
  int64_t off;
  int n;
  if (!chunk_of(tab, chunk_tensor, n_tensors, blockIdx.x, t, off, n)) return;
  const naju_adamw_group h = ga.g[t.group & (NAJU_OPTIM_MAX_GROUPS - 1)];
  const float coef = coefp ? *coefp : 1.f;
  float* __restrict__ P = t.param + off;
  const float* __restrict__ G = t.grad + off;
  float* __restrict__ M = t.exp_avg + off;
  float* __restrict__ V = t.exp_avg_sq + off;
  const int tid = threadIdx.x;
  if (n == kChunk && aligned16(P) && aligned16(G) && aligned16(M) && aligned16(V)) {
    float4* P4 = (float4*)P;
    const float4* G4 = (const float4*)G;
    float4* M4 = (float4*)M;
    float4* V4 = (float4*)V;
#pragma unroll
    for (int b = 0; b < kVec4; b += kBatch) {
      float4 p[kBatch], g[kBatch], m[kBatch], v[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int i = (b + k) * kThreads + tid;
        p[k] = P4[i];
        g[k] = G4[i];
        m[k] = M4[i];
        v[k] = V4[i];
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int i = (b + k) * kThreads + tid;
        adamw4(p[k], g[k], m[k], v[k], h, coef);
        P4[i] = p[k];
        M4[i] = m[k];
        V4[i] = v[k];
      }
    }
    return;
  }
  // a tensor's last (partial) chunk, or unaligned tensors: element by element
  for (int i = tid; i < n; i += kThreads) {
    float p = P[i], m = M[i], v = V[i];
    adamw1(p, G[i] * coef, m, v, h);
    P[i] = p;
    M[i] = m;
    V[i] = v;
  }
}

// part[c] = sum of grad^2 over chunk c (float32; per thread, then the wave's
// lanes by butterfly, then the waves in wave order).
__global__ __launch_bounds__(kThreads) void sqnorm_kernel(const naju_adamw_tensor* __restrict__ tab,
                                                          const int32_t* __restrict__ chunk_tensor, int n_tensors,
                                                          float* __restrict__ part) {
  __shared__ float s_w[kThreads / 64];
  const int64_t c = blockIdx.x;
  naju_adamw_tensor t;
  int64_t off;
  int n;
  if (!chunk_of(tab, chunk_tensor, n_tensors, c, t, off, n)) {
    if (threadIdx.x == 0) part[c] = 0.f;
    return;
  }
  const float* __restrict__ G = t.grad + off;
  const int tid = threadIdx.x;
  float s = 0.f;
  if (n == kChunk && aligned16(G)) {
    const float4* G4 = (const float4*)G;
#pragma unroll
    for (int b = 0; b < kVec4; b += 2 * kBatch) {
      float4 g[2 * kBatch];
#pragma unroll
      for (int k = 0; k < 2 * kBatch; ++k) g[k] = G4[(b + k) * kThreads + tid];
#pragma unroll
      for (int k = 0; k < 2 * kBatch; ++k) s += (g[k].x * g[k].x + g[k].y * g[k].y) + (g[k].z * g[k].z + g[k].w * g[k].w);
    }
  } else {
    for (int i = tid; i < n; i += kThreads) s += G[i] * G[i];
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
  if ((tid & 63) == 0) s_w[tid >> 6] = s;
  __syncthreads();
  if (tid == 0) {
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) tot += s_w[w];
    part[c] = tot;
  }
}

// norm = sqrt(sum of the chunk sums): thread i adds chunks i, i + 1024, ...
// in float64, then a fixed-order tree over the threads.
__global__ __launch_bounds__(1024) void norm_final_kernel(const float* __restrict__ part, int64_t n_chunks,
                                                          float max_norm, float* __restrict__ norm,
                                                          float* __restrict__ coef) {
  __shared__ double s_d[1024];
  const int tid = threadIdx.x;
  double s = 0.0;
  for (int64_t i = tid; i < n_chunks; i += 1024) s += (double)part[i];
  s_d[tid] = s;
  __syncthreads();
  for (int h = 512; h >= 1; h >>= 1) {
    if (tid < h) s_d[tid] += s_d[tid + h];
    __syncthreads();
  }
  if (tid == 0) {
    const float nrm = (float)sqrt(s_d[0]);
    norm[0] = nrm;
    if (coef) {
      // clip_grad_norm_: max_norm / (total_norm + 1e-6), clamped at 1 (NaN stays NaN)
      const float cc = max_norm / (nrm + 1e-6f);
      coef[0] = cc > 1.f ? 1.f : cc;
    }
  }
}

template <typename TO>
using out4_t = TO __attribute__((ext_vector_type(4)));

// naju_cast_multi: one workgroup per chunk; a full aligned chunk issues all
// eight float4 loads of a thread before its first store.
template <typename TO>
__global__ __launch_bounds__(kThreads) void cast_kernel(const naju_cast_tensor* __restrict__ tab,
                                                        const int32_t* __restrict__ chunk_tensor, int n_tensors,
                                                        TO* __restrict__ dst) {
  naju_cast_tensor t;
  int64_t off;
  int n;
  if (!chunk_of(tab, chunk_tensor, n_tensors, blockIdx.x, t, off, n)) return;
  const float* __restrict__ S = t.src ? t.src + off : nullptr;
  TO* __restrict__ D = dst + t.dst_offset + off;
  const int tid = threadIdx.x;
  if (n == kChunk && (!S || aligned16(S)) && ((uintptr_t)D & 7u) == 0) {
    float4 v[kVec4];
#pragma unroll
    for (int k = 0; k < kVec4; ++k) v[k] = S ? ((const float4*)S)[k * kThreads + tid] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < kVec4; ++k) {
      out4_t<TO> o;
      o.x = (TO)v[k].x;
      o.y = (TO)v[k].y;
      o.z = (TO)v[k].z;
      o.w = (TO)v[k].w;
      ((out4_t<TO>*)D)[k * kThreads + tid] = o;
    }
    return;
  }
  for (int i = tid; i < n; i += kThreads) D[i] = S ? (TO)S[i] : (TO)0.f;
}

thread_local char g_err[256] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_table(const naju_adamw_tensor* tensors, const int32_t* chunk_tensor, int n_tensors, int64_t n_chunks) {
  if (n_tensors < 0 || n_chunks < 0) return fail(NAJU_ERR_INVALID, "negative table size");
  if (n_chunks > 0x7fffffff) return fail(NAJU_ERR_UNSUPPORTED, "too many chunks (%lld)", (long long)n_chunks);
  if (n_chunks > 0 && (!tensors || !chunk_tensor || n_tensors == 0))
    return fail(NAJU_ERR_INVALID, "null tensor table or chunk map");
  return NAJU_OK;
}

}  // namespace

extern "C" {

const char* naju_optim_last_error(void) { return g_err; }

size_t naju_grad_norm_workspace_bytes(int64_t n_chunks) {
  if (n_chunks < 0) return 0;
  return (size_t)n_chunks * sizeof(float) + 256;
}

int naju_grad_norm(const naju_adamw_tensor* tensors, const int32_t* chunk_tensor, int n_tensors, int64_t n_chunks,
                   float max_norm, float* norm, float* coef, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  int rc = check_table(tensors, chunk_tensor, n_tensors, n_chunks);
  if (rc) return rc;
  if (!norm) return fail(NAJU_ERR_INVALID, "null norm pointer");
  const size_t need = naju_grad_norm_workspace_bytes(n_chunks);
  if (!workspace || workspace_bytes < need)
    return fail(NAJU_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need,
                workspace ? workspace_bytes : (size_t)0);
  hipStream_t st = (hipStream_t)stream;
  float* part = (float*)workspace;
  if (n_chunks > 0)
    hipLaunchKernelGGL(sqnorm_kernel, dim3((unsigned)n_chunks), dim3(kThreads), 0, st, tensors, chunk_tensor,
                       n_tensors, part);
  // no chunks: the empty sum, norm 0 (as torch's clip_grad_norm_ of no gradients)
  hipLaunchKernelGGL(norm_final_kernel, dim3(1), dim3(1024), 0, st, part, n_chunks, max_norm, norm, coef);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return NAJU_OK;
}

int naju_adamw_step(const naju_adamw_tensor* tensors, const int32_t* chunk_tensor, int n_tensors, int64_t n_chunks,
                    const naju_adamw_group* groups, int n_groups, const float* grad_coef, void* stream) {
  g_err[0] = 0;
  int rc = check_table(tensors, chunk_tensor, n_tensors, n_chunks);
  if (rc) return rc;
  if (n_groups < 1 || n_groups > NAJU_OPTIM_MAX_GROUPS || !groups)
    return fail(NAJU_ERR_INVALID, "n_groups must be in [1, %d] with a groups array", NAJU_OPTIM_MAX_GROUPS);
  for (int i = 0; i < n_groups; ++i)
    if (!(groups[i].bias_correction2_sqrt > 0.f))
      return fail(NAJU_ERR_INVALID, "group %d: bias_correction2_sqrt must be positive (step >= 1)", i);
  if (n_chunks == 0) return NAJU_OK;
  GroupArgs ga = {};
  for (int i = 0; i < n_groups; ++i) ga.g[i] = groups[i];
  hipLaunchKernelGGL(adamw_kernel, dim3((unsigned)n_chunks), dim3(kThreads), 0, (hipStream_t)stream, tensors,
                     chunk_tensor, n_tensors, ga, grad_coef);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return NAJU_OK;
}

int naju_cast_multi(const naju_cast_tensor* tensors, const int32_t* chunk_tensor, int n_tensors, int64_t n_chunks,
                    void* dst, int dst_dtype, void* stream) {
  g_err[0] = 0;
  if (n_tensors < 0 || n_chunks < 0) return fail(NAJU_ERR_INVALID, "negative table size");
  if (n_chunks > 0x7fffffff) return fail(NAJU_ERR_UNSUPPORTED, "too many chunks (%lld)", (long long)n_chunks);
  if (n_chunks > 0 && (!tensors || !chunk_tensor || n_tensors == 0 || !dst))
    return fail(NAJU_ERR_INVALID, "null tensor table, chunk map or destination");
  if (dst_dtype != NAJU_DTYPE_BF16 && dst_dtype != NAJU_DTYPE_F16)
    return fail(NAJU_ERR_UNSUPPORTED, "destination dtype %d: bf16 or f16 only", dst_dtype);
  if (n_chunks == 0) return NAJU_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dst_dtype == NAJU_DTYPE_BF16)
    hipLaunchKernelGGL(cast_kernel<__bf16>, dim3((unsigned)n_chunks), dim3(kThreads), 0, st, tensors, chunk_tensor,
                       n_tensors, (__bf16*)dst);
  else
    hipLaunchKernelGGL(cast_kernel<_Float16>, dim3((unsigned)n_chunks), dim3(kThreads), 0, st, tensors,
                       chunk_tensor, n_tensors, (_Float16*)dst);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return NAJU_OK;
}

}  // extern "C"
