// scan_internal.h -- definitions shared by the scan's translation units
// (naju_scan.hip: the N = 1 kernels, the direct general-N kernels and the C
// ABI; naju_scan_mc.hip: the chunked matrix-core kernels for 9 <= N <= 64).
// Internal to the library; not part of the C ABI.
#ifndef NAJU_SCAN_INTERNAL_H
#define NAJU_SCAN_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "naju_scan.h"

namespace naju_detail {

typedef __bf16 bf16_t;
typedef _Float16 f16_t;

// ------------------------------------------------------------------ helpers

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return (float)x; }
__device__ __forceinline__ float to_f32(f16_t x) { return (float)x; }

template <typename T>
__device__ __forceinline__ T from_f32(float x) {
  return (T)x;
}

// sigmoid(x) = 1 / (1 + 2^(-x*log2 e)); exact 0 and 1 at -inf and +inf,
// so hard-reset (f=0) and pure-retention (f=1) gates stay exact.
__device__ __forceinline__ float sigm(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

// Load with a runtime dtype code (B_t / C_t scalars and other small streams).
__device__ __forceinline__ float ld_any(const void* p, int dt, int64_t i) {
  if (dt == NAJU_DTYPE_F32) return ((const float*)p)[i];
  if (dt == NAJU_DTYPE_BF16) return (float)((const bf16_t*)p)[i];
  return (float)((const f16_t*)p)[i];
}
__device__ __forceinline__ void st_any(void* p, int dt, int64_t i, float v) {
  if (dt == NAJU_DTYPE_F32)
    ((float*)p)[i] = v;
  else if (dt == NAJU_DTYPE_BF16)
    ((bf16_t*)p)[i] = (bf16_t)v;
  else
    ((f16_t*)p)[i] = (f16_t)v;
}

// Workspace header, a fixed-size region that no other part of any layout
// ever overlaps (so its counters, which must start at zero, are only ever
// written by the ticket logic below): word 0 is the status word; word 1 the
// device epoch (look-back tags of launches recorded into a HIP graph, see
// epoch_bump_kernel); tile t's ticket counter is word kCtrBase + t*kCtrStride,
// t < kMaxTiles.
enum { HDR_STATUS = 0, HDR_EPOCH = 1 };
constexpr int kCtrBase = 64;
constexpr int kCtrStride = 4;
constexpr int kMaxTiles = 1 << 16;
constexpr size_t kHeaderBytes = ((size_t)kCtrBase + (size_t)kMaxTiles * kCtrStride) * sizeof(uint32_t);
// Bound on idle polls of one look-back. A poll is a few device-scope loads
// plus a short sleep (~1 us), so the bound is about a second, far beyond any
// legitimate wait (microseconds); past it the carry becomes NaN and the
// status word records the failure, so every wave still exits.
constexpr uint32_t kSpinLimit = 1u << 20;

// Kernel arguments (one struct for every kernel; unused fields are null).
struct ScanArgs {
  const void* u;
  const void* fl;
  const void* il;
  const void* Bm;
  const void* Cm;
  const float* Dsk;
  const float* h0;
  const void* dy;
  void* y;
  float* ckpt;
  float* hT;
  void* du;
  void* dfl;
  void* dil;
  float* dh0;
  float* partB;  // [n_dtiles][batch][T][N]
  float* partC;
  float* partD;  // N = 1: [batch][K][D]; N > 1: [batch][nseg][D]
  float* segF;   // N > 1, per time segment: [batch][nseg][D] decay over the segment
  float* segZ;   // [batch][nseg][D][N] the segment's state map from a zero state
  float* seg0;   // [batch][nseg][D][N] the state (adjoint carry) entering each segment
  int nseg;      // N > 1: time segments (one workgroup each per channel tile)
  int seg_sc;    // N > 1: sub-chunks per time segment
  uint32_t* hdr;
  uint64_t* agg;   // [K][n_tiles][2][CH]
  uint64_t* incl;  // [K][n_tiles][CH]
  int64_t T;
  int64_t D;
  int64_t ldbc;  // elements between rows of B and C (N unless strided; the matrix-core path only)
  int64_t ldg;   // elements between rows of dfl and dil (D unless strided; the matrix-core backward only)
  float* partG;  // [2][batch * nseg][D]: per-segment sums of dfl, dil (matrix-core backward; NULL: none)
  int N;
  int batch;
  int bc_dt;
  int n_dtiles;
  int n_tiles;
  int K;
  int ck_rows;  // rows per checkpoint interval of ckpt
  int Kc;       // number of checkpoint intervals of ckpt
  // Chunked matrix-core forward map launch with recomp = 1: the backward's
  // recompute of the state entering every sub-block (into ckpt, Kc of them)
  // from the forward's checkpoint ck_src (Kc_src intervals, one segment
  // each) instead of a segment map.
  // (With a checkpoint interval longer than the sub-block the forward's time
  // segments start at interval boundaries, so every state the recompute
  // starts from is a checkpoint entry.)
  const float* ck_src;
  int Kc_src;
  int recomp;
  // N = 1: this launch's look-back tag. Nonzero: a host tag (odd, new for
  // every eager launch). Zero: the launch was recorded into a HIP graph, and
  // the tag comes from the device epoch, which the one-thread
  // epoch_bump_kernel recorded right before it advances on every replay.
  uint32_t tag;
  int strict;    // N = 1: take carries from the immediate predecessor's inclusive carry only
  // N = 1: idle look-back rounds before a hand-off gives up (kSpinLimit;
  // 0 = give up at once, a test hook that makes every hand-off fail while
  // every kernel still exits normally)
  uint32_t spin_limit;
};

// Lane exchange for the butterfly steps below: the value of the partner lane
// that differs in bit log2(m) (and, for m = 8 / 4, in the lower bits too:
// row_mirror pairs i with 15 - i, row_half_mirror i with 7 - i).
template <int m>
__device__ __forceinline__ float dpp_partner(float x) {
  constexpr int ctrl = m == 8 ? 0x140 : m == 4 ? 0x141 : m == 2 ? 0x4E : 0xB1;
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), ctrl, 0xF, 0xF, false));
}

// (lo, hi) -> lanes with bit log2(m) clear get lo + partner's lo, lanes with
// it set get hi + partner's hi, m = 32 or 16 (one lane-swap instruction).
template <int m>
__device__ __forceinline__ float swap_sum(float lo, float hi) {
  if constexpr (m == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}

// Transposing butterfly over aligned groups of LG lanes of the M entries of
// v (the same scheme as tr_reduce, with DPP and lane-swap exchanges). On
// return, lane l of a group holds the group sums of entries
// [l*M/LG, (l+1)*M/LG) in v[0 ..) when M >= LG, else entry l / (LG/M) in
// v[0]. Fixed order: run-to-run identical.
template <int LG, int K, int M>
__device__ __forceinline__ void trd_step(float (&v)[M], int lane) {
  if constexpr (LG > 1) {
    constexpr int m = LG / 2;
    if constexpr (K >= 2) {
      constexpr int h = K / 2;
      if constexpr (m >= 16) {
#pragma unroll
        for (int j = 0; j < h; ++j) v[j] = swap_sum<m>(v[j], v[j + h]);
      } else {
        const bool hi = (lane & m) != 0;
#pragma unroll
        for (int j = 0; j < h; ++j) {
          const float keep = hi ? v[j + h] : v[j], send = hi ? v[j] : v[j + h];
          v[j] = keep + dpp_partner<m>(send);
        }
      }
      trd_step<m, h, M>(v, lane);
    } else {
      if constexpr (m >= 16)
        v[0] = swap_sum<m>(v[0], v[0]);
      else
        v[0] += dpp_partner<m>(v[0]);
      trd_step<m, 1, M>(v, lane);
    }
  }
}

// ------------------------------------------ chunked matrix-core path (N > 8)
//
// naju_scan_mc.hip. Workgroups of kMcW waves own kMcDT channels of one batch
// row and walk one time segment in sub-blocks of kMcQ rows; the state entering
// each checkpoint interval of a.ck_rows rows (a multiple of kMcQ) is written
// to the checkpoint as [batch][a.Kc][D][N].
constexpr int kMcQ = 16;
constexpr int kMcW = 4;
constexpr int kMcDT = 16 * kMcW;
// the backward's workgroups: kMcWB waves over kMcDTB channels (its dB / dC
// partial sums are per kMcDTB-channel tile)
constexpr int kMcWB = 8;
constexpr int kMcDTB = 16 * kMcWB;

// Below this decay over a sub-block (product of its 16 f of one channel),
// the chunked kernels form the intra-sub-block decay terms as exact
// products; at or above it, as ratios Pf[t] / Pf[s] of the running products
// from the sub-block's first row, which turns those terms into matrix
// products. 1 / Pf then stays at most 2^30, far from overflow, and Pf dy
// leaves the normal range only for |dy| below about 2^-96. A hard reset
// (f = 0) is always below it.
constexpr float kMcRatioMin = 0x1p-30f;

// True when the chunked kernels serve this state size.
inline bool mc_ok(int64_t N) { return N > 8 && N <= 64; }

// Forward: map = true computes the maps of segments 0 .. nseg-2 (segF /
// segZ); map = false the scan itself from h0 or the carried segment states.
hipError_t mc_fwd_launch(const ScanArgs& a, bool map, int x_dt, int g_dt, int y_dt, hipStream_t st);
// Backward: map = true the adjoint maps of segments 1 .. nseg-1; map = false
// du, dfl, dil, dh0 and the dB / dC / dD partials.
hipError_t mc_bwd_launch(const ScanArgs& a, bool map, int x_dt, int g_dt, int du_dt, int dg_dt, hipStream_t st);

}  // namespace naju_detail

#endif  // NAJU_SCAN_INTERNAL_H
