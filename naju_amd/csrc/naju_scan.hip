// naju_scan.hip -- MI355X (gfx950) kernels and C ABI of the Naju gated scan.
//
// Recurrence (reference naju/scan.py:15-19, naju_scan_reference :79-93):
//   f_t = sigmoid(fl_t), i_t = sigmoid(il_t)
//   x_t = f_t * x_{t-1} + i_t * B_t * u_t ,  y_t = sum_n C_t x_t + D u_t
//
// Design (one HBM pass per direction):
//  * Lanes run over channels d (the contiguous axis of [B,T,D]), V channels
//    per lane, so every load and store of the u / gate / dy / grad streams is
//    a coalesced 8- or 16-byte vector access. B_t and C_t are uniform across
//    the lanes of a batch row and come in through scalar loads.
//  * A workgroup owns a tile of 64*V channels and a chunk of L = W*R
//    timesteps; wave w holds rows [w*R, w*R+R) of the chunk in registers.
//  * Each wave scans its rows from a zero state and reduces them to an affine
//    map s -> F*s + Z (the composition rule of reference
//    naju/chunk_affine_triton.py:3-5). The W maps are composed through LDS.
//  * Chunks hand their carries to each other through a decoupled look-back:
//    a workgroup publishes its chunk map (the "aggregate"), then walks back
//    over its predecessors' published maps until it meets an "inclusive"
//    carry, and publishes its own inclusive carry. Published words are
//    64-bit {float value, 32-bit tag} pairs written and read with relaxed
//    device-scope atomics, so no cache-wide fences are needed and stale words
//    from earlier launches (older tags) are never mistaken for fresh ones.
//    Chunks are handed out in order through an atomic ticket, so a workgroup
//    waits only on workgroups that are already running: no deadlock at any
//    occupancy. Every wait is bounded.
//  * The backward is the same machinery run in reverse time for the adjoint
//    x̄_t = C_t dy_t + f_{t+1} x̄_{t+1}; the forward state inside a chunk is
//    recomputed from the checkpoint the forward wrote at the chunk start.
//    du, dfl, dil come out of that single pass; dB, dC (sums over channels)
//    and dD (sum over batch and time) are written as per-tile partial sums
//    and folded by one small kernel in a fixed order (deterministic).
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <atomic>
#include <mutex>
#include <type_traits>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "naju_scan.h"
#include "scan_internal.h"

namespace {

using namespace naju_detail;

// V consecutive elements starting at element d0 of row `p`, by access mode:
//   kVecAll : one aligned vector access, no bounds check (the caller knows
//             the whole tile is inside [0, D));
//   kVecLane: one aligned vector access if d0 < D (the host guarantees
//             D % V == 0), else zeros;
//   kElem   : element-wise, each element checked against D.
// Out-of-range elements read as 0 and are not written.
enum { kVecAll = 0, kVecLane = 1, kElem = 2 };

// V consecutive elements of a row as loaded: the raw bits (one 32-bit word
// per two 2-byte elements), turned into floats where they are used. Chunk
// rows are loaded long before pass 1 reaches them; kept raw, 2-byte rows take
// half the registers of converted ones.
template <typename T, int V>
struct RawRow {
  static constexpr int NW = (V * (int)sizeof(T) + 3) / 4;
  uint32_t w[NW];
  __device__ __forceinline__ float get(int j) const {
    if constexpr (sizeof(T) == 4) {
      return __builtin_bit_cast(float, w[j]);
    } else {
      const uint32_t x = w[j >> 1];
      const uint16_t h = (j & 1) ? (uint16_t)(x >> 16) : (uint16_t)(x & 0xffffu);
      return to_f32(__builtin_bit_cast(T, h));
    }
  }
};

// ld_row into a RawRow from row pointer p (uniform: the row at the tile's
// first channel) at lane element offset lo, channel d0 = tile start + lo.
// The byte offset is a 32-bit lane value, so the load takes the row address
// in scalar registers and one offset register shared by every row.
// Out-of-range elements read as 0 (all-zero bits).
template <typename T>
__device__ __forceinline__ const T* at_lane(const T* p, uint32_t lo) {
  return (const T*)((const char*)p + lo * (uint32_t)sizeof(T));
}
template <typename T>
__device__ __forceinline__ T* at_lane(T* p, uint32_t lo) {
  return (T*)((char*)p + lo * (uint32_t)sizeof(T));
}

// A uniform pointer held in scalar registers through an opaque copy: loads
// at it plus a lane's 32-bit offset then use the scalar-base address form,
// instead of the compiler deriving every row's 64-bit address from the
// previous row's in vector registers.
template <typename T>
__device__ __forceinline__ T* sreg(T* p) {
  uint64_t v = (uint64_t)p;
  asm("s_mov_b64 %0, %1" : "=s"(v) : "s"(v));
  // back through a global (address space 1) pointer, so the accesses stay
  // global ones rather than flat ones
  return (T*)(__attribute__((address_space(1))) T*)v;
}

// NT: a non-temporal load (a stream read once per call).
template <typename T, int V, int MODE, bool NT = false>
__device__ __forceinline__ void ld_row_raw(const T* __restrict__ p, uint32_t lo, int64_t d0, int64_t D,
                                           RawRow<T, V>& o) {
  constexpr int NW = RawRow<T, V>::NW;
  if constexpr (MODE != kElem && (V * sizeof(T)) % 4 == 0) {
    // a clang vector type: HIP's uint2 / uint4 member reads become one
    // 4-byte load each
    typedef uint32_t vw __attribute__((ext_vector_type(NW)));
    if (MODE == kVecAll || d0 < D) {
      const vw v = NT ? __builtin_nontemporal_load(reinterpret_cast<const vw*>(at_lane(p, lo)))
                      : *reinterpret_cast<const vw*>(at_lane(p, lo));
#pragma unroll
      for (int k = 0; k < NW; ++k) o.w[k] = v[k];
    } else {
#pragma unroll
      for (int k = 0; k < NW; ++k) o.w[k] = 0u;
    }
  } else {
#pragma unroll
    for (int k = 0; k < NW; ++k) o.w[k] = 0u;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const bool ok = MODE == kElem ? d0 + j < D : (MODE == kVecAll || d0 < D);
      if constexpr (sizeof(T) == 4) {
        o.w[j] = ok ? __builtin_bit_cast(uint32_t, at_lane(p, lo)[j]) : 0u;
      } else {
        const uint32_t h = ok ? (uint32_t)__builtin_bit_cast(uint16_t, at_lane(p, lo)[j]) : 0u;
        o.w[j >> 1] |= (j & 1) ? h << 16 : h;
      }
    }
  }
}

// st_row at row pointer p (uniform, the tile's first channel) and lane
// element offset lo (channel d0 = tile start + lo). The rows stored here are
// the N = 1 kernels' outputs (y; du, dfl, dil), written once per call and
// not read again by the scan: non-temporal stores, so they do not take the
// caches' room from the input streams, which the backward reads again after
// the forward (at config 2 the step went from 187 to 165 us with them, with
// the dy loads below from 165 to 150; at configs 3 and 4, whose streams far
// exceed the last-level cache, 3-5% per step).
template <typename T, int V, int MODE>
__device__ __forceinline__ void st_row_at(T* __restrict__ p, uint32_t lo, int64_t d0, int64_t D,
                                          const float (&x)[V]) {
  typedef T vec_t __attribute__((ext_vector_type(V)));
  if constexpr (MODE == kElem) {
#pragma unroll
    for (int j = 0; j < V; ++j)
      if (d0 + j < D) __builtin_nontemporal_store(from_f32<T>(x[j]), at_lane(p, lo) + j);
  } else {
    if (MODE == kVecAll || d0 < D) {
      vec_t v;
#pragma unroll
      for (int j = 0; j < V; ++j) v[j] = from_f32<T>(x[j]);
      __builtin_nontemporal_store(v, reinterpret_cast<vec_t*>(at_lane(p, lo)));
    }
  }
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}

// Wave-wide sums of the M entries of v (M a power of two, M <= 64): a
// transposing butterfly (each lane keeps half of its entries and trades the
// other half with its partner, masks 32, 16, ...) until one entry is left,
// then a plain butterfly over the remaining lane bits. Afterwards lane l
// holds the sum of entry l / (64 / M) in v[0]. Fixed order.
template <int MASK, int K, int M>
__device__ __forceinline__ void wave_sums_step(float (&v)[M], int lane) {
  if constexpr (K > 1) {
    const bool hi = (lane & MASK) != 0;
#pragma unroll
    for (int j = 0; j < K / 2; ++j) {
      const float lo_v = v[j], hi_v = v[j + K / 2];
      v[j] = (hi ? hi_v : lo_v) + __shfl_xor(hi ? lo_v : hi_v, MASK, 64);
    }
    wave_sums_step<MASK / 2, K / 2, M>(v, lane);
  } else {
#pragma unroll
    for (int m = MASK; m >= 1; m >>= 1) v[0] += __shfl_xor(v[0], m, 64);
  }
}
template <int M>
__device__ __forceinline__ void wave_sums(float (&v)[M], int lane) {
  static_assert(M >= 1 && M <= 64 && (M & (M - 1)) == 0, "M must be a power of two <= 64");
  wave_sums_step<32, M, M>(v, lane);
}

// Tagged words of the look-back: {value bits, tag} in one 64-bit atomic.
__device__ __forceinline__ uint64_t ld_word(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_word(uint64_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool word_ok(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }
__device__ __forceinline__ float word_val(uint64_t w) { return __uint_as_float((uint32_t)w); }

// Look-back tag of a launch from the device epoch E: even and nonzero, so it
// never equals a host tag (odd) or the tag 0 of a zero-filled workspace.
__device__ __forceinline__ uint32_t epoch_tag(uint32_t e) { return (e & 0x7fffffffu) << 1; }

// Advances the device epoch by one (skipping the values whose tag would be
// 0). Recorded into a HIP graph before each N = 1 scan launch, so every
// replay of that launch sees a new tag: look-back words left by an earlier
// replay carry an older tag and are never taken for fresh ones. Stream order
// makes the new value visible to the scan launch that follows.
__global__ void epoch_bump_kernel(uint32_t* hdr) {
  uint32_t e = hdr[HDR_EPOCH] + 1u;
  if (epoch_tag(e) == 0u) e += 1u;
  hdr[HDR_EPOCH] = e;
}

// Workgroup blockIdx.x serves tile blockIdx.x % n_tiles; the chunk comes from
// that tile's ticket counter, so a tile's chunks are handed out in the order
// its workgroups start and every chunk a workgroup waits on is already held
// by a running workgroup. The workgroup that draws the tile's last ticket
// rewinds the counter for the next launch (all K tickets are taken by then).
// Also returns the launch's look-back tag in *s_tag (a.tag, or the device
// epoch's tag when a.tag is 0: read next to the ticket, in the same round
// trip; nothing changes the epoch while the launch runs).
// Returns the ticket (uniform). A ticket outside [0, K) means a workspace
// that was not zero-filled: it is recorded in the status word and the
// caller poisons its blockIdx chunk instead of computing it.
__device__ __forceinline__ uint32_t take_ticket(const ScanArgs& a, int tile, uint32_t* s_ticket, uint32_t* s_tag) {
  if (threadIdx.x == 0) {
    uint32_t* ctr = a.hdr + kCtrBase + (int64_t)tile * kCtrStride;
    uint32_t e = 0;
    if (a.tag == 0u) e = __hip_atomic_load(a.hdr + HDR_EPOCH, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t t = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (t == (uint32_t)a.K - 1) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (t >= (uint32_t)a.K) __hip_atomic_store(a.hdr + HDR_STATUS, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_ticket = t;
    *s_tag = a.tag != 0u ? a.tag : epoch_tag(e);
  }
  __syncthreads();
  return __builtin_amdgcn_readfirstlane(*s_ticket);
}

// ------------------------------------------------ workgroup-wide look-back
//
// A chunk's map, published as "aggregate" words, and its inclusive carry,
// published as "inclusive" words, live in the workspace at
//   agg [chunk][tile][2][CH]   (F block, then Z block)
//   incl[chunk][tile][CH]
// with channel slot cs = j*64 + lane (j < V), so every wave-wide access of
// one j touches 64 consecutive 8-byte words.
//
// Each round, wave w polls predecessors base + dir*(p*W + w), p < P, so one
// memory round trip covers a window of W*P predecessors. A predecessor is
// usable when all CH channels of a word kind carry the current tag (a wave
// vote). Wave 0 then walks the window in order: aggregates are composed
// until the first inclusive carry, which ends the walk; a predecessor that
// is not ready yet ends the round and the next round resumes there.
template <int V, int W, int P>
struct LookShared {
  float S[W * P][64 * V];
  float F[W * P][64 * V];
  float Z[W * P][64 * V];
  int stat[W * P];  // 0 = not ready, 1 = aggregate, 2 = inclusive
  int ctl[2];       // done, number of predecessors consumed
};

// One round's polled words, as this wave loaded them: predecessor slot
// p*W + wv of the round (p < P), V channel words of each kind.
template <int V, int P>
struct LookPoll {
  uint64_t wi[P][V], wf[P][V], wz[P][V];
};

// Issue this wave's polls of the round whose first predecessor is `base`.
template <int V, int W, int P>
__device__ __forceinline__ void lb_issue(const ScanArgs& a, int base, int tile, int dir, int lane, int wv,
                                         LookPoll<V, P>& q) {
  constexpr int CH = 64 * V;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = base + dir * (p * W + wv);
    const bool inr = c >= 0 && c < a.K;
    const uint64_t* pi = a.incl + ((int64_t)c * a.n_tiles + tile) * CH + lane;
    const uint64_t* pa = a.agg + ((int64_t)c * a.n_tiles + tile) * 2 * CH + lane;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      // values (not struct members) assigned on both paths, so the words
      // stay in registers
      uint64_t wi = 0, wf = 0, wz = 0;
      if (inr) {
        wi = ld_word(pi + j * 64);
        wf = ld_word(pa + j * 64);
        wz = ld_word(pa + CH + j * 64);
      }
      q.wi[p][j] = wi;
      q.wf[p][j] = wf;
      q.wz[p][j] = wz;
    }
  }
}

// Finish one round from its polled words: stage them in LDS, wave 0 walks
// the window in order (aggregates composed into aF, aZ until the first
// inclusive carry, which ends the walk into `out`; a predecessor that is
// not ready ends the round). Returns true when the carry is known; else
// advances base past the predecessors consumed.
template <int V, int W, int P>
__device__ __forceinline__ bool lb_consume(const ScanArgs& a, LookShared<V, W, P>& sh, int& base, int dir,
                                           uint32_t tag, int lane, int wv, const LookPoll<V, P>& q, float (&aF)[V],
                                           float (&aZ)[V], float (&out)[V], uint32_t& idle) {
  constexpr int WP = W * P;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int slot = p * W + wv;
    const int c = base + dir * slot;
    const bool inr = c >= 0 && c < a.K;
    bool iok = inr, aok = inr;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      iok = iok && word_ok(q.wi[p][j], tag);
      aok = aok && word_ok(q.wf[p][j], tag) && word_ok(q.wz[p][j], tag);
      sh.S[slot][j * 64 + lane] = word_val(q.wi[p][j]);
      sh.F[slot][j * 64 + lane] = word_val(q.wf[p][j]);
      sh.Z[slot][j * 64 + lane] = word_val(q.wz[p][j]);
    }
    iok = __all(iok);
    aok = __all(aok);
    if (lane == 0) sh.stat[slot] = iok ? 2 : (aok ? 1 : 0);
  }
  __syncthreads();
  if (wv == 0) {
    int consumed = 0, done = 0;
    for (int slot = 0; slot < WP; ++slot) {
      const int st = sh.stat[slot];
      if (st == 2) {
#pragma unroll
        for (int j = 0; j < V; ++j) out[j] = fmaf(aF[j], sh.S[slot][j * 64 + lane], aZ[j]);
        done = 1;
        break;
      }
      // strict: never compose aggregates, wait for the predecessor's
      // inclusive carry (a fixed composition order)
      if (st != 1 || a.strict) break;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        aZ[j] = fmaf(aF[j], sh.Z[slot][j * 64 + lane], aZ[j]);
        aF[j] *= sh.F[slot][j * 64 + lane];
      }
      ++consumed;
    }
    if (!done && consumed == 0 && ++idle > a.spin_limit) {
      // Bounded wait exceeded: record it and end with a NaN carry.
      if (lane == 0) __hip_atomic_store(a.hdr + HDR_STATUS, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int j = 0; j < V; ++j) out[j] = __builtin_nanf("");
      done = 1;
    }
    if (lane == 0) {
      sh.ctl[0] = done;
      sh.ctl[1] = consumed;
    }
  }
  __syncthreads();
  const int done = sh.ctl[0];
  const int consumed = sh.ctl[1];
  base += dir * consumed;
  if (!done && consumed == 0) __builtin_amdgcn_s_sleep(2);
  return done != 0;
}

// Carry entering chunk k (dir = -1: forward, predecessors k-1, k-2, ...;
// dir = +1: backward, k+1, k+2, ...). Result valid in wave 0's lanes.
template <int V, int W, int P>
__device__ __forceinline__ void wg_look_back(const ScanArgs& a, LookShared<V, W, P>& sh, int k, int tile, int dir,
                                             uint32_t tag, int lane, int wv, float (&out)[V]) {
  float aF[V], aZ[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    aF[j] = 1.f;
    aZ[j] = 0.f;
    out[j] = 0.f;
  }
  if (a.spin_limit == 0u) {
    // the host asked every hand-off to give up at once (a test hook): the
    // failure path of an exceeded wait, taken without polling
    if (wv == 0) {
      if (lane == 0) __hip_atomic_store(a.hdr + HDR_STATUS, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int j = 0; j < V; ++j) out[j] = __builtin_nanf("");
    }
    return;
  }
  int base = k + dir;
  uint32_t idle = 0;
  while (true) {
    LookPoll<V, P> q;
    lb_issue<V, W, P>(a, base, tile, dir, lane, wv, q);
    if (lb_consume<V, W, P>(a, sh, base, dir, tag, lane, wv, q, aF, aZ, out, idle)) break;
  }
}

// Rows [t0, t0+R) (rowbase = b*T + t0) of one [batch,T,D] stream, p at the
// tile's first channel. ROWCHK: rows at or beyond T read as 0.
template <typename T, int V, int R, int MODE, bool ROWCHK, bool NT = false>
__device__ __forceinline__ void ld_rows_raw(const T* __restrict__ p, int64_t rowbase, int t0, int64_t Tn, int64_t D,
                                            uint32_t lo, int64_t d0, RawRow<T, V> (&o)[R]) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (!ROWCHK || t0 + r < Tn) {
      ld_row_raw<T, V, MODE, NT>(sreg(p + (rowbase + r) * D), lo, d0, D, o[r]);
    } else {
#pragma unroll
      for (int k = 0; k < RawRow<T, V>::NW; ++k) o[r].w[k] = 0u;
    }
  }
}

// B_t and C_t of rows [t0, t0+R) into scalar registers: lane r < R loads
// B_t0+r and lane R + r loads C_t0+r (one vector register for the wave),
// then each value is read out of its lane. Held as vector registers, the
// 2R values uniform across the wave would take 2R of them.
template <typename T, int R, bool ROWCHK>
__device__ __forceinline__ void ld_bc(const T* __restrict__ pb, const T* __restrict__ pc, int64_t rowbase, int t0,
                                      int64_t Tn, int lane, float (&bt)[R], float (&ct)[R]) {
  static_assert(2 * R <= 64, "one lane per value");
  const int r = lane < R ? lane : lane - R;
  float v = 0.f;
  if (lane < 2 * R && (!ROWCHK || t0 + r < Tn)) v = to_f32((lane < R ? pb : pc)[rowbase + r]);
#pragma unroll
  for (int q = 0; q < R; ++q) {
    bt[q] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), q));
    ct[q] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), R + q));
  }
}

// ------------------------------------------------------------ N = 1 forward
//
// One workgroup = (batch row b, tile of CH = 64*V channels, chunk k of
// L = W*R timesteps). Forward chunk order: ticket -> (k, tile), chunk-major,
// so every predecessor (k-1, same tile) holds a smaller ticket. Lane `lane`
// owns channels d0 .. d0+V-1 (d0 = tile start + lane*V); its slot for
// channel j in LDS and workspace arrays is j*64 + lane. A workgroup whose
// chunk and tile lie wholly inside [0,T) x [0,D) runs the FULL body: no
// bounds checks, all loads issued back to back; edge workgroups check.
template <typename TU, typename TG, typename TB, int V, int R, int W, int P, bool VEC, bool F32O, bool FULL>
__device__ __forceinline__ void n1_fwd_body(const ScanArgs& a, int k, int tile, int lane, int wv, uint32_t tag,
                                            bool poison,
                                            float (&s_F)[W][64 * V], float (&s_Z)[W][64 * V], float (&s_in)[64 * V],
                                            LookShared<V, W, P>& s_lb) {
  using TY = std::conditional_t<F32O, float, TU>;  // y dtype
  constexpr int CH = 64 * V;
  constexpr int L = W * R;
  constexpr int M = FULL ? kVecAll : (VEC ? kVecLane : kElem);
  const int b = tile / a.n_dtiles;
  const int dtile = tile - b * a.n_dtiles;
  const int64_t T = a.T, D = a.D;
  const int64_t dbase = (int64_t)dtile * CH;  // the tile's first channel
  const uint32_t lo = (uint32_t)(lane * V);
  const int64_t d0 = dbase + lo;
  const int t0 = k * L + wv * R;
  const int64_t rowbase = (int64_t)b * T + t0;

  float Dv[V];
  bool dok[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    dok[j] = FULL || d0 + j < D;
    Dv[j] = dok[j] ? a.Dsk[d0 + j] : 0.f;
  }

  // ---- load the wave's R rows
  RawRow<TU, V> xu[R];
  RawRow<TG, V> xf[R], xi[R];
  float Bt[R], Ct[R];
  ld_rows_raw<TU, V, R, M, !FULL>((const TU*)a.u + dbase, rowbase, t0, T, D, lo, d0, xu);
  ld_rows_raw<TG, V, R, M, !FULL>((const TG*)a.fl + dbase, rowbase, t0, T, D, lo, d0, xf);
  ld_rows_raw<TG, V, R, M, !FULL>((const TG*)a.il + dbase, rowbase, t0, T, D, lo, d0, xi);
  ld_bc<TB, R, !FULL>((const TB*)a.Bm, (const TB*)a.Cm, rowbase, t0, T, lane, Bt, Ct);

  // ---- pass 1: local scan from zero; keep y = yl + q * (carry) per element
  float F[V], Z[V];
  float yl[R][V], q[R][V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    F[j] = 1.f;
    Z[j] = 0.f;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const bool tv = FULL || t0 + r < T;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const bool v = tv && dok[j];
      const float f = v ? sigm(xf[r].get(j)) : 1.f;
      const float ig = v ? sigm(xi[r].get(j)) : 0.f;
      const float x = xu[r].get(j);
      Z[j] = fmaf(f, Z[j], ig * Bt[r] * x);
      F[j] *= f;
      yl[r][j] = fmaf(Ct[r], Z[j], Dv[j] * x);
      q[r][j] = Ct[r] * F[j];
      // formed here: otherwise the compiler moves parts of this row's
      // arithmetic past the look-back and keeps more values live across it
      asm volatile("" : "+v"(yl[r][j]), "+v"(q[r][j]));
    }
  }
#pragma unroll
  for (int j = 0; j < V; ++j) {
    s_F[wv][j * 64 + lane] = F[j];
    s_Z[wv][j * 64 + lane] = Z[j];
  }
  __syncthreads();

  // ---- chunk map (wave 0), publish, look back, publish the inclusive carry
  float Fw[V], Zw[V], sin[V];
  uint64_t* my_agg = a.agg + ((int64_t)k * a.n_tiles + tile) * 2 * CH + lane;
  uint64_t* my_incl = a.incl + ((int64_t)k * a.n_tiles + tile) * CH + lane;
  if (wv == 0) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      Fw[j] = 1.f;
      Zw[j] = 0.f;
    }
#pragma unroll
    for (int w = 0; w < W; ++w)
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float f = s_F[w][j * 64 + lane];
        Zw[j] = fmaf(f, Zw[j], s_Z[w][j * 64 + lane]);
        Fw[j] *= f;
      }
    if (poison) {
      // no valid ticket: this chunk's outputs become NaN, nothing is published
#pragma unroll
      for (int j = 0; j < V; ++j) sin[j] = __builtin_nanf("");
    } else if (k > 0) {
#pragma unroll
      for (int j = 0; j < V; ++j) {
        st_word(my_agg + j * 64, Fw[j], tag);
        st_word(my_agg + CH + j * 64, Zw[j], tag);
      }
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) sin[j] = (a.h0 && dok[j]) ? a.h0[(int64_t)b * D + d0 + j] : 0.f;
    }
  }
  if (k > 0 && !poison) wg_look_back<V, W, P>(a, s_lb, k, tile, -1, tag, lane, wv, sin);
  if (wv == 0) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      if (!poison) st_word(my_incl + j * 64, fmaf(Fw[j], sin[j], Zw[j]), tag);
      s_in[j * 64 + lane] = sin[j];
    }
    if (a.hT && k == a.K - 1) {
#pragma unroll
      for (int j = 0; j < V; ++j)
        if (dok[j]) a.hT[(int64_t)b * D + d0 + j] = fmaf(Fw[j], sin[j], Zw[j]);
    }
  }
  __syncthreads();

  // ---- pass 2: this wave's carry, then y
  float s[V];
#pragma unroll
  for (int j = 0; j < V; ++j) s[j] = s_in[j * 64 + lane];
  for (int w = 0; w < wv; ++w)
#pragma unroll
    for (int j = 0; j < V; ++j) s[j] = fmaf(s_F[w][j * 64 + lane], s[j], s_Z[w][j * 64 + lane]);
  // the state entering a checkpoint interval of the backward pass
  if (a.ckpt && t0 % a.ck_rows == 0 && (FULL || t0 < T)) {
#pragma unroll
    for (int j = 0; j < V; ++j)
      if (dok[j]) a.ckpt[((int64_t)b * a.Kc + t0 / a.ck_rows) * D + d0 + j] = s[j];
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < V; ++j) yl[r][j] = fmaf(q[r][j], s[j], yl[r][j]);
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (FULL || t0 + r < T) st_row_at<TY, V, M>((TY*)a.y + (rowbase + r) * D + dbase, lo, d0, D, yl[r]);
}

template <typename TU, typename TG, typename TB, int V, int R, int W, int P, bool VEC, bool F32O>
__global__ __launch_bounds__(64 * W) void n1_fwd_kernel(const ScanArgs a) {
  constexpr int CH = 64 * V;
  constexpr int L = W * R;
  __shared__ uint32_t s_ticket, s_tag;
  __shared__ float s_F[W][CH];
  __shared__ float s_Z[W][CH];
  __shared__ float s_in[CH];
  __shared__ LookShared<V, W, P> s_lb;

  const int tile = (int)(blockIdx.x % (uint32_t)a.n_tiles);
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int dtile = tile % a.n_dtiles;
  const int kx = (int)(blockIdx.x / (uint32_t)a.n_tiles);
  const uint32_t t = take_ticket(a, tile, &s_ticket, &s_tag);
  // an out-of-range ticket (a workspace that was not zero-filled) poisons
  // the chunk this workgroup's index names, so no output is left unwritten
  const bool poison = t >= (uint32_t)a.K;
  const int k = poison ? kx : (int)t;
  const uint32_t tag = __builtin_amdgcn_readfirstlane(s_tag);
  if constexpr (VEC) {
    if ((int64_t)(k + 1) * L <= a.T && (int64_t)(dtile + 1) * CH <= a.D) {
      n1_fwd_body<TU, TG, TB, V, R, W, P, VEC, F32O, true>(a, k, tile, lane, wv, tag, poison, s_F, s_Z, s_in, s_lb);
      return;
    }
  }
  n1_fwd_body<TU, TG, TB, V, R, W, P, VEC, F32O, false>(a, k, tile, lane, wv, tag, poison, s_F, s_Z, s_in, s_lb);
}

// ----------------------------------------------------------- N = 1 backward
//
// Adjoint in carry form: with g = f_{t+1} x̄_{t+1} entering row t from the
// future, x̄_t = C_t dy_t + g and the carry leaving is f_t x̄_t. Rows [t0,t1)
// map g_in -> A g_in + Zb with A = prod f. Chunks run in reverse order
// (ticket -> chunk K-1-k), so the look-back walks towards larger t. The
// forward state entering the chunk comes from the forward's checkpoint.
template <typename TU, typename TG, typename TB, int V, int R, int W, int P, bool VEC, bool F32O, bool FULL>
__device__ __forceinline__ void n1_bwd_body(const ScanArgs& a, int k, int tile, int lane, int wv, uint32_t tag,
                                            bool poison,
                                            float (&s_F)[W][64 * V], float (&s_Z)[W][64 * V],
                                            float (&s_Zb)[W][64 * V], float (&s_g)[64 * V],
                                            float (&s_dD)[W][64 * V], LookShared<V, W, P>& s_lb,
                                            float (&s_pq)[W][2 * R][64]) {
  using TDU = std::conditional_t<F32O, float, TU>;  // du dtype
  using TDG = std::conditional_t<F32O, float, TG>;  // dfl, dil dtype
  constexpr int CH = 64 * V;
  constexpr int L = W * R;
  constexpr int M = FULL ? kVecAll : (VEC ? kVecLane : kElem);
  const int b = tile / a.n_dtiles;
  const int dtile = tile - b * a.n_dtiles;
  const int64_t T = a.T, D = a.D;
  const int64_t dbase = (int64_t)dtile * CH;  // the tile's first channel
  const uint32_t lo = (uint32_t)(lane * V);
  const int64_t d0 = dbase + lo;
  const int t0 = k * L + wv * R;
  const int64_t rowbase = (int64_t)b * T + t0;

  float Dv[V];
  bool dok[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    dok[j] = FULL || d0 + j < D;
    Dv[j] = dok[j] ? a.Dsk[d0 + j] : 0.f;
  }

  // rows as loaded (u and dy stay raw until used; the gate logits become
  // gates in pass 1)
  RawRow<TU, V> xu[R], xg[R];
  RawRow<TG, V> lf[R], li[R];
  float xf[R][V], xi[R][V];
  float Bt[R], Ct[R];
  ld_rows_raw<TU, V, R, M, !FULL>((const TU*)a.u + dbase, rowbase, t0, T, D, lo, d0, xu);
  ld_rows_raw<TG, V, R, M, !FULL>((const TG*)a.fl + dbase, rowbase, t0, T, D, lo, d0, lf);
  ld_rows_raw<TG, V, R, M, !FULL>((const TG*)a.il + dbase, rowbase, t0, T, D, lo, d0, li);
  // dy is read once per call (non-temporal loads, like the output stores)
  ld_rows_raw<TU, V, R, M, !FULL, true>((const TU*)a.dy + dbase, rowbase, t0, T, D, lo, d0, xg);
  ld_bc<TB, R, !FULL>((const TB*)a.Bm, (const TB*)a.Cm, rowbase, t0, T, lane, Bt, Ct);
  float s[V];
#pragma unroll
  for (int j = 0; j < V; ++j) s[j] = dok[j] ? a.ckpt[((int64_t)b * a.K + k) * D + d0 + j] : 0.f;

  // ---- pass 1: gates, w = i*B*u, forward map (F, Z) and adjoint map (F, Zb)
  float F[V], Z[V], G[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    F[j] = 1.f;
    Z[j] = 0.f;
    G[j] = 0.f;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const bool tv = FULL || t0 + r < T;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const bool v = tv && dok[j];
      xf[r][j] = v ? sigm(lf[r].get(j)) : 1.f;  // f
      xi[r][j] = v ? sigm(li[r].get(j)) : 0.f;  // i
      Z[j] = fmaf(xf[r][j], Z[j], xi[r][j] * Bt[r] * xu[r].get(j));
      F[j] *= xf[r][j];
      // only the gates (and the raw rows) cross the look-back, not products
      // that pass 2 would otherwise share with this pass
      asm volatile("" : "+v"(xf[r][j]), "+v"(xi[r][j]));
    }
  }
#pragma unroll
  for (int r = R - 1; r >= 0; --r)
#pragma unroll
    for (int j = 0; j < V; ++j) G[j] = xf[r][j] * fmaf(xg[r].get(j), Ct[r], G[j]);
  // this wave's dD terms sum_t dy u (they need no scan): summed over the
  // workgroup by wave 0 behind the barrier below
  float dDs[V];
#pragma unroll
  for (int j = 0; j < V; ++j) dDs[j] = 0.f;
#pragma unroll
  for (int r = R - 1; r >= 0; --r)
#pragma unroll
    for (int j = 0; j < V; ++j) dDs[j] = fmaf(xg[r].get(j), xu[r].get(j), dDs[j]);
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int k2 = 0; k2 < RawRow<TU, V>::NW; ++k2) asm volatile("" : "+v"(xu[r].w[k2]), "+v"(xg[r].w[k2]));
#pragma unroll
  for (int j = 0; j < V; ++j) {
    s_F[wv][j * 64 + lane] = F[j];
    s_Z[wv][j * 64 + lane] = Z[j];
    s_Zb[wv][j * 64 + lane] = G[j];
    s_dD[wv][j * 64 + lane] = dDs[j];
  }
  __syncthreads();

  // ---- chunk adjoint map (wave 0), publish, look ahead, publish inclusive
  float A[V], Zb[V], gin[V];
  uint64_t* my_agg = a.agg + ((int64_t)k * a.n_tiles + tile) * 2 * CH + lane;
  uint64_t* my_incl = a.incl + ((int64_t)k * a.n_tiles + tile) * CH + lane;
  if (wv == 0) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      A[j] = 1.f;
      Zb[j] = 0.f;
      gin[j] = 0.f;
    }
#pragma unroll
    for (int w = W - 1; w >= 0; --w)
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float f = s_F[w][j * 64 + lane];
        Zb[j] = fmaf(f, Zb[j], s_Zb[w][j * 64 + lane]);
        A[j] *= f;
      }
    if (poison) {
      // no valid ticket: this chunk's outputs become NaN, nothing is published
#pragma unroll
      for (int j = 0; j < V; ++j) gin[j] = __builtin_nanf("");
    } else if (k < a.K - 1) {
#pragma unroll
      for (int j = 0; j < V; ++j) {
        st_word(my_agg + j * 64, A[j], tag);
        st_word(my_agg + CH + j * 64, Zb[j], tag);
      }
    }
    if (a.partD) {
      // the chunk's dD partial: the waves' sums in wave order
#pragma unroll
      for (int j = 0; j < V; ++j) {
        float acc = 0.f;
        for (int w = 0; w < W; ++w) acc += s_dD[w][j * 64 + lane];
        if (dok[j]) a.partD[((int64_t)b * a.K + k) * D + d0 + j] = acc;
      }
    }
  }
  if (k < a.K - 1 && !poison) wg_look_back<V, W, P>(a, s_lb, k, tile, +1, tag, lane, wv, gin);
  if (wv == 0) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float gout = fmaf(A[j], gin[j], Zb[j]);
      if (!poison) st_word(my_incl + j * 64, gout, tag);
      s_g[j * 64 + lane] = gin[j];
      if (a.dh0 && k == 0 && dok[j]) a.dh0[(int64_t)b * D + d0 + j] = gout;
    }
  }
  __syncthreads();

  // ---- pass 2: exact carries of this wave's rows
  float g[V];
#pragma unroll
  for (int j = 0; j < V; ++j) g[j] = s_g[j * 64 + lane];
  for (int w = 0; w < wv; ++w)
#pragma unroll
    for (int j = 0; j < V; ++j) s[j] = fmaf(s_F[w][j * 64 + lane], s[j], s_Z[w][j * 64 + lane]);
  for (int w = W - 1; w > wv; --w)
#pragma unroll
    for (int j = 0; j < V; ++j) g[j] = fmaf(s_F[w][j * 64 + lane], g[j], s_Zb[w][j * 64 + lane]);

  // forward states x_t of every row (x_{t0-1} = s0)
  float xs[R][V], s0[V];
#pragma unroll
  for (int j = 0; j < V; ++j) s0[j] = s[j];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < V; ++j) {
      s[j] = fmaf(xf[r][j], s[j], xi[r][j] * Bt[r] * xu[r].get(j));
      xs[r][j] = s[j];
    }

  // reverse sweep: gradients (naju/cuda/naju_cuda.cu:116-140 restated);
  // f(1-f) and i(1-i) as fma(-f, f, f), exactly 0 at f in {0, 1}.
  // This lane's terms of the dB / dC sums of row r go to s_pq[wv][r] /
  // s_pq[wv][R + r] (in LDS rather than registers: 2R fewer live VGPRs).
#pragma unroll
  for (int r = R - 1; r >= 0; --r) {
    float pb = 0.f, pc = 0.f;
    float du[V], dfl[V], dil[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float f = xf[r][j], ig = xi[r][j], x = xu[r].get(j), gy = xg[r].get(j);
      const float xprev = r > 0 ? xs[r - 1][j] : s0[j];
      const float xb = fmaf(gy, Ct[r], g[j]);
      const float iu = ig * x;
      const float dws = xb * Bt[r];
      pb = fmaf(xb, iu, pb);
      pc = fmaf(gy, xs[r][j], pc);
      g[j] = f * xb;
      dfl[j] = fmaf(-f, f, f) * (xb * xprev);
      dil[j] = fmaf(-ig, ig, ig) * (dws * x);
      du[j] = fmaf(ig, dws, Dv[j] * gy);
    }
    s_pq[wv][r][lane] = pb;
    s_pq[wv][R + r][lane] = pc;
    // each row's gradients are stored as soon as they are formed
    if (FULL || t0 + r < T) {
      const int64_t ro = (rowbase + r) * D + dbase;
      if (a.du) st_row_at<TDU, V, M>(sreg((TDU*)a.du + ro), lo, d0, D, du);
      if (a.dfl) st_row_at<TDG, V, M>(sreg((TDG*)a.dfl + ro), lo, d0, D, dfl);
      if (a.dil) st_row_at<TDG, V, M>(sreg((TDG*)a.dil + ro), lo, d0, D, dil);
    }
  }
  if (a.partB || a.partC) {
    // partial sums over this tile's channels, stored [dtile][b*T + t]: the Q
    // lanes 64i/2R .. of entry i (row r of dB, i < R, or of dC) each add
    // SPAN of the wave's terms (in a rotated order that keeps the eight lanes
    // of a 16-byte LDS read on distinct banks), then combine in lane order
    static_assert(64 % (2 * R) == 0, "2R must divide the wave");
    constexpr int Q = 64 / (2 * R);
    constexpr int SPAN = 64 / Q;
    static_assert(SPAN % 4 == 0, "16-byte reads");
    asm volatile("" ::: "memory");  // the wave reads back its own stores
    const int i = lane / Q, part = lane % Q;
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < SPAN; c += 4) {
      const int col = part * SPAN + ((c + 4 * i + 16 * part) % SPAN);
      const float4 v = *(const float4*)&s_pq[wv][i][col];
      acc += (v.x + v.y) + (v.z + v.w);
    }
#pragma unroll
    for (int m = 1; m < Q; m <<= 1) acc += __shfl_xor(acc, m, 64);
    const int r = i < R ? i : i - R;
    const int64_t t = t0 + r;
    if (part == 0 && (FULL || t < T)) {
      float* dst = i < R ? a.partB : a.partC;
      if (dst) dst[(int64_t)dtile * a.batch * T + (int64_t)b * T + t] = acc;
    }
  }
}

template <typename TU, typename TG, typename TB, int V, int R, int W, int P, bool VEC, bool F32O>
__global__ __launch_bounds__(64 * W) void n1_bwd_kernel(const ScanArgs a) {
  constexpr int CH = 64 * V;
  constexpr int L = W * R;
  __shared__ uint32_t s_ticket, s_tag;
  __shared__ float s_F[W][CH];
  __shared__ float s_Z[W][CH];
  __shared__ float s_Zb[W][CH];
  __shared__ float s_g[CH];
  __shared__ float s_dD[W][CH];
  __shared__ LookShared<V, W, P> s_lb;
  __shared__ __align__(16) float s_pq[W][2 * R][64];

  const int tile = (int)(blockIdx.x % (uint32_t)a.n_tiles);
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int dtile = tile % a.n_dtiles;
  const int kx = (int)(blockIdx.x / (uint32_t)a.n_tiles);
  const uint32_t t = take_ticket(a, tile, &s_ticket, &s_tag);
  // an out-of-range ticket (a workspace that was not zero-filled) poisons
  // the chunk this workgroup's index names, so no output is left unwritten
  const bool poison = t >= (uint32_t)a.K;
  const int k = poison ? kx : a.K - 1 - (int)t;
  const uint32_t tag = __builtin_amdgcn_readfirstlane(s_tag);
  if constexpr (VEC) {
    if ((int64_t)(k + 1) * L <= a.T && (int64_t)(dtile + 1) * CH <= a.D) {
      n1_bwd_body<TU, TG, TB, V, R, W, P, VEC, F32O, true>(a, k, tile, lane, wv, tag, poison, s_F, s_Z, s_Zb, s_g, s_dD,
                                                             s_lb, s_pq);
      return;
    }
  }
  n1_bwd_body<TU, TG, TB, V, R, W, P, VEC, F32O, false>(a, k, tile, lane, wv, tag, poison, s_F, s_Z, s_Zb, s_g, s_dD,
                                                        s_lb, s_pq);
}

// Sum over q < n_parts of p[q*stride + i], in q order, with the loads of
// eight parts issued together.
__device__ __forceinline__ float sum_parts(const float* __restrict__ p, int n_parts, int64_t stride, int64_t i) {
  float sm = 0.f;
  int q = 0;
  for (; q + 8 <= n_parts; q += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = p[(int64_t)(q + u) * stride + i];
#pragma unroll
    for (int u = 0; u < 8; ++u) sm += v[u];
  }
  for (; q < n_parts; ++q) sm += p[(int64_t)q * stride + i];
  return sm;
}

// Folds the backward's partial sums, in a fixed order (run-to-run
// identical), in one launch:
//   blocks [0, n_bc_blocks): dB, dC [i] = sum over the channel tiles q of
//     partB/partC[q*btn + i] (consecutive threads read consecutive i);
//   blocks [n_bc_blocks, ...): per-channel vectors v = 0 .. n_vec-1 (dD,
//     and the gate gradients' sums when asked for), ceil(D / 64) blocks
//     each: out_v[d] = sum over the n_rows rows of part_v[row][d], 64
//     channels per block; wave w of 16 sums rows w, w+16, ... (32 loads in
//     flight) with four interleaved accumulators, then the 16 wave sums are
//     added in wave order.
struct FoldVecs {
  const float* part[3];
  float* out[3];
  int n;
};

__global__ __launch_bounds__(1024) void fold_kernel(const float* __restrict__ partB,
                                                    const float* __restrict__ partC, int n_parts, int64_t btn,
                                                    void* dB, void* dC, int bc_dt, int n_bc_blocks, FoldVecs fv,
                                                    int64_t n_rows, int64_t D, int bc_split, int64_t N,
                                                    int64_t ld_out) {
  // entry i of the [batch * T][N] sums lands at row i / N, column i % N of
  // dB / dC, whose rows are ld_out elements apart
  auto out = [&](int64_t i) { return ld_out == N ? i : (i / N) * ld_out + (i - (i / N) * N); };
  __shared__ float s_acc[16][64];
  __shared__ float4 s_b4[16][64], s_c4[16][64];
  if ((int)blockIdx.x < n_bc_blocks) {
    const int64_t stride = (int64_t)n_bc_blocks * blockDim.x;
    if (bc_split) {
      // few entries (btn % 4 == 0): a block takes 64 float4 entries and its
      // 16 waves split the parts, wave k summing the k-th run of
      // ceil(n_parts / 16) consecutive parts; the 16 runs are then added in
      // run order, so far more workgroups share the reads
      const int j = (int)threadIdx.x & 63, k = (int)threadIdx.x >> 6;
      const int64_t n4 = btn / 4;
      const int64_t i4 = (int64_t)blockIdx.x * 64 + j;
      const int per = (n_parts + 15) / 16;
      const int q0 = k * per, q1 = q0 + per < n_parts ? q0 + per : n_parts;
      float4 sb = make_float4(0.f, 0.f, 0.f, 0.f), sc = sb;
      if (i4 < n4) {
        const float4* pb = reinterpret_cast<const float4*>(partB);
        const float4* pc = reinterpret_cast<const float4*>(partC);
        for (int q = q0; q < q1; ++q) {
          if (dB) {
            const float4 v = pb[(int64_t)q * n4 + i4];
            sb.x += v.x, sb.y += v.y, sb.z += v.z, sb.w += v.w;
          }
          if (dC) {
            const float4 v = pc[(int64_t)q * n4 + i4];
            sc.x += v.x, sc.y += v.y, sc.z += v.z, sc.w += v.w;
          }
        }
      }
      s_b4[k][j] = sb;
      s_c4[k][j] = sc;
      __syncthreads();
      if (k == 0 && i4 < n4) {
        float4 tb = s_b4[0][j], tc = s_c4[0][j];
#pragma unroll
        for (int m = 1; m < 16; ++m) {
          const float4 vb = s_b4[m][j], vc = s_c4[m][j];
          tb.x += vb.x, tb.y += vb.y, tb.z += vb.z, tb.w += vb.w;
          tc.x += vc.x, tc.y += vc.y, tc.z += vc.z, tc.w += vc.w;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (dB) st_any(dB, bc_dt, out(4 * i4 + e), (&tb.x)[e]);
          if (dC) st_any(dC, bc_dt, out(4 * i4 + e), (&tc.x)[e]);
        }
      }
      return;
    }
    if (btn % 4 == 0) {
      // four consecutive entries per thread, the parts of dB and dC loaded
      // four at a time with 16-byte loads, added in part order (the same
      // order, so the same sums, as the scalar loop below)
      const int64_t n4 = btn / 4;
      const float4* pb = reinterpret_cast<const float4*>(partB);
      const float4* pc = reinterpret_cast<const float4*>(partC);
      for (int64_t i4 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i4 < n4; i4 += stride) {
        float sb[4] = {0.f, 0.f, 0.f, 0.f}, sc[4] = {0.f, 0.f, 0.f, 0.f};
        int q = 0;
        // eight parts of each quantity in flight per thread
        for (; q + 8 <= n_parts; q += 8) {
          float4 vb[8], vc[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            if (dB) vb[u] = pb[(int64_t)(q + u) * n4 + i4];
            if (dC) vc[u] = pc[(int64_t)(q + u) * n4 + i4];
          }
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            sb[0] += vb[u].x, sb[1] += vb[u].y, sb[2] += vb[u].z, sb[3] += vb[u].w;
            sc[0] += vc[u].x, sc[1] += vc[u].y, sc[2] += vc[u].z, sc[3] += vc[u].w;
          }
        }
        for (; q < n_parts; ++q) {
          if (dB) {
            const float4 v = pb[(int64_t)q * n4 + i4];
            sb[0] += v.x, sb[1] += v.y, sb[2] += v.z, sb[3] += v.w;
          }
          if (dC) {
            const float4 v = pc[(int64_t)q * n4 + i4];
            sc[0] += v.x, sc[1] += v.y, sc[2] += v.z, sc[3] += v.w;
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (dB) st_any(dB, bc_dt, out(4 * i4 + e), sb[e]);
          if (dC) st_any(dC, bc_dt, out(4 * i4 + e), sc[e]);
        }
      }
      return;
    }
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < btn; i += stride) {
      if (dB) st_any(dB, bc_dt, out(i), sum_parts(partB, n_parts, btn, i));
      if (dC) st_any(dC, bc_dt, out(i), sum_parts(partC, n_parts, btn, i));
    }
    return;
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t per_vec = (D + 63) / 64;
  const int64_t bi = (int64_t)blockIdx.x - n_bc_blocks;
  const int vi = (int)(bi / per_vec);
  if (vi >= fv.n) return;
  // (selected, not indexed: a dynamic index into the argument would go
  // through scratch memory)
  const float* __restrict__ partD = vi == 0 ? fv.part[0] : (vi == 1 ? fv.part[1] : fv.part[2]);
  float* __restrict__ dD = vi == 0 ? fv.out[0] : (vi == 1 ? fv.out[1] : fv.out[2]);
  const int64_t d = (bi - vi * per_vec) * 64 + lane;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (d < D) {
    // 32 rows of a wave in flight per round: at N = 1 a wave's whole share
    // (512 rows over 16 waves at B = 8, T = 4096) is one memory round trip
    int64_t r = w;
    for (; r + 16 * 31 < n_rows; r += 16 * 32) {
      float v[32];
#pragma unroll
      for (int u = 0; u < 32; ++u) v[u] = partD[(r + 16 * u) * D + d];
#pragma unroll
      for (int u = 0; u < 32; ++u) acc[u & 3] += v[u];
    }
    for (int u = 0; r < n_rows; r += 16, ++u) acc[u & 3] += partD[r * D + d];
  }
  s_acc[w][lane] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  __syncthreads();
  if (w == 0 && d < D) {
    float sm = 0.f;
    for (int q = 0; q < 16; ++q) sm += s_acc[q][lane];
    dD[d] = sm;
  }
}

// ------------------------------------------------------ general N (N >= 2)
//
// Lanes run over the state index n (a wave instruction covers G = 64/LG
// channels, LG = min(NP, 64) lanes each, S = NP/LG states per lane; NP is
// N rounded up to a power of two, states n >= N stay 0). One workgroup owns
// a tile of 64 channels of one batch row for the whole sequence and walks T
// in sub-chunks of kGnCK rows. Per-channel gates and inputs of a sub-chunk
// are staged in LDS with coalesced loads and read back as broadcasts; B_t and
// C_t rows are staged as [row][n]. Sums over n use fixed-order butterflies.
//   forward : x_t = f x_{t-1} + i u B_t per lane; y_t = sum_n C_t x_t + D u;
//             the state entering every sub-chunk is checkpointed.
//   backward: sub-chunks in reverse; the forward states of a sub-chunk are
//             recomputed from its checkpoint into registers, then the adjoint
//             x̄_t = C_t dy_t + f_{t+1} x̄_{t+1} runs backwards with its carry
//             kept in registers across sub-chunks (no inter-workgroup waits).
//             dB, dC are summed over the tile's channels (lanes of other
//             channel groups, then waves in wave order) into per-tile partials.
constexpr int kGnCK = 32;  // rows per sub-chunk = checkpoint interval
constexpr int kGnDT = 64;  // channels per workgroup
constexpr int kGnW = 8;    // waves per workgroup

template <int LG>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = LG / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Sums over aligned groups of LG lanes of the M entries of v, by a
// transposing butterfly: at each step a lane keeps half of its entries and
// trades the other half with its partner, so the M sums cost M-1 lane
// exchanges instead of M*log2(LG). Afterwards lane l of a group holds the
// sums of entries [l*M/LG, (l+1)*M/LG) in v[0 .. M/LG). Fixed order, so the
// sums are run-to-run identical.
template <int LG, int K, int M>
__device__ __forceinline__ void tr_reduce_step(float (&v)[M], int lane) {
  if constexpr (LG > 1) {
    constexpr int m = LG / 2;
    const bool hi = (lane & m) != 0;
#pragma unroll
    for (int j = 0; j < K / 2; ++j) {
      const float lo_v = v[j], hi_v = v[j + K / 2];
      v[j] = (hi ? hi_v : lo_v) + __shfl_xor(hi ? lo_v : hi_v, m, 64);
    }
    tr_reduce_step<m, K / 2, M>(v, lane);
  }
}
template <int LG, int M>
__device__ __forceinline__ void tr_reduce(float (&v)[M], int lane) {
  tr_reduce_step<LG, M, M>(v, lane);
}

constexpr int kGnThreads = 64 * kGnW;
constexpr int kGnE = kGnCK * kGnDT / kGnThreads;  // tile elements per thread

// This thread's kGnE elements (element k = e*kGnThreads + tid is row k/kGnDT,
// channel k%kGnDT) of a [kGnCK][kGnDT] tile of one [batch,T,D] stream
// starting at row t0, channel dbase. Rows past T and channels past D read a
// clamped in-bounds element, which the caller replaces. The dtype switch is
// outside the element loop, so the loads issue back to back.
__device__ __forceinline__ void gn_ld_tile(const ScanArgs& a, const void* p, int dt, int b, int64_t t0,
                                           int64_t dbase, float (&v)[kGnE]) {
  int64_t idx[kGnE];
#pragma unroll
  for (int e = 0; e < kGnE; ++e) {
    const int k = e * kGnThreads + (int)threadIdx.x;
    const int64_t t = t0 + k / kGnDT, d = dbase + k % kGnDT;
    idx[e] = ((int64_t)b * a.T + (t < a.T ? t : a.T - 1)) * a.D + (d < a.D ? d : a.D - 1);
  }
  if (dt == NAJU_DTYPE_F32) {
#pragma unroll
    for (int e = 0; e < kGnE; ++e) v[e] = ((const float*)p)[idx[e]];
  } else if (dt == NAJU_DTYPE_BF16) {
#pragma unroll
    for (int e = 0; e < kGnE; ++e) v[e] = (float)((const bf16_t*)p)[idx[e]];
  } else {
#pragma unroll
    for (int e = 0; e < kGnE; ++e) v[e] = (float)((const f16_t*)p)[idx[e]];
  }
}

// The same for a [kGnCK][NP] tile of B or C ([batch,T,N]); entries past T or
// N are replaced by the caller.
template <int NP, int EB, int NT = kGnThreads>
__device__ __forceinline__ void gn_ld_bc(const ScanArgs& a, const void* p, int b, int64_t t0, float (&v)[EB]) {
  int64_t idx[EB];
#pragma unroll
  for (int e = 0; e < EB; ++e) {
    const int k = e * NT + (int)threadIdx.x;
    const int64_t t = t0 + k / NP;
    const int n = k % NP;
    idx[e] = ((int64_t)b * a.T + (t < a.T ? t : a.T - 1)) * a.N + (n < a.N ? n : a.N - 1);
  }
  if (a.bc_dt == NAJU_DTYPE_F32) {
#pragma unroll
    for (int e = 0; e < EB; ++e) v[e] = ((const float*)p)[idx[e]];
  } else if (a.bc_dt == NAJU_DTYPE_BF16) {
#pragma unroll
    for (int e = 0; e < EB; ++e) v[e] = (float)((const bf16_t*)p)[idx[e]];
  } else {
#pragma unroll
    for (int e = 0; e < EB; ++e) v[e] = (float)((const f16_t*)p)[idx[e]];
  }
}

// The same from a uniform tile base plus 32-bit lane offsets (the gq
// forward's staging; the segmented forward keeps gn_ld_bc, which measured
// faster there).
template <int NP, int EB, int NT = kGnThreads>
__device__ __forceinline__ void gq_ld_bc(const ScanArgs& a, const void* p, int b, int64_t t0, float (&v)[EB]) {
  static_assert(NT % NP == 0, "staging rows");
  // A uniform base (row t0 of batch row b) plus a 32-bit per-lane offset
  // (at most kGnCK rows x N < 2^12 elements): rows past T are clamped to the
  // last row, states past N to N - 1.
  const int64_t tb = t0 < a.T ? t0 : a.T - 1;
  const int rmax = (int)(a.T - tb < kGnCK ? a.T - tb : kGnCK) - 1;
  const int64_t row0 = ((int64_t)b * a.T + tb) * a.N;
  const int n = (int)threadIdx.x % NP;
  const uint32_t nn = (uint32_t)(n < a.N ? n : a.N - 1);
  uint32_t off[EB];
#pragma unroll
  for (int e = 0; e < EB; ++e) {
    const int r = e * (NT / NP) + (int)threadIdx.x / NP;
    off[e] = (uint32_t)(r < rmax ? r : rmax) * (uint32_t)a.N + nn;
  }
  if (a.bc_dt == NAJU_DTYPE_F32) {
    const float* q = (const float*)p + row0;
#pragma unroll
    for (int e = 0; e < EB; ++e) v[e] = q[off[e]];
  } else if (a.bc_dt == NAJU_DTYPE_BF16) {
    const bf16_t* q = (const bf16_t*)p + row0;
#pragma unroll
    for (int e = 0; e < EB; ++e) v[e] = (float)q[off[e]];
  } else {
    const f16_t* q = (const f16_t*)p + row0;
#pragma unroll
    for (int e = 0; e < EB; ++e) v[e] = (float)q[off[e]];
  }
}

// Writes a prefetched B/C tile into LDS, zero where the row is past T or the
// state index past N.
template <int NP, int EB>
__device__ __forceinline__ void gn_st_bc(const ScanArgs& a, int64_t t0, const float (&vb)[EB],
                                         const float (&vc)[EB], float (&sB)[kGnCK][NP], float (&sC)[kGnCK][NP]) {
#pragma unroll
  for (int e = 0; e < EB; ++e) {
    const int k = e * kGnThreads + (int)threadIdx.x;
    if (k < kGnCK * NP) {
      const int r = k / NP, n = k % NP;
      const bool ok = t0 + r < a.T && n < a.N;
      sB[r][n] = ok ? vb[e] : 0.f;
      sC[r][n] = ok ? vc[e] : 0.f;
    }
  }
}

// Writes one prefetched [kGnCK][NP] tile of B or C into LDS (zeros outside).
template <int NP, int EB>
__device__ __forceinline__ void gn_st_one(const ScanArgs& a, int64_t t0, const float (&v)[EB], float (&sv)[kGnCK][NP]) {
#pragma unroll
  for (int e = 0; e < EB; ++e) {
    const int k = e * kGnThreads + (int)threadIdx.x;
    if (k < kGnCK * NP) {
      const int r = k / NP, n = k % NP;
      sv[r][n] = (t0 + r < a.T && n < a.N) ? v[e] : 0.f;
    }
  }
}

// Time segments. With nseg > 1 the sub-chunks of T are split into nseg
// segments of seg_sc sub-chunks, each scanned by its own workgroup per
// channel tile (grid = tiles * segments, tile = blockIdx % tiles). The state
// entering a segment comes from three steps: every segment's map from a zero
// state (gc_fwd_kernel<NP, true>: decay F and state Z per channel), a carry
// pass over the segments (gn_seg_carry_kernel), then the full scan from the
// carried state. The backward mirrors this with the adjoint carry
// (gn_bwd_map_kernel, the carry in reverse, gn_bwd_kernel).

// Adjoint map of segment blockIdx / n_tiles + 1 (segments 1 .. nseg-1): the
// carry leaving the segment's first row towards the past, from a zero carry
// entering its last row (segZ), and the product of its gates (segF). Lanes
// over n as in gn_bwd_kernel; each sub-chunk's f, dy and C are staged in LDS
// transposed ([channel][row], [n][row]) so a 16-byte read yields four rows,
// with the next sub-chunk's loads in flight while this one is walked. Rows
// past T are staged as f = 1, dy = 0 and change nothing.
constexpr int kGmRP = kGnCK + 4;  // LDS row pitch of the transposed tiles

template <int NP>
__global__ __launch_bounds__(64 * kGnW) void gn_bwd_map_kernel(const ScanArgs a, int x_dt, int g_dt) {
  constexpr int LG = NP < 64 ? NP : 64;
  constexpr int S = NP / LG;
  constexpr int G = 64 / LG;
  constexpr int NPASS = kGnDT / G;
  constexpr int PPW = (NPASS + kGnW - 1) / kGnW;
  constexpr int EB = kGnCK * NP >= kGnThreads ? kGnCK * NP / kGnThreads : 1;
  constexpr int BCT = kGnCK * NP / EB;
  static_assert(kGnCK == 4 * kGnW, "tile shape");
  __shared__ __align__(16) float s_x[2][kGnDT][kGmRP];  // [0] f, [1] dy
  __shared__ __align__(16) float s_c[NP][kGmRP];
  const int N = a.N;
  const int mdt = (int)((a.D + kGnDT - 1) / kGnDT);  // this kernel's channel tiles
  const int mtiles = a.batch * mdt;
  const int tile = (int)(blockIdx.x % (uint32_t)mtiles);
  const int seg = (int)(blockIdx.x / (uint32_t)mtiles) + 1;
  const int b = tile / mdt;
  const int dtile = tile - b * mdt;
  const int64_t T = a.T, D = a.D;
  const int64_t dbase = (int64_t)dtile * kGnDT;
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gl = lane / LG, nl = lane - gl * LG;
  const int KC = (int)((T + kGnCK - 1) / kGnCK);
  const int sc0 = seg * a.seg_sc;
  const int sc1 = sc0 + a.seg_sc < KC ? sc0 + a.seg_sc : KC;
  const int64_t dl = dbase + lane;
  const bool dl_ok = dl < D;
  const uint32_t lane_c = (uint32_t)(dl_ok ? dl : D - 1) - (uint32_t)dbase;
  const int bn = tid % NP, bn_r0 = (tid / NP) * EB;
  const bool bn_act = tid < BCT;
  const int bnc = bn < N ? bn : N - 1;

  float gc[PPW][S], Ac[PPW];
#pragma unroll
  for (int q = 0; q < PPW; ++q) {
    Ac[q] = 1.f;
#pragma unroll
    for (int s2 = 0; s2 < S; ++s2) gc[q][s2] = 0.f;
  }
  float vf[4], vg[4], vc[EB];
  // this thread's rows 4*wv .. 4*wv+3 of channel lane (f, dy) and rows
  // bn_r0 .. of state bn (C) of the sub-chunk at t0 (rows clamped in bounds)
  auto load = [&](int64_t t0) {
    const int rows = (int)((T - t0) < kGnCK ? (T - t0) : kGnCK);
    const int64_t xrow0 = ((int64_t)b * T + t0) * D + dbase;
    uint32_t xo[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int rr = 4 * wv + e < rows ? 4 * wv + e : rows - 1;
      xo[e] = (uint32_t)rr * (uint32_t)D + lane_c;
    }
    auto ld4 = [&](const void* p, int dt, float (&o)[4]) {
      if (dt == NAJU_DTYPE_F32) {
        const char* q = (const char*)((const float*)p + xrow0);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = *(const float*)(q + xo[e] * 4u);
      } else if (dt == NAJU_DTYPE_BF16) {
        const char* q = (const char*)((const bf16_t*)p + xrow0);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = (float)*(const bf16_t*)(q + xo[e] * 2u);
      } else {
        const char* q = (const char*)((const f16_t*)p + xrow0);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = (float)*(const f16_t*)(q + xo[e] * 2u);
      }
    };
    ld4(a.fl, g_dt, vf);
    ld4(a.dy, x_dt, vg);
    if (bn_act) {
      const int64_t brow0 = ((int64_t)b * T + t0) * N;
#pragma unroll
      for (int e = 0; e < EB; ++e) {
        const int rr = bn_r0 + e < rows ? bn_r0 + e : rows - 1;
        const uint32_t o = (uint32_t)rr * (uint32_t)N + (uint32_t)bnc;
        if (a.bc_dt == NAJU_DTYPE_F32)
          vc[e] = *(const float*)((const char*)((const float*)a.Cm + brow0) + o * 4u);
        else if (a.bc_dt == NAJU_DTYPE_BF16)
          vc[e] = (float)*(const bf16_t*)((const char*)((const bf16_t*)a.Cm + brow0) + o * 2u);
        else
          vc[e] = (float)*(const f16_t*)((const char*)((const f16_t*)a.Cm + brow0) + o * 2u);
      }
    }
  };
  load((int64_t)(sc1 - 1) * kGnCK);
  for (int sc = sc1 - 1; sc >= sc0; --sc) {
    const int64_t t0 = (int64_t)sc * kGnCK;
    __syncthreads();  // the previous sub-chunk's tiles are consumed
    {
      float4 F4, Y4;
      float* pF = &F4.x;
      float* pY = &Y4.x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool ok = dl_ok && t0 + 4 * wv + e < T;
        pF[e] = ok ? sigm(vf[e]) : 1.f;
        pY[e] = ok ? vg[e] : 0.f;
      }
      *(float4*)&s_x[0][lane][4 * wv] = F4;
      *(float4*)&s_x[1][lane][4 * wv] = Y4;
      if (bn_act) {
#pragma unroll
        for (int e = 0; e < EB; ++e) s_c[bn][bn_r0 + e] = (t0 + bn_r0 + e < T && bn < N) ? vc[e] : 0.f;
      }
    }
    __syncthreads();
    if (sc > sc0) load(t0 - kGnCK);  // next (earlier) sub-chunk, while this one runs
#pragma unroll
    for (int q = 0; q < PPW; ++q) {
      const int pass = wv + q * kGnW;
      // only when some waves have fewer passes: a branch here would let the
      // LDS reads of later passes be hoisted above it
      if constexpr (NPASS % kGnW != 0) {
        if (pass >= NPASS) break;
      }
      const int c = pass * G + gl;
#pragma unroll
      for (int r4 = kGnCK - 4; r4 >= 0; r4 -= 4) {
        // reads issued per block: hoisted across the unrolled passes and
        // blocks they would need hundreds of registers
        __builtin_amdgcn_sched_barrier(0);
        const float4 f4 = *(const float4*)&s_x[0][c][r4], y4 = *(const float4*)&s_x[1][c][r4];
        float4 C4[S];
#pragma unroll
        for (int s2 = 0; s2 < S; ++s2) C4[s2] = *(const float4*)&s_c[nl + 64 * s2][r4];
#pragma unroll
        for (int e = 3; e >= 0; --e) {
          const float f = (&f4.x)[e], gy = (&y4.x)[e];
          Ac[q] *= f;
#pragma unroll
          for (int s2 = 0; s2 < S; ++s2) gc[q][s2] = f * fmaf(gy, (&C4[s2].x)[e], gc[q][s2]);
        }
      }
    }
  }
#pragma unroll
  for (int q = 0; q < PPW; ++q) {
    const int pass = wv + q * kGnW;
    if (pass >= NPASS) break;
    const int64_t d = dbase + (int64_t)pass * G + gl;
    if (d >= D) continue;
    const int64_t o = ((int64_t)b * a.nseg + seg) * D + d;
#pragma unroll
    for (int s2 = 0; s2 < S; ++s2) {
      const int n = nl + 64 * s2;
      if (n < N) a.segZ[o * N + n] = gc[q][s2];
    }
    if (nl == 0) a.segF[o] = Ac[q];
  }
}

// ----------------------------------------------- general N forward, lanes over d
//
// The forward of N > 1 runs with one channel per lane and its NP states in
// VGPRs (NP = N rounded up to a power of two; states n >= N see B = C = 0 and
// stay 0). A wave owns 64 consecutive channels of one batch row, a workgroup
// kGcW waves, for one time segment. B_t and C_t rows of a kGnCK-row sub-chunk
// are staged in LDS (converted to f32) and read back as broadcasts, so a row
// costs 2 FMA + 1 multiply per state and no cross-lane sums. Per-lane inputs
// are loaded in groups of kGcRG rows, the next group while the current one
// is scanned. MAP: the segment's map from a zero state (decay F and state Z
// per channel) for the carry pass; otherwise the scan itself from the
// segment's entering state, with y, the checkpoint and hT.
constexpr int kGcW = 4;            // waves per workgroup
constexpr int kGcCH = 64 * kGcW;   // channels per workgroup
constexpr int kGcRG = 8;           // rows per input group

// The lane's channel's values of rows t0 .. t0+kGcRG-1 (clamped in bounds).
__device__ __forceinline__ void gc_ld_rows(const void* p, int dt, int64_t rowbase, int64_t t0, int64_t T, int64_t D,
                                           int64_t d, float (&v)[kGcRG]) {
  int64_t idx[kGcRG];
#pragma unroll
  for (int r = 0; r < kGcRG; ++r) idx[r] = (rowbase + (t0 + r < T ? t0 + r : T - 1)) * D + d;
  if (dt == NAJU_DTYPE_F32) {
#pragma unroll
    for (int r = 0; r < kGcRG; ++r) v[r] = ((const float*)p)[idx[r]];
  } else if (dt == NAJU_DTYPE_BF16) {
#pragma unroll
    for (int r = 0; r < kGcRG; ++r) v[r] = (float)((const bf16_t*)p)[idx[r]];
  } else {
#pragma unroll
    for (int r = 0; r < kGcRG; ++r) v[r] = (float)((const f16_t*)p)[idx[r]];
  }
}

template <int NP, bool MAP>
__global__ __launch_bounds__(64 * kGcW) void gc_fwd_kernel(const ScanArgs a, int x_dt, int g_dt, int y_dt) {
  constexpr int EB = (kGnCK * NP + 64 * kGcW - 1) / (64 * kGcW);
  __shared__ float s_B[kGnCK][NP];
  __shared__ float s_C[MAP ? 1 : kGnCK][NP];
  const int N = a.N;
  const int64_t T = a.T, D = a.D;
  const int ndt = (int)((D + kGcCH - 1) / kGcCH);
  const int ntl = a.batch * ndt;
  const int tile = (int)(blockIdx.x % (uint32_t)ntl);
  const int seg = (int)(blockIdx.x / (uint32_t)ntl);
  const int b = tile / ndt;
  const int dtile = tile - b * ndt;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t d = (int64_t)dtile * kGcCH + wv * 64 + lane;
  const bool dok = d < D;
  const int64_t dc = dok ? d : D - 1;  // clamped channel for loads
  const int KC = (int)((T + kGnCK - 1) / kGnCK);
  const int sc0 = seg * a.seg_sc;
  const int sc1 = sc0 + a.seg_sc < KC ? sc0 + a.seg_sc : KC;
  const int64_t rowbase = (int64_t)b * T;
  const int64_t t_beg = (int64_t)sc0 * kGnCK;
  const int64_t t_end = (int64_t)sc1 * kGnCK < T ? (int64_t)sc1 * kGnCK : T;

  float x[NP];
  {
    const float* xin = MAP ? nullptr
                           : (a.nseg > 1 ? a.seg0 + ((int64_t)b * a.nseg + seg) * D * N
                                         : (a.h0 ? a.h0 + (int64_t)b * D * N : nullptr));
#pragma unroll
    for (int n = 0; n < NP; ++n) x[n] = (xin && dok && n < N) ? xin[dc * N + n] : 0.f;
  }
  float Fd = 1.f;
  const float Dv = MAP ? 0.f : a.Dsk[dc];

  float gu[kGcRG], gf[kGcRG], gi[kGcRG];  // the next input group
  gc_ld_rows(a.u, x_dt, rowbase, t_beg, T, D, dc, gu);
  gc_ld_rows(a.fl, g_dt, rowbase, t_beg, T, D, dc, gf);
  gc_ld_rows(a.il, g_dt, rowbase, t_beg, T, D, dc, gi);
  float vb[EB], vc[EB];  // B (and C) rows of the next sub-chunk
  gn_ld_bc<NP, EB, 64 * kGcW>(a, a.Bm, b, t_beg, vb);
  if (!MAP) gn_ld_bc<NP, EB, 64 * kGcW>(a, a.Cm, b, t_beg, vc);
  for (int sc = sc0; sc < sc1; ++sc) {
    const int64_t t0 = (int64_t)sc * kGnCK;
    __syncthreads();  // the previous sub-chunk's B/C rows are consumed
    {
      // stage B (and C) rows of the sub-chunk, f32, zero outside [0,T) x [0,N)
#pragma unroll
      for (int e = 0; e < EB; ++e) {
        const int k = e * 64 * kGcW + (int)threadIdx.x;
        if (k < kGnCK * NP) {
          const int r = k / NP, n = k % NP;
          const bool ok = t0 + r < T && n < N;
          s_B[r][n] = ok ? vb[e] : 0.f;
          if (!MAP) s_C[MAP ? 0 : r][n] = ok ? vc[e] : 0.f;
        }
      }
    }
    __syncthreads();
    if (sc + 1 < sc1) {
      gn_ld_bc<NP, EB, 64 * kGcW>(a, a.Bm, b, t0 + kGnCK, vb);
      if (!MAP) gn_ld_bc<NP, EB, 64 * kGcW>(a, a.Cm, b, t0 + kGnCK, vc);
    }
    if (!MAP && a.ckpt && dok) {
      float* ck = a.ckpt + (((int64_t)b * KC + sc) * D + d) * N;
#pragma unroll
      for (int n = 0; n < NP; ++n)
        if (n < N) ck[n] = x[n];
    }
    const int rows = (int)((T - t0) < kGnCK ? (T - t0) : kGnCK);
#pragma unroll 1
    for (int r0 = 0; r0 < rows; r0 += kGcRG) {
      float cu[kGcRG], cf[kGcRG], ci[kGcRG];
#pragma unroll
      for (int r = 0; r < kGcRG; ++r) {
        cu[r] = gu[r];
        cf[r] = gf[r];
        ci[r] = gi[r];
      }
      const int64_t tn = t0 + r0 + kGcRG;
      if (tn < t_end) {
        gc_ld_rows(a.u, x_dt, rowbase, tn, T, D, dc, gu);
        gc_ld_rows(a.fl, g_dt, rowbase, tn, T, D, dc, gf);
        gc_ld_rows(a.il, g_dt, rowbase, tn, T, D, dc, gi);
      }
      float yv[kGcRG];
#pragma unroll
      for (int r = 0; r < kGcRG; ++r) {
        yv[r] = 0.f;
        if (r0 + r < rows) {
          const float f = sigm(cf[r]);
          const float w = sigm(ci[r]) * cu[r];
          const int rr = r0 + r;
          if (MAP) {
            Fd *= f;
#pragma unroll
            for (int n = 0; n < NP; ++n) {
              // f*x then + w*B as two in-place updates of x (a multiply and
              // an accumulating FMA): no temporary per state and no register
              // move of the loop-carried state
              x[n] *= f;
              x[n] = fmaf(w, s_B[rr][n], x[n]);
            }
          } else {
            float y4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int n = 0; n < NP; ++n) {
              x[n] *= f;
              x[n] = fmaf(w, s_B[rr][n], x[n]);
              y4[n & 3] = fmaf(s_C[MAP ? 0 : rr][n], x[n], y4[n & 3]);
            }
            yv[r] = fmaf(Dv, cu[r], (y4[0] + y4[1]) + (y4[2] + y4[3]));
          }
        }
      }
      if (!MAP && dok) {
        const int64_t o = (rowbase + t0 + r0) * D + d;
        if (y_dt == NAJU_DTYPE_F32) {
#pragma unroll
          for (int r = 0; r < kGcRG; ++r)
            if (r0 + r < rows) ((float*)a.y)[o + (int64_t)r * D] = yv[r];
        } else if (y_dt == NAJU_DTYPE_BF16) {
#pragma unroll
          for (int r = 0; r < kGcRG; ++r)
            if (r0 + r < rows) ((bf16_t*)a.y)[o + (int64_t)r * D] = (bf16_t)yv[r];
        } else {
#pragma unroll
          for (int r = 0; r < kGcRG; ++r)
            if (r0 + r < rows) ((f16_t*)a.y)[o + (int64_t)r * D] = (f16_t)yv[r];
        }
      }
    }
  }
  if (!dok) return;
  if (MAP) {
    const int64_t o = ((int64_t)b * a.nseg + seg) * D + d;
#pragma unroll
    for (int n = 0; n < NP; ++n)
      if (n < N) a.segZ[o * N + n] = x[n];
    a.segF[o] = Fd;
  } else if (a.hT && seg == a.nseg - 1) {
#pragma unroll
    for (int n = 0; n < NP; ++n)
      if (n < N) a.hT[((int64_t)b * D + d) * N + n] = x[n];
  }
}

// Carry over the time segments, one thread per (b, d, n): the state entering
// each segment (dir = +1, from h0) or the adjoint carry entering it from the
// future (dir = -1, from zero), into seg0.
__global__ void gn_seg_carry_kernel(const ScanArgs a, int dir) {
  const int64_t DN = a.D * (int64_t)a.N;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.batch * DN) return;
  const int64_t b = i / DN, dn = i - b * DN, d = dn / a.N;
  const int ns = a.nseg;
  if (dir > 0) {
    float x = a.h0 ? a.h0[i] : 0.f;
    for (int sg = 0; sg < ns; ++sg) {
      const int64_t o = (b * ns + sg) * a.D + d;
      a.seg0[o * a.N + (dn - d * a.N)] = x;
      if (sg + 1 < ns) x = fmaf(a.segF[o], x, a.segZ[o * a.N + (dn - d * a.N)]);
    }
  } else {
    float g = 0.f;
    for (int sg = ns - 1; sg >= 0; --sg) {
      const int64_t o = (b * ns + sg) * a.D + d;
      a.seg0[o * a.N + (dn - d * a.N)] = g;
      if (sg > 0) g = fmaf(a.segF[o], g, a.segZ[o * a.N + (dn - d * a.N)]);
    }
  }
}


// ------------------------------------------------- general N backward kernel
//
// One workgroup per (batch row, 64-channel tile, time segment), 8 waves.
// Lanes run over the state index n (LG = min(NP, 64) lanes per channel, S
// states per lane, G channels per wave instruction). A wave walks its
// channel passes one after another; per kGnCK-row sub-chunk (the checkpoint
// interval, walked from the last to the first) and per 16-row half (the later
// half first) it
//   1. recomputes the forward states of the half's rows from the checkpoint
//      (the earlier half's rows first, unstored, when it is the later half),
//   2. runs the adjoint x̄_t = C_t dy_t + g, g <- f_t x̄_t backwards over
//      the rows, with this lane's terms of sum_n x̄_t x_{t-1} (dfl) and
//      sum_n x̄_t B_t (dws), and of the dB / dC sums over the channels,
//   3. reduces the dfl / dws terms over the channel's lanes every 8 rows with
//      a transposing butterfly made of DPP and lane-swap moves, and writes
//      du, dfl, dil over the consumed inputs in LDS.
// The inputs of a sub-chunk are staged in LDS transposed, as [channel][row]
// and [n][row], so one 16-byte read yields four rows of a channel (or of a
// state) and a row costs a quarter of an LDS instruction per stream. Rows
// past T and channels past D are staged as the neutral step (f = 1, i = u =
// dy = 0, B = C = 0), so the loops carry no row guards; the stores skip them.
constexpr int kGnH = 16;          // rows per adjoint half
constexpr int kGnRG = 8;          // rows per reduction group
constexpr int kGnRP = kGnCK + 4;  // LDS row pitch (floats) of the transposed tiles

// Value of lane l ^ m for the lanes with bit log2(m) clear.
template <int m>
__device__ __forceinline__ float from_upper(float x) {
  if constexpr (m == 32) {
    return __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false)[1]);
  } else if constexpr (m == 16) {
    return __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false)[1]);
  } else {
    return __shfl_xor(x, m, 64);
  }
}

// General-N forward with Q = NP/4 lanes per channel, four states per lane,
// over the whole of T: lane (channel c, quarter q) holds x[n] for
// n = 4q .. 4q+3. With Q times the lanes per channel of gc_fwd_kernel it
// needs no time segments (no segment-map pass, no carry pass) once the
// batch x channel-group grid fills the GPU on its own. Per
// 32-row sub-chunk the workgroup stages B and C ([row][n]) and the channels'
// gates f, w = i*u and u ([row][channel]) in LDS, each value computed once;
// a lane's part of y_t = sum_n C_t[n] x_t[n] is summed over the channel's Q
// lanes by a transposing butterfly over 8 rows at a time, and y goes back
// through LDS so that its stores are row-contiguous.
constexpr int kGqW = 4;   // waves per workgroup
constexpr int kGqRG = 8;  // rows per reduction group

template <int NP>
__global__ __launch_bounds__(64 * kGqW) void gq_fwd_kernel(const ScanArgs a, int x_dt, int g_dt, int y_dt) {
  constexpr int Q = NP / 4;          // lanes per channel
  constexpr int CPW = 64 / Q;        // channels per wave
  constexpr int CPB = CPW * kGqW;    // channels per workgroup
  constexpr int NT = 64 * kGqW;      // threads
  constexpr int EB = kGnCK * NP / NT;   // B / C values staged per thread
  constexpr int EG = kGnCK * CPB / NT;  // gate values staged per thread
  static_assert(Q >= 4 && Q <= 16 && EB >= 1 && EG >= 1, "tile shape");
  __shared__ __align__(16) float s_B[kGnCK][NP];
  __shared__ __align__(16) float s_C[kGnCK][NP];
  __shared__ float s_f[kGnCK][CPB], s_w[kGnCK][CPB], s_u[kGnCK][CPB], s_y[kGnCK][CPB];
  const int N = a.N;
  const int64_t T = a.T, D = a.D;
  const int ndt = (int)((D + CPB - 1) / CPB);
  const int b = (int)(blockIdx.x / (uint32_t)ndt);
  const int dtile = (int)(blockIdx.x - (uint32_t)b * (uint32_t)ndt);
  const int64_t dbase = (int64_t)dtile * CPB;
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int cl = wv * CPW + lane / Q;  // this lane's channel within the workgroup
  const int q = lane % Q;
  const int64_t d = dbase + cl;
  const bool dok = d < D;
  const int64_t rowbase = (int64_t)b * T;
  const int KC = (int)((T + kGnCK - 1) / kGnCK);
  const int sc0 = 0, sc1 = KC;
  const float* xin = a.h0 ? a.h0 + (int64_t)b * D * N : nullptr;
  float x[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int n = 4 * q + k;
    x[k] = (xin && dok && n < N) ? xin[d * N + n] : 0.f;
  }
  // staging roles for the gates: entry k = e * NT + tid -> (row, channel)
  // two register sets of staged inputs: sub-chunk sc is loaded while
  // sc - 2 is computed (a wave's compute of one sub-chunk is shorter than
  // the load latency)
  float gu0[EG], gf0[EG], gi0[EG], vb0[EB], vc0[EB];
  float gu1[EG], gf1[EG], gi1[EG], vb1[EB], vc1[EB];
  auto load = [&](int64_t t0, float (&gu)[EG], float (&gf)[EG], float (&gi)[EG], float (&vb)[EB],
                  float (&vc)[EB]) {
#pragma unroll
    for (int e = 0; e < EG; ++e) {
      const int k = e * NT + tid;
      const int r = k / CPB, c = k % CPB;
      const int64_t t = t0 + r < T ? t0 + r : T - 1;
      const int64_t dc = dbase + c < D ? dbase + c : D - 1;
      const int64_t o = (rowbase + t) * D + dc;
      gu[e] = ld_any(a.u, x_dt, o);
      gf[e] = ld_any(a.fl, g_dt, o);
      gi[e] = ld_any(a.il, g_dt, o);
    }
    gq_ld_bc<NP, EB, NT>(a, a.Bm, b, t0, vb);
    gq_ld_bc<NP, EB, NT>(a, a.Cm, b, t0, vc);
  };
  auto body = [&](int sc, float (&gu)[EG], float (&gf)[EG], float (&gi)[EG], float (&vb)[EB], float (&vc)[EB]) {
    const int64_t t0 = (int64_t)sc * kGnCK;
    const int rows = (int)((T - t0) < kGnCK ? (T - t0) : kGnCK);
    __syncthreads();  // the previous sub-chunk's tiles are consumed, its y stored
#pragma unroll
    for (int e = 0; e < EG; ++e) {
      const int k = e * NT + tid;
      const int r = k / CPB, c = k % CPB;
      const bool ok = r < rows && dbase + c < D;
      const float f = sigm(gf[e]);
      s_f[r][c] = ok ? f : 1.f;
      s_w[r][c] = ok ? sigm(gi[e]) * gu[e] : 0.f;
      s_u[r][c] = ok ? gu[e] : 0.f;
    }
#pragma unroll
    for (int e = 0; e < EB; ++e) {
      const int k = e * NT + tid;
      const int r = k / NP, n = k % NP;
      const bool ok = r < rows && n < N;
      s_B[r][n] = ok ? vb[e] : 0.f;
      s_C[r][n] = ok ? vc[e] : 0.f;
    }
    __syncthreads();
    if (sc + 2 < sc1) load(t0 + 2 * kGnCK, gu, gf, gi, vb, vc);  // while this one runs
    // the state entering this sub-chunk: the backward's checkpoint
    if (a.ckpt && dok) {
      float* ck = a.ckpt + (((int64_t)b * KC + sc) * D + d) * N;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (4 * q + k < N) ck[4 * q + k] = x[k];
    }
#pragma unroll
    for (int g = 0; g < kGnCK; g += kGqRG) {
      float yp[kGqRG];
#pragma unroll
      for (int rr = 0; rr < kGqRG; ++rr) {
        const int r = g + rr;
        const float f = s_f[r][cl], w = s_w[r][cl];
        const float4 b4 = *(const float4*)&s_B[r][4 * q];
        const float4 c4 = *(const float4*)&s_C[r][4 * q];
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          x[k] *= f;
          x[k] = fmaf(w, (&b4.x)[k], x[k]);
          acc = fmaf((&c4.x)[k], x[k], acc);
        }
        yp[rr] = acc;
      }
      // sums over the channel's Q lanes: lane q then holds row q / (Q / 8)
      // of the group (Q >= 8), or rows 2q, 2q+1 (Q = 4)
      trd_step<Q, kGqRG, kGqRG>(yp, lane);
      if constexpr (Q >= kGqRG) {
        constexpr int SP = Q / kGqRG;
        if (q % SP == 0) {
          const int r = g + q / SP;
          s_y[r][cl] = fmaf(a.Dsk[dok ? d : 0], s_u[r][cl], yp[0]);
        }
      } else {
        constexpr int PER = kGqRG / Q;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
          const int r = g + q * PER + j;
          s_y[r][cl] = fmaf(a.Dsk[dok ? d : 0], s_u[r][cl], yp[j]);
        }
      }
    }
    __syncthreads();
    // y of the sub-chunk, row-contiguous stores
#pragma unroll
    for (int e = 0; e < EG; ++e) {
      const int k = e * NT + tid;
      const int r = k / CPB, c = k % CPB;
      if (r < rows && dbase + c < D) st_any(a.y, y_dt, (rowbase + t0 + r) * D + dbase + c, s_y[r][c]);
    }
  };
  load((int64_t)sc0 * kGnCK, gu0, gf0, gi0, vb0, vc0);
  if (sc0 + 1 < sc1) load((int64_t)(sc0 + 1) * kGnCK, gu1, gf1, gi1, vb1, vc1);
  for (int sc = sc0; sc < sc1; sc += 2) {
    body(sc, gu0, gf0, gi0, vb0, vc0);
    if (sc + 1 < sc1) body(sc + 1, gu1, gf1, gi1, vb1, vc1);
  }
  if (a.hT && dok) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (4 * q + k < N) a.hT[((int64_t)b * D + d) * N + 4 * q + k] = x[k];
  }
}

template <int NP, int DT, int W>
__global__ __launch_bounds__(64 * W) void gn_bwd_kernel(const ScanArgs a, int x_dt, int g_dt, int du_dt,
                                                           int dg_dt) {
  constexpr int LG = NP < 64 ? NP : 64;
  constexpr int S = NP / LG;
  constexpr int G = 64 / LG;
  constexpr int TH = 64 * W;         // threads
  constexpr int RGS = TH / DT;        // staging row groups of 4 rows
  constexpr int NPASS = DT / G;
  constexpr int PPW = (NPASS + W - 1) / W;
  static_assert(RGS * 4 == kGnCK && kGnCK == 2 * kGnH && kGnH == 2 * kGnRG, "tile shape");
  // B / C staging: thread -> state n = tid % NP, rows [rb*EB, rb*EB + EB)
  constexpr int EB = kGnCK * NP >= TH ? kGnCK * NP / TH : 1;
  constexpr int BCT = kGnCK * NP / EB;  // threads that stage B / C
  // one object per tile family, so a lane addresses all of them from one
  // base register plus immediate offsets: [0] f, [1] i, [2] u, [3] dy
  // ([channel][row]); [0] B, [1] C ([n][row])
  __shared__ __align__(16) float s_x[4][DT][kGnRP];
  __shared__ __align__(16) float s_bc[2][NP][kGnRP];
  __shared__ float s_pB[kGnCK][NP], s_pC[kGnCK][NP];
  __shared__ float s_dD[RGS][DT];
  __shared__ float s_Dsk[DT];
  const int N = a.N;
  const int tile = (int)(blockIdx.x % (uint32_t)a.n_tiles);
  const int seg = (int)(blockIdx.x / (uint32_t)a.n_tiles);
  const int b = tile / a.n_dtiles;
  const int dtile = tile - b * a.n_dtiles;
  const int64_t T = a.T, D = a.D;
  const int64_t dbase = (int64_t)dtile * DT;
  const int tid = (int)threadIdx.x;
  if (tid < DT) s_Dsk[tid] = dbase + tid < D ? a.Dsk[dbase + tid] : 0.f;  // read after the first barrier
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gl = lane / LG, nl = lane - gl * LG;
  const int KC = (int)((T + kGnCK - 1) / kGnCK);
  const int64_t btn = (int64_t)a.batch * T * N;
  const int sc0 = seg * a.seg_sc;
  const int sc1 = sc0 + a.seg_sc < KC ? sc0 + a.seg_sc : KC;
  // staging roles: channel sch, rows 4*srg .. 4*srg+3; B / C state bn, rows
  // bn_r0 .. bn_r0+EB-1
  const int sch = tid % DT, srg = tid / DT;
  const int64_t dl = dbase + sch;
  const bool dl_ok = dl < D;
  const uint32_t lane_c = (uint32_t)(dl_ok ? dl : D - 1) - (uint32_t)dbase;  // clamped channel offset
  const int bn = tid % NP, bn_r0 = (tid / NP) * EB;
  const bool bn_act = tid < BCT;
  const int bnc = bn < N ? bn : N - 1;

  // adjoint carry f_{t+1} x̄_{t+1} per channel pass: zero past the end of T,
  // else the carry entering the segment from the future
  const float* gin = a.nseg > 1 ? a.seg0 + ((int64_t)b * a.nseg + seg) * D * N : nullptr;
  float gc[PPW][S];
#pragma unroll
  for (int q = 0; q < PPW; ++q) {
    const int64_t d = dbase + (int64_t)(wv + q * W) * G + gl;
#pragma unroll
    for (int s2 = 0; s2 < S; ++s2) {
      const int n = nl + 64 * s2;
      gc[q][s2] = (gin && n < N && d < D) ? gin[d * N + n] : 0.f;
    }
  }
  float dDacc = 0.f;

  for (int sc = sc1 - 1; sc >= sc0; --sc) {
    const int64_t t0 = (int64_t)sc * kGnCK;
    const int rows = (int)((T - t0) < kGnCK ? (T - t0) : kGnCK);
    // this sub-chunk's inputs and checkpointed states
    // Global addresses are a uniform 64-bit base (this sub-chunk's first
    // row) plus a 32-bit per-lane element offset (clamped in bounds), so a
    // stream costs one address register per lane.
    const int64_t xrow0 = ((int64_t)b * T + t0) * D + dbase;  // [B,T,D] element of (t0, dbase)
    const int64_t brow0 = ((int64_t)b * T + t0) * N;          // [B,T,N] element of (t0, 0)
    float vu[4], vf[4], vi[4], vg[4], vb[EB], vc[EB];
    {
      uint32_t xo[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int rr = 4 * srg + e < rows ? 4 * srg + e : rows - 1;
        xo[e] = (uint32_t)rr * (uint32_t)D + lane_c;
      }
      auto ld4 = [&](const void* p, int dt, float (&o)[4]) {
        if (dt == NAJU_DTYPE_F32) {
          const char* q = (const char*)((const float*)p + xrow0);
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = *(const float*)(q + xo[e] * 4u);
        } else if (dt == NAJU_DTYPE_BF16) {
          const char* q = (const char*)((const bf16_t*)p + xrow0);
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = (float)*(const bf16_t*)(q + xo[e] * 2u);
        } else {
          const char* q = (const char*)((const f16_t*)p + xrow0);
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = (float)*(const f16_t*)(q + xo[e] * 2u);
        }
      };
      ld4(a.u, x_dt, vu);
      ld4(a.fl, g_dt, vf);
      ld4(a.il, g_dt, vi);
      ld4(a.dy, x_dt, vg);
      uint32_t bo[EB];
#pragma unroll
      for (int e = 0; e < EB; ++e) {
        const int rr = bn_r0 + e < rows ? bn_r0 + e : rows - 1;
        bo[e] = (uint32_t)rr * (uint32_t)N + (uint32_t)bnc;
      }
      if (bn_act) {
        if (a.bc_dt == NAJU_DTYPE_F32) {
          const char* qb = (const char*)((const float*)a.Bm + brow0);
          const char* qc = (const char*)((const float*)a.Cm + brow0);
#pragma unroll
          for (int e = 0; e < EB; ++e) vb[e] = *(const float*)(qb + bo[e] * 4u), vc[e] = *(const float*)(qc + bo[e] * 4u);
        } else if (a.bc_dt == NAJU_DTYPE_BF16) {
          const char* qb = (const char*)((const bf16_t*)a.Bm + brow0);
          const char* qc = (const char*)((const bf16_t*)a.Cm + brow0);
#pragma unroll
          for (int e = 0; e < EB; ++e)
            vb[e] = (float)*(const bf16_t*)(qb + bo[e] * 2u), vc[e] = (float)*(const bf16_t*)(qc + bo[e] * 2u);
        } else {
          const char* qb = (const char*)((const f16_t*)a.Bm + brow0);
          const char* qc = (const char*)((const f16_t*)a.Cm + brow0);
#pragma unroll
          for (int e = 0; e < EB; ++e)
            vb[e] = (float)*(const f16_t*)(qb + bo[e] * 2u), vc[e] = (float)*(const f16_t*)(qc + bo[e] * 2u);
        }
      }
    }
    float x0[PPW][S];
    {
      const float* ck = a.ckpt + (((int64_t)b * KC + sc) * D + dbase) * N;
#pragma unroll
      for (int q = 0; q < PPW; ++q) {
        const int cq = (wv + q * W) * G;  // first channel of the pass (uniform)
        const float* ckq = ck + (int64_t)cq * N;
#pragma unroll
        for (int s2 = 0; s2 < S; ++s2) {
          const int n = nl + 64 * s2;
          const bool ok = n < N && dbase + cq + gl < D && wv + q * W < NPASS;
          x0[q][s2] = ok ? *(const float*)((const char*)ckq + ((uint32_t)gl * (uint32_t)N + (uint32_t)n) * 4u) : 0.f;
        }
      }
    }
    __syncthreads();  // the previous sub-chunk's LDS tiles are stored
    {
      float4 F, I, U, Y;
      float* pF = &F.x;
      float* pI = &I.x;
      float* pU = &U.x;
      float* pY = &Y.x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool ok = dl_ok && t0 + 4 * srg + e < T;
        pF[e] = ok ? sigm(vf[e]) : 1.f;
        pI[e] = ok ? sigm(vi[e]) : 0.f;
        // the tile holds w = i*u, the only form the recompute and the
        // adjoint use (dil is formed from it below)
        pU[e] = ok ? pI[e] * vu[e] : 0.f;
        pY[e] = ok ? vg[e] : 0.f;
        dDacc = fmaf(pY[e], ok ? vu[e] : 0.f, dDacc);
      }
      *(float4*)&s_x[0][sch][4 * srg] = F;
      *(float4*)&s_x[1][sch][4 * srg] = I;
      *(float4*)&s_x[2][sch][4 * srg] = U;
      *(float4*)&s_x[3][sch][4 * srg] = Y;
      if (bn_act) {
#pragma unroll
        for (int e = 0; e < EB; ++e) {
          const bool ok = t0 + bn_r0 + e < T && bn < N;
          s_bc[0][bn][bn_r0 + e] = ok ? vb[e] : 0.f;
          s_bc[1][bn][bn_r0 + e] = ok ? vc[e] : 0.f;
        }
      }
    }
    __syncthreads();

    for (int h = 1; h >= 0; --h) {
      const int hr0 = h * kGnH;
      if (hr0 >= rows) continue;  // uniform over the workgroup
      float accB[kGnH][S], accC[kGnH][S];
#pragma unroll
      for (int r = 0; r < kGnH; ++r)
#pragma unroll
        for (int s2 = 0; s2 < S; ++s2) accB[r][s2] = accC[r][s2] = 0.f;
#pragma unroll
      for (int q = 0; q < PPW; ++q) {
        const int pass = wv + q * W;
        if constexpr (NPASS % W != 0) {
          if (pass >= NPASS) break;
        }
        // passes are independent: keep the scheduler from interleaving them
        // (their live registers would add up)
        __builtin_amdgcn_sched_barrier(0);
        const int c = pass * G + gl;
        float xs[S];
#pragma unroll
        for (int s2 = 0; s2 < S; ++s2) xs[s2] = x0[q][s2];
        // forward states: rows [0, hr0) unstored, then the half's rows
        for (int r4 = 0; r4 < hr0; r4 += 4) {
          const float4 f4 = *(const float4*)&s_x[0][c][r4];
          const float4 u4 = *(const float4*)&s_x[2][c][r4];
          float4 B4[S];
#pragma unroll
          for (int s2 = 0; s2 < S; ++s2) B4[s2] = *(const float4*)&s_bc[0][nl + 64 * s2][r4];
          const float* pf = &f4.x;
          const float* pu = &u4.x;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float iu = pu[e];
#pragma unroll
            for (int s2 = 0; s2 < S; ++s2) xs[s2] = fmaf(iu, (&B4[s2].x)[e], xs[s2] * pf[e]);
          }
        }
        float xin[S], hist[kGnH][S];
#pragma unroll
        for (int s2 = 0; s2 < S; ++s2) xin[s2] = xs[s2];
        // The LDS reads of each 4-row block are issued right before the
        // block (scheduling fences): hoisting all of a half's reads would
        // hold 16 rows of operands in registers at once.
#pragma unroll
        for (int r4 = 0; r4 < kGnH; r4 += 4) {
          __builtin_amdgcn_sched_barrier(0);
          const int r = hr0 + r4;
          const float4 f4 = *(const float4*)&s_x[0][c][r];
          const float4 u4 = *(const float4*)&s_x[2][c][r];
          float4 B4[S];
#pragma unroll
          for (int s2 = 0; s2 < S; ++s2) B4[s2] = *(const float4*)&s_bc[0][nl + 64 * s2][r];
          const float* pf = &f4.x;
          const float* pu = &u4.x;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float iu = pu[e];
#pragma unroll
            for (int s2 = 0; s2 < S; ++s2) {
              xs[s2] = fmaf(iu, (&B4[s2].x)[e], xs[s2] * pf[e]);
              hist[r4 + e][s2] = xs[s2];
            }
          }
        }
        // adjoint over the half's rows, last first, reduced every kGnRG rows.
        // The memory clobber makes it read its operands from LDS again
        // instead of keeping the recompute's 16 rows of them in registers.
        asm volatile("" ::: "memory");
#pragma unroll
        for (int grp = kGnH / kGnRG - 1; grp >= 0; --grp) {
          float v[2 * kGnRG];  // [0, kGnRG): dfl terms, [kGnRG, 2 kGnRG): dws terms
#pragma unroll
          for (int r4 = kGnRG - 4; r4 >= 0; r4 -= 4) {
            __builtin_amdgcn_sched_barrier(0);
            const int lr = grp * kGnRG + r4;  // local row of the half
            const int r = hr0 + lr;
            const float4 f4 = *(const float4*)&s_x[0][c][r];
            const float4 u4 = *(const float4*)&s_x[2][c][r], y4 = *(const float4*)&s_x[3][c][r];
            float4 B4[S], C4[S];
#pragma unroll
            for (int s2 = 0; s2 < S; ++s2) {
              B4[s2] = *(const float4*)&s_bc[0][nl + 64 * s2][r];
              C4[s2] = *(const float4*)&s_bc[1][nl + 64 * s2][r];
            }
            const float* pf = &f4.x;
            const float* pu = &u4.x;
            const float* py = &y4.x;
#pragma unroll
            for (int e = 3; e >= 0; --e) {
              const int j = r4 + e;  // row within the group
              const float iu = pu[e], gy = py[e];
              float tf = 0.f, tw = 0.f;
#pragma unroll
              for (int s2 = 0; s2 < S; ++s2) {
                const float xprev = lr + e > 0 ? hist[lr + e - 1][s2] : xin[s2];
                const float xb = fmaf(gy, (&C4[s2].x)[e], gc[q][s2]);
                tf = fmaf(xb, xprev, tf);
                tw = fmaf(xb, (&B4[s2].x)[e], tw);
                accB[lr + e][s2] = fmaf(xb, iu, accB[lr + e][s2]);
                accC[lr + e][s2] = fmaf(gy, hist[lr + e][s2], accC[lr + e][s2]);
                // keep the updates here: sunk to the end of the pass they
                // would hold every row's operands in registers
                asm volatile("" : "+v"(accB[lr + e][s2]), "+v"(accC[lr + e][s2]));
                gc[q][s2] = pf[e] * xb;
              }
              v[j] = tf;
              v[kGnRG + j] = tw;
            }
          }
          __builtin_amdgcn_sched_barrier(0);
          trd_step<LG, 2 * kGnRG, 2 * kGnRG>(v, lane);
          // lanes holding dfl sums (the lower half of the group) take the
          // matching dws sums from the upper half and write the outputs over
          // the consumed f, i, u of their rows
          constexpr int KF = 2 * kGnRG >= LG ? 2 * kGnRG / LG : 1;
          constexpr int SPREAD = 2 * kGnRG >= LG ? 1 : LG / (2 * kGnRG);
          float vw[KF];
#pragma unroll
          for (int j = 0; j < KF; ++j) vw[j] = from_upper<LG / 2>(v[j]);
          if (nl < LG / 2 && nl % SPREAD == 0) {
            const int e0 = (nl / SPREAD) * KF;
#pragma unroll
            for (int j = 0; j < KF; ++j) {
              const int r = hr0 + grp * kGnRG + e0 + j;
              const float f = s_x[0][c][r], ig = s_x[1][c][r], w = s_x[2][c][r], gy = s_x[3][c][r];
              s_x[1][c][r] = fmaf(ig, vw[j], s_Dsk[c] * gy);     // du
              s_x[0][c][r] = fmaf(-f, f, f) * v[j];              // dfl
              s_x[2][c][r] = (1.f - ig) * (vw[j] * w);           // dil = i(1-i) u dws
            }
          }
        }
      }
      // dB / dC partials of the half's rows: over the channel groups of this
      // wave, then over the waves in wave order
      if constexpr (G > 1) {
#pragma unroll
        for (int r = 0; r < kGnH; ++r)
#pragma unroll
          for (int s2 = 0; s2 < S; ++s2) {
#pragma unroll
            for (int m = 32; m >= LG; m >>= 1) {
              accB[r][s2] += __shfl_xor(accB[r][s2], m, 64);
              accC[r][s2] += __shfl_xor(accC[r][s2], m, 64);
            }
          }
      }
      for (int w = 0; w < W; ++w) {
        if (wv == w && gl == 0) {
#pragma unroll
          for (int r = 0; r < kGnH; ++r)
#pragma unroll
            for (int s2 = 0; s2 < S; ++s2) {
              const int n = nl + 64 * s2;
              s_pB[hr0 + r][n] = (w == 0 ? 0.f : s_pB[hr0 + r][n]) + accB[r][s2];
              s_pC[hr0 + r][n] = (w == 0 ? 0.f : s_pC[hr0 + r][n]) + accC[r][s2];
            }
        }
        __syncthreads();
      }
    }
    // stores: dB / dC partials, then du / dfl / dil (channel lane, rows
    // 4*wv .. 4*wv+3, one 16-byte LDS read per stream)
    {
      float* pB = a.partB ? a.partB + (int64_t)dtile * btn + brow0 : nullptr;
      float* pC = a.partC ? a.partC + (int64_t)dtile * btn + brow0 : nullptr;
      for (int e = tid; e < kGnCK * NP; e += TH) {
        const int r = e / NP, n = e - r * NP;
        if (r < rows && n < N) {
          const uint32_t o = ((uint32_t)r * (uint32_t)N + (uint32_t)n) * 4u;
          if (pB) *(float*)((char*)pB + o) = s_pB[r][n];
          if (pC) *(float*)((char*)pC + o) = s_pC[r][n];
        }
      }
    }
    if (dl_ok) {
      const float4 o0 = *(const float4*)&s_x[1][sch][4 * srg];
      const float4 o1 = *(const float4*)&s_x[0][sch][4 * srg];
      const float4 o2 = *(const float4*)&s_x[2][sch][4 * srg];
      auto st4 = [&](void* p, int dt, const float4& v) {
        if (!p) return;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (4 * srg + e < rows) {
            uint32_t o = (uint32_t)(4 * srg + e) * (uint32_t)D + (uint32_t)sch;
            // computed here: addresses hoisted to the top of the sub-chunk
            // would occupy registers through the whole scan
            asm volatile("" : "+v"(o));
            const float x = (&v.x)[e];
            if (dt == NAJU_DTYPE_F32)
              *(float*)((char*)((float*)p + xrow0) + o * 4u) = x;
            else if (dt == NAJU_DTYPE_BF16)
              *(bf16_t*)((char*)((bf16_t*)p + xrow0) + o * 2u) = (bf16_t)x;
            else
              *(f16_t*)((char*)((f16_t*)p + xrow0) + o * 2u) = (f16_t)x;
          }
        }
      };
      st4(a.du, du_dt, o0);
      st4(a.dfl, dg_dt, o1);
      st4(a.dil, dg_dt, o2);
    }
  }
#pragma unroll
  for (int q = 0; q < PPW; ++q) {
    const int pass = wv + q * W;
    if (pass >= NPASS) break;
    const int64_t d = dbase + (int64_t)pass * G + gl;
    if (d >= D) continue;
    if (a.dh0 && seg == 0) {
#pragma unroll
      for (int s2 = 0; s2 < S; ++s2) {
        const int n = nl + 64 * s2;
        if (n < N) a.dh0[((int64_t)b * D + d) * N + n] = gc[q][s2];
      }
    }
  }
  // dD = sum dy * u over this segment's rows, in wave order
  s_dD[srg][sch] = dDacc;
  __syncthreads();
  if (tid < DT && dbase + tid < D && a.partD) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < RGS; ++w) s += s_dD[w][tid];
    a.partD[((int64_t)b * a.nseg + seg) * D + dbase + tid] = s;
  }
}

// Fills n float32 values with src[i] (or 0 when src is null); used for the
// empty-shape edge cases (hT = h0 when T == 0, zero gradients).
__global__ void fill_kernel(float* dst, const float* src, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    dst[i] = src ? src[i] : 0.f;
}
__global__ void zero_any_kernel(void* dst, int dt, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) st_any(dst, dt, i, 0.f);
}

// ------------------------------------------------------------- host side

thread_local char g_err[512] = "";

// Host tags of the look-back words: one new odd value per eager launch,
// process-wide (zero-filled workspaces hold tag 0; device-epoch tags of
// graph-recorded launches are even, so the two kinds never meet).
std::atomic<uint32_t> g_tag{0};
uint32_t next_tag() { return (g_tag.fetch_add(1, std::memory_order_relaxed) << 1) | 1u; }

// The look-back tag of an N = 1 launch on stream st. Eager: a host tag.
// While st is being captured into a HIP graph, a host tag would be frozen
// into the graph and every replay would accept the words of the previous
// replay as its own; the launch then takes its tag from the device epoch
// instead, and the one-thread epoch_bump_kernel recorded just before it
// advances the epoch on every replay. Returns the tag (0 = device epoch), or
// -1 after recording a launch error.
int64_t launch_tag(uint32_t* hdr, hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess) cs = hipStreamCaptureStatusNone;
  if (cs != hipStreamCaptureStatusActive) return next_tag();
  hipLaunchKernelGGL(epoch_bump_kernel, dim3(1), dim3(1), 0, st, hdr);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return -1;
  return 0;
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

size_t dsize(int dt) { return dt == NAJU_DTYPE_F32 ? 4 : 2; }

// The look-back's bound on idle rounds: kSpinLimit, or a smaller value from
// the environment variable NAJU_DEBUG_SPIN_LIMIT (read at every call). A
// test hook: 0 makes every carry hand-off give up at once, so the failure
// path (NaN outputs, status word 1) runs while every kernel exits normally.
uint32_t spin_limit() {
  const char* s = getenv("NAJU_DEBUG_SPIN_LIMIT");
  if (!s || !*s) return kSpinLimit;
  char* end = nullptr;
  const unsigned long v = strtoul(s, &end, 10);
  return (end && *end == 0 && v < kSpinLimit) ? (uint32_t)v : kSpinLimit;
}

// Tile geometry of the N = 1 kernels, per direction: V channels per lane,
// R rows per wave, W waves per workgroup (chunk L = W*R rows), P look-back
// slots polled per wave and round (window W*P chunks). The checkpoint holds
// the state entering every backward chunk, so its layout follows the
// backward chunk length.
#ifndef NAJU_F_V
#define NAJU_F_V 2
#endif
#ifndef NAJU_F_R
#define NAJU_F_R 16
#endif
#ifndef NAJU_F_W
#define NAJU_F_W 8
#endif
#ifndef NAJU_F_P
#define NAJU_F_P 1
#endif
#ifndef NAJU_B_V
#define NAJU_B_V 2
#endif
#ifndef NAJU_B_R
#define NAJU_B_R 8
#endif
#ifndef NAJU_B_W
#define NAJU_B_W 8
#endif
#ifndef NAJU_B_P
#define NAJU_B_P 1
#endif
constexpr int kFV = NAJU_F_V, kFR = NAJU_F_R, kFW = NAJU_F_W, kFP = NAJU_F_P;
constexpr int kBV = NAJU_B_V, kBR = NAJU_B_R, kBW = NAJU_B_W, kBP = NAJU_B_P;
constexpr int kFChunk = kFR * kFW;
constexpr int kBChunk = kBR * kBW;
// The forward writes the state entering every backward chunk: at the start
// of a forward wave's rows.
static_assert(kFChunk % kBChunk == 0 && kBChunk % kFR == 0, "backward chunks must tile forward chunks by waves");

int n1_vec_width(bool bwd) { return bwd ? kBV : kFV; }

struct Layout {
  int V, CH, L, K, n_dtiles, n_tiles;
  int nseg, seg_sc;  // N > 1: time segments
  int ck_rows;       // the forward's checkpoint interval
  size_t off_agg, off_incl, off_partB, off_partC, off_partD, off_partG, off_segF, off_segZ, off_seg0, off_dense, total;
};

// N > 1: enough time segments that about kGnTargetWgs workgroups run per
// launch (each segment keeps at least one sub-chunk).
#ifndef NAJU_GN_TARGET_WGS
#define NAJU_GN_TARGET_WGS 1536  // two rounds of three 4-wave workgroups per CU
#endif
constexpr int kGnTargetWgs = NAJU_GN_TARGET_WGS;
// The chunked matrix-core kernels' time segments: the forward holds up to
// four 4-wave workgroups per CU and wants at least three (for latency
// hiding); the backward holds one 8-wave workgroup per CU and wants two per
// CU over the launch (measured at the C2 shape: 4, 8 and 12 segments took
// 696, 689 and 709 us), so that one workgroup's start-up overlaps another's
// tail.
#ifndef NAJU_MC_FWD_MIN_PER_CU
#define NAJU_MC_FWD_MIN_PER_CU 3
#endif
#ifndef NAJU_MC_BWD_MIN_PER_CU
#define NAJU_MC_BWD_MIN_PER_CU 2
#endif
constexpr int kCUs = 256;  // MI355X
// The matrix-core forward's time segments are whole multiples of this many
// sub-blocks (128 rows), so that they start at interval boundaries of every
// served checkpoint interval (32, 64 and 128 rows).
constexpr int kMcSegUnit = 8;
constexpr int kGcTargetWaves = 2048;

// Sub-blocks per time segment of a chunked matrix-core launch over n_tiles
// channel tiles and K sub-blocks: the segmentation whose busiest CU walks
// the fewest sub-blocks, ceil(n_tiles s / CUs) * (sub-blocks per segment),
// among those that give every CU at least min_per_cu workgroups; the fewest
// segments on a tie, since each one past the first costs the segment-map
// pass over its rows and a start-up. Segments are a multiple of `unit`
// sub-blocks long (the forward with a checkpoint interval of unit
// sub-blocks: every segment then starts where an interval does).
int mc_seg_sc(int64_t n_tiles, int K, bool bwd, int unit) {
  const int64_t min_wg = (int64_t)kCUs * (bwd ? NAJU_MC_BWD_MIN_PER_CU : NAJU_MC_FWD_MIN_PER_CU);
  int best = K;
  int64_t best_cost = -1;
  for (int s = 1; s <= K; ++s) {
    const int sc = ((K + s - 1) / s + unit - 1) / unit * unit;
    const int ns = unit == 1 ? s : (K + sc - 1) / sc;
    const int64_t wg = n_tiles * ns;
    if (wg < min_wg && s < K) continue;
    const int64_t cost = (wg + kCUs - 1) / kCUs * sc;
    if (best_cost < 0 || cost < best_cost) best_cost = cost, best = sc;
    if (wg >= 8 * min_wg) break;
  }
  return best;
}
// gq_fwd_kernel serves a forward whose batch x channel-group grid holds at
// least three 4-wave workgroups per CU (256 CUs); smaller grids take the
// segmented gc_fwd_kernel, whose time segments supply the parallelism.
constexpr int kGqMinWgs = 768;

size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

int np_of(int64_t N);
bool gq_ok(int64_t N, int64_t batch, int64_t D);
// The chunked matrix-core kernels serve 9 <= N <= 64 in the directions that
// have them.
constexpr bool kMcBwd = true;
bool use_mc(int64_t N, bool bwd) { return mc_ok(N) && (!bwd || kMcBwd); }
// Rows per checkpoint interval of the general-N forward: the chunked
// backward reads the state entering every kMcQ-row sub-block.
int64_t gn_ck_rows(int64_t N) { return use_mc(N, true) ? kMcQ : kGnCK; }
// The checkpoint interval the flags ask for (NAJU_CKPT_ROWS; 0 = the
// default: the backward's chunk at N = 1, gn_ck_rows at N > 1), or -1 when
// the shape does not serve it: longer intervals than the default only on the
// matrix-core path, whose backward recomputes the states between.
int ckpt_rows(int flags, int64_t N) {
  const int r = ((flags & NAJU_CKPT_MASK) >> NAJU_CKPT_SHIFT) * 16;
  const int def = N == 1 ? kBChunk : (int)gn_ck_rows(N);
  if (r == 0 || r == def) return def;
  // 2, 4, ... kMcSegUnit sub-blocks: intervals that divide the forward's
  // segment unit
  const bool served = r > kMcQ && r <= kMcQ * kMcSegUnit && (kMcQ * kMcSegUnit) % r == 0;
  return (N > 1 && use_mc(N, true) && served) ? r : -1;
}
int gq_channels(int64_t N);
int gn_bwd_dt(int np);

// Byte offsets of the workspace regions for the layout's K, tiles and
// segments (the backward's partial sums only when bwd).
void place_regions(Layout& l, int64_t batch, int64_t T, int64_t D, int64_t N, bool bwd) {
  size_t off = align_up(kHeaderBytes);
  const size_t units = N == 1 ? (size_t)l.K * l.n_tiles : 0;
  l.off_agg = off;
  off = align_up(off + units * 2 * l.CH * sizeof(uint64_t));
  l.off_incl = off;
  off = align_up(off + units * l.CH * sizeof(uint64_t));
  const size_t part_bc = bwd ? (size_t)l.n_dtiles * batch * T * N * sizeof(float) : 0;
  l.off_partB = off;
  off = align_up(off + part_bc);
  l.off_partC = off;
  off = align_up(off + part_bc);
  l.off_partD = off;
  off = align_up(off + (bwd ? (size_t)batch * (N == 1 ? l.K : l.nseg) * D * sizeof(float) : 0));
  // the matrix-core backward's per-segment sums of dfl and dil (when asked for)
  l.off_partG = off;
  off = align_up(off + (bwd && N > 1 && use_mc(N, true) ? (size_t)2 * batch * l.nseg * D * sizeof(float) : 0));
  const size_t seg_units = l.nseg > 1 ? (size_t)batch * l.nseg * D : 0;
  l.off_segF = off;
  off = align_up(off + seg_units * sizeof(float));
  l.off_segZ = off;
  off = align_up(off + seg_units * N * sizeof(float));
  l.off_seg0 = off;
  off = align_up(off + seg_units * N * sizeof(float));
  // the backward's recomputed state at every sub-block when the forward's
  // checkpoint interval is longer than the sub-block
  const bool dense = bwd && N > 1 && use_mc(N, true) && l.ck_rows > kMcQ;
  l.off_dense = off;
  off = align_up(off + (dense ? (size_t)batch * ((T + kMcQ - 1) / kMcQ) * D * N * sizeof(float) : 0));
  l.total = off;
}

// cap: at N > 1, fewer time segments (down to one) until the workspace fits
// in cap bytes; the N = 1 layout has no such freedom.
// cap: at N > 1, fewer time segments (down to one) until the workspace fits
// in cap bytes; the N = 1 layout has no such freedom. ck_rows: the
// checkpoint interval (0 = the default; it sizes the backward's recomputed
// states). The matrix-core forward's time segments are a multiple of
// kMcSegUnit sub-blocks long, for every interval: every segment then starts
// at an interval boundary of each served interval, so the checkpoint holds
// every state the backward's recompute starts from, and the segmentation
// (hence every output bit) does not depend on the interval.
Layout make_layout(int64_t batch, int64_t T, int64_t D, int64_t N, int x_dt, int g_dt, bool bwd,
                   size_t cap = SIZE_MAX, int ck_rows = 0) {
  Layout l{};
  l.ck_rows = ck_rows;
  (void)x_dt;
  (void)g_dt;
  const bool mc = use_mc(N, bwd);
  if (N == 1) {
    l.V = n1_vec_width(bwd);
    l.CH = 64 * l.V;
    l.L = bwd ? kBChunk : kFChunk;
  } else if (mc) {  // chunked matrix-core kernels: kMcDT (kMcDTB) channels, kMcQ-row sub-blocks
    l.V = 1;
    l.CH = bwd ? kMcDTB : kMcDT;
    l.L = kMcQ;
  } else {  // general N: channel tiles walking T, checkpoint every kGnCK rows
    l.V = 1;
    l.CH = bwd ? gn_bwd_dt(np_of(N)) : kGnDT;  // the backward kernel's tiles (dB/dC partials)
    l.L = kGnCK;
  }
  l.K = (int)((T + l.L - 1) / l.L);
  l.n_dtiles = (int)((D + l.CH - 1) / l.CH);
  l.n_tiles = (int)(batch * l.n_dtiles);
  l.nseg = 1;
  l.seg_sc = l.K;
  // sub-blocks per segment must be a multiple of this (the matrix-core
  // forward: kMcSegUnit, whatever the checkpoint interval)
  const int unit = (mc && !bwd) ? kMcSegUnit : 1;
  if (N > 1 && l.n_tiles > 0 && l.K > 0 && (mc || bwd || !gq_ok(N, batch, D))) {
    if (mc) {
      l.seg_sc = mc_seg_sc(l.n_tiles, l.K, bwd, unit);
    } else {
      // forward (lanes over channels): about kGcTargetWaves waves; backward
      // (8-wave workgroups over 64 channels): about kGnTargetWgs workgroups
      const int64_t per_seg = bwd ? l.n_tiles : batch * ((D + 63) / 64);
      // (the 8-wave NP = 128 backward runs one workgroup per CU: 1024)
      const int64_t target = bwd ? (np_of(N) <= 64 ? kGnTargetWgs : 1024) : kGcTargetWaves;
      int64_t want = (target + per_seg - 1) / per_seg;
      if (want > l.K) want = l.K;
      if (want < 1) want = 1;
      l.seg_sc = (int)((l.K + want - 1) / want);
    }
    l.nseg = (l.K + l.seg_sc - 1) / l.seg_sc;
  }
  place_regions(l, batch, T, D, N, bwd);
  while (l.total > cap && l.nseg > 1) {
    const int want = l.nseg / 2;
    l.seg_sc = ((l.K + want - 1) / want + unit - 1) / unit * unit;
    l.nseg = (l.K + l.seg_sc - 1) / l.seg_sc;
    place_regions(l, batch, T, D, N, bwd);
  }
  return l;
}

bool dt_ok(int dt) { return dt == NAJU_DTYPE_F32 || dt == NAJU_DTYPE_BF16 || dt == NAJU_DTYPE_F16; }

int check_common(int64_t batch, int64_t T, int64_t D, int64_t N, int x_dt, int g_dt, int bc_dt) {
  if (batch < 0 || T < 0 || D < 0) return fail(NAJU_ERR_INVALID, "negative shape (batch=%lld T=%lld D=%lld)",
                                               (long long)batch, (long long)T, (long long)D);
  if (N < 1) return fail(NAJU_ERR_INVALID, "N (d_state) must be >= 1, got %lld", (long long)N);
  if (!dt_ok(x_dt) || !dt_ok(g_dt) || !dt_ok(bc_dt))
    return fail(NAJU_ERR_INVALID, "unknown dtype code (x=%d gate=%d bc=%d)", x_dt, g_dt, bc_dt);
  if (g_dt != NAJU_DTYPE_F32 && g_dt != x_dt)
    return fail(NAJU_ERR_UNSUPPORTED, "gate dtype must be float32 or equal to the u dtype");
  if (bc_dt != NAJU_DTYPE_F32 && bc_dt != x_dt)
    return fail(NAJU_ERR_UNSUPPORTED, "B/C dtype must be float32 or equal to the u dtype");
  if (x_dt == NAJU_DTYPE_F32 && g_dt != NAJU_DTYPE_F32)
    return fail(NAJU_ERR_UNSUPPORTED, "float32 u needs float32 gates");
  if (N > 128) return fail(NAJU_ERR_UNSUPPORTED, "N (d_state) must be <= 128, got %lld", (long long)N);
  if (T > (1ll << 30) || D > (1ll << 30) || batch > (1ll << 30))
    return fail(NAJU_ERR_INVALID, "dimension exceeds 2^30");
  // The general-N kernels address a sub-chunk's [32 rows x channels] tiles
  // with 32-bit offsets from the tile's first element.
  if (N > 1 && D >= (1ll << 25))
    return fail(NAJU_ERR_UNSUPPORTED, "N > 1 needs D < 2^25 channels, got %lld", (long long)D);
  return NAJU_OK;
}

bool aligned(const void* p, size_t a) { return p == nullptr || ((uintptr_t)p % a) == 0; }

typedef void (*kern_t)(ScanArgs);

template <typename TU, typename TG, typename TB, bool VEC, bool F32O>
kern_t pick_n1(bool bwd) {
  return bwd ? (kern_t)n1_bwd_kernel<TU, TG, TB, kBV, kBR, kBW, kBP, VEC, F32O>
             : (kern_t)n1_fwd_kernel<TU, TG, TB, kFV, kFR, kFW, kFP, VEC, F32O>;
}

template <typename TU, typename TG, bool VEC, bool F32O>
kern_t pick_n1_bc(int bc_dt, bool bwd) {
  return bc_dt == NAJU_DTYPE_F32 ? pick_n1<TU, TG, float, VEC, F32O>(bwd) : pick_n1<TU, TG, TU, VEC, F32O>(bwd);
}

template <bool VEC, bool F32O>
kern_t pick_n1_dt(int x_dt, int g_dt, int bc_dt, bool bwd) {
  if (x_dt == NAJU_DTYPE_F32) return pick_n1<float, float, float, VEC, F32O>(bwd);
  if (x_dt == NAJU_DTYPE_BF16)
    return g_dt == NAJU_DTYPE_F32 ? pick_n1_bc<bf16_t, float, VEC, F32O>(bc_dt, bwd)
                                  : pick_n1_bc<bf16_t, bf16_t, VEC, F32O>(bc_dt, bwd);
  return g_dt == NAJU_DTYPE_F32 ? pick_n1_bc<f16_t, float, VEC, F32O>(bc_dt, bwd)
                                : pick_n1_bc<f16_t, f16_t, VEC, F32O>(bc_dt, bwd);
}

kern_t pick_n1_all(bool vec, bool f32o, int x_dt, int g_dt, int bc_dt, bool bwd) {
  if (vec)
    return f32o ? pick_n1_dt<true, true>(x_dt, g_dt, bc_dt, bwd) : pick_n1_dt<true, false>(x_dt, g_dt, bc_dt, bwd);
  return f32o ? pick_n1_dt<false, true>(x_dt, g_dt, bc_dt, bwd) : pick_n1_dt<false, false>(x_dt, g_dt, bc_dt, bwd);
}

typedef void (*gn_fwd_t)(ScanArgs, int, int, int);
typedef void (*gn_bwd_t)(ScanArgs, int, int, int, int);

int np_of(int64_t N) {
  int np = 2;
  while (np < N) np <<= 1;
  return np;
}


// Backward workgroup shape per NP: 32 channels in 4 waves (three workgroups
// fit a CU: 149 VGPRs, 54 KB of LDS) up to NP = 64; 64 channels in 8 waves
// at NP = 128, whose B/C tiles would not leave room for three.
int gn_bwd_dt(int np) { return np <= 64 ? 32 : 64; }
int gn_bwd_waves(int np) { return np <= 64 ? 4 : 8; }

gn_bwd_t pick_gn_bwd(int np) {
  switch (np) {
    case 2: return gn_bwd_kernel<2, 32, 4>;
    case 4: return gn_bwd_kernel<4, 32, 4>;
    case 8: return gn_bwd_kernel<8, 32, 4>;
    case 16: return gn_bwd_kernel<16, 32, 4>;
    case 32: return gn_bwd_kernel<32, 32, 4>;
    case 64: return gn_bwd_kernel<64, 32, 4>;
    default: return gn_bwd_kernel<128, 64, 8>;
  }
}

// Workgroups per time segment of the general-N forward.
int64_t gc_tiles(int64_t batch, int64_t D) { return batch * ((D + kGcCH - 1) / kGcCH); }

// The forward without time segments (gq_fwd_kernel): 16 <= NP <= 64 and a
// grid that fills the GPU.
int gq_channels(int64_t N) { return 64 / (np_of((int)N) / 4) * kGqW; }
bool gq_ok(int64_t N, int64_t batch, int64_t D) {
  const int np = np_of((int)N);
  return N > 1 && np >= 16 && np <= 64 && batch * ((D + gq_channels(N) - 1) / gq_channels(N)) >= kGqMinWgs;
}
gn_fwd_t pick_gq_fwd(int np) {
  switch (np) {
    case 16: return gq_fwd_kernel<16>;
    case 32: return gq_fwd_kernel<32>;
    default: return gq_fwd_kernel<64>;
  }
}

gn_fwd_t pick_gc_fwd(int np, bool map) {
  switch (np) {
    case 2: return map ? gc_fwd_kernel<2, true> : gc_fwd_kernel<2, false>;
    case 4: return map ? gc_fwd_kernel<4, true> : gc_fwd_kernel<4, false>;
    case 8: return map ? gc_fwd_kernel<8, true> : gc_fwd_kernel<8, false>;
    case 16: return map ? gc_fwd_kernel<16, true> : gc_fwd_kernel<16, false>;
    case 32: return map ? gc_fwd_kernel<32, true> : gc_fwd_kernel<32, false>;
    case 64: return map ? gc_fwd_kernel<64, true> : gc_fwd_kernel<64, false>;
    default: return map ? gc_fwd_kernel<128, true> : gc_fwd_kernel<128, false>;
  }
}

typedef void (*gn_map_t)(ScanArgs, int, int);

gn_map_t pick_gn_bwd_map(int np) {
  switch (np) {
    case 2: return gn_bwd_map_kernel<2>;
    case 4: return gn_bwd_map_kernel<4>;
    case 8: return gn_bwd_map_kernel<8>;
    case 16: return gn_bwd_map_kernel<16>;
    case 32: return gn_bwd_map_kernel<32>;
    case 64: return gn_bwd_map_kernel<64>;
    default: return gn_bwd_map_kernel<128>;
  }
}

// N > 1 with time segments: the segment maps and the carry pass that give
// every segment its entering state (dir +1) or adjoint carry (dir -1).
int gn_segments(const ScanArgs& a, const Layout& l, int x_dt, int g_dt, bool bwd, hipStream_t st) {
  if (l.nseg <= 1) return NAJU_OK;
  if (bwd) {
    // the map kernel tiles channels by kGnDT, independently of the main kernel
    const unsigned grid = (unsigned)((int64_t)a.batch * ((a.D + kGnDT - 1) / kGnDT) * (l.nseg - 1));
    hipLaunchKernelGGL(pick_gn_bwd_map(np_of(a.N)), dim3(grid), dim3(64 * kGnW), 0, st, a, x_dt, g_dt);
  } else {
    const unsigned grid = (unsigned)(gc_tiles(a.batch, a.D) * (l.nseg - 1));
    hipLaunchKernelGGL(pick_gc_fwd(np_of(a.N), true), dim3(grid), dim3(64 * kGcW), 0, st, a, x_dt, g_dt, 0);
  }
  const int64_t n = (int64_t)a.batch * a.D * a.N;
  hipLaunchKernelGGL(gn_seg_carry_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a, bwd ? -1 : 1);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return NAJU_OK;
}

int launch(kern_t k, unsigned grid, unsigned block, hipStream_t st, const ScanArgs& a) {
  hipLaunchKernelGGL(k, dim3(grid), dim3(block), 0, st, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return NAJU_OK;
}

unsigned small_grid(int64_t n) {
  const int64_t g = (n + 255) / 256;
  return (unsigned)(g < 1 ? 1 : (g > 4096 ? 4096 : g));
}

}  // namespace

extern "C" {

int naju_scan_version(void) { return (0 << 16) | 1; }

const char* naju_scan_last_error(void) { return g_err; }

int64_t naju_scan_ckpt_elems_ex(int64_t batch, int64_t T, int64_t D, int64_t N, int x_dtype, int gate_dtype,
                                int bc_dtype, int flags) {
  if (check_common(batch, T, D, N, x_dtype, gate_dtype, bc_dtype) != NAJU_OK) return -1;
  const int rows = ckpt_rows(flags, N);
  if (rows < 0) return fail(NAJU_ERR_UNSUPPORTED, "checkpoint interval %d rows is not served at N=%lld (served: 32, 64 and 128 rows at 9 <= N <= 64)",
                            ((flags & NAJU_CKPT_MASK) >> NAJU_CKPT_SHIFT) * 16, (long long)N), -1;
  // N = 1: one state per backward chunk; N > 1: the state every `rows` rows
  if (N > 1) return batch * ((T + rows - 1) / rows) * D * N;
  const Layout l = make_layout(batch, T, D, N, x_dtype, gate_dtype, true);
  return batch * (int64_t)l.K * D * N;
}

int64_t naju_scan_ckpt_elems(int64_t batch, int64_t T, int64_t D, int64_t N, int x_dtype, int gate_dtype,
                             int bc_dtype) {
  return naju_scan_ckpt_elems_ex(batch, T, D, N, x_dtype, gate_dtype, bc_dtype, 0);
}

size_t naju_scan_workspace_bytes_ex(int64_t batch, int64_t T, int64_t D, int64_t N, int x_dtype, int gate_dtype,
                                    int bc_dtype, int flags) {
  if (check_common(batch, T, D, N, x_dtype, gate_dtype, bc_dtype) != NAJU_OK) return 0;
  const int rows = ckpt_rows(flags, N);
  if (rows < 0) return fail(NAJU_ERR_UNSUPPORTED, "checkpoint interval %d rows is not served at N=%lld (served: 32, 64 and 128 rows at 9 <= N <= 64)",
                            ((flags & NAJU_CKPT_MASK) >> NAJU_CKPT_SHIFT) * 16, (long long)N), 0;
  const size_t f = make_layout(batch, T, D, N, x_dtype, gate_dtype, false, SIZE_MAX, rows).total;
  const size_t b = make_layout(batch, T, D, N, x_dtype, gate_dtype, true, SIZE_MAX, rows).total;
  return f > b ? f : b;
}

size_t naju_scan_workspace_bytes(int64_t batch, int64_t T, int64_t D, int64_t N, int x_dtype, int gate_dtype,
                                 int bc_dtype) {
  return naju_scan_workspace_bytes_ex(batch, T, D, N, x_dtype, gate_dtype, bc_dtype, 0);
}

}  // extern "C"

namespace {

// B / C (or dB / dC) with rows ld elements apart: ld = N always; another
// ld only on the matrix-core path (9 <= N <= 64), a multiple of 4 with both
// pointers aligned to four elements (the staging loads of the kernels).
int check_bc_ld(const void* p, const void* q, int64_t N, int dt, int64_t ld, bool bwd) {
  if (ld == N) return NAJU_OK;
  if (ld < N) return fail(NAJU_ERR_INVALID, "B / C row stride (%lld) must be >= N (%lld)", (long long)ld, (long long)N);
  if (N <= 1 || !use_mc(N, bwd))
    return fail(NAJU_ERR_UNSUPPORTED, "a B / C row stride other than N is served at 9 <= N <= 64 only");
  // the kernels address a sub-block's rows with 32-bit offsets
  if (ld > (1 << 24)) return fail(NAJU_ERR_UNSUPPORTED, "B / C row stride (%lld) above 2^24", (long long)ld);
  const size_t a4 = 4 * dsize(dt);
  if (ld % 4 || (p && !aligned(p, a4)) || (q && !aligned(q, a4)))
    return fail(NAJU_ERR_UNSUPPORTED, "strided B / C need a row stride that is a multiple of 4 and %zu-byte "
                "aligned pointers", a4);
  return NAJU_OK;
}

// The forward of naju_scan_fwd and naju_scan_fwd_noalloc. cap bounds the
// layout (time segments at N > 1) to the bytes available.
int scan_fwd_impl(const void* u, const void* f_logit, const void* i_logit, const void* B, const void* C,
                  const float* D_skip, const float* h0, void* y, float* ckpt, float* hT, int64_t batch, int64_t T,
                  int64_t D, int64_t N, int x_dtype, int gate_dtype, int bc_dtype, int flags, void* workspace,
                  size_t workspace_bytes, void* stream, size_t cap, int64_t ldbc) {
  g_err[0] = 0;
  int rc = check_common(batch, T, D, N, x_dtype, gate_dtype, bc_dtype);
  if (rc) return rc;
  if ((rc = check_bc_ld(B, C, N, bc_dtype, ldbc, false))) return rc;
  if (flags & ~(NAJU_FLAG_OUT_F32 | NAJU_FLAG_DETERMINISTIC | NAJU_CKPT_MASK))
    return fail(NAJU_ERR_INVALID, "unknown flag bits 0x%x", flags);
  const int ck_rows = ckpt_rows(flags, N);
  if (ck_rows < 0)
    return fail(NAJU_ERR_UNSUPPORTED, "checkpoint interval %d rows is not served at N=%lld (served: 32, 64 and 128 rows at 9 <= N <= 64)",
                ((flags & NAJU_CKPT_MASK) >> NAJU_CKPT_SHIFT) * 16, (long long)N);
  const int out_f32 = flags & NAJU_FLAG_OUT_F32;
  hipStream_t st = (hipStream_t)stream;
  if (batch == 0 || D == 0) return NAJU_OK;
  if (T == 0) {
    if (hT) {
      hipLaunchKernelGGL(fill_kernel, dim3(small_grid(batch * D * N)), dim3(256), 0, st, hT, h0, batch * D * N);
      if (hipGetLastError() != hipSuccess) return fail(NAJU_ERR_LAUNCH, "fill launch failed");
    }
    return NAJU_OK;
  }
  if (!u || !f_logit || !i_logit || !B || !C || !D_skip || !y)
    return fail(NAJU_ERR_INVALID, "null input/output pointer (u, f_logit, i_logit, B, C, D_skip and y are required)");
  const Layout l = make_layout(batch, T, D, N, x_dtype, gate_dtype, false, cap, ck_rows);
  if (!workspace || workspace_bytes < l.total)
    return fail(NAJU_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", l.total,
                workspace ? workspace_bytes : (size_t)0);
  if (!aligned(workspace, 256)) return fail(NAJU_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  const size_t va_x = l.V * dsize(x_dtype), va_g = l.V * dsize(gate_dtype);
  const size_t va_y = l.V * (out_f32 ? 4 : dsize(x_dtype));
  const bool vec = (D % l.V == 0) && aligned(u, va_x) && aligned(y, va_y) && aligned(f_logit, va_g) &&
                   aligned(i_logit, va_g);
  ScanArgs a{};
  a.u = u;
  a.fl = f_logit;
  a.il = i_logit;
  a.Bm = B;
  a.Cm = C;
  a.Dsk = D_skip;
  a.h0 = h0;
  a.y = y;
  a.ckpt = ckpt;
  a.hT = hT;
  char* ws = (char*)workspace;
  a.hdr = (uint32_t*)ws;
  a.agg = (uint64_t*)(ws + l.off_agg);
  a.incl = (uint64_t*)(ws + l.off_incl);
  a.T = T;
  a.D = D;
  a.ldbc = ldbc;
  a.N = (int)N;
  a.batch = (int)batch;
  a.bc_dt = bc_dtype;
  a.n_dtiles = l.n_dtiles;
  a.n_tiles = l.n_tiles;
  a.K = l.K;
  if (N > 1) {
    const int y_dt = out_f32 ? (int)NAJU_DTYPE_F32 : x_dtype;
    a.nseg = l.nseg;
    a.seg_sc = l.seg_sc;
    a.segF = (float*)(ws + l.off_segF);
    a.segZ = (float*)(ws + l.off_segZ);
    a.seg0 = (float*)(ws + l.off_seg0);
    if (use_mc(N, false)) {
      // chunked matrix-core forward: segment maps, their carry, the scan
      a.n_dtiles = l.n_dtiles;
      a.n_tiles = l.n_tiles;
      a.ck_rows = ck_rows;
      a.Kc = (int)((T + a.ck_rows - 1) / a.ck_rows);
      if ((int64_t)l.n_tiles * l.nseg > 0x7fffffff) return fail(NAJU_ERR_UNSUPPORTED, "problem too large");
      hipError_t e = hipSuccess;
      if (l.nseg > 1) {
        e = mc_fwd_launch(a, true, x_dtype, gate_dtype, y_dt, st);
        if (e == hipSuccess) {
          const int64_t n = (int64_t)a.batch * a.D * a.N;
          hipLaunchKernelGGL(gn_seg_carry_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a, 1);
          e = hipGetLastError();
        }
      }
      if (e == hipSuccess) e = mc_fwd_launch(a, false, x_dtype, gate_dtype, y_dt, st);
      if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
      return NAJU_OK;
    }
    if (gq_ok(N, batch, D)) {
      // one workgroup per (batch row, channel group), over all of T
      const int64_t grid = batch * ((D + gq_channels(N) - 1) / gq_channels(N));
      if (grid > 0x7fffffff) return fail(NAJU_ERR_UNSUPPORTED, "problem too large");
      hipLaunchKernelGGL(pick_gq_fwd(np_of(N)), dim3((unsigned)grid), dim3(64 * kGqW), 0, st, a, x_dtype, gate_dtype,
                         y_dt);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
      return NAJU_OK;
    }
    if (gc_tiles(batch, D) * l.nseg > 0x7fffffff) return fail(NAJU_ERR_UNSUPPORTED, "problem too large");
    rc = gn_segments(a, l, x_dtype, gate_dtype, false, st);
    if (rc) return rc;
    hipLaunchKernelGGL(pick_gc_fwd(np_of(N), false), dim3((unsigned)(gc_tiles(batch, D) * l.nseg)), dim3(64 * kGcW),
                       0, st, a, x_dtype, gate_dtype, y_dt);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
    return NAJU_OK;
  }
  const int64_t wgs = (int64_t)l.K * l.n_tiles;
  if (wgs > 0x7fffffff || l.n_tiles > kMaxTiles)
    return fail(NAJU_ERR_UNSUPPORTED, "problem too large (%lld workgroups, %d channel tiles)", (long long)wgs,
                l.n_tiles);
  const int64_t tg = launch_tag(a.hdr, st);
  if (tg < 0) return fail(NAJU_ERR_LAUNCH, "epoch launch failed");
  a.tag = (uint32_t)tg;
  a.strict = (flags & NAJU_FLAG_DETERMINISTIC) != 0;
  a.spin_limit = spin_limit();
  a.ck_rows = kBChunk;
  a.Kc = (int)((T + kBChunk - 1) / kBChunk);
  kern_t k = pick_n1_all(vec, out_f32 != 0, x_dtype, gate_dtype, bc_dtype, false);
  return launch(k, (unsigned)wgs, 64 * kFW, st, a);
}

// ------------------------------------------- allocation-free forward scratch
//
// naju_scan_fwd_noalloc runs the forward on a file-scope device array instead
// of a caller workspace. Each GPU the library runs on holds its own copy of
// `scratch` until the process ends. Host code never passes the array's name
// to a kernel (in host code it is only a stand-in for the symbol): at the
// first call on a device, with that device current, hipGetSymbolAddress gives
// the array's device address there, kept per device in g_scratch_ptr, and the
// launches use that address. Every call on a device shares that device's
// array, so calls that overlap in time on one GPU race.
constexpr size_t kScratchBytes = NAJU_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Zeroes the status word and every ticket counter of a workspace header (a
// kernel, not a memset, so a graph that records it replays it correctly).
// The device epoch (word 1) is left alone: resetting it inside a recorded
// graph would give every replay the same tag.
__global__ void clear_header_kernel(uint32_t* hdr) {
  const int64_t n = (int64_t)(kHeaderBytes / sizeof(uint32_t));
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    if (i != HDR_EPOCH) hdr[i] = 0u;
}

// This device's scratch address; at the first call on a device also clears
// its header on `st`. Returns null after recording an error.
void* scratch_for_current_device(hipStream_t st) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(NAJU_ERR_LAUNCH, "no current HIP device (or device index >= %d)", kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev]) return g_scratch_ptr[dev];
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr) {
    fail(NAJU_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
    return nullptr;
  }
  hipLaunchKernelGGL(clear_header_kernel, dim3(256), dim3(256), 0, st, (uint32_t*)p);
  const hipError_t le = hipGetLastError();
  if (le != hipSuccess) {
    fail(NAJU_ERR_LAUNCH, "scratch clear launch failed: %s", hipGetErrorString(le));
    return nullptr;
  }
  g_scratch_ptr[dev] = p;
  return p;
}

}  // namespace

extern "C" {

int naju_scan_fwd(const void* u, const void* f_logit, const void* i_logit, const void* B, const void* C,
                  const float* D_skip, const float* h0, void* y, float* ckpt, float* hT, int64_t batch, int64_t T,
                  int64_t D, int64_t N, int x_dtype, int gate_dtype, int bc_dtype, int flags, void* workspace,
                  size_t workspace_bytes, void* stream) {
  return scan_fwd_impl(u, f_logit, i_logit, B, C, D_skip, h0, y, ckpt, hT, batch, T, D, N, x_dtype, gate_dtype,
                       bc_dtype, flags, workspace, workspace_bytes, stream, SIZE_MAX, N);
}

int naju_scan_fwd_strided(const void* u, const void* f_logit, const void* i_logit, const void* B, const void* C,
                          const float* D_skip, const float* h0, void* y, float* ckpt, float* hT, int64_t batch,
                          int64_t T, int64_t D, int64_t N, int64_t bc_ld, int x_dtype, int gate_dtype, int bc_dtype,
                          int flags, void* workspace, size_t workspace_bytes, void* stream) {
  return scan_fwd_impl(u, f_logit, i_logit, B, C, D_skip, h0, y, ckpt, hT, batch, T, D, N, x_dtype, gate_dtype,
                       bc_dtype, flags, workspace, workspace_bytes, stream, SIZE_MAX, bc_ld);
}

int naju_scan_fwd_noalloc(const void* u, const void* f_logit, const void* i_logit, const void* B, const void* C,
                          const float* D_skip, const float* h0, void* y, float* ckpt, float* hT, int64_t batch,
                          int64_t T, int64_t D, int64_t N, int x_dtype, int gate_dtype, int bc_dtype, int flags,
                          void* stream) {
  g_err[0] = 0;
  const int rc = check_common(batch, T, D, N, x_dtype, gate_dtype, bc_dtype);
  if (rc) return rc;
  if (batch > 0 && T > 0 && D > 0) {
    const int rows = ckpt_rows(flags, N);
    const Layout l = make_layout(batch, T, D, N, x_dtype, gate_dtype, false, kScratchBytes, rows < 0 ? 0 : rows);
    if (l.total > kScratchBytes)
      return fail(NAJU_ERR_WORKSPACE,
                  "naju_scan_fwd_noalloc: this shape needs %zu bytes of scratch, the static maximum is %zu "
                  "(use naju_scan_fwd with a workspace)",
                  l.total, kScratchBytes);
  }
  hipStream_t st = (hipStream_t)stream;
  void* ws = scratch_for_current_device(st);
  if (!ws) return NAJU_ERR_LAUNCH;
  return scan_fwd_impl(u, f_logit, i_logit, B, C, D_skip, h0, y, ckpt, hT, batch, T, D, N, x_dtype, gate_dtype,
                       bc_dtype, flags, ws, kScratchBytes, stream, kScratchBytes, N);
}

// The gate-gradient options of naju_scan_bwd_ex: dfl / dil rows ldg apart in
// dg_req (-1: the default type), their sums over batch and time. Served on
// the matrix-core path (9 <= N <= 64); a stride other than D needs a
// multiple of 4 and pointers aligned to four elements.
int check_gate_ext(const void* dfl, const void* dil, int64_t N, int64_t D, int64_t ldg, int dg_req, int dg_dt,
                   bool sums) {
  if (ldg == D && dg_req < 0 && !sums) return NAJU_OK;
  if (N <= 1 || !use_mc(N, true))
    return fail(NAJU_ERR_UNSUPPORTED, "gate-gradient strides, types and sums are served at 9 <= N <= 64");
  if (ldg < D) return fail(NAJU_ERR_INVALID, "dfl / dil row stride (%lld) must be >= D (%lld)", (long long)ldg,
                           (long long)D);
  if (ldg > (1 << 24)) return fail(NAJU_ERR_UNSUPPORTED, "dfl / dil row stride (%lld) above 2^24", (long long)ldg);
  if (dg_req >= 0 && !dt_ok(dg_req)) return fail(NAJU_ERR_INVALID, "unknown dtype code %d", dg_req);
  const size_t a4 = 4 * dsize(dg_dt);
  if (ldg != D && (ldg % 4 || (dfl && !aligned(dfl, a4)) || (dil && !aligned(dil, a4))))
    return fail(NAJU_ERR_UNSUPPORTED, "strided dfl / dil need a row stride that is a multiple of 4 and %zu-byte "
                "aligned pointers", a4);
  return NAJU_OK;
}

static int scan_bwd_impl(const void* u, const void* f_logit, const void* i_logit, const void* B, const void* C,
                         const float* D_skip, const float* ckpt, const void* dy, void* du, void* dfl, void* dil,
                         void* dB, void* dC, float* dD, float* dh0, int64_t batch, int64_t T, int64_t D, int64_t N,
                         int x_dtype, int gate_dtype, int bc_dtype, int flags, void* workspace,
                         size_t workspace_bytes, void* stream, int64_t ldbc, int64_t lddbc, int64_t ldg = -1,
                         int dg_req = -1, float* dfl_sum = nullptr, float* dil_sum = nullptr) {
  g_err[0] = 0;
  int rc = check_common(batch, T, D, N, x_dtype, gate_dtype, bc_dtype);
  if (rc) return rc;
  if ((rc = check_bc_ld(B, C, N, bc_dtype, ldbc, true))) return rc;
  if ((rc = check_bc_ld(dB, dC, N, (flags & NAJU_FLAG_OUT_F32) ? (int)NAJU_DTYPE_F32 : bc_dtype, lddbc, true)))
    return rc;
  if (lddbc != N && batch * T > 0 && D == 0)
    return fail(NAJU_ERR_UNSUPPORTED, "strided dB / dC need D > 0");
  if (ldg < 0) ldg = D;
  // the type dfl and dil are written in
  const int dg_dt = dg_req >= 0 ? dg_req : ((flags & NAJU_FLAG_OUT_F32) ? (int)NAJU_DTYPE_F32 : gate_dtype);
  if ((rc = check_gate_ext(dfl, dil, N, D, ldg, dg_req, dg_dt, dfl_sum || dil_sum))) return rc;
  if (flags & ~(NAJU_FLAG_OUT_F32 | NAJU_FLAG_DETERMINISTIC | NAJU_CKPT_MASK))
    return fail(NAJU_ERR_INVALID, "unknown flag bits 0x%x", flags);
  const int ck_rows = ckpt_rows(flags, N);
  if (ck_rows < 0)
    return fail(NAJU_ERR_UNSUPPORTED, "checkpoint interval %d rows is not served at N=%lld (served: 32, 64 and 128 rows at 9 <= N <= 64)",
                ((flags & NAJU_CKPT_MASK) >> NAJU_CKPT_SHIFT) * 16, (long long)N);
  const int out_f32 = flags & NAJU_FLAG_OUT_F32;
  hipStream_t st = (hipStream_t)stream;
  if (batch == 0 || T == 0 || D == 0) {
    // Gradients of an empty scan: the reductions over the empty axes are 0.
    if (dD) hipLaunchKernelGGL(fill_kernel, dim3(small_grid(D)), dim3(256), 0, st, dD, (const float*)nullptr, D);
    if (dfl_sum)
      hipLaunchKernelGGL(fill_kernel, dim3(small_grid(D)), dim3(256), 0, st, dfl_sum, (const float*)nullptr, D);
    if (dil_sum)
      hipLaunchKernelGGL(fill_kernel, dim3(small_grid(D)), dim3(256), 0, st, dil_sum, (const float*)nullptr, D);
    if (dh0)
      hipLaunchKernelGGL(fill_kernel, dim3(small_grid(batch * D * N)), dim3(256), 0, st, dh0,
                         (const float*)nullptr, batch * D * N);
    if (dB) hipLaunchKernelGGL(zero_any_kernel, dim3(small_grid(batch * T * N)), dim3(256), 0, st, dB, bc_dtype,
                               batch * T * N);
    if (dC) hipLaunchKernelGGL(zero_any_kernel, dim3(small_grid(batch * T * N)), dim3(256), 0, st, dC, bc_dtype,
                               batch * T * N);
    if (hipGetLastError() != hipSuccess) return fail(NAJU_ERR_LAUNCH, "fill launch failed");
    return NAJU_OK;
  }
  if (!u || !f_logit || !i_logit || !B || !C || !D_skip || !dy)
    return fail(NAJU_ERR_INVALID, "null input pointer (u, f_logit, i_logit, B, C, D_skip and dy are required)");
  if (!ckpt) return fail(NAJU_ERR_INVALID, "ckpt is required (write it with naju_scan_fwd)");
  const Layout l = make_layout(batch, T, D, N, x_dtype, gate_dtype, true, SIZE_MAX, ck_rows);
  if (!workspace || workspace_bytes < l.total)
    return fail(NAJU_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", l.total,
                workspace ? workspace_bytes : (size_t)0);
  if (!aligned(workspace, 256)) return fail(NAJU_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  const size_t va_x = l.V * dsize(x_dtype), va_g = l.V * dsize(gate_dtype);
  const size_t vo_x = out_f32 ? l.V * 4 : va_x, vo_g = out_f32 ? l.V * 4 : va_g;
  const bool vec = (D % l.V == 0) && aligned(u, va_x) && aligned(dy, va_x) && aligned(du, vo_x) &&
                   aligned(f_logit, va_g) && aligned(i_logit, va_g) && aligned(dfl, vo_g) && aligned(dil, vo_g);
  ScanArgs a{};
  a.u = u;
  a.fl = f_logit;
  a.il = i_logit;
  a.Bm = B;
  a.Cm = C;
  a.Dsk = D_skip;
  a.dy = dy;
  a.ckpt = (float*)ckpt;
  a.du = du;
  a.dfl = dfl;
  a.dil = dil;
  a.dh0 = dh0;
  char* ws = (char*)workspace;
  a.hdr = (uint32_t*)ws;
  a.agg = (uint64_t*)(ws + l.off_agg);
  a.incl = (uint64_t*)(ws + l.off_incl);
  a.partB = dB ? (float*)(ws + l.off_partB) : nullptr;
  a.partC = dC ? (float*)(ws + l.off_partC) : nullptr;
  a.partD = dD ? (float*)(ws + l.off_partD) : nullptr;
  a.partG = (dfl_sum || dil_sum) ? (float*)(ws + l.off_partG) : nullptr;
  a.T = T;
  a.D = D;
  a.ldbc = ldbc;
  a.ldg = ldg;
  a.N = (int)N;
  a.batch = (int)batch;
  a.bc_dt = bc_dtype;
  a.n_dtiles = l.n_dtiles;
  a.n_tiles = l.n_tiles;
  a.K = l.K;
  if (N > 1) {
    const int du_dt = out_f32 ? (int)NAJU_DTYPE_F32 : x_dtype;
    a.nseg = l.nseg;
    a.seg_sc = l.seg_sc;
    a.segF = (float*)(ws + l.off_segF);
    a.segZ = (float*)(ws + l.off_segZ);
    a.seg0 = (float*)(ws + l.off_seg0);
    if ((int64_t)l.n_tiles * l.nseg > 0x7fffffff) return fail(NAJU_ERR_UNSUPPORTED, "problem too large");
    if (use_mc(N, true)) {
      // chunked matrix-core backward: adjoint segment maps, their carry, the
      // backward itself
      hipError_t e = hipSuccess;
      if (ck_rows > kMcQ) {
        // memory-light checkpoint: the state entering every sub-block,
        // recomputed from the forward's checkpoint into the workspace by the
        // forward's kernels (one workgroup per checkpoint interval and
        // kMcDT channels), bitwise as the forward computed it
        ScanArgs r = a;
        r.recomp = 1;
        r.ck_src = ckpt;
        r.Kc_src = (int)((T + ck_rows - 1) / ck_rows);
        r.ckpt = (float*)(ws + l.off_dense);
        r.Kc = (int)((T + kMcQ - 1) / kMcQ);
        r.seg_sc = ck_rows / kMcQ;
        r.nseg = r.Kc_src + 1;  // the map launch runs segments 0 .. nseg - 2
        r.n_dtiles = (int)((D + kMcDT - 1) / kMcDT);
        r.n_tiles = (int)(batch * r.n_dtiles);
        if ((int64_t)r.n_tiles * r.Kc_src > 0x7fffffff) return fail(NAJU_ERR_UNSUPPORTED, "problem too large");
        e = mc_fwd_launch(r, true, x_dtype, gate_dtype, x_dtype, st);
        a.ckpt = r.ckpt;
      }
      a.ck_rows = kMcQ;
      a.Kc = (int)((T + kMcQ - 1) / kMcQ);
      if (e == hipSuccess && l.nseg > 1) {
        e = mc_bwd_launch(a, true, x_dtype, gate_dtype, du_dt, dg_dt, st);
        if (e == hipSuccess) {
          const int64_t n = (int64_t)a.batch * a.D * a.N;
          hipLaunchKernelGGL(gn_seg_carry_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a, -1);
          e = hipGetLastError();
        }
      }
      if (e == hipSuccess) e = mc_bwd_launch(a, false, x_dtype, gate_dtype, du_dt, dg_dt, st);
      if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
      goto fold;
    }
    rc = gn_segments(a, l, x_dtype, gate_dtype, true, st);
    if (rc) return rc;
    hipLaunchKernelGGL(pick_gn_bwd(np_of(N)), dim3((unsigned)((int64_t)l.n_tiles * l.nseg)),
                       dim3(64 * gn_bwd_waves(np_of(N))), 0, st,
                       a, x_dtype, gate_dtype, du_dt, dg_dt);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(NAJU_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  } else {
    const int64_t wgs = (int64_t)l.K * l.n_tiles;
    if (wgs > 0x7fffffff || l.n_tiles > kMaxTiles)
      return fail(NAJU_ERR_UNSUPPORTED, "problem too large (%lld workgroups, %d channel tiles)", (long long)wgs,
                  l.n_tiles);
    const int64_t tg = launch_tag(a.hdr, st);
    if (tg < 0) return fail(NAJU_ERR_LAUNCH, "epoch launch failed");
    a.tag = (uint32_t)tg;
    a.strict = (flags & NAJU_FLAG_DETERMINISTIC) != 0;
    a.spin_limit = spin_limit();
    kern_t k = pick_n1_all(vec, out_f32 != 0, x_dtype, gate_dtype, bc_dtype, true);
    rc = launch(k, (unsigned)wgs, 64 * kBW, st, a);
    if (rc) return rc;
  }
fold:
  if (dB || dC || dD || a.partG) {
    const int64_t btn = batch * T * N;
    // enough workgroups for about one pass of the threads over the entries
    // (four per thread when btn % 4 == 0), at most 1024
    // (when that leaves fewer than 128 workgroups and btn % 4 == 0, 64
    // entries per workgroup with the parts split over its waves instead)
    const int64_t per = btn % 4 == 0 ? 4 * 1024 : 1024;
    const int64_t n_plain = (btn + per - 1) / per;
    const int bc_split = btn % 4 == 0 && n_plain < 128 ? 1 : 0;
    const int64_t n_bc64 = bc_split ? (btn / 4 + 63) / 64 : (n_plain < 1024 ? n_plain : 1024);
    const int n_bc = (dB || dC) ? (int)n_bc64 : 0;
    const int64_t n_rows = batch * (int64_t)(N == 1 ? l.K : l.nseg);
    FoldVecs fv{};
    auto add_vec = [&](const float* part, float* out) {
      fv.part[fv.n] = part;
      fv.out[fv.n] = out;
      ++fv.n;
    };
    if (dD) add_vec(a.partD, dD);
    if (dfl_sum) add_vec(a.partG, dfl_sum);
    if (dil_sum) add_vec(a.partG + n_rows * D, dil_sum);
    const int n_d = fv.n * (int)((D + 63) / 64);
    hipLaunchKernelGGL(fold_kernel, dim3((unsigned)(n_bc + n_d)), dim3(1024), 0, st, a.partB, a.partC, l.n_dtiles,
                       btn, dB, dC, out_f32 ? (int)NAJU_DTYPE_F32 : bc_dtype, n_bc, fv, n_rows, D, bc_split, N,
                       lddbc);
    if (hipGetLastError() != hipSuccess) return fail(NAJU_ERR_LAUNCH, "fold launch failed");
  }
  return NAJU_OK;
}

int naju_scan_bwd(const void* u, const void* f_logit, const void* i_logit, const void* B, const void* C,
                  const float* D_skip, const float* ckpt, const void* dy, void* du, void* dfl, void* dil, void* dB,
                  void* dC, float* dD, float* dh0, int64_t batch, int64_t T, int64_t D, int64_t N, int x_dtype,
                  int gate_dtype, int bc_dtype, int flags, void* workspace, size_t workspace_bytes,
                  void* stream) {
  return scan_bwd_impl(u, f_logit, i_logit, B, C, D_skip, ckpt, dy, du, dfl, dil, dB, dC, dD, dh0, batch, T, D, N,
                       x_dtype, gate_dtype, bc_dtype, flags, workspace, workspace_bytes, stream, N, N);
}

int naju_scan_bwd_strided(const void* u, const void* f_logit, const void* i_logit, const void* B, const void* C,
                          const float* D_skip, const float* ckpt, const void* dy, void* du, void* dfl, void* dil,
                          void* dB, void* dC, float* dD, float* dh0, int64_t batch, int64_t T, int64_t D, int64_t N,
                          int64_t bc_ld, int64_t dbc_ld, int x_dtype, int gate_dtype, int bc_dtype, int flags,
                          void* workspace, size_t workspace_bytes, void* stream) {
  return scan_bwd_impl(u, f_logit, i_logit, B, C, D_skip, ckpt, dy, du, dfl, dil, dB, dC, dD, dh0, batch, T, D, N,
                       x_dtype, gate_dtype, bc_dtype, flags, workspace, workspace_bytes, stream, bc_ld, dbc_ld);
}

int naju_scan_bwd_ex(const void* u, const void* f_logit, const void* i_logit, const void* B, const void* C,
                     const float* D_skip, const float* ckpt, const void* dy, void* du, void* dfl, void* dil,
                     void* dB, void* dC, float* dD, float* dh0, int64_t batch, int64_t T, int64_t D, int64_t N,
                     int x_dtype, int gate_dtype, int bc_dtype, int flags, const naju_scan_bwd_layout* layout,
                     void* workspace, size_t workspace_bytes, void* stream) {
  if (!layout) return naju_scan_bwd(u, f_logit, i_logit, B, C, D_skip, ckpt, dy, du, dfl, dil, dB, dC, dD, dh0,
                                    batch, T, D, N, x_dtype, gate_dtype, bc_dtype, flags, workspace,
                                    workspace_bytes, stream);
  const naju_scan_bwd_layout& o = *layout;
  return scan_bwd_impl(u, f_logit, i_logit, B, C, D_skip, ckpt, dy, du, dfl, dil, dB, dC, dD, dh0, batch, T, D, N,
                       x_dtype, gate_dtype, bc_dtype, flags, workspace, workspace_bytes, stream,
                       o.bc_ld > 0 ? o.bc_ld : N, o.dbc_ld > 0 ? o.dbc_ld : N, o.dg_ld > 0 ? o.dg_ld : D,
                       o.dg_dtype, o.dfl_sum, o.dil_sum);
}

int naju_scan_workspace_status(const void* workspace, void* stream, uint32_t* status) {
  if (!workspace || !status) return fail(NAJU_ERR_INVALID, "null workspace or status pointer");
  hipStream_t st = (hipStream_t)stream;
  uint32_t hdr[4];
  if (hipMemcpyAsync(hdr, workspace, sizeof(hdr), hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return fail(NAJU_ERR_LAUNCH, "could not read the workspace header");
  *status = hdr[HDR_STATUS];
  if (hdr[HDR_STATUS] != 0) {
    // Clear the status word and rewind every ticket counter (a status of 2
    // means some counter was out of range); the device epoch is kept, so
    // look-back words of earlier graph replays keep older tags.
    char* w = (char*)workspace;
    if (hipMemsetAsync(w + HDR_STATUS * sizeof(uint32_t), 0, sizeof(uint32_t), st) != hipSuccess ||
        hipMemsetAsync(w + kCtrBase * sizeof(uint32_t), 0, kHeaderBytes - kCtrBase * sizeof(uint32_t), st) !=
            hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
      return fail(NAJU_ERR_LAUNCH, "could not clear the workspace header");
  }
  return NAJU_OK;
}

int naju_scan_noalloc_status(void* stream, uint32_t* status) {
  g_err[0] = 0;
  if (!status) return fail(NAJU_ERR_INVALID, "null status pointer");
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(NAJU_ERR_LAUNCH, "no current HIP device (or device index >= %d)", kMaxDevices);
  void* p = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    p = g_scratch_ptr[dev];
  }
  if (!p) {  // no naju_scan_fwd_noalloc call on this device yet
    *status = 0;
    return NAJU_OK;
  }
  return naju_scan_workspace_status(p, stream, status);
}

}  // extern "C"
