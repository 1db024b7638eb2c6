// naju_scan_mc.hip -- chunked matrix-core kernels of the Naju scan for
// 9 <= N <= 64 (the mixer's d_state = 64 among them).
//
// Recurrence (reference naju/scan.py:15-19): x_t = f_t x_{t-1} + w_t B_t,
// y_t = C_t . x_t + D u_t, f = sigmoid(f_logit), w = sigmoid(i_logit) u.
//
// The direct recurrence costs about 3N vector operations per (row, channel)
// forward. Over a sub-block of Q = 16 rows with entering state X [N x ch],
// the same outputs are
//   y_t   = Pf_t (C_t . X) + sum_{s<=t} G[t][s] P[t,s] w_s + D u_t
//   X_out = Pall X + B^T (Pe (.) w)
// with G = C B^T [Q x Q] (shared by all channels of a batch row), the
// per-channel decays P[t,s] = prod_{s<q<=t} f_q, Pf_t = prod_{q<=t} f_q,
// Pe_t = prod_{q>t} f_q and Pall = Pf_{Q-1}: the O(N) work per element
// becomes the two matrix products C X and B^T (Pe w), which run on the
// matrix cores (v_mfma_f32_16x16x4_f32, exact float32 products), and the
// vector units keep O(Q) work per element. Every decay is a product of
// gates formed directly (no logarithms, no divisions), so gates that are
// exactly 0 or 1 stay exact and no input range needs a guard. This is the
// chunked form of the reference's Triton pass 1 (naju/chunk_triton.py:121-
// 139), without its exp(+-cumsum(log f)) factorisation.
//
// Lane layout. A wave owns 16 channels (lane l: channel j = l % 16) and
// holds, in the MFMA accumulator layout, the rows t = 4r + g of its channel
// (g = l / 16, value r = 0..3) and the state entries n = 16m + 4g + r. That
// layout is at the same time the B operand of C X (k-step 4m + r) and the
// output of B^T (Pe w), whose B operand (Pe w)[4s + g][j] is the lane's own
// value s: the state chain needs no data movement between lanes.
#include <hip/hip_runtime.h>

#include "naju_scan.h"
#include "scan_internal.h"

namespace naju_detail {
namespace {

typedef float f4_t __attribute__((ext_vector_type(4)));

// D += A B for one 16x16x4 float32 tile: lane l supplies A[l%16][l/16] and
// B[l/16][l%16] and holds D[4(l/16) + r][l%16] in value r.
__device__ __forceinline__ f4_t mma(float a, float b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Four values that are exact in the 2-byte stream type TT (B and C as
// staged: converted from TT, zero rows included) packed as TT pairs.
template <typename TT>
__device__ __forceinline__ void pack4(const float (&x)[4], uint32_t (&w)[2]) {
  if constexpr (__is_same(TT, bf16_t)) {
    // the upper halves of the float bits (exact: the low halves are zero)
#pragma unroll
    for (int k = 0; k < 2; ++k)
      w[k] = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, x[2 * k + 1]), __builtin_bit_cast(uint32_t, x[2 * k]),
                                   0x07060302u);
  } else {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      const h2 h = {(_Float16)x[2 * k], (_Float16)x[2 * k + 1]};
      w[k] = __builtin_bit_cast(uint32_t, h);
    }
  }
}

// D += A B with K = 32 on the 16-bit matrix-core path, for operands exact in
// TT (bf16 or f16): lane l supplies A[l%16][k] and B[k][l%16] for its eight
// k of the product, a0 and b0 (then a1 and b1) packed by pack4 from the same
// four k each, so that any assignment of the lane's values to k pairs A and
// B alike. The products are exact in float32 and only the accumulation
// rounds, as on the float32 path, at one instruction in place of eight.
template <typename TT>
__device__ __forceinline__ f4_t mma_k32(const uint32_t (&a0)[2], const uint32_t (&a1)[2], const uint32_t (&b0)[2],
                                        const uint32_t (&b1)[2], f4_t c) {
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  const u4 av = {a0[0], a0[1], a1[0], a1[1]}, bv = {b0[0], b0[1], b1[0], b1[1]};
  if constexpr (__is_same(TT, bf16_t)) {
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, av), __builtin_bit_cast(v8, bv), c, 0, 0,
                                                   0);
  } else {
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8, av), __builtin_bit_cast(v8, bv), c, 0, 0, 0);
  }
}

// x[k] = hi + mid + lo exactly, in three bf16 parts packed in pairs like
// pack4: hi keeps the top 8 significant bits of x (truncated), mid the next
// 8 of the remainder and lo the at most 8 left, so each part is exact in
// bf16 and each difference exact in float32. (x = +-inf or nan gives nan
// parts; the states and adjoints split here are finite for finite inputs.)
__device__ __forceinline__ void split4_bf16(const float (&x)[4], uint32_t (&h)[2], uint32_t (&md)[2],
                                            uint32_t (&lo)[2]) {
  uint32_t hb[4], mb[4], lb[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    // x as rounded: the subtraction below must not be fused with the
    // product that formed x (the parts would then sum to the unrounded
    // product, differently wherever the compiler chose to fuse)
    float xk = x[k];
    asm volatile("" : "+v"(xk));
    hb[k] = __builtin_bit_cast(uint32_t, xk) & 0xffff0000u;
    const float r = xk - __builtin_bit_cast(float, hb[k]);
    mb[k] = __builtin_bit_cast(uint32_t, r) & 0xffff0000u;
    lb[k] = __builtin_bit_cast(uint32_t, r - __builtin_bit_cast(float, mb[k]));
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    h[k] = __builtin_amdgcn_perm(hb[2 * k + 1], hb[2 * k], 0x07060302u);
    md[k] = __builtin_amdgcn_perm(mb[2 * k + 1], mb[2 * k], 0x07060302u);
    lo[k] = __builtin_amdgcn_perm(lb[2 * k + 1], lb[2 * k], 0x07060302u);
  }
}

// D += A B over the lane's four k (the k-steps of four 16x16x4 float32
// products) with A exact in bf16 (a: packed by pack4) and B float32 given by
// its split4_bf16 parts: hi and mid in one K = 32 product, lo (with zeros)
// in a second. Each product is exact; the result matches the float32 path
// up to the accumulation's rounding, at two instructions in place of four.
// (The K = 16 form, v_mfma_f32_16x16x16_bf16, took the lo part at first and
// gave run-to-run different results in this position on gfx950 with the
// compiler's default scheduling; the K = 32 form is used throughout.)
__device__ __forceinline__ f4_t mma_x3(const uint32_t (&a)[2], const uint32_t (&h)[2], const uint32_t (&md)[2],
                                       const uint32_t (&lo)[2], f4_t c) {
  c = mma_k32<bf16_t>(a, a, h, md, c);
  const uint32_t z[2] = {0u, 0u};
  return mma_k32<bf16_t>(a, z, lo, z, c);
}

constexpr int Q = kMcQ;    // rows per sub-block
constexpr int TP = Q + 4;  // pitch of the per-wave [channel][row] tiles

// Decays of the own rows t = 4r + g (g = the lane group, 0..3) from the
// channel's gates fa[0 .. Q): pf[r] = prod_{q <= t} fa[q] and
// pe[r] = prod_{q > t} fa[q], plus Pall = prod_q fa[q]. The group's part is
// a masked product of fixed elements: selecting fa[4r + g] by the lane's
// group would be turned into an indexed array in scratch memory.
__device__ __forceinline__ float own_decays(const float (&fa)[Q], int g, float (&pf)[4], float (&pe)[4]) {
  float run = 1.f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float a1 = g >= 1 ? fa[4 * r + 1] : 1.f;
    const float a2 = g >= 2 ? fa[4 * r + 2] : 1.f;
    const float a3 = g >= 3 ? fa[4 * r + 3] : 1.f;
    pf[r] = ((run * fa[4 * r]) * a1) * (a2 * a3);
    run *= (fa[4 * r] * fa[4 * r + 1]) * (fa[4 * r + 2] * fa[4 * r + 3]);
  }
  const float all = run;
  run = 1.f;
#pragma unroll
  for (int r = 3; r >= 0; --r) {
    const float b3 = g < 3 ? fa[4 * r + 3] : 1.f;
    const float b2 = g < 2 ? fa[4 * r + 2] : 1.f;
    const float b1 = g < 1 ? fa[4 * r + 1] : 1.f;
    pe[r] = (run * b3) * (b2 * b1);
    run *= (fa[4 * r + 3] * fa[4 * r + 2]) * (fa[4 * r + 1] * fa[4 * r]);
  }
  return all;
}

// Four consecutive elements of a stream of element type TT at element
// offset i from p (4-element aligned when VEC), as float.
template <typename TT, bool VEC>
__device__ __forceinline__ void ld4v(const TT* __restrict__ p, uint32_t i, float (&o)[4]) {
  if constexpr (VEC) {
    typedef TT v4 __attribute__((ext_vector_type(4)));
    const v4 v = *reinterpret_cast<const v4*>(p + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = to_f32(v[e]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = to_f32(p[i + e]);
  }
}

// Four consecutive elements of a stream as loaded: the raw bits (8 bytes
// for 2-byte types, 16 for float), turned into floats only where they are
// used. A conversion right after the load would make the wave wait for the
// load there, so data loaded a sub-block ahead stays raw until its turn.
template <typename TT>
struct Raw4 {
  static constexpr int NW = sizeof(TT) == 2 ? 2 : 4;
  uint32_t w[NW];
  __device__ __forceinline__ float get(int e) const {
    if constexpr (sizeof(TT) == 4) {
      return __builtin_bit_cast(float, w[e]);
    } else {
      const uint32_t x = w[e >> 1];
      const uint16_t h = (e & 1) ? (uint16_t)(x >> 16) : (uint16_t)(x & 0xffffu);
      return to_f32(__builtin_bit_cast(TT, h));
    }
  }
};

// Raw4 load of elements i .. i+3 at p (4-element aligned; VEC: one 8- or
// 16-byte load) or of the elements at offsets o[0..3] (clamped edge lanes).
template <typename TT>
__device__ __forceinline__ void ld4r(const TT* __restrict__ p, uint32_t i, Raw4<TT>& r) {
  // a clang vector type (not HIP's uint2 / uint4 structs, whose member
  // reads are split into one 4-byte load each)
  typedef uint32_t vw __attribute__((ext_vector_type(Raw4<TT>::NW)));
  const vw v = *reinterpret_cast<const vw*>(p + i);
#pragma unroll
  for (int k = 0; k < Raw4<TT>::NW; ++k) r.w[k] = v[k];
}
template <typename TT>
__device__ __forceinline__ void ld4r_at(const TT* __restrict__ p, const uint32_t (&o)[4], Raw4<TT>& r) {
  if constexpr (sizeof(TT) == 2) {
    uint32_t h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = __builtin_bit_cast(uint16_t, p[o[e]]);
    r.w[0] = h[0] | (h[1] << 16), r.w[1] = h[2] | (h[3] << 16);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) r.w[e] = __builtin_bit_cast(uint32_t, p[o[e]]);
  }
}

// LDS tiles of a sub-block's B and C, staged once per workgroup:
//   Bn, C [t][n]  (row-major; pitch NP + 4 makes 16-byte reads of 16
//                  different rows conflict-free),
//   Bt [n][p(t)]  (B transposed, time rows permuted p(4s + g) = 4g + s, so
//                  the four rows 4s + g (s = 0..3) a lane feeds to the state
//                  update are one 16-byte read).
template <int NP, bool MAP>
struct McBC {
  static constexpr int P = NP + 4;
  float Bn[2][MAP ? 1 : kMcQ][MAP ? 4 : P];
  float C[2][MAP ? 1 : kMcQ][MAP ? 4 : P];
  float Bt[2][NP][TP];
};

// One sub-block's inputs as a lane loads them: row rho of the wave's 16
// channels cq .. cq+3 (clamped in bounds; rows past T and channels past D
// become the neutral step when the gates are formed), and the workgroup's B
// (and C) groups of four entries: thread tid < 4 NP takes row (4 tid) / NP,
// entries n0 .. n0+3 with n0 = (4 tid) % NP.
template <int NP, bool MAP, typename TU, typename TG, typename TB>
struct McIn {
  Raw4<TG> f, i;
  Raw4<TU> u;
  Raw4<TB> b, c;

  __device__ __forceinline__ void load(const ScanArgs& a, int b_row, int64_t t0, int64_t dw, int rho, int cq,
                                       int tid, bool vec) {
    const int64_t T = a.T, D = a.D;
    const int64_t rows = T - t0 < kMcQ ? T - t0 : kMcQ;
    // row t0 of the batch row (uniform) plus a 32-bit in-bounds offset:
    // row min(rho, rows - 1) (< 16 rows of D < 2^25 channels), channel
    // clamped to D - 1 (a wave may lie wholly past D)
    const int64_t base = ((int64_t)b_row * T + t0) * D;
    const uint32_t off = (uint32_t)((rho < rows ? rho : rows - 1) * D);
    if (vec) {  // the wave's 16 channels lie inside [0, D), D % 4 == 0
      const uint32_t o = off + (uint32_t)(dw + cq);
      ld4r<TG>((const TG*)a.fl + base, o, f);
      ld4r<TG>((const TG*)a.il + base, o, i);
      ld4r<TU>((const TU*)a.u + base, o, u);
    } else {
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = off + (uint32_t)(dw + cq + e < D ? dw + cq + e : D - 1);
      ld4r_at<TG>((const TG*)a.fl + base, o, f);
      ld4r_at<TG>((const TG*)a.il + base, o, i);
      ld4r_at<TU>((const TU*)a.u + base, o, u);
    }
    if (tid < 4 * NP) {
      const int N = a.N;
      const int row = (4 * tid) / NP, n0 = (4 * tid) % NP;
      const int64_t bb = ((int64_t)b_row * T + t0) * a.ldbc;  // (t0, 0), uniform
      const uint32_t ro = (uint32_t)((row < rows ? row : rows - 1) * a.ldbc);
      if (N == NP) {
        ld4r<TB>((const TB*)a.Bm + bb, ro + n0, b);
        if constexpr (!MAP) ld4r<TB>((const TB*)a.Cm + bb, ro + n0, c);
      } else {
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = ro + (uint32_t)(n0 + e < N ? n0 + e : N - 1);
        ld4r_at<TB>((const TB*)a.Bm + bb, o, b);
        if constexpr (!MAP) ld4r_at<TB>((const TB*)a.Cm + bb, o, c);
      }
    }
  }

  // Waits for these loads here. Used on the first sub-block's inputs before
  // the loop: the compiler's wait counting would otherwise still see them
  // pending at their uses inside the loop, and since every other iteration
  // has the next sub-block's loads issued after them, it would wait there
  // for those too, leaving nothing in flight while the sub-block is worked.
  __device__ __forceinline__ void settle() {
#pragma unroll
    for (int k = 0; k < Raw4<TG>::NW; ++k) asm volatile("" : "+v"(f.w[k]), "+v"(i.w[k]));
#pragma unroll
    for (int k = 0; k < Raw4<TU>::NW; ++k) asm volatile("" : "+v"(u.w[k]));
#pragma unroll
    for (int k = 0; k < Raw4<TB>::NW; ++k) asm volatile("" : "+v"(b.w[k]), "+v"(c.w[k]));
  }

  // B (and C) into LDS buffer buf; zeros past T and past N. (Each 16 lanes
  // read one 64-entry row of B and C, coalesced; the backward's staging takes
  // another lane map, which the forward measured slower with.)
  __device__ __forceinline__ void stage(McBC<NP, MAP>& sh, int buf, const ScanArgs& a, int64_t t0, int tid) const {
    if (tid < 4 * NP) {
      const int row = (4 * tid) / NP, n0 = (4 * tid) % NP;
      const bool rok = t0 + row < a.T;
      float vb[4], vc[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool ok = rok && n0 + e < a.N;
        vb[e] = ok ? b.get(e) : 0.f;
        if constexpr (!MAP) vc[e] = ok ? c.get(e) : 0.f;
        sh.Bt[buf][n0 + e][4 * (row & 3) + (row >> 2)] = vb[e];
      }
      if constexpr (!MAP) {
        *(float4*)&sh.Bn[buf][row][n0] = make_float4(vb[0], vb[1], vb[2], vb[3]);
        *(float4*)&sh.C[buf][row][n0] = make_float4(vc[0], vc[1], vc[2], vc[3]);
      }
    }
  }
};

// The wave's 16 channels x 64 state entries (X in the D layout: lane (j, g)
// value r of X[m] is entry 16m + 4g + r of channel j), stored as the
// contiguous 4 KB run [channel][entry] at ckw. Stored straight from the D
// layout, each store would write sixteen 64-byte pieces; transposed through
// tt (16 x 36 floats of the wave's own LDS, free at the call), each store
// writes eight whole 128-byte lines. Two halves of 32 entries per channel.
// (MT = 4 only: the callers test N == 64)
template <int MT>
__device__ __forceinline__ void store_state64(float* ckw, const f4_t (&X)[MT], float* tt, int j, int g, int lane) {
  static_assert(16 * 36 <= 2 * 16 * TP, "the transposition fits a wave's two gate tiles");
  if constexpr (MT == 4) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      asm volatile("" ::: "memory");
#pragma unroll
      for (int k = 0; k < 2; ++k)
        *(float4*)(tt + j * 36 + 16 * k + 4 * g) =
            make_float4(X[2 * h + k][0], X[2 * h + k][1], X[2 * h + k][2], X[2 * h + k][3]);
      asm volatile("" ::: "memory");
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const int c = 8 * s2 + (lane >> 3), q = 4 * (lane & 7);
        const float4 v = *(const float4*)(tt + c * 36 + q);
        *(float4*)(ckw + c * 64 + 32 * h + q) = v;
      }
    }
    asm volatile("" ::: "memory");
  }
}

// ------------------------------------------------------------------ forward
//
// One workgroup per (batch row, kMcDT channels, time segment); the segment's
// sub-blocks are walked in order, the inputs of sub-block sb + 1 loaded while
// sb is computed and staged at its end, B and C double-buffered
// in LDS (one barrier per sub-block). MAP: the segment's map from a zero
// state (decay per channel into segF, state into segZ) for the carry pass
// over the segments, or with a.recomp the states entering the segment's
// sub-blocks, from its checkpoint (one segment per checkpoint interval),
// into a.ckpt; otherwise y, the checkpoint and hT from the entering state
// (h0, or seg0 when T is split into segments).
template <int NP, bool MAP, typename TU, typename TG, typename TB>
__global__ __launch_bounds__(64 * kMcW) __attribute__((amdgpu_waves_per_eu(3))) void mc_fwd_kernel(const ScanArgs a, int y_dt) {
  constexpr int MT = NP / 16;  // 16-entry tiles of the state index
  using In = McIn<NP, MAP, TU, TG, TB>;
  __shared__ __align__(16) McBC<NP, MAP> sh;
  // per wave: f (later G for the exact path, then y) and w = i u as [channel][row]
  __shared__ __align__(16) float s_t[kMcW][2][16][TP];

  const int N = a.N;
  const int64_t T = a.T, D = a.D;
  const int tile = (int)(blockIdx.x % (uint32_t)a.n_tiles);
  const int seg = (int)(blockIdx.x / (uint32_t)a.n_tiles);
  const int b = tile / a.n_dtiles;
  const int dtile = tile - b * a.n_dtiles;
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int64_t dw = (int64_t)dtile * kMcDT + 16 * wv;  // the wave's first channel
  const int64_t d = dw + j;
  const bool dok = d < D;
  const int KS = (int)((T + Q - 1) / Q);
  const int sb0 = seg * a.seg_sc;
  const int sb1 = sb0 + a.seg_sc < KS ? sb0 + a.seg_sc : KS;
  const int ck_sb = a.ck_rows / Q;
  const bool vec = dw + 16 <= D && D % 4 == 0;

  // state entries n = 16m + 4g + r of channel d
  f4_t X[MT];
  {
    const float* xin = MAP ? (a.recomp ? a.ck_src + ((int64_t)b * a.Kc_src + seg) * D * N : nullptr)
                           : (a.nseg > 1 ? a.seg0 + ((int64_t)b * a.nseg + seg) * D * N
                                         : (a.h0 ? a.h0 + (int64_t)b * D * N : nullptr));
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = 16 * m + 4 * g + r;
        X[m][r] = (xin && dok && n < N) ? xin[d * N + n] : 0.f;
      }
    // loaded before the loop, waited for here (as McIn::settle)
#pragma unroll
    for (int m = 0; m < MT; ++m) asm volatile("" : "+v"(X[m]));
  }
  float Fseg = 1.f;
  // load role: row rho, channels cq .. cq+3 of the wave's 16
  const int rho = lane >> 2, cq = (lane & 3) * 4;
  // channels of the load role inside [0, D) (0..4), formed once: past D a
  // channel is the neutral step
  const int ncq0 = (int)(D - dw - cq < 4 ? (D - dw - cq < 0 ? 0 : D - dw - cq) : 4);
  // D of the load role's channels (the D u term of y is added there)
  float Dvc[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) Dvc[e] = (!MAP && dw + cq + e < D) ? a.Dsk[dw + cq + e] : 0.f;
  asm volatile("" : "+v"(Dvc[0]), "+v"(Dvc[1]), "+v"(Dvc[2]), "+v"(Dvc[3]));

  // inputs of sub-blocks sb (cur) and sb + 1 (nxt), loaded one sub-block
  // ahead of their use
  In cur, nxt;
  if (sb0 < sb1) {
    cur.load(a, b, (int64_t)sb0 * Q, dw, rho, cq, tid, vec);
    cur.settle();
    cur.stage(sh, 0, a, (int64_t)sb0 * Q, tid);
  }
  for (int sb = sb0; sb < sb1; ++sb) {
    // The lane's indices, recomputed every sub-block from an opaque copy of
    // the lane id (they shadow the ones above), so that the lane-dependent
    // LDS and global addresses are not all hoisted out of the loop and held.
    int lane_l = lane;
    asm volatile("" : "+v"(lane_l));
    const int j = lane_l & 15, g = lane_l >> 4;
    const int rho = lane_l >> 2, cq = (lane_l & 3) * 4;
    const int arow = 4 * (j & 3) + (j >> 2);
    const int64_t d = dw + j;
    const bool dok = d < D;
    const int tid = 64 * wv + lane_l;
    const int buf = (sb - sb0) & 1;
    const int64_t t0 = (int64_t)sb * Q;
    if (sb + 1 < sb1) nxt.load(a, b, t0 + Q, dw, rho, cq, tid, vec);
    // gates in the load layout, each element computed once; rows past T
    // and channels past D are the neutral step f = 1, w = u = 0
    // (32-bit tests: rows left in the sub-block, uniform, and ncq0)
    const int rl = (int)(T - t0 < Q ? T - t0 : Q);
    const bool rok = rho < rl;
    float uu[4];  // u of the load role (0 past T / D), for the D u term
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool ok = rok && e < ncq0;
      // both gates formed on every lane, then selected (no branch per element)
      float sf = sigm(cur.f.get(e)), sw = sigm(cur.i.get(e)) * cur.u.get(e);
      asm volatile("" : "+v"(sf), "+v"(sw));
      s_t[wv][0][cq + e][rho] = ok ? sf : 1.f;
      s_t[wv][1][cq + e][rho] = ok ? sw : 0.f;
      uu[e] = ok ? cur.u.get(e) : 0.f;
    }
    __syncthreads();  // B / C of sb are staged; every wave is done with sb - 1
    // G[t][s] = C_t . B_s of the sub-block, in the layout of an A operand
    // whose MFMA row i is time row arow(i): Gp[r] = G[arow(j)][4r + g]
    // (the product B_(arow) C_(arow)^T transposed; k-step (q, r') takes
    // n = 16q + 4k + r')
    f4_t Gp = {0.f, 0.f, 0.f, 0.f};
    if constexpr (!MAP && sizeof(TB) == 2 && NP >= 32) {
      // B and C exact in TB: two 16-entry groups of n per K = 32 product
#pragma unroll
      for (int q = 0; q < NP / 16; q += 2) {
        uint32_t pb[2][2], pc[2][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float4 c4 = *(const float4*)&sh.C[buf][arow][16 * (q + h) + 4 * g];
          const float4 b4 = *(const float4*)&sh.Bn[buf][arow][16 * (q + h) + 4 * g];
          pack4<TB>({b4.x, b4.y, b4.z, b4.w}, pb[h]);
          pack4<TB>({c4.x, c4.y, c4.z, c4.w}, pc[h]);
        }
        Gp = mma_k32<TB>(pb[0], pb[1], pc[0], pc[1], Gp);
      }
    } else if constexpr (!MAP) {
#pragma unroll
      for (int q = 0; q < NP / 16; ++q) {
        const float4 c4 = *(const float4*)&sh.C[buf][arow][16 * q + 4 * g];
        const float4 b4 = *(const float4*)&sh.Bn[buf][arow][16 * q + 4 * g];
        Gp = mma(b4.x, c4.x, Gp);
        Gp = mma(b4.y, c4.y, Gp);
        Gp = mma(b4.z, c4.z, Gp);
        Gp = mma(b4.w, c4.w, Gp);
      }
    }
    // (the wave reads back what its own lanes wrote: LDS keeps a wave's
    // accesses in order, the compiler must not move them)
    asm volatile("" ::: "memory");
    // this lane's channel over all Q rows, and its own rows 4r + g
    float fa[Q];
#pragma unroll
    for (int q4 = 0; q4 < Q; q4 += 4) {
      const float4 f4 = *(const float4*)&s_t[wv][0][j][q4];
      fa[q4] = f4.x, fa[q4 + 1] = f4.y, fa[q4 + 2] = f4.z, fa[q4 + 3] = f4.w;
    }
    float w_o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) w_o[r] = s_t[wv][1][j][4 * r + g];
    // decays of the own rows: pf = prod_{q <= t} f, pe = prod_{q > t} f
    float pf[4], pe[4];
    const float Pall = own_decays(fa, g, pf, pe);

    if constexpr (!MAP) {
      // intra-sub-block part of y for the own rows t = 4r + g,
      // S[t] = sum_{s<=t} P[t,s] G[t][s] w_s.
      float S[4];
      if (__all(Pall >= kMcRatioMin)) {
        // Every channel of the wave keeps its decay over the sub-block above
        // kMcRatioMin: P[t,s] = Pf[t] / Pf[s] (products from row 0) in
        // floating point, and S = Pf * (masked G) (w / Pf) is one 16 x 16 x 16
        // product: MFMA row i is time row arow(i), k-step e takes row
        // s = 4e + g, whose w / Pf this lane holds (its own row e).
        f4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float gm = 4 * e + g <= arow ? Gp[e] : 0.f;
          acc = mma(gm, w_o[e] * __builtin_amdgcn_rcpf(pf[e]), acc);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) S[r] = pf[r] * acc[r];
      } else {
        // exact products: Horner S_k = f_k S_{k-1} + G[t][k] w_k for
        // k = 0 .. t; rows k <= 4r are in every lane's range, rows
        // 4r+1 .. 4r+3 only in some. G goes through the f tile (read into
        // fa already) as [t][s].
        float (*TGt)[TP] = s_t[wv][0];
#pragma unroll
        for (int r = 0; r < 4; ++r) TGt[arow][4 * r + g] = Gp[r];
        asm volatile("" ::: "memory");
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 4 * r + g;
          float acc = 0.f;
#pragma unroll
          for (int s4 = 0; s4 <= 4 * r; s4 += 4) {
            // w of rows s4 .. s4+3 read where used (fewer live registers)
            const float4 G4 = *(const float4*)&TGt[t][s4];
            const float4 W4 = *(const float4*)&s_t[wv][1][j][s4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int s = s4 + e;
              if (s <= 4 * r) {
                acc = fmaf(acc, fa[s], (&G4.x)[e] * (&W4.x)[e]);
              } else {
                const bool in = s <= t;
                acc = fmaf(acc, in ? fa[s] : 1.f, in ? (&G4.x)[e] * (&W4.x)[e] : 0.f);
              }
            }
          }
          S[r] = acc;
        }
      }
      // C X for the own rows (MFMA row i = 4g + r is time row 4r + g)
      f4_t cx = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float4 c4 = *(const float4*)&sh.C[buf][arow][16 * m + 4 * g];
        cx = mma(c4.x, X[m][0], cx);
        cx = mma(c4.y, X[m][1], cx);
        cx = mma(c4.z, X[m][2], cx);
        cx = mma(c4.w, X[m][3], cx);
      }
      // B / C of sb + 1 into the other buffer (free since the barrier
      // above), before this sub-block's stores are issued: waiting for the
      // next sub-block's loads after them would wait for the stores as well
      if (sb + 1 < sb1) {
        nxt.settle();
        nxt.stage(sh, buf ^ 1, a, t0 + Q, tid);
      }
      // the state entering this sub-block is the backward's checkpoint
      if (NP == 64 && N == 64 && a.ckpt && dw + 16 <= D && sb % ck_sb == 0) {
        store_state64(a.ckpt + (((int64_t)b * a.Kc + sb / ck_sb) * D + dw) * N, X, &s_t[wv][0][0][0], j, g, lane_l);
      } else if (a.ckpt && dok && sb % ck_sb == 0) {
        float* ck = a.ckpt + (((int64_t)b * a.Kc + sb / ck_sb) * D + d) * N;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const int n = 16 * m + 4 * g;
          if ((N & 3) == 0) {
            if (n < N) *(float4*)(ck + n) = make_float4(X[m][0], X[m][1], X[m][2], X[m][3]);
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (n + r < N) ck[n + r] = X[m][r];
          }
        }
      }
      // y of the own rows (less D u) through the f tile, then stored in the
      // load layout (row rho, channels cq .. cq+3) with D u added
      asm volatile("" ::: "memory");
#pragma unroll
      for (int r = 0; r < 4; ++r) s_t[wv][0][j][4 * r + g] = fmaf(pf[r], cx[r], S[r]);
      asm volatile("" ::: "memory");
      if (rok) {
        float yv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) yv[e] = fmaf(Dvc[e], uu[e], s_t[wv][0][cq + e][rho]);
        const int64_t o = ((int64_t)b * T + t0 + rho) * D + dw + cq;
        if (y_dt == NAJU_DTYPE_F32) {
          if (vec)
            *(float4*)((float*)a.y + o) = make_float4(yv[0], yv[1], yv[2], yv[3]);
          else
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (dw + cq + e < D) ((float*)a.y)[o + e] = yv[e];
        } else {
          typedef TU v4 __attribute__((ext_vector_type(4)));
          if (vec) {
            v4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (TU)yv[e];
            *(v4*)((TU*)a.y + o) = v;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (dw + cq + e < D) ((TU*)a.y)[o + e] = (TU)yv[e];
          }
        }
      }
    } else {
      Fseg *= Pall;
      if (NP == 64 && N == 64 && a.recomp && dw + 16 <= D) {
        // the state entering sb, as the scan's checkpoint holds it (the
        // wave's gate tiles are free: f and w are in registers)
        store_state64(a.ckpt + (((int64_t)b * a.Kc + sb) * D + dw) * N, X, &s_t[wv][0][0][0], j, g, lane_l);
      } else if (a.recomp && dok) {
        // the state entering sb, as the scan's checkpoint holds it
        float* ck = a.ckpt + (((int64_t)b * a.Kc + sb) * D + d) * N;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const int n = 16 * m + 4 * g;
          if ((N & 3) == 0) {
            if (n < N) *(float4*)(ck + n) = make_float4(X[m][0], X[m][1], X[m][2], X[m][3]);
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (n + r < N) ck[n + r] = X[m][r];
          }
        }
      }
    }
    // X <- Pall X + B^T (Pe w): k-step s takes rows 4s + k
    float wp[4];
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) wp[s2] = pe[s2] * w_o[s2];
    if constexpr (__is_same(TB, bf16_t)) {
      // B exact in bf16: Pe w split in three bf16 parts (the 16-bit path)
      uint32_t wh[2], wm[2], wl[2];
      split4_bf16(wp, wh, wm, wl);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        X[m] *= Pall;
        const float4 bt = *(const float4*)&sh.Bt[buf][16 * m + j][4 * g];
        uint32_t ab[2];
        pack4<TB>({bt.x, bt.y, bt.z, bt.w}, ab);
        X[m] = mma_x3(ab, wh, wm, wl, X[m]);
      }
    } else {
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        X[m] *= Pall;
        const float4 bt = *(const float4*)&sh.Bt[buf][16 * m + j][4 * g];
        X[m] = mma(bt.x, wp[0], X[m]);
        X[m] = mma(bt.y, wp[1], X[m]);
        X[m] = mma(bt.z, wp[2], X[m]);
        X[m] = mma(bt.w, wp[3], X[m]);
      }
    }
    // the map's B of sb + 1 into the other buffer, as late as possible so
    // that its loads have the whole sub-block to land
    if (MAP && sb + 1 < sb1) nxt.stage(sh, buf ^ 1, a, t0 + Q, tid);
    cur = nxt;
  }
  if (!dok) return;
  if (MAP) {
    if (a.recomp) return;
    const int64_t o = ((int64_t)b * a.nseg + seg) * D + d;
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = 16 * m + 4 * g + r;
        if (n < N) a.segZ[o * N + n] = X[m][r];
      }
    if (g == 0) a.segF[o] = Fseg;
  } else if (a.hT && seg == a.nseg - 1) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = 16 * m + 4 * g + r;
        if (n < N) a.hT[((int64_t)b * D + d) * N + n] = X[m][r];
      }
  }
}

// ----------------------------------------------------------------- backward
//
// Adjoint in carry form: g_t is the carry entering row t from the future
// (f_{t+1} xbar_{t+1}), xbar_t = C_t dy_t + g_t. Over a sub-block with
// entering state X [N x ch] (the forward's checkpoint, every kMcQ rows) and
// carry ghat entering its last row:
//   xbar_t = sum_{s>=t} P[s,t] C_s dy_s + Pe_t ghat
//   dws_t  = xbar_t . B_t = sum_{s>=t} P[s,t] dy_s G[s][t] + Pe_t (B_t . ghat)
//   xbar_t . x_t = Pf_t sum_{s>=t} P[s,t] dy_s (C_s . X)
//                + sum_{s>=t>=r} P[s,r] dy_s w_r G[s][r]          (rectangle)
//                + Pe_t Pf_t (ghat . X) + Pe_t sum_{r<=t} P[t,r] w_r (B_r . ghat)
//   dfl_t  = (1 - f_t) (xbar_t . x_t - w_t dws_t)  (= f(1-f) xbar_t . x_{t-1},
//            no division; exactly 0 at f = 1, and set to 0 at f = 0)
//   du_t   = i_t dws_t + D dy_t,   dil_t = (1 - i_t) dws_t w_t
//   dC_t   = sum_d (dy Pf)_t[d] X[.][d] + sum_{r<=t} H[t][r] B_r
//   dB_t   = sum_d (w Pe)_t[d] ghat[.][d] + sum_{s>=t} H[s][t] C_s
//            with H[s][r] = sum_d dy_s P[s,r] w_r (the wave's 16 channels)
//   ghat'  = Pall ghat + C^T (Pf dy)   (the carry leaving the first row)
// (naju/cuda/naju_cuda.cu:104-141 restated per sub-block.) C X, B ghat,
// G = C B^T, the dB / dC products and the carry update run on the matrix
// cores; the per-channel sums over pairs of rows on the vector units.
//
// Layouts. "D layout" as in the forward: lane (j, g) value r holds row
// 4r + g of channel j, or state entry n = 16m + 4g + r of channel j. "T
// layout": lane (j, g) value r holds entry n = 16m + j of channel 4g + r.
// ghat is kept in both (the two carry updates read the same operands with
// the A and B roles swapped); X is read from the checkpoint in both.
//
// LDS per workgroup (NP = 64): B / C staged as Bn, C [t][n] and Bt, Ct
// [n][p(t)] (19 KB), per wave the gate tiles f, w, dy, i [channel][row]
// (5 KB) and a pool of seven [16][TP] tiles (8.75 KB) that holds G, G^T,
// gathers, the rectangle sums' partials, (dy Pf) / (w Pe), H / H^T and
// finally the wave's dB / dC, which the workgroup adds in wave order.
template <int NP, bool MAP>
struct McBwdLds {
  static constexpr int P = NP + 4;
  static constexpr int POOL = 9 * 16 * TP;  // floats of a wave's pool
  float Bn[MAP ? 1 : kMcQ][MAP ? 4 : P];
  float C[MAP ? 1 : kMcQ][MAP ? 4 : P];
  float Bt[MAP ? 1 : NP][TP];
  float Ct[NP][TP];
  float gate[kMcWB][MAP ? 2 : 4][16][TP];  // f, dy, w, i as [channel][row]; later dfl, du, dil
  float pool[MAP ? 1 : kMcWB][POOL];
};

template <int NP, bool MAP, typename TU, typename TG, typename TB>
struct McInB {
  Raw4<TG> f, i;
  Raw4<TU> dy, u;
  Raw4<TB> b, c;

  __device__ __forceinline__ void load(const ScanArgs& a, int b_row, int64_t t0, int64_t dw, int rho, int cq,
                                       int tid, bool vec) {
    const int64_t T = a.T, D = a.D;
    const int64_t rows = T - t0 < kMcQ ? T - t0 : kMcQ;
    // row t0 of the batch row (uniform) plus a 32-bit in-bounds offset:
    // row min(rho, rows - 1), channel clamped to D - 1
    const int64_t base = ((int64_t)b_row * T + t0) * D;
    const uint32_t off = (uint32_t)((rho < rows ? rho : rows - 1) * D);
    if (vec) {
      const uint32_t o = off + (uint32_t)(dw + cq);
      ld4r<TG>((const TG*)a.fl + base, o, f);
      ld4r<TU>((const TU*)a.dy + base, o, dy);
      if constexpr (!MAP) {
        ld4r<TG>((const TG*)a.il + base, o, i);
        ld4r<TU>((const TU*)a.u + base, o, u);
      }
    } else {
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = off + (uint32_t)(dw + cq + e < D ? dw + cq + e : D - 1);
      ld4r_at<TG>((const TG*)a.fl + base, o, f);
      ld4r_at<TU>((const TU*)a.dy + base, o, dy);
      if constexpr (!MAP) {
        ld4r_at<TG>((const TG*)a.il + base, o, i);
        ld4r_at<TU>((const TU*)a.u + base, o, u);
      }
    }
    if (tid < 4 * NP) {
      const int N = a.N;
      const int row = tid % kMcQ, n0 = 4 * (tid / kMcQ);
      const int64_t bb = ((int64_t)b_row * T + t0) * a.ldbc;
      const uint32_t ro = (uint32_t)((row < rows ? row : rows - 1) * a.ldbc);
      if (N == NP) {
        ld4r<TB>((const TB*)a.Cm + bb, ro + n0, c);
        if constexpr (!MAP) ld4r<TB>((const TB*)a.Bm + bb, ro + n0, b);
      } else {
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = ro + (uint32_t)(n0 + e < N ? n0 + e : N - 1);
        ld4r_at<TB>((const TB*)a.Cm + bb, o, c);
        if constexpr (!MAP) ld4r_at<TB>((const TB*)a.Bm + bb, o, b);
      }
    }
  }

  // waits for these loads here (as McIn::settle)
  __device__ __forceinline__ void settle() {
#pragma unroll
    for (int k = 0; k < Raw4<TG>::NW; ++k) asm volatile("" : "+v"(f.w[k]), "+v"(i.w[k]));
#pragma unroll
    for (int k = 0; k < Raw4<TU>::NW; ++k) asm volatile("" : "+v"(dy.w[k]), "+v"(u.w[k]));
#pragma unroll
    for (int k = 0; k < Raw4<TB>::NW; ++k) asm volatile("" : "+v"(b.w[k]), "+v"(c.w[k]));
  }

  // B and C into LDS. Thread tid < 4 NP takes row tid % 16, entries n0 ..
  // n0+3 with n0 = 4 (tid / 16): a half-wave holds all 16 rows of two
  // groups of entries, so the transposed tiles' 4-byte writes fall on 32
  // different banks, and each [t][n] tile takes one 16-byte write per lane
  // (the forward's row-per-16-lanes map costs 14 and 6 extra LDS cycles per
  // write there, about 1.4% of this kernel).
  __device__ __forceinline__ void stage(McBwdLds<NP, MAP>& sh, const ScanArgs& a, int64_t t0, int tid) const {
    if (tid < 4 * NP) {
      const int row = tid % kMcQ, n0 = 4 * (tid / kMcQ);
      const bool rok = t0 + row < a.T;
      const int pr = 4 * (row & 3) + (row >> 2);
      float vb[4], vc[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool ok = rok && n0 + e < a.N;
        vc[e] = ok ? c.get(e) : 0.f;
        sh.Ct[n0 + e][pr] = vc[e];
        if constexpr (!MAP) {
          vb[e] = ok ? b.get(e) : 0.f;
          sh.Bt[n0 + e][pr] = vb[e];
        }
      }
      if constexpr (!MAP) {
        *(float4*)&sh.Bn[row][n0] = make_float4(vb[0], vb[1], vb[2], vb[3]);
        *(float4*)&sh.C[row][n0] = make_float4(vc[0], vc[1], vc[2], vc[3]);
      }
    }
  }
};

// Four floats at p (16-byte aligned) as an array.
__device__ __forceinline__ void rd4(const float* p, float (&o)[4]) {
  const float4 v = *(const float4*)p;
  o[0] = v.x, o[1] = v.y, o[2] = v.z, o[3] = v.w;
}

// The adjoint carry's update ghat <- Pall ghat + C^T (Pf dy) for the lane's
// entries (k-step e takes rows 4e + g; on the 16-bit path when C is bf16).
template <typename TB, int MT>
__device__ __forceinline__ void carry_update(f4_t (&gh)[MT], const float (*Ct)[TP], float Pall, const float (&pfdy)[4],
                                             int j, int g) {
  if constexpr (__is_same(TB, bf16_t)) {
    uint32_t qh[2], qm[2], ql[2];
    split4_bf16(pfdy, qh, qm, ql);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float ct4[4];
      rd4(&Ct[16 * m + j][4 * g], ct4);
      uint32_t ac[2];
      pack4<TB>(ct4, ac);
      gh[m] *= Pall;
      gh[m] = mma_x3(ac, qh, qm, ql, gh[m]);
    }
  } else {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float ct4[4];
      rd4(&Ct[16 * m + j][4 * g], ct4);
      gh[m] *= Pall;
#pragma unroll
      for (int e = 0; e < 4; ++e) gh[m] = mma(ct4[e], pfdy[e], gh[m]);
    }
  }
}

__device__ __forceinline__ void wr4(float* p, float a0, float a1, float a2, float a3) {
  *(float4*)p = make_float4(a0, a1, a2, a3);
}

// The checkpointed state entering sub-block sb of batch row b for channel
// dcl, in the D layout: x[m][r] = entry 16m + 4g + r (clamped in bounds;
// the entries past N and the channels past D are zeroed where used, by
// ckpt_val, so that a load a sub-block ahead does not wait for its data).
template <int MT>
__device__ __forceinline__ void load_ckpt(f4_t (&x)[MT], const ScanArgs& a, int b, int sb, int64_t dcl, int g) {
  const int N = a.N;
  const float* ck = a.ckpt + ((int64_t)b * a.Kc + sb) * a.D * N;  // uniform
  const uint32_t co = (uint32_t)(dcl * N);
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const int n = 16 * m + 4 * g;
    if ((N & 3) == 0) {
      const float4 v = *(const float4*)(ck + (co + (uint32_t)(n < N ? n : N - 4)));
      x[m][0] = v.x, x[m][1] = v.y, x[m][2] = v.z, x[m][3] = v.w;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) x[m][r] = ck[co + (uint32_t)(n + r < N ? n + r : N - 1)];
    }
  }
}
// Entry 16m + 4g + r of a load_ckpt state, zero past N and for channels
// past D.
__device__ __forceinline__ float ckpt_val(const f4_t& xm, int r, int n, int N, bool dok) {
  return (dok && n + r < N) ? xm[r] : 0.f;
}

// Four values of the load layout (row rho, channels cq .. cq+3) from a
// [channel][row] tile into a [batch, T, D] stream of element type TT at
// (uniform) base p plus the 32-bit element offset o.
template <typename TT>
__device__ __forceinline__ void store_row4(void* p, uint32_t o, const float (*tl)[TP], int cq, int rho, bool vec,
                                           int nval) {
  typedef TT v4 __attribute__((ext_vector_type(4)));
  v4 x;
#pragma unroll
  for (int e = 0; e < 4; ++e) x[e] = (TT)tl[cq + e][rho];
  TT* q = (TT*)p;
  if (vec) {
    *(v4*)(q + o) = x;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (e < nval) q[o + e] = x[e];
  }
}

template <int NP, bool MAP, typename TU, typename TG, typename TB>
__global__ __launch_bounds__(64 * kMcWB) void mc_bwd_kernel(const ScanArgs a, int du_dt, int dg_dt) {
  constexpr int MT = NP / 16;
  constexpr int P = NP + 4;
  using In = McInB<NP, MAP, TU, TG, TB>;
  __shared__ __align__(16) McBwdLds<NP, MAP> sh;

  const int N = a.N;
  const int64_t T = a.T, D = a.D;
  const int tile = (int)(blockIdx.x % (uint32_t)a.n_tiles);
  const int seg = (int)(blockIdx.x / (uint32_t)a.n_tiles) + (MAP ? 1 : 0);
  const int b = tile / a.n_dtiles;
  const int dtile = tile - b * a.n_dtiles;
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int64_t dw = (int64_t)dtile * kMcDTB + 16 * wv;
  const int64_t d = dw + j;
  const bool dok = d < D;
  const int KS = (int)((T + Q - 1) / Q);
  const int sb0 = seg * a.seg_sc;
  const int sb1 = sb0 + a.seg_sc < KS ? sb0 + a.seg_sc : KS;
  const bool vec = dw + 16 <= D && D % 4 == 0;
  const int rho = lane >> 2, cq = (lane & 3) * 4;
  const int ncq = (int)(D - dw - cq < 4 ? (D - dw - cq < 0 ? 0 : D - dw - cq) : 4);  // valid of cq .. cq+3
  float Dv = (!MAP && dok) ? a.Dsk[d] : 0.f;
  asm volatile("" : "+v"(Dv));

  // adjoint carry in the D layout: gh[m][r] = entry 16m + 4g + r of channel j
  f4_t gh[MT];
  {
    const float* gin = (!MAP && a.nseg > 1) ? a.seg0 + ((int64_t)b * a.nseg + seg) * D * N : nullptr;
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = 16 * m + 4 * g + r;
        gh[m][r] = (gin && dok && n < N) ? gin[d * N + n] : 0.f;
      }
    // loaded before the loop, waited for here (as McIn::settle)
#pragma unroll
    for (int m = 0; m < MT; ++m) asm volatile("" : "+v"(gh[m]));
  }
  float Fseg = 1.f;
  float dDacc[4] = {0.f, 0.f, 0.f, 0.f};
  float sgf = 0.f, sgi = 0.f;  // dfl, dil summed over this lane's rows (channel j)

  float (*Tf)[TP] = sh.gate[wv][0];
  float (*Tdy)[TP] = sh.gate[wv][1];

  // inputs of sub-blocks sb (cur) and sb - 1 (nxt), loaded one sub-block
  // ahead and kept raw until staged (two sets: cur's registers are free
  // once staged, so nxt can take them without a copy)
  In cur, nxt;
  // the checkpointed state entering the current (xc) and the next (xn)
  // sub-block, loaded one sub-block ahead like the inputs
  f4_t xc[MAP ? 1 : MT], xn[MAP ? 1 : MT];
  if (sb0 < sb1) {
    cur.load(a, b, (int64_t)(sb1 - 1) * Q, dw, rho, cq, tid, vec);
    cur.settle();
    if constexpr (!MAP) {
      load_ckpt<MT>(xc, a, b, sb1 - 1, dok ? d : D - 1, g);
#pragma unroll
      for (int m = 0; m < MT; ++m) asm volatile("" : "+v"(xc[m]));
    }
  }
  for (int sb = sb1 - 1; sb >= sb0; --sb) {
    // The lane's indices, recomputed every sub-block from an opaque copy of
    // the lane id (they shadow the ones above): otherwise every
    // lane-dependent LDS and global address is hoisted out of the loop, and
    // holding them all costs more registers than recomputing them.
    int lane_l = lane;
    asm volatile("" : "+v"(lane_l));
    const int j = lane_l & 15, g = lane_l >> 4;
    const int rho = lane_l >> 2, cq = (lane_l & 3) * 4;
    const int arow = 4 * (j & 3) + (j >> 2);
    const int ncq = (int)(D - dw - cq < 4 ? (D - dw - cq < 0 ? 0 : D - dw - cq) : 4);
    const int64_t d = dw + j;
    const bool dok = d < D;
    const int64_t dcl = dok ? d : D - 1;
    const int tid = 64 * wv + lane_l;
    const int64_t t0 = (int64_t)sb * Q;
    // ---- stage B / C; gates in the load layout (each element once; rows
    // past T and channels past D are the neutral step f = 1, i = w = dy = 0)
    cur.stage(sh, a, t0, tid);
    const int rl = (int)(T - t0 < Q ? T - t0 : Q);  // rows left (uniform)
    const bool rok = rho < rl;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool ok = rok && e < ncq;
      // gates formed on every lane, then selected (no branch per element)
      float sf = sigm(cur.f.get(e));
      asm volatile("" : "+v"(sf));
      Tf[cq + e][rho] = ok ? sf : 1.f;
      Tdy[cq + e][rho] = ok ? cur.dy.get(e) : 0.f;
      if constexpr (!MAP) {
        float si = sigm(cur.i.get(e));
        asm volatile("" : "+v"(si));
        const float ig = ok ? si : 0.f;
        sh.gate[wv][3][cq + e][rho] = ig;
        sh.gate[wv][2][cq + e][rho] = ok ? ig * cur.u.get(e) : 0.f;
        dDacc[e] = fmaf(ok ? cur.dy.get(e) : 0.f, ok ? cur.u.get(e) : 0.f, dDacc[e]);
      }
    }
    __syncthreads();  // staging visible
    if (sb - 1 >= sb0) {
      nxt.load(a, b, t0 - Q, dw, rho, cq, tid, vec);
      if constexpr (!MAP) load_ckpt<MT>(xn, a, b, sb - 1, dcl, g);
    }
    asm volatile("" ::: "memory");

    // this lane's channel: gates and dy over all rows, decays of the own rows
    float fa[Q];
#pragma unroll
    for (int q4 = 0; q4 < Q; q4 += 4) {
      float f4[4];
      rd4(&Tf[j][q4], f4);
#pragma unroll
      for (int e = 0; e < 4; ++e) fa[q4 + e] = f4[e];
    }
    float pf[4], pe[4], dy_o[4], pfdy[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) dy_o[r] = Tdy[j][4 * r + g];
    const float Pall = own_decays(fa, g, pf, pe);
#pragma unroll
    for (int r = 0; r < 4; ++r) pfdy[r] = pf[r] * dy_o[r];

    if constexpr (!MAP) {
      float (*Tw)[TP] = sh.gate[wv][2];
      float (*Ti)[TP] = sh.gate[wv][3];
      float* pl = sh.pool[wv];
      float (*TGm)[TP] = (float (*)[TP])(pl + 0 * 16 * TP);  // G[s][t]
      float (*TGT)[TP] = (float (*)[TP])(pl + 1 * 16 * TP);  // G[s][t] at [t][s]
      float (*Tx1)[TP] = (float (*)[TP])(pl + 2 * 16 * TP);  // gathers, then row sums
      float (*Tx2)[TP] = (float (*)[TP])(pl + 3 * 16 * TP);
      // H in the pool's last two tiles, past the dC / dB partials (which take
      // its first 32 P floats) and the scratch tiles: other waves read it
      // after the partial-sum barrier
      constexpr int kPH = McBwdLds<NP, MAP>::POOL - 32 * TP;
      static_assert(32 * P <= kPH && 7 * 16 * TP <= kPH, "H tiles clear of the partials and scratch tiles");
      float (*TH)[TP] = (float (*)[TP])(pl + kPH);             // H[t][p(r)]
      float (*THT)[TP] = (float (*)[TP])(pl + kPH + 16 * TP);  // H[s][t] at [t][p(s)]
      // ---- G[t][s] = C_t . B_s in the layout of an A operand whose MFMA row
      // i is time row arow(i): Gp[r] = G[arow(j)][4r + g] (k-step (q, r')
      // takes n = 16q + 4k + r'); C X and B ghat for the own rows (MFMA row
      // 4g + r = time row 4r + g) and ghat . X per channel from the same reads
      f4_t Gp = {0.f, 0.f, 0.f, 0.f}, cx = {0.f, 0.f, 0.f, 0.f}, bg = {0.f, 0.f, 0.f, 0.f};
      float gX = 0.f;
      // (B and C exact in TB: G on the 16-bit path, two groups of n per
      // product, the even group's values packed until the odd one's)
      constexpr bool g16 = sizeof(TB) == 2 && NP >= 32;
      uint32_t pb[2], pc[2];
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        float c4[4], b4[4];
        rd4(&sh.C[arow][16 * m + 4 * g], c4);
        rd4(&sh.Bn[arow][16 * m + 4 * g], b4);
        constexpr bool bx = g16 && __is_same(TB, bf16_t);
        if constexpr (g16) {
          if (m & 1) {
            uint32_t qb[2], qc[2];
            pack4<TB>(b4, qb);
            pack4<TB>(c4, qc);
            Gp = mma_k32<TB>(pb, qb, pc, qc, Gp);
            if constexpr (bx) {
              // C X and B ghat over the pair of entry groups m - 1, m: X and
              // ghat split in three bf16 parts, three K = 32 products each
              float xe[4], xo[4], ge4[4], go4[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                xe[e] = ckpt_val(xc[m - 1], e, 16 * (m - 1) + 4 * g, N, dok);
                xo[e] = ckpt_val(xc[m], e, 16 * m + 4 * g, N, dok);
                ge4[e] = gh[m - 1][e];
                go4[e] = gh[m][e];
              }
              uint32_t h0[2], m0[2], l0[2], h1[2], m1[2], l1[2];
              split4_bf16(xe, h0, m0, l0);
              split4_bf16(xo, h1, m1, l1);
              cx = mma_k32<TB>(pc, qc, h0, h1, cx);
              cx = mma_k32<TB>(pc, qc, m0, m1, cx);
              cx = mma_k32<TB>(pc, qc, l0, l1, cx);
              split4_bf16(ge4, h0, m0, l0);
              split4_bf16(go4, h1, m1, l1);
              bg = mma_k32<TB>(pb, qb, h0, h1, bg);
              bg = mma_k32<TB>(pb, qb, m0, m1, bg);
              bg = mma_k32<TB>(pb, qb, l0, l1, bg);
            }
          } else {
            pack4<TB>(b4, pb);
            pack4<TB>(c4, pc);
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float xv = ckpt_val(xc[m], e, 16 * m + 4 * g, N, dok);
          if constexpr (!g16) Gp = mma(b4[e], c4[e], Gp);
          if constexpr (!bx) {
            cx = mma(c4[e], xv, cx);
            bg = mma(b4[e], gh[m][e], bg);
          }
          gX = fmaf(gh[m][e], xv, gX);
        }
      }
      gX += __shfl_xor(gX, 16, 64);
      gX += __shfl_xor(gX, 32, 64);
      // ---- the decay terms of the own rows t:
      //   V1_t = sum_{s>=t} P[s,t] dy_s G[s][t], V2_t = sum_{s>=t} P[s,t] dy_s (C X)_s,
      //   V3_t = sum_{r<=t} P[t,r] w_r (B ghat)_r,
      //   A3_t = sum_{s>=t>=r} M[s][r], M[s][r] = P[s,r] dy_s w_r G[s][r],
      // and H[s][r] = sum over the wave's channels of P[s,r] dy_s w_r.
      float V1[4], V2[4], V3[4], A3[4];
      if (__all(Pall >= kMcRatioMin)) {
        // Every channel's decay over the sub-block stays above kMcRatioMin:
        // P[s,t] = Pf[s] / Pf[t] in floating point, with a = Pf dy and
        // b = w / Pf, and every term is a 16 x 16 x 16 product (MFMA row i =
        // time row arow(i), k-step e = row 4e + g, whose a and b this lane
        // holds): V1 = (masked G^T a) / Pf, V2 = (masked ones (a C X)) / Pf,
        // V3 = Pf (masked ones (b B ghat)), rowsum = a (masked G b),
        // colsum = b (masked G^T a), A3 = suffix sums of rowsum minus strict
        // suffix sums of colsum; H = a^T b over the channels (k = channel).
        float ip[4], ra[4], rb[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          ip[r] = __builtin_amdgcn_rcpf(pf[r]);
          ra[r] = pf[r] * dy_o[r];
          rb[r] = Tw[j][4 * r + g] * ip[r];
        }
        float (*TGs)[TP] = TGm;  // G[t][s]
        float (*Ta)[TP] = TGT;   // a as [channel][row]
        float (*Tb)[TP] = Tx1;   // b as [channel][row]
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          TGs[arow][4 * r + g] = Gp[r];
          Ta[j][4 * r + g] = ra[r];
          Tb[j][4 * r + g] = rb[r];
        }
        asm volatile("" ::: "memory");
        f4_t D1 = {0.f, 0.f, 0.f, 0.f}, D2 = D1, D3 = D1, R1 = D1, DH = D1, D4 = D1;
        // the 0 / 1 masks are exact in bf16: the masked sums take the 16-bit
        // path with the float32 operand split (mask_pk: four masks packed)
        const auto mask_pk = [](bool m0, bool m1, bool m2, bool m3, uint32_t (&w)[2]) {
          w[0] = (m0 ? 0x3f80u : 0u) | (m1 ? 0x3f800000u : 0u);
          w[1] = (m2 ? 0x3f80u : 0u) | (m3 ? 0x3f800000u : 0u);
        };
        float v2[4], v3[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int s = 4 * e + g;
          const bool ge = s >= arow, le = s <= arow;
          D1 = mma(ge ? TGs[s][arow] : 0.f, ra[e], D1);
          v2[e] = ra[e] * cx[e];
          v3[e] = rb[e] * bg[e];
          R1 = mma(le ? Gp[e] : 0.f, rb[e], R1);
          DH = mma(Ta[s][j], Tb[s][j], DH);
        }
        uint32_t mge[2], mle[2], mgt[2];
        mask_pk(g >= arow, 4 + g >= arow, 8 + g >= arow, 12 + g >= arow, mge);
        mask_pk(g <= arow, 4 + g <= arow, 8 + g <= arow, 12 + g <= arow, mle);
        mask_pk(g > arow, 4 + g > arow, 8 + g > arow, 12 + g > arow, mgt);
        {
          uint32_t h[2], md[2], lo[2];
          split4_bf16(v2, h, md, lo);
          D2 = mma_x3(mge, h, md, lo, D2);
          split4_bf16(v3, h, md, lo);
          D3 = mma_x3(mle, h, md, lo, D3);
        }
        {
          float v4[4], v5[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v4[e] = ra[e] * R1[e], v5[e] = -(rb[e] * D1[e]);
          uint32_t h4[2], m4[2], l4[2], h5[2], m5[2], l5[2];
          split4_bf16(v4, h4, m4, l4);
          split4_bf16(v5, h5, m5, l5);
          D4 = mma_k32<bf16_t>(mge, mgt, h4, h5, D4);
          D4 = mma_k32<bf16_t>(mge, mgt, m4, m5, D4);
          D4 = mma_k32<bf16_t>(mge, mgt, l4, l5, D4);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          V1[r] = D1[r] * ip[r];
          V2[r] = D2[r] * ip[r];
          V3[r] = D3[r] * pf[r];
          A3[r] = D4[r];
          // lane (j, g) holds H[4g + r][j], zero for j > 4g + r
          const float h = j <= 4 * g + r ? DH[r] : 0.f;
          TH[4 * g + r][4 * (j & 3) + (j >> 2)] = h;
          THT[j][4 * r + g] = h;
        }
      } else {
        // exact products: G as [t][s] and [s][t] tiles, Horner chains and a
        // butterfly over the channels
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          TGm[arow][4 * r + g] = Gp[r];
          TGT[4 * r + g][arow] = Gp[r];
        }
        // ---- V1 = sum_{s>=t} P[s,t] dy_s G[s][t], V2 = sum_{s>=t} P[s,t] dy_s (C X)_s
        // (Horner from s = 15 down), V3 = sum_{r<=t} P[t,r] w_r (B ghat)_r
#pragma unroll
        for (int r = 0; r < 4; ++r) Tx1[j][4 * r + g] = cx[r], Tx2[j][4 * r + g] = bg[r];
        asm volatile("" ::: "memory");
        // (operands are read from the tiles in 4-row chunks as they are needed,
        // which keeps the live registers low)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 4 * r + g;
          float a1 = 0.f, a2 = 0.f;
#pragma unroll
          for (int s4 = 12; s4 >= 4 * r; s4 -= 4) {
            float gt4[4], y4[4], c4[4];
            rd4(&TGT[t][s4], gt4);
            rd4(&Tdy[j][s4], y4);
            rd4(&Tx1[j][s4], c4);
#pragma unroll
            for (int e = 3; e >= 0; --e) {
              const int s = s4 + e;
              const float fs = s < Q - 1 ? fa[s + 1] : 1.f;
              if (s >= 4 * r + 3) {
                a1 = fmaf(a1, fs, y4[e] * gt4[e]);
                a2 = fmaf(a2, fs, y4[e] * c4[e]);
              } else {
                const bool in = s >= t;
                a1 = in ? fmaf(a1, fs, y4[e] * gt4[e]) : a1;
                a2 = in ? fmaf(a2, fs, y4[e] * c4[e]) : a2;
              }
            }
          }
          V1[r] = a1;
          V2[r] = a2;
          float a3 = 0.f;
#pragma unroll
          for (int q4 = 0; q4 <= 4 * r; q4 += 4) {
            float w4[4], b4[4];
            rd4(&Tw[j][q4], w4);
            rd4(&Tx2[j][q4], b4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int q = q4 + e;
              if (q <= 4 * r) {
                a3 = fmaf(a3, fa[q], w4[e] * b4[e]);
              } else {
                const bool in = q <= t;
                a3 = fmaf(a3, in ? fa[q] : 1.f, in ? w4[e] * b4[e] : 0.f);
              }
            }
          }
          V3[r] = a3;
        }
        // ---- rectangle sums A3_t = sum_{s>=t>=r} M[s][r] with M = K G[s][r],
        // K[s][r] = P[s,r] dy_s w_r; per row block r the K of the own row
        // s = 4r + g (16 slots, q <= 4r + 3) are summed over the wave's 16
        // channels by a transposing butterfly in each 16-lane row, after which
        // lane j holds slot q = j: H[s][j]
        float cp[Q], rs[4];
#pragma unroll
        for (int q = 0; q < Q; ++q) cp[q] = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int s = 4 * r + g;
          float hv[Q];
          float Pz = 0.f, rsum = 0.f;
#pragma unroll
          for (int q4 = 4 * r; q4 >= 0; q4 -= 4) {
            float w4[4], g4[4];
            rd4(&Tw[j][q4], w4);
            rd4(&TGm[s][q4], g4);
#pragma unroll
            for (int e = 3; e >= 0; --e) {
              const int q = q4 + e;
              // Pz = P[s, q] = prod_{q < q' <= s} f for q <= s, 0 for q > s
              // (a product chain with no masked multiply, so that it stays
              // straight-line code)
              if (q == 4 * r + 3) {
                Pz = q == s ? 1.f : 0.f;
              } else if (q >= 4 * r) {
                Pz = q == s ? 1.f : Pz * fa[q + 1];
              } else {
                Pz = Pz * fa[q + 1];
              }
              const float kv = Pz * (dy_o[r] * w4[e]);
              hv[q] = kv;
              const float mv = kv * g4[e];
              rsum += mv;
              cp[q] += mv;
            }
          }
#pragma unroll
          for (int q = 4 * r + 4; q < Q; ++q) hv[q] = 0.f;
          rs[r] = rsum;
          trd_step<16, Q, Q>(hv, lane);
          // lane j: H[s][j] (zero for j > s: every slot past s held zeros);
          // over r and the lanes every entry of both tiles is written
          TH[s][4 * (j & 3) + (j >> 2)] = hv[0];
          THT[j][4 * (s & 3) + (s >> 2)] = hv[0];
        }
        // row sums of all 16 rows, and column sums over the channel's lanes
        // (group g's partials in pool tile 4 + g for g < 3, tile 3 for g = 3)
#pragma unroll
        for (int r = 0; r < 4; ++r) Tx1[j][4 * r + g] = rs[r];
        {
          float* tc = pl + (g < 3 ? 4 + g : 3) * 16 * TP;
#pragma unroll
          for (int q4 = 0; q4 < Q; q4 += 4) wr4(tc + j * TP + q4, cp[q4], cp[q4 + 1], cp[q4 + 2], cp[q4 + 3]);
        }
        asm volatile("" ::: "memory");
        // A3_t = sum_{s>=t} rowsum[s] - sum_{q>t} colsum[q]
        {
          float sufR = 0.f, sufC = 0.f;
#pragma unroll
          for (int r = 3; r >= 0; --r) {
            float r4[4], c0[4], c1[4], c2[4], c3[4], cs[4];
            rd4(&Tx1[j][4 * r], r4);
            rd4(pl + 4 * 16 * TP + j * TP + 4 * r, c0);
            rd4(pl + 5 * 16 * TP + j * TP + 4 * r, c1);
            rd4(pl + 6 * 16 * TP + j * TP + 4 * r, c2);
            rd4(pl + 3 * 16 * TP + j * TP + 4 * r, c3);
#pragma unroll
            for (int e = 0; e < 4; ++e) cs[e] = (c0[e] + c1[e]) + (c2[e] + c3[e]);
            const float sR = sufR + r4[3] + (g <= 2 ? r4[2] : 0.f) + (g <= 1 ? r4[1] : 0.f) + (g <= 0 ? r4[0] : 0.f);
            const float sC = sufC + (g < 3 ? cs[3] : 0.f) + (g < 2 ? cs[2] : 0.f) + (g < 1 ? cs[1] : 0.f);
            A3[r] = sR - sC;
            sufR += (r4[0] + r4[1]) + (r4[2] + r4[3]);
            sufC += (cs[0] + cs[1]) + (cs[2] + cs[3]);
          }
        }
      }
      // ---- outputs of the own rows into the gate tiles (dfl over f, du over
      // i, dil over w), stored in the load layout
      float q1[4], q2[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float f_o = Tf[j][4 * r + g], i_o = Ti[j][4 * r + g], w_o = Tw[j][4 * r + g];
        const float dws = fmaf(pe[r], bg[r], V1[r]);
        const float xx = fmaf(pf[r], V2[r], A3[r]) + pe[r] * fmaf(pf[r], gX, V3[r]);
        const float dfl = f_o == 0.f ? 0.f : (1.f - f_o) * fmaf(-w_o, dws, xx);
        const float du = fmaf(i_o, dws, Dv * dy_o[r]);
        const float dil = (1.f - i_o) * (dws * w_o);
        q1[r] = pfdy[r];
        q2[r] = w_o * pe[r];
        sgf += dfl;
        sgi += dil;
        Tf[j][4 * r + g] = dfl;
        Ti[j][4 * r + g] = du;
        Tw[j][4 * r + g] = dil;
      }
      asm volatile("" ::: "memory");
      // the next sub-block's loads are waited for here, before this
      // sub-block's stores are issued: waiting for them after the stores
      // (at the end of the sub-block) would wait for the stores as well
      if (sb - 1 >= sb0) {
        nxt.settle();
#pragma unroll
        for (int m = 0; m < MT; ++m) asm volatile("" : "+v"(xn[m]));
      }
      if (rok && ncq > 0) {
        const int64_t ob = ((int64_t)b * T + t0) * D;  // uniform
        const uint32_t o = (uint32_t)(rho * D + dw + cq);
        void* du_p = a.du ? (char*)a.du + ob * (du_dt == NAJU_DTYPE_F32 ? 4 : 2) : nullptr;
        // dfl, dil: rows a.ldg elements apart, in dg_dt
        const int64_t obg = ((int64_t)b * T + t0) * a.ldg;  // uniform
        const uint32_t og = (uint32_t)(rho * a.ldg + dw + cq);
        const int gsz = dg_dt == NAJU_DTYPE_F32 ? 4 : 2;
        void* dfl_p = a.dfl ? (char*)a.dfl + obg * gsz : nullptr;
        void* dil_p = a.dil ? (char*)a.dil + obg * gsz : nullptr;
        if (du_p) {
          if (du_dt == NAJU_DTYPE_F32) store_row4<float>(du_p, o, Ti, cq, rho, vec, ncq);
          else store_row4<TU>(du_p, o, Ti, cq, rho, vec, ncq);
        }
        if (dg_dt == NAJU_DTYPE_F32) {
          if (dfl_p) store_row4<float>(dfl_p, og, Tf, cq, rho, vec, ncq);
          if (dil_p) store_row4<float>(dil_p, og, Tw, cq, rho, vec, ncq);
        } else if (dg_dt == NAJU_DTYPE_BF16) {
          if (dfl_p) store_row4<bf16_t>(dfl_p, og, Tf, cq, rho, vec, ncq);
          if (dil_p) store_row4<bf16_t>(dil_p, og, Tw, cq, rho, vec, ncq);
        } else {
          if (dfl_p) store_row4<f16_t>(dfl_p, og, Tf, cq, rho, vec, ncq);
          if (dil_p) store_row4<f16_t>(dil_p, og, Tw, cq, rho, vec, ncq);
        }
      }
      // ---- dC^T [n][t] and dB^T [n][t] per 16-entry tile of n (channel part:
      // K = channel 4g + kk; H part: K = row 4kk + g). The MFMA A operands X
      // and ghat (entering this sub-block) per channel and entry come through
      // this wave's pool as [16 channels][P] tiles, written in the D layout
      // and read transposed.
      // (tiles 0 and 1: the decay phase is done with them)
      float (*TQ1)[TP] = (float (*)[TP])(pl + 0 * 16 * TP);  // (dy Pf)[t][d]
      float (*TQ2)[TP] = (float (*)[TP])(pl + 1 * 16 * TP);  // (w Pe)[t][d]
#pragma unroll
      for (int r = 0; r < 4; ++r) TQ1[4 * r + g][j] = q1[r], TQ2[4 * r + g][j] = q2[r];
      asm volatile("" ::: "memory");
      float qv1[4], qv2[4];
      rd4(&TQ1[j][4 * g], qv1);
      rd4(&TQ2[j][4 * g], qv2);
      asm volatile("" ::: "memory");
      float* TX = pl;           // X [channel][n]
      float* TGh = pl + 16 * P;  // ghat [channel][n]
      {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const int n = 16 * m + 4 * g;
          wr4(TX + j * P + n, ckpt_val(xc[m], 0, n, N, dok), ckpt_val(xc[m], 1, n, N, dok),
              ckpt_val(xc[m], 2, n, N, dok), ckpt_val(xc[m], 3, n, N, dok));
          wr4(TGh + j * P + n, gh[m][0], gh[m][1], gh[m][2], gh[m][3]);
        }
      }
      asm volatile("" ::: "memory");
      // the wave's channel part: X^T (dy Pf) and ghat^T (w Pe) over its 16
      // channels (the H part, B^T H and C^T H^T, is formed once per
      // workgroup from the waves' summed H after the partial-sum barrier)
      f4_t dCt[MT], dBt[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        f4_t accC = {0.f, 0.f, 0.f, 0.f}, accB = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          accC = mma(TX[(4 * g + e) * P + 16 * m + j], qv1[e], accC);
          accB = mma(TGh[(4 * g + e) * P + 16 * m + j], qv2[e], accB);
        }
        dCt[m] = accC;
        dBt[m] = accB;
      }
      // ---- carry update: ghat <- Pall ghat + C^T (Pf dy)
      carry_update<TB, MT>(gh, sh.Ct, Pall, pfdy, j, g);
      // ---- the wave's dC / dB [t][n] into its pool (its reads of the pool
      // are done; other waves read it after the barrier), then the workgroup
      // adds the waves' in wave order
      asm volatile("" ::: "memory");
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        wr4(pl + (0 * 16 + j) * P + 16 * m + 4 * g, dCt[m][0], dCt[m][1], dCt[m][2], dCt[m][3]);
        wr4(pl + (1 * 16 + j) * P + 16 * m + 4 * g, dBt[m][0], dBt[m][1], dBt[m][2], dBt[m][3]);
      }
      __syncthreads();
      static_assert(2 * MT <= kMcWB, "one output tile per wave");
      if (wv < 2 * MT) {
        // wave w forms output tile w: dC (qd = 0) or dB (qd = 1) for entries
        // n = 16m .. 16m+15 and the sub-block's 16 rows, in the MFMA output
        // layout (lane (j, g) holds n = 16m + 4g + r of row t = j): the
        // waves' channel parts summed in wave order, plus B^T (sum H) or
        // C^T (sum H)^T with H summed over the waves in wave order
        const int qd = wv / MT, m = wv - qd * MT;
        float hs[4] = {0.f, 0.f, 0.f, 0.f}, acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < kMcWB; ++w) {
          const float* pw = sh.pool[w];
          float h4[4], v4[4];
          rd4(pw + kPH + qd * 16 * TP + j * TP + 4 * g, h4);
          rd4(pw + (qd * 16 + j) * P + 16 * m + 4 * g, v4);
#pragma unroll
          for (int e = 0; e < 4; ++e) hs[e] += h4[e], acc[e] += v4[e];
        }
        float a4[4];
        rd4(qd == 0 ? &sh.Bt[16 * m + j][4 * g] : &sh.Ct[16 * m + j][4 * g], a4);
        f4_t hp = {0.f, 0.f, 0.f, 0.f};
        if constexpr (__is_same(TB, bf16_t)) {
          uint32_t ab[2], hh[2], hm[2], hl[2];
          pack4<TB>(a4, ab);
          split4_bf16(hs, hh, hm, hl);
          hp = mma_x3(ab, hh, hm, hl, hp);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) hp = mma(a4[e], hs[e], hp);
        }
        float* dst = qd == 0 ? a.partC : a.partB;
        const int n = 16 * m + 4 * g;
        if (dst && t0 + j < T && n < N) {
          const int64_t btn = (int64_t)a.batch * T * N;
          float* q = dst + (int64_t)dtile * btn + ((int64_t)b * T + t0) * N;  // uniform
          const uint32_t o = (uint32_t)(j * N + n);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] += hp[r];
          if ((N & 3) == 0) {
            *(float4*)(q + o) = make_float4(acc[0], acc[1], acc[2], acc[3]);
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (n + r < N) q[o + r] = acc[r];
          }
        }
      }
    } else {
      // MAP: the adjoint map of the segment (ghat from zero, decay product)
      Fseg *= Pall;
      carry_update<TB, MT>(gh, sh.Ct, Pall, pfdy, j, g);
    }
    // every wave is done with the staged B / C (and, in the scan, with the
    // pools and H tiles its output tile reads) before they are restaged
    __syncthreads();
    cur = nxt;
    if constexpr (!MAP) {
#pragma unroll
      for (int m = 0; m < MT; ++m) xc[m] = xn[m];
    }
  }
  if constexpr (MAP) {
    if (!dok) return;
    const int64_t o = ((int64_t)b * a.nseg + seg) * D + d;
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = 16 * m + 4 * g + r;
        if (n < N) a.segZ[o * N + n] = gh[m][r];
      }
    if (g == 0) a.segF[o] = Fseg;
  } else {
    if (a.dh0 && seg == 0 && dok) {
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int n = 16 * m + 4 * g + r;
          if (n < N) a.dh0[((int64_t)b * D + d) * N + n] = gh[m][r];
        }
    }
    // dD of the segment: lanes with the same cq hold the same four channels
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v = dDacc[e];
      v += __shfl_xor(v, 4, 64);
      v += __shfl_xor(v, 8, 64);
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      dDacc[e] = v;
    }
    if (a.partD && rho == 0) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (e < ncq) a.partD[((int64_t)b * a.nseg + seg) * D + dw + cq + e] = dDacc[e];
    }
    // the gate gradients' sums of the segment: channel j's four lane groups
    // added (groups 0 + 1, 2 + 3, then the pairs)
    if (a.partG) {
      sgf += __shfl_xor(sgf, 16, 64);
      sgi += __shfl_xor(sgi, 16, 64);
      sgf += __shfl_xor(sgf, 32, 64);
      sgi += __shfl_xor(sgi, 32, 64);
      if (g == 0 && dok) {
        const int64_t o = ((int64_t)b * a.nseg + seg) * D + d;
        a.partG[o] = sgf;
        a.partG[(int64_t)a.batch * a.nseg * D + o] = sgi;
      }
    }
  }
}

int np16(int64_t N) { return N <= 16 ? 16 : (N <= 32 ? 32 : 64); }

}  // namespace

typedef void (*mc_fwd_t)(ScanArgs, int);

template <typename TU, typename TG, typename TB>
mc_fwd_t pick_fwd_np(int np, bool map) {
  switch (np) {
    case 16: return map ? mc_fwd_kernel<16, true, TU, TG, TB> : mc_fwd_kernel<16, false, TU, TG, TB>;
    case 32: return map ? mc_fwd_kernel<32, true, TU, TG, TB> : mc_fwd_kernel<32, false, TU, TG, TB>;
    default: return map ? mc_fwd_kernel<64, true, TU, TG, TB> : mc_fwd_kernel<64, false, TU, TG, TB>;
  }
}

// The served dtype combinations (u; gates f32 or u's; B/C f32 or u's).
template <typename TU>
mc_fwd_t pick_fwd_u(int g_dt, int bc_dt, int np, bool map) {
  const bool gf = g_dt == NAJU_DTYPE_F32, bf = bc_dt == NAJU_DTYPE_F32;
  if (gf) return bf ? pick_fwd_np<TU, float, float>(np, map) : pick_fwd_np<TU, float, TU>(np, map);
  return bf ? pick_fwd_np<TU, TU, float>(np, map) : pick_fwd_np<TU, TU, TU>(np, map);
}

typedef void (*mc_bwd_t)(ScanArgs, int, int);

template <typename TU, typename TG, typename TB>
mc_bwd_t pick_bwd_np(int np, bool map) {
  switch (np) {
    case 16: return map ? mc_bwd_kernel<16, true, TU, TG, TB> : mc_bwd_kernel<16, false, TU, TG, TB>;
    case 32: return map ? mc_bwd_kernel<32, true, TU, TG, TB> : mc_bwd_kernel<32, false, TU, TG, TB>;
    default: return map ? mc_bwd_kernel<64, true, TU, TG, TB> : mc_bwd_kernel<64, false, TU, TG, TB>;
  }
}

template <typename TU>
mc_bwd_t pick_bwd_u(int g_dt, int bc_dt, int np, bool map) {
  const bool gf = g_dt == NAJU_DTYPE_F32, bf = bc_dt == NAJU_DTYPE_F32;
  if (gf) return bf ? pick_bwd_np<TU, float, float>(np, map) : pick_bwd_np<TU, float, TU>(np, map);
  return bf ? pick_bwd_np<TU, TU, float>(np, map) : pick_bwd_np<TU, TU, TU>(np, map);
}

hipError_t mc_fwd_launch(const ScanArgs& a, bool map, int x_dt, int g_dt, int y_dt, hipStream_t st) {
  const int segs = map ? a.nseg - 1 : a.nseg;
  const unsigned grid = (unsigned)((int64_t)a.n_tiles * segs);
  if (grid == 0) return hipSuccess;
  const int np = np16(a.N);
  mc_fwd_t k = x_dt == NAJU_DTYPE_F32    ? pick_fwd_np<float, float, float>(np, map)
               : x_dt == NAJU_DTYPE_BF16 ? pick_fwd_u<bf16_t>(g_dt, a.bc_dt, np, map)
                                         : pick_fwd_u<f16_t>(g_dt, a.bc_dt, np, map);
  hipLaunchKernelGGL(k, dim3(grid), dim3(64 * kMcW), 0, st, a, y_dt);
  return hipGetLastError();
}

hipError_t mc_bwd_launch(const ScanArgs& a, bool map, int x_dt, int g_dt, int du_dt, int dg_dt, hipStream_t st) {
  const int segs = map ? a.nseg - 1 : a.nseg;
  const unsigned grid = (unsigned)((int64_t)a.n_tiles * segs);
  if (grid == 0) return hipSuccess;
  const int np = np16(a.N);
  mc_bwd_t k = x_dt == NAJU_DTYPE_F32    ? pick_bwd_np<float, float, float>(np, map)
               : x_dt == NAJU_DTYPE_BF16 ? pick_bwd_u<bf16_t>(g_dt, a.bc_dt, np, map)
                                         : pick_bwd_u<f16_t>(g_dt, a.bc_dt, np, map);
  hipLaunchKernelGGL(k, dim3(grid), dim3(64 * kMcWB), 0, st, a, du_dt, dg_dt);
  return hipGetLastError();
}

}  // namespace naju_detail
