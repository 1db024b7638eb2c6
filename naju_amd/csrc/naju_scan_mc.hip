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
  float f[4], i[4], u[4], b[4], c[MAP ? 1 : 4];

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
      ld4v<TG, true>((const TG*)a.fl + base, o, f);
      ld4v<TG, true>((const TG*)a.il + base, o, i);
      ld4v<TU, true>((const TU*)a.u + base, o, u);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t dd = dw + cq + e < D ? dw + cq + e : D - 1;
        const uint32_t o = off + (uint32_t)dd;
        f[e] = to_f32(((const TG*)a.fl + base)[o]);
        i[e] = to_f32(((const TG*)a.il + base)[o]);
        u[e] = to_f32(((const TU*)a.u + base)[o]);
      }
    }
    if (tid < 4 * NP) {
      const int N = a.N;
      const int row = (4 * tid) / NP, n0 = (4 * tid) % NP;
      const int64_t bb = ((int64_t)b_row * T + t0) * N;  // (t0, 0), uniform
      const uint32_t ro = (uint32_t)((row < rows ? row : rows - 1) * N);
      if (N == NP) {
        ld4v<TB, true>((const TB*)a.Bm + bb, ro + n0, b);
        if constexpr (!MAP) ld4v<TB, true>((const TB*)a.Cm + bb, ro + n0, c);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t o = ro + (uint32_t)(n0 + e < N ? n0 + e : N - 1);
          b[e] = to_f32(((const TB*)a.Bm + bb)[o]);
          if constexpr (!MAP) c[e] = to_f32(((const TB*)a.Cm + bb)[o]);
        }
      }
    }
  }

  // B (and C) into LDS buffer buf; zeros past T and past N
  __device__ __forceinline__ void stage(McBC<NP, MAP>& sh, int buf, const ScanArgs& a, int64_t t0, int tid) const {
    if (tid < 4 * NP) {
      const int row = (4 * tid) / NP, n0 = (4 * tid) % NP;
      const bool rok = t0 + row < a.T;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool ok = rok && n0 + e < a.N;
        const float vb = ok ? b[e] : 0.f;
        sh.Bt[buf][n0 + e][4 * (row & 3) + (row >> 2)] = vb;
        if constexpr (!MAP) {
          sh.Bn[buf][row][n0 + e] = vb;
          sh.C[buf][row][n0 + e] = ok ? c[e] : 0.f;
        }
      }
    }
  }
};

// ------------------------------------------------------------------ forward
//
// One workgroup per (batch row, kMcDT channels, time segment); the segment's
// sub-blocks are walked in order, the inputs of sub-block sb + 1 loaded while
// sb is computed, B and C double-buffered in LDS (one barrier per
// sub-block). MAP: the segment's map from a zero state (decay per channel
// into segF, state into segZ) for the carry pass over the segments; otherwise
// y, the checkpoint and hT from the entering state (h0, or seg0 when T is
// split into segments).
template <int NP, bool MAP, typename TU, typename TG, typename TB>
__global__ __launch_bounds__(64 * kMcW) void mc_fwd_kernel(const ScanArgs a, int y_dt) {
  constexpr int MT = NP / 16;  // 16-entry tiles of the state index
  using In = McIn<NP, MAP, TU, TG, TB>;
  __shared__ __align__(16) McBC<NP, MAP> sh;
  __shared__ __align__(16) float s_t[kMcW][3][16][TP];  // per wave: f, w, u (then y) as [channel][row]
  __shared__ __align__(16) float s_G[MAP ? 1 : kMcW][Q][Q + 4];  // per wave: G = C B^T

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
    const float* xin = MAP ? nullptr
                           : (a.nseg > 1 ? a.seg0 + ((int64_t)b * a.nseg + seg) * D * N
                                         : (a.h0 ? a.h0 + (int64_t)b * D * N : nullptr));
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = 16 * m + 4 * g + r;
        X[m][r] = (xin && dok && n < N) ? xin[d * N + n] : 0.f;
      }
  }
  float Fseg = 1.f;
  const float Dv = (!MAP && dok) ? a.Dsk[d] : 0.f;
  // load role: row rho, channels cq .. cq+3 of the wave's 16
  const int rho = lane >> 2, cq = (lane & 3) * 4;
  // A-operand row of C X: MFMA row i = lane % 16 holds time row 4(i%4) + i/4
  const int arow = 4 * (j & 3) + (j >> 2);

  In cur, nxt;
  if (sb0 < sb1) {
    cur.load(a, b, (int64_t)sb0 * Q, dw, rho, cq, tid, vec);
    cur.stage(sh, 0, a, (int64_t)sb0 * Q, tid);
  }
  for (int sb = sb0; sb < sb1; ++sb) {
    const int buf = (sb - sb0) & 1;
    const int64_t t0 = (int64_t)sb * Q;
    if (sb + 1 < sb1) nxt.load(a, b, t0 + Q, dw, rho, cq, tid, vec);
    // gates in the load layout, each element computed once; rows past T
    // and channels past D are the neutral step f = 1, w = u = 0
    const bool rok = t0 + rho < T;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool ok = rok && dw + cq + e < D;
      s_t[wv][0][cq + e][rho] = ok ? sigm(cur.f[e]) : 1.f;
      s_t[wv][1][cq + e][rho] = ok ? sigm(cur.i[e]) * cur.u[e] : 0.f;
      s_t[wv][2][cq + e][rho] = ok ? cur.u[e] : 0.f;
    }
    __syncthreads();  // B / C of sb are staged; every wave is done with sb - 1
    if (sb + 1 < sb1) nxt.stage(sh, buf ^ 1, a, t0 + Q, tid);  // the other buffer is free now
    if constexpr (!MAP) {
      // G = C B^T of the sub-block, G[t][s] = sum_n C[t][n] B[s][n] (k-step
      // (q, r') takes n = 16q + 4k + r'), into this wave's LDS tile
      f4_t G = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < NP / 16; ++q) {
        const float4 c4 = *(const float4*)&sh.C[buf][j][16 * q + 4 * g];
        const float4 b4 = *(const float4*)&sh.Bn[buf][j][16 * q + 4 * g];
        G = mma(c4.x, b4.x, G);
        G = mma(c4.y, b4.y, G);
        G = mma(c4.z, b4.z, G);
        G = mma(c4.w, b4.w, G);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) s_G[wv][4 * g + r][j] = G[r];
    }
    // (the wave reads back what its own lanes wrote: LDS keeps a wave's
    // accesses in order, the compiler must not move them)
    asm volatile("" ::: "memory");
    // this lane's channel over all Q rows, and its own rows 4r + g
    float fa[Q], wa[Q];
#pragma unroll
    for (int q4 = 0; q4 < Q; q4 += 4) {
      const float4 f4 = *(const float4*)&s_t[wv][0][j][q4];
      const float4 w4 = *(const float4*)&s_t[wv][1][j][q4];
      fa[q4] = f4.x, fa[q4 + 1] = f4.y, fa[q4 + 2] = f4.z, fa[q4 + 3] = f4.w;
      wa[q4] = w4.x, wa[q4 + 1] = w4.y, wa[q4 + 2] = w4.z, wa[q4 + 3] = w4.w;
    }
    float w_o[4], u_o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      w_o[r] = s_t[wv][1][j][4 * r + g];
      u_o[r] = s_t[wv][2][j][4 * r + g];
    }
    // decays of the own rows: pf = prod_{q <= t} f, pe = prod_{q > t} f
    float pf[4], pe[4];
    const float Pall = own_decays(fa, g, pf, pe);

    if constexpr (!MAP) {
      // intra-sub-block part of y for the own rows t = 4r + g:
      // S_k = f_k S_{k-1} + G[t][k] w_k for k = 0 .. t (Horner); rows k <= 4r
      // are in every lane's range, rows 4r+1 .. 4r+3 only in some
      float S[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 4 * r + g;
        float acc = 0.f;
#pragma unroll
        for (int s4 = 0; s4 <= 4 * r; s4 += 4) {
          const float4 G4 = *(const float4*)&s_G[wv][t][s4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int s = s4 + e;
            if (s <= 4 * r) {
              acc = fmaf(acc, fa[s], (&G4.x)[e] * wa[s]);
            } else {
              const bool in = s <= t;
              acc = fmaf(acc, in ? fa[s] : 1.f, in ? (&G4.x)[e] * wa[s] : 0.f);
            }
          }
        }
        S[r] = acc;
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
      // the state entering this sub-block is the backward's checkpoint
      if (a.ckpt && dok && sb % ck_sb == 0) {
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
      // y of the own rows into the u tile, then stored in the load layout
      // (row rho, channels cq .. cq+3)
#pragma unroll
      for (int r = 0; r < 4; ++r) s_t[wv][2][j][4 * r + g] = fmaf(pf[r], cx[r], fmaf(Dv, u_o[r], S[r]));
      asm volatile("" ::: "memory");
      if (rok) {
        float yv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) yv[e] = s_t[wv][2][cq + e][rho];
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
    }
    // X <- Pall X + B^T (Pe w): k-step s takes rows 4s + k
    float wp[4];
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) wp[s2] = pe[s2] * w_o[s2];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      X[m] *= Pall;
      const float4 bt = *(const float4*)&sh.Bt[buf][16 * m + j][4 * g];
      X[m] = mma(bt.x, wp[0], X[m]);
      X[m] = mma(bt.y, wp[1], X[m]);
      X[m] = mma(bt.z, wp[2], X[m]);
      X[m] = mma(bt.w, wp[3], X[m]);
    }
    cur = nxt;
  }
  if (!dok) return;
  if (MAP) {
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
  (void)a, (void)map, (void)x_dt, (void)g_dt, (void)du_dt, (void)dg_dt, (void)st;
  return hipErrorNotSupported;
}

}  // namespace naju_detail
