// na_mfma.h — shared pieces of the matrix-core (gfx950 MFMA) kernels:
// operand traits and layouts, tile decoding, key/query boxes, chunk
// walking and masks, and the host-side tile choice.  See na_mfma.hip for
// the tiling scheme.
#pragma once

#include <cmath>
#include <cstdlib>

#include "na_common.h"
#include "na_launch.h"

namespace na {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename T>
struct Mf;
template <>
struct Mf<bf16_t> {
  typedef __bf16 e;
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  typedef __bf16 v4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mf<f16_t> {
  typedef _Float16 e;
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  typedef _Float16 v4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <typename T>
__device__ __forceinline__ typename Mf<T>::v8 ld8(const T *p) {
  return *reinterpret_cast<const typename Mf<T>::v8 *>(p);
}

template <typename T>
__device__ __forceinline__ typename Mf<T>::v8 zero8() {
  typename Mf<T>::v8 z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = (typename Mf<T>::e)0.f;
  return z;
}

// B operand from 8 fp32 scores (the lane's keys 8i+4h+j for i = 2b, 2b+1).
template <typename T>
__device__ __forceinline__ typename Mf<T>::v8 pack8(const float *x) {
  typename Mf<T>::v8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (typename Mf<T>::e)x[i];
  return r;
}

// A operand from an LDS row of a transposed chunk: elements 4h..4h+3 and
// 8+4h..8+4h+3 of the 16-wide k-block starting at `row`.
template <typename T>
__device__ __forceinline__ typename Mf<T>::v8 lds_a(const typename Mf<T>::e *row,
                                                  int h) {
  typedef typename Mf<T>::v4 v4;
  const v4 lo = *reinterpret_cast<const v4 *>(row + 4 * h);
  const v4 hi = *reinterpret_cast<const v4 *>(row + 8 + 4 * h);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

constexpr int kRow = 36;  // LDS row stride (elements) of a transposed chunk

__device__ __forceinline__ int xcd_tile(int bid, int n_launch) {
  // Workgroups are dealt to the 8 XCDs round-robin; give each XCD a
  // contiguous range of tiles so neighbouring tiles share its L2.
  return (bid & 7) * (n_launch >> 3) + (bid >> 3);
}

__device__ __forceinline__ int ceil_log2(int x) {
  int l = 0;
  while ((1 << l) < x) ++l;
  return l;
}

// Window of sub-grid query i (phase r) on axis a, as sub-grid [lo, hi).
__device__ __forceinline__ void sub_window(const Prob &P, const Tiling &Tl,
                                           int a, int L, int r, int i, int &lo,
                                           int &hi) {
  const Axis &x = P.ax[a];
  if (P.dense) {
    lo = 0;
    hi = L;
    return;
  }
  if (x.d == 1) {
    const AxisWin w = axis_window(i, L, x.K, 1, x.causal);
    lo = w.lo;
    hi = w.hi;
    return;
  }
  const AxisWin w = axis_window(r + x.d * i, L, x.K, x.d, x.causal);
  lo = (int)fdiv((uint32_t)(w.lo - r), Tl.fd[a]);
  hi = (int)fdiv((uint32_t)(w.hi - r + x.d - 1), Tl.fd[a]);
}

// Sub-grid queries [qlo, qhi] whose windows contain sub-grid key j.
__device__ __forceinline__ void sub_inverse(const Prob &P, const Tiling &Tl,
                                            int a, int L, int r, int Lr, int j,
                                            int &qlo, int &qhi) {
  const Axis &x = P.ax[a];
  if (P.dense) {
    qlo = 0;
    qhi = Lr - 1;
    return;
  }
  if (x.causal) {
    qlo = j;
    qhi = min(j + x.K - 1, Lr - 1);
    return;
  }
  if (x.d * x.K <= L) {  // clamped windows: start = clamp(i - K/2, 0, Lr - K)
    const int nh = x.K / 2;
    qlo = j <= x.K - 1 ? 0 : j - nh;
    qhi = j >= Lr - x.K ? Lr - 1 : j + nh;
    return;
  }
  // general odd K: window bounds are non-decreasing in i
  int a0 = 0, b0 = Lr, lo, hi;
  while (a0 < b0) {
    const int mid = (a0 + b0) >> 1;
    sub_window(P, Tl, a, L, r, mid, lo, hi);
    if (hi > j) b0 = mid; else a0 = mid + 1;
  }
  qlo = a0;
  a0 = 0;
  b0 = Lr;
  while (a0 < b0) {
    const int mid = (a0 + b0) >> 1;
    sub_window(P, Tl, a, L, r, mid, lo, hi);
    if (lo > j) b0 = mid; else a0 = mid + 1;
  }
  qhi = a0 - 1;
}

// Per-wave tile context: phase, sub-grid origin and valid counts per axis.
struct TileCtx {
  int b, head;
  int r[3], i0[3], nv[3], nt[3];  // nv: valid in sample, nt: valid in tensor
  int L[3];                       // sample extents
};

__device__ __forceinline__ TileCtx decode_tile(const Prob &P, const Tiling &Tl,
                                               int id, const FastDiv &fHn) {
  TileCtx c;
  int g[3];
  uint32_t rest = (uint32_t)id;
#pragma unroll
  for (int a = 2; a >= 0; --a) {
    const uint32_t qd = fdiv(rest, Tl.fG[a]);
    g[a] = (int)(rest - qd * Tl.fG[a].d);
    rest = qd;
  }
  const uint32_t bq = fdiv(rest, fHn);
  c.head = (int)(rest - bq * fHn.d);
  c.b = (int)bq;
  int O[3];
  sample_extents(P, c.b, c.L, O);
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    const Axis &x = P.ax[a];
    const uint32_t rr = fdiv((uint32_t)g[a], Tl.fnt[a]);
    c.r[a] = (int)rr;
    c.i0[a] = (g[a] - (int)rr * Tl.nt[a]) * Tl.T[a];
    int Ls, Lt;
    if (x.d == 1) {
      Ls = c.L[a];
      Lt = x.L;
    } else {
      Ls = c.L[a] > c.r[a] ? (int)fdiv((uint32_t)(c.L[a] - 1 - c.r[a]), Tl.fd[a]) + 1 : 0;
      Lt = x.L > c.r[a] ? (int)fdiv((uint32_t)(x.L - 1 - c.r[a]), Tl.fd[a]) + 1 : 0;
    }
    c.nv[a] = max(0, min(Ls - c.i0[a], Tl.T[a]));
    c.nt[a] = max(0, min(Lt - c.i0[a], Tl.T[a]));
  }
  return c;
}

// Coordinates of slot n (0..31) inside a T0 x T1 x T2 tile.
__device__ __forceinline__ void tile_slot(const Tiling &Tl, int n, int u[3]) {
  u[2] = n & (Tl.T[2] - 1);
  u[1] = (n >> Tl.lgT[2]) & (Tl.T[1] - 1);
  u[0] = n >> (Tl.lgT[2] + Tl.lgT[1]);
}

// A row-major box of sub-grid points, innermost extent padded to 2^lgP.
struct Box {
  int lo[3], E[3];
  int lgP;     // padding of the innermost axis (30: the box is one row)
  int slots;   // padded number of points
};

__device__ __forceinline__ void box_init(Box &bx) {
  const int rows = bx.E[0] * bx.E[1];
  if (rows == 1) {
    bx.lgP = 30;
    bx.slots = bx.E[2];
  } else {
    bx.lgP = max(3, ceil_log2(bx.E[2]));
    bx.slots = rows << bx.lgP;
  }
}

__device__ __forceinline__ int uni(int x) {
  return __builtin_amdgcn_readfirstlane(x);
}

// Row coordinates (e0, e1) of padded-box row R, advanced incrementally so
// the chunk loop never divides; the cursor is wave-uniform.
struct RowCursor {
  int R, e0, e1;
};

// Advance (e0, e1) by dr rows, 0 <= dr <= 3 (a chunk spans at most 4
// rows), without branches: e1 + dr wraps at most three times.
__device__ __forceinline__ void row_add(int &e0, int &e1, int dr, int E1) {
  const int x = e1 + dr;
  const int wraps = (int)(x >= E1) + (int)(x >= 2 * E1) + (int)(x >= 3 * E1);
  e1 = x - wraps * E1;
  e0 += wraps;
}

// First row of a 32-slot chunk (wave-uniform).
struct ChunkRows {
  int R0, e0, e1;
};

// Move the cursor to the chunk starting at slot g0 (rows only advance).
__device__ __forceinline__ ChunkRows chunk_rows(RowCursor &rc, const Box &bx,
                                                int g0) {
  const int R = uni(g0 >> bx.lgP);
  while (rc.R + 3 < R) {
    row_add(rc.e0, rc.e1, 3, bx.E[1]);
    rc.R += 3;
  }
  row_add(rc.e0, rc.e1, R - rc.R, bx.E[1]);
  rc.R = R;
  rc.e0 = uni(rc.e0);
  rc.e1 = uni(rc.e1);
  return ChunkRows{R, rc.e0, rc.e1};
}

// Box coordinates of padded slot g0 + n, clamped into the box; returns
// false when the slot is padding (its clamped point is a real box point).
__device__ __forceinline__ bool box_point(const Box &bx, const ChunkRows &cr,
                                          int g0, int n, int e[3]) {
  const int g = g0 + n;
  e[2] = g & ((1 << bx.lgP) - 1);
  e[0] = cr.e0;
  e[1] = cr.e1;
  row_add(e[0], e[1], (g >> bx.lgP) - cr.R0, bx.E[1]);
  const bool inside = (e[2] < bx.E[2]) & (e[0] < bx.E[0]);
  e[2] = min(e[2], bx.E[2] - 1);
  e[0] = min(e[0], bx.E[0] - 1);
  return inside;
}

// Per-chunk mask helper: for the 4 groups i of a lane's 16 elements
// (slots g0 + 8i + 4h + j), the row of group i is wave-uniform; the
// element is inside [wlo, wlo + ww) on every axis iff rowok(i) and
// its innermost coordinate xb(i) + 4h + j is.
__device__ __forceinline__ void chunk_mask(const Box &bx, const ChunkRows &cr,
                                           int g0, int h, const int wlo[3],
                                           const int ww[3], bool ok[16]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int g = g0 + 8 * i;
    const int xb = g & ((1 << bx.lgP) - 1);
    int e0 = cr.e0, e1 = cr.e1;
    row_add(e0, e1, uni((g >> bx.lgP) - cr.R0), bx.E[1]);
    const bool rowok = ((unsigned)(e1 - wlo[1]) < (unsigned)ww[1]) &
                       ((unsigned)(e0 - wlo[0]) < (unsigned)ww[0]);
    const int x0 = xb + 4 * h - wlo[2];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      ok[4 * i + j] = rowok & ((unsigned)(x0 + j) < (unsigned)ww[2]);
  }
}


// In-wave LDS ordering: this wave's LDS operations are complete.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS ops done
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
}

// Element offset of box point e: base + e0*S0 + e1*S1 + e2*S2 (wave-uniform
// base and strides, so the chunk loops carry four scalars for addressing).
struct BoxAddr {
  int64_t base;
  int S[3];
};

// Box of sub-grid points of phase tc.r, origin bx.lo, rows of `heads`
// heads: token strides along each axis times the dilation.
__device__ __forceinline__ BoxAddr box_addr(const Prob &P, const TileCtx &tc,
                                            const Box &bx, int head,
                                            int heads) {
  BoxAddr ba;
  int p[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) p[a] = tc.r[a] + P.ax[a].d * bx.lo[a];
  const int row = heads * P.D;
  ba.base = tok_in(P, tc.b, p[0], p[1], p[2]) * row + (int64_t)head * P.D;
  ba.S[2] = uni(P.ax[2].d * row);
  ba.S[1] = uni(P.ax[1].d * P.ax[2].L * row);
  ba.S[0] = uni(P.ax[0].d * P.ax[1].L * P.ax[2].L * row);
  return ba;
}

__device__ __forceinline__ int box_off(const BoxAddr &ba, const int e[3]) {
  return e[0] * ba.S[0] + e[1] * ba.S[1] + e[2] * ba.S[2];
}

// First global chunk index >= lo that wave w of W owns (c == w mod W).
__device__ __forceinline__ int first_owned(int lo, int w, int W) {
  return lo + (((w - lo) % W) + W) % W;
}

// Load the K and V rows of one chunk (A-operand layout: lane (key, h)
// holds elements 16t + 8h .. 16t + 8h + 7).
template <typename T, int D>
__device__ __forceinline__ void load_kv(const T *kp, const T *vp,
                                        typename Mf<T>::v8 *kf,
                                        typename Mf<T>::v8 *vf, int h) {
#pragma unroll
  for (int t = 0; t < D / 16; ++t) {
    kf[t] = ld8(kp + 16 * t + 8 * h);
    vf[t] = ld8(vp + 16 * t + 8 * h);
  }
}


// Query-tile setup shared by the forward and the dQ role: the lane's
// query, its window relative to the tile's key box, and the box itself.
struct QTile {
  TileCtx tc;
  bool q_valid, q_tensor, any;
  int64_t qtok;
  Box bx;
  int wlo[3], ww[3];
  int nbox, nextra;
};

__device__ __forceinline__ QTile query_tile(const Prob &P, const Tiling &Tl,
                                            const TileCtx &tc0, int n) {
  QTile Q;
  Q.tc = tc0;
  const TileCtx &tc = Q.tc;
  int u[3];
  tile_slot(Tl, n, u);
  Q.q_tensor = (u[0] < tc.nt[0]) & (u[1] < tc.nt[1]) & (u[2] < tc.nt[2]);
  Q.q_valid = (u[0] < tc.nv[0]) & (u[1] < tc.nv[1]) & (u[2] < tc.nv[2]);
  Q.any = (tc.nv[0] > 0) & (tc.nv[1] > 0) & (tc.nv[2] > 0);
  int pos[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) pos[a] = tc.r[a] + P.ax[a].d * (tc.i0[a] + u[a]);
  Q.qtok = tok_in(P, tc.b, pos[0], pos[1], pos[2]);
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    int lo0 = 0, hi0 = 0, lo1 = 0, hi1 = 0;
    if (Q.any) {
      sub_window(P, Tl, a, tc.L[a], tc.r[a], tc.i0[a], lo0, hi0);
      sub_window(P, Tl, a, tc.L[a], tc.r[a], tc.i0[a] + tc.nv[a] - 1, lo1, hi1);
    }
    Q.bx.lo[a] = uni(lo0);
    Q.bx.E[a] = uni(Q.any ? hi1 - lo0 : 1);
    int lo = 0, hi = 0;
    if (Q.q_valid)
      sub_window(P, Tl, a, tc.L[a], tc.r[a], tc.i0[a] + u[a], lo, hi);
    Q.wlo[a] = lo - Q.bx.lo[a];
    Q.ww[a] = Q.q_valid ? hi - lo : 0;
  }
  box_init(Q.bx);
  Q.bx.lgP = uni(Q.bx.lgP);
  Q.nbox = uni(Q.any ? (Q.bx.slots + 31) >> 5 : 0);
  Q.nextra = uni(Q.any ? (P.n_extra + 31) >> 5 : 0);
  return Q;
}

// Mask of a chunk of additional tokens (global chunk index c >= nbox).
__device__ __forceinline__ void extra_mask(bool q_valid, int first, int n_extra,
                                           int h, bool ok[16]) {
#pragma unroll
  for (int e = 0; e < 16; ++e)
    ok[e] = q_valid & (first + 8 * (e >> 2) + 4 * h + (e & 3) < n_extra);
}


// ---------------------------------------------------------------------------

int ilog2(int x) {
  int l = 0;
  while ((1 << l) < x) ++l;
  return l;
}

// Estimated 32-wide chunks per tile and tile count of a tiling.
struct TileCost {
  double tiles, chunks;
};

TileCost tiling_cost(const Prob &P, const int T[3]) {
  double tiles = 1.0, rows = 1.0;
  int e2 = 1;
  for (int a = 0; a < 3; ++a) {
    const Axis &x = P.ax[a];
    const int Lr = (x.L + x.d - 1) / x.d;
    const int nt = (Lr + T[a] - 1) / T[a];
    tiles *= (double)x.d * nt;
    const int e = P.dense ? Lr : min(min(T[a], Lr) + x.K - 1, Lr);
    if (a < 2) rows *= e; else e2 = e;
  }
  const double slots =
      rows == 1.0 ? e2 : rows * (double)(1 << max(3, ilog2(e2)));
  return {tiles, std::ceil(slots / 32.0) + std::ceil(P.n_extra / 32.0)};
}

Tiling choose_tiling(const Prob &P, int heads_q, int heads_kv, double *chunks) {
  Tiling best{};
  double best_cost = 1e300;
  for (int l0 = 0; l0 <= 5; ++l0)
    for (int l1 = 0; l0 + l1 <= 5; ++l1) {
      const int l2 = 5 - l0 - l1;
      const int T[3] = {1 << l0, 1 << l1, 1 << l2};
      bool ok = true;
      for (int a = 0; a < 3; ++a)
        if (P.ax[a].L == 1 && T[a] != 1) ok = false;
      if (!ok) continue;
      const TileCost c = tiling_cost(P, T);
      if (c.tiles * c.chunks < best_cost) {
        best_cost = c.tiles * c.chunks;
        *chunks = c.chunks;
        for (int a = 0; a < 3; ++a) best.T[a] = T[a];
      }
    }
  int grid = 1;
  for (int a = 0; a < 3; ++a) {
    best.lgT[a] = ilog2(best.T[a]);
    const Axis &x = P.ax[a];
    const int Lr = (x.L + x.d - 1) / x.d;
    best.nt[a] = (Lr + best.T[a] - 1) / best.T[a];
    grid *= x.d * best.nt[a];
  }
  best.n_q = P.B * heads_q * grid;
  best.n_k = P.B * heads_kv * grid;
  for (int a = 0; a < 3; ++a) {
    best.fG[a] = make_fastdiv((uint32_t)(P.ax[a].d * best.nt[a]));
    best.fnt[a] = make_fastdiv((uint32_t)best.nt[a]);
    best.fd[a] = make_fastdiv((uint32_t)P.ax[a].d);
  }
  best.fH = make_fastdiv((uint32_t)heads_q);
  best.fHk = make_fastdiv((uint32_t)heads_kv);
  best.fRep1 = make_fastdiv((uint32_t)(heads_q / heads_kv + 1));
  return best;
}

// Waves per tile: one per ~6 chunks, at most `cap` (2 for the backward at
// head_dim 128, to stay within 64 KB of LDS).  NATTEN_AMD_FWD_WAVES /
// NATTEN_AMD_BWD_WAVES override the choice (tuning aid; still capped).
int waves_for(double chunks, int cap, const char *env) {
  int w = (int)std::ceil(chunks / 6.0);
  if (const char *o = std::getenv(env)) {
    const int v = std::atoi(o);
    if (v > 0) w = v;
  }
  return max(1, min(w, cap));
}


}  // namespace
}  // namespace na
