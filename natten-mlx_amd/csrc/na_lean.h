// na_lean.h — pieces shared by the lean matrix-core (gfx950) workgroup
// kernels: the fused forward / backward (na_lean.hip) and the split ops
// (na_lsplit.hip).  Problem and tile description (LAx, LProb, LTile), the
// window rules on a dilation phase's sub-grid, the wave sub-box walk, the
// staging of a box of rows into LDS, the lane-swap reductions and the
// host-side choice of wave tile, workgroup and LDS layout.
#pragma once

#include <cstring>

#include <cmath>
#include <cstdlib>
#include <type_traits>

#include "na_common.h"
#include "na_launch.h"

namespace na {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct L16;
template <>
struct L16<bf16_t> {
  typedef __bf16 e;
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  typedef __bf16 v4 __attribute__((ext_vector_type(4)));
  typedef __bf16 v2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ f32x4 mma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ v4 tr(const e *p) {
    typedef __attribute__((address_space(3))) v4 lv4;
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lv4 *)(p));
  }
  static __device__ __forceinline__ float dot2(v2 a, v2 b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false);
  }
};
template <>
struct L16<f16_t> {
  typedef _Float16 e;
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  typedef _Float16 v4 __attribute__((ext_vector_type(4)));
  typedef _Float16 v2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ f32x4 mma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ v4 tr(const e *p) {
    typedef __fp16 h4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
    typedef __attribute__((address_space(3))) h4 lh4;
    return __builtin_bit_cast(v4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lh4 *)(p)));
  }
  static __device__ __forceinline__ float dot2(v2 a, v2 b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
  }
};

// One spatial axis of a lean problem (unit axes: L = K = T = d = 1).
struct LAx {
  int32_t L, K, d, causal, nh;
  int32_t Lq, Lrem;   // L / d and L % d: phase r holds Lq + (r < Lrem) points
  int32_t T, lgT;     // wave tile extent (power of two)
  int32_t TW, lgTW;   // workgroup tile extent: T, times W on the stack axis
  int32_t nt;         // workgroup tiles per phase (of the longest phase)
  int32_t Em;         // workgroup key-box extent of the LDS layout (maximum)
  int32_t tok;        // token stride of one position step along this axis
  FastDiv fG;         // tile-grid extent d * nt
  FastDiv fnt;        // nt
  FastDiv fd;         // d (per-sample phase extents)
};

struct LProb {
  LAx ax[3];
  int32_t B, H, Hkv, D;
  int32_t Ltot;       // tokens per sample
  float sl2;          // scale * log2(e)
  int32_t n_tiles, n_launch;
  int32_t sa;         // stack axis: the workgroup's waves tile this axis
  int32_t ebox;       // staged rows: Em2 (rank 1) or Em0 * Em1 * 2^lgP2
  int32_t lgP2;       // rank >= 2: staged box rows are 2^lgP2 >= Em2 wide
  int32_t rep;        // query heads per key/value head
  int32_t sl;         // rank 3: box layers (axis 0) staged at a time
  float scale;
  FastDiv fH, fRep;
  FastDiv fHkv;       // key/value heads
  FastDiv fGrid;      // spatial tiles per (batch, head): prod of d * nt
  FastDiv fE1;        // rank 3: box row -> (e0, e1)
  const int32_t *se;  // per-sample extents [B, rank] or nullptr
  int32_t nx;         // additional key/value tokens per sample
  int32_t nxr;        // their LDS rows (nx rounded up to 16), before the box
  int32_t kp;         // kernel slots per query (K0 K1 K2), split ops
  int32_t kst0, kst1; // slot strides of axes 0 and 1 (K1 K2, K2)
  int32_t hl;         // forward (VX): query heads a workgroup runs over one
                      // staged box (a divisor of rep; 0: one head per
                      // workgroup, decoded per query head)
  FastDiv fHg;        // rep / hl: head groups per key/value head
};

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ int xcd_tile(int bid, int n_launch) {
  // Workgroups are dealt to the 8 XCDs round-robin; give each XCD a
  // contiguous range of tiles so neighbouring tiles share its L2.
  return (bid & 7) * (n_launch >> 3) + (bid >> 3);
}

// Window [start, end) of sub-grid index i on an axis whose phase has Lr
// points (branch-free: both rules are evaluated and one is selected).
__device__ __forceinline__ int wstart(const LAx &x, int i, int Lr) {
  const int nc = min(max(i - x.nh, 0), Lr - x.K);
  const int ca = max(i - x.K + 1, 0);
  const int sel = -x.causal;
  return (ca & sel) | (nc & ~sel);
}
__device__ __forceinline__ int wend(const LAx &x, int i, int Lr) {
  const int nc = min(max(i - x.nh, 0), Lr - x.K) + x.K;
  const int sel = -x.causal;
  return ((i + 1) & sel) | (nc & ~sel);
}

// Queries [start, end) whose windows hold sub-grid key j: on a non-causal
// axis the clamped windows give [j <= K-1 ? 0 : j - K/2, j >= Lr-K ? Lr :
// j + K/2 + 1); on a causal axis [j, min(j + K, Lr)).  Both bounds are
// non-decreasing in j.
__device__ __forceinline__ int iwstart(const LAx &x, int j, int Lr) {
  const int nc = j <= x.K - 1 ? 0 : j - x.nh;
  const int sel = -x.causal;
  return (j & sel) | (nc & ~sel);
}
__device__ __forceinline__ int iwend(const LAx &x, int j, int Lr) {
  const int nc = j >= Lr - x.K ? Lr : j + x.nh + 1;
  const int ca = min(j + x.K, Lr);
  const int sel = -x.causal;
  return (ca & sel) | (nc & ~sel);
}

// Staged rows interleave two tensors: [x row | 8 | y row | 8] elements, so
// both are addressed from one lane base with constant offsets.  The 16
// bytes after each row spread the rows over the LDS banks; in a query box
// the pair after the Q row holds (lse * log2(e), -delta) of the row.
constexpr int lds_row(int D) { return 2 * (D + 8); }
constexpr int lds_y(int D) { return D + 8; }
// Key rows of slack after a staged box: a chunk read near the box end may
// run up to 15 rows past it.
constexpr int kSlack = 16;

// Workgroup tile: everything wave-uniform about a tile of 16 W queries and
// its key box [lo, lo + E) per axis.
struct LTile {
  int b, head, hk;
  int r[3], i0[3], nv[3], Lr[3];
  int nvt[3];         // rows of the tensor (nv: rows of the sample)
  int lo[3], E[3];
  int kbase;          // element offset of box point (0,0,0), head hk
  int SK[3];          // element stride of one box step per axis (K/V)
};

// Origin of spatial tile `sp` (row-major over the per-axis grids d * nt):
// phase, first sub-grid index and valid count per axis.  VX: sample t.b
// has its own extent per axis (P.se); its phase extent Lr is then that of
// the sample (on a non-causal axis at least K, so every window stays inside
// the tensor whatever the extents hold), nv counts the sample's rows and
// nvt the tensor's.
template <int R, bool VX = false>
__device__ __forceinline__ bool tile_origin(const LProb &P, uint32_t sp,
                                            LTile &t) {
  int g[3] = {0, 0, 0};
#pragma unroll
  for (int a = 2; a >= 3 - R; --a) {
    if (a == 3 - R) {
      g[a] = (int)sp;
    } else {
      const uint32_t qd = fdiv(sp, P.ax[a].fG);
      g[a] = (int)(sp - qd * P.ax[a].fG.d);
      sp = qd;
    }
  }
  bool any = true;
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    const LAx &x = P.ax[a];
    if (a < 3 - R) {
      t.r[a] = 0; t.i0[a] = 0; t.nv[a] = 1; t.Lr[a] = 1;
      continue;
    }
    const int rr = (int)fdiv((uint32_t)g[a], x.fnt);
    t.r[a] = rr;
    t.i0[a] = (g[a] - rr * x.nt) * x.TW;  // TW: any wave count times T
    t.Lr[a] = x.Lq + (rr < x.Lrem ? 1 : 0);
    t.nvt[a] = min(t.Lr[a] - t.i0[a], x.TW);
    if (VX && P.se != nullptr) {
      const int Lb = min(max(P.se[min(t.b, P.B - 1) * R + a - (3 - R)], 0), x.L);
      const int lq = (int)fdiv((uint32_t)Lb, x.fd);
      const int lr = lq + (rr < Lb - lq * x.d ? 1 : 0);
      t.Lr[a] = x.causal ? lr : max(lr, x.K);
    }
    t.nv[a] = min(t.Lr[a] - t.i0[a], x.TW);
    any = any & (t.nv[a] > 0);
  }
  return any;
}

// The tile's box (INV: the queries whose windows hold its keys; else the
// keys its queries' windows hold) and its addressing for rows of head
// `head` in a tensor of `heads` heads.
template <int R, bool INV>
__device__ __forceinline__ void tile_box(const LProb &P, LTile &t, int head,
                                         int heads) {
  int tok0 = t.b * P.Ltot;
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    const LAx &x = P.ax[a];
    if (a < 3 - R) {
      t.lo[a] = 0; t.E[a] = 1; t.SK[a] = 0;
      continue;
    }
    const int i1 = t.i0[a] + max(t.nv[a], 1) - 1;
    t.lo[a] = INV ? iwstart(x, t.i0[a], t.Lr[a]) : wstart(x, t.i0[a], t.Lr[a]);
    t.E[a] = (INV ? iwend(x, i1, t.Lr[a]) : wend(x, i1, t.Lr[a])) - t.lo[a];
    tok0 += (t.r[a] + x.d * t.lo[a]) * x.tok;
    t.SK[a] = x.d * x.tok * heads * P.D;
  }
  t.kbase = (tok0 * heads + head) * P.D;
}

// Tile of (sample, key/value head, group of P.hl query heads): t.head is
// the group's first query head.
template <int R>
__device__ __forceinline__ bool decode_tile_group(const LProb &P, int tile,
                                                  LTile &t) {
  const uint32_t rest = fdiv((uint32_t)tile, P.fGrid);
  const uint32_t sp = (uint32_t)tile - rest * P.fGrid.d;
  const uint32_t r2 = fdiv(rest, P.fHg);
  const int sub = (int)(rest - r2 * P.fHg.d);
  const uint32_t bq = fdiv(r2, P.fHkv);
  t.hk = (int)(r2 - bq * P.fHkv.d);
  t.b = (int)bq;
  t.head = t.hk * P.rep + sub * P.hl;
  const bool any = tile_origin<R, true>(P, sp, t);
  tile_box<R, false>(P, t, t.hk, P.Hkv);
  return any & (t.b < P.B);
}

template <int R, bool VX = false>
__device__ __forceinline__ bool decode_tile(const LProb &P, int tile,
                                            LTile &t) {
  // tiles at or beyond n_tiles decode to a batch index >= B
  const uint32_t rest = fdiv((uint32_t)tile, P.fGrid);
  const uint32_t sp = (uint32_t)tile - rest * P.fGrid.d;
  const uint32_t bq = fdiv(rest, P.fH);
  t.head = (int)(rest - bq * P.fH.d);
  t.b = (int)bq;
  t.hk = (int)fdiv((uint32_t)t.head, P.fRep);
  const bool any = tile_origin<R, VX>(P, sp, t);
  tile_box<R, false>(P, t, t.hk, P.Hkv);
  return any & (t.b < P.B);
}

// A wave's part of a workgroup tile: its 16 queries (wave tile w along the
// stack axis) and the sub-box of the workgroup box their windows cover,
// walked as rows (e0, e1) x column segments of 16 keys from ws2.
struct WSub {
  int i0[3], nv[3], nvt[3];
  int ws[3], we[3];
  int cpr, nchunks;
  bool any;
};

template <int R, bool INV = false>
__device__ __forceinline__ WSub wave_sub(const LProb &P, const LTile &t,
                                         int w) {
  WSub s;
  s.any = true;
  int rows = 1;
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    if (a < 3 - R) {
      s.i0[a] = 0; s.nv[a] = 1; s.nvt[a] = 1; s.ws[a] = 0; s.we[a] = 1;
      continue;
    }
    const LAx &x = P.ax[a];
    const int off = a == P.sa ? w * x.T : 0;
    s.i0[a] = t.i0[a] + off;
    s.nv[a] = min(t.nv[a] - off, x.T);
    s.nvt[a] = min(t.nvt[a] - off, x.T);
    s.any = s.any & (s.nv[a] > 0);
    const int nvc = max(s.nv[a], 1);
    s.ws[a] = (INV ? iwstart(x, s.i0[a], t.Lr[a]) : wstart(x, s.i0[a], t.Lr[a])) -
              t.lo[a];
    s.we[a] = (INV ? iwend(x, s.i0[a] + nvc - 1, t.Lr[a])
                   : wend(x, s.i0[a] + nvc - 1, t.Lr[a])) - t.lo[a];
    if (a < 2) rows *= s.we[a] - s.ws[a];
  }
  s.cpr = (s.we[2] - s.ws[2] + 15) >> 4;
  s.nchunks = rows * s.cpr;
  return s;
}

// Chunk cursor over a wave's sub-box (chunks are visited in order).
struct Cursor {
  int e0, e1, cs;
};

__device__ __forceinline__ void advance(Cursor &cu, const WSub &s) {
  // branch-free: selects on wave-uniform values
  const int cs = cu.cs + 1;
  const bool w1 = cs == s.cpr;
  cu.cs = w1 ? 0 : cs;
  const int e1 = cu.e1 + (w1 ? 1 : 0);
  const bool w2 = e1 == s.we[1];
  cu.e1 = w2 ? s.ws[1] : e1;
  cu.e0 += w2 ? 1 : 0;
}

// 16-byte load at a 32-bit element offset from a wave-uniform base (the
// offset stays a 32-bit register operand, no 64-bit address arithmetic).
template <typename T>
__device__ __forceinline__ typename L16<T>::v8 ld8(const T *base, int off) {
  return *reinterpret_cast<const typename L16<T>::v8 *>(
      reinterpret_cast<const char *>(base) + (size_t)((uint32_t)off * 2u));
}
__device__ __forceinline__ float ldf(const float *base, int off) {
  return *reinterpret_cast<const float *>(reinterpret_cast<const char *>(base) +
                                          (size_t)((uint32_t)off * 4u));
}

// Element offset of staged-box unit (row kk of the LDS layout, 16-byte unit
// o): box coordinates from the layout (shifts; rank 3 divides by Em1 and
// adds the first staged layer s0), clamped onto the tile's true box, then
// 24-bit products with the strides.
template <int R>
__device__ __forceinline__ int unit_offset(const LProb &P, const LTile &t,
                                           int kk, int o, int s0) {
  int e0 = 0, e1 = 0, e2 = kk;
  if (R >= 2) {
    const int row = kk >> P.lgP2;
    e2 = kk & ((1 << P.lgP2) - 1);
    if (R == 2) {
      e1 = row;
    } else {
      e0 = (int)fdiv((uint32_t)row, P.fE1);
      e1 = row - e0 * P.ax[1].Em;
      e0 += s0;
    }
  }
  int off = t.kbase + 8 * o;
  if (R == 3) off += __umul24((unsigned)min(e0, t.E[0] - 1), (unsigned)t.SK[0]);
  if (R >= 2) off += __umul24((unsigned)min(e1, t.E[1] - 1), (unsigned)t.SK[1]);
  off += __umul24((unsigned)min(e2, t.E[2] - 1), (unsigned)t.SK[2]);
  return off;
}

// Global element offsets g[j] and LDS element offsets la[j] (layout row
// stride RS) of a lane's NU staging units u0 + j nthr + tid, j < NU (u0 a
// multiple of NU nthr, nthr of OCT): layout row kk_j = (u0 + tid) / OCT +
// j nthr / OCT, unit o = tid % OCT.  Rank 1, and rank 2 (or rank 3 staging
// one layer per slab) when a step of nthr / OCT layout rows is a whole
// number of box rows, step the box row (two adds, a min and a 24-bit
// product per unit); otherwise unit_offset per unit.  Units past the layout take its last row (the lane's unit of
// it): real rows, staged again with the same values, and every row's OCT
// units are held by OCT consecutive lanes.
template <int R, int OCT, int RS, int NU = 4, bool LAYER3 = true>
__device__ __forceinline__ void unit_walk(const LProb &P, const LTile &t,
                                          int u0, int tid, int nthr, int s0,
                                          int (&g)[NU], int (&la)[NU]) {
  const int step = nthr / OCT;
  const int kk0 = u0 / OCT + tid / OCT, o = tid % OCT;
  const int P2 = R >= 2 ? 1 << P.lgP2 : 1;
  if (R == 1) {
    const int base = t.kbase + 8 * o;
#pragma unroll
    for (int j = 0; j < NU; ++j) {
      const int kk = min(kk0 + j * step, P.ebox - 1);
      g[j] = base + __umul24((unsigned)min(kk, t.E[2] - 1), (unsigned)t.SK[2]);
      la[j] = __umul24(kk, RS) + 8 * o;
    }
    return;
  }
  // rank 2, and rank 3 staged one box layer (axis 0 = s0) per slab: step
  // box rows of the layer
  if ((R == 2 || (R == 3 && LAYER3 && P.sl == 1)) && (step & (P2 - 1)) == 0) {
    const int e2 = kk0 & (P2 - 1);
    const int row0 = kk0 >> P.lgP2, drow = step >> P.lgP2;
    int base = t.kbase + 8 * o + __umul24((unsigned)min(e2, t.E[2] - 1), (unsigned)t.SK[2]);
    if (R == 3) base += __umul24((unsigned)min(s0, t.E[0] - 1), (unsigned)t.SK[0]);
    const int Em1 = P.ax[1].Em;
#pragma unroll
    for (int j = 0; j < NU; ++j) {
      const int row = min(row0 + j * drow, Em1 - 1);
      g[j] = base + __umul24((unsigned)min(row, t.E[1] - 1), (unsigned)t.SK[1]);
      la[j] = __umul24((row << P.lgP2) + e2, RS) + 8 * o;
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < NU; ++j) {
    const int kk = min(kk0 + j * step, P.ebox - 1);
    g[j] = unit_offset<R>(P, t, kk, o, s0);
    la[j] = __umul24(kk, RS) + 8 * o;
  }
}

__device__ __forceinline__ f32x4 zero4() {
  f32x4 z = {0.f, 0.f, 0.f, 0.f};
  return z;
}

// Sum over G (4, 8 or 16) consecutive lanes, complete in the group's first
// lane, by DPP lane moves (no LDS traffic): swaps within quads (the
// butterfly's first two steps), then the row shifts by 4 and 8 that bring
// the upper half of the group to its first lane.
template <int G>
__device__ __forceinline__ float dpp_group_sum(float x) {
  auto dpp = [](float v, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v),
                                                      decltype(ctrl)::value, 0xf, 0xf, false));
  };
  x += dpp(x, std::integral_constant<int, 0xb1>());    // quad_perm [1,0,3,2]
  x += dpp(x, std::integral_constant<int, 0x4e>());    // quad_perm [2,3,0,1]
  if (G >= 8) x += dpp(x, std::integral_constant<int, 0x104>());   // row_shl:4
  if (G >= 16) x += dpp(x, std::integral_constant<int, 0x108>());  // row_shl:8
  return x;
}

// Max / sum over the four lanes l, l ^ 16, l ^ 32, l ^ 48 that hold one
// query's scores (two lane-swap butterflies, no LDS traffic).
__device__ __forceinline__ float quad_max(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x),
                                                  __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x),
                                                  __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float quad_sum(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x),
                                                  __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x),
                                                  __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Window mask carried by the score accumulator: the MFMA starts from 0 for
// the lane's 4 elements inside the window and from -inf outside, so S comes
// out masked (-inf plus a finite product is -inf).  cb: the column part
// (0 / -inf per element), rowok: the chunk row is inside the window.
__device__ __forceinline__ void col_bias(int x0, int ww2, float cb[4]) {
#pragma unroll
  for (int r = 0; r < 4; ++r)
    cb[r] = (unsigned)(x0 + r) < (unsigned)ww2 ? 0.f : -INFINITY;
}
__device__ __forceinline__ f32x4 mask_init(bool rowok, const float cb[4]) {
  f32x4 c;
#pragma unroll
  for (int r = 0; r < 4; ++r) c[r] = rowok ? cb[r] : -INFINITY;
  return c;
}

// In-wave LDS ordering: this wave's LDS operations are complete.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
}

// Slack rows after a staged box: zero (a chunk read near the end of the box
// may include them; zero rows keep every MFMA operand finite).
template <typename T, int D>
__device__ __forceinline__ void zero_slack(const LProb &P,
                                           typename L16<T>::e *xs, int tid,
                                           int nthr) {
  typedef typename L16<T>::v8 v8;
  constexpr int SLU = kSlack * lds_row(D) / 8;  // 16-byte units of slack
  for (int u = tid; u < SLU; u += nthr) {
    v8 z;
#pragma unroll
    for (int i = 0; i < 8; ++i) z[i] = (typename L16<T>::e)0.f;
    *reinterpret_cast<v8 *>(xs + P.ebox * lds_row(D) + 8 * u) = z;
  }
}

// Stage a workgroup's box of rows of two tensors (x, y: K and V, or Q and
// dO) into LDS: box point (e0, e1, e2) at layout row ((e0 * Em1 + e1) <<
// lgP2) + e2 (rank 1: e2), element row * lds_row(D); layout points past the
// tile's true box are clamped onto it (their rows are real rows, so every
// staged value is finite).  Four 16-byte units per lane at a time, all in
// flight together.
template <typename T, int D, int R>
__device__ __forceinline__ void stage_box(const LProb &P, const LTile &t,
                                          const T *__restrict__ x,
                                          const T *__restrict__ y,
                                          typename L16<T>::e *xs,
                                          typename L16<T>::e *ys, int tid,
                                          int nthr, int s0) {
  typedef typename L16<T>::v8 v8;
  constexpr int OCT = D / 8;  // 16-byte units per row
  constexpr int RSE = lds_row(D);
  const int nun = P.ebox * OCT;
  for (int u0 = 0; u0 < nun; u0 += 4 * nthr) {
    v8 xr[4], yr[4];
    int g[4], la[4];
    unit_walk<R, OCT, RSE>(P, t, u0, tid, nthr, s0, g, la);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xr[j] = ld8(x, g[j]);
      yr[j] = ld8(y, g[j]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      *reinterpret_cast<v8 *>(xs + la[j]) = xr[j];
      *reinterpret_cast<v8 *>(ys + la[j]) = yr[j];
    }
  }
  zero_slack<T, D>(P, xs, tid, nthr);
}

// A slab of the box of two tensors staged in two steps, so its loads can be
// in flight while the previous slab is computed: load() issues every unit
// of the lane (two rounds of four, the units of stage_box) into registers,
// store() writes them to LDS.  Used where a box is staged in several slabs
// and two rounds cover a slab (ebox * D / 8 <= 8 * nthr).
template <typename T, int D, int R>
struct SlabPrefetch {
  typedef typename L16<T>::v8 v8;
  static constexpr int OCT = D / 8;
  static constexpr int RSE = lds_row(D);
  v8 x[2][4], y[2][4];
  int la[2][4];
  __device__ __forceinline__ void load(const LProb &P, const LTile &t,
                                       const T *__restrict__ xg,
                                       const T *__restrict__ yg, int tid, int nthr,
                                       int s0) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      int g[4];
      // a round past the layout clamps to its last row (real rows,
      // rewritten with the same values)
      unit_walk<R, OCT, RSE>(P, t, r * 4 * nthr, tid, nthr, s0, g, la[r]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[r][j] = ld8(xg, g[j]);
        y[r][j] = ld8(yg, g[j]);
      }
    }
  }
  __device__ __forceinline__ void store(typename L16<T>::e *xs,
                                        typename L16<T>::e *ys) const {
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        *reinterpret_cast<v8 *>(xs + la[r][j]) = x[r][j];
        *reinterpret_cast<v8 *>(ys + la[r][j]) = y[r][j];
      }
  }
};

// ---------------------------------------------------------------------------
// Host side.

int ilog2c(int x) {
  int l = 0;
  while ((1 << l) < x) ++l;
  return l;
}

constexpr size_t kLdsBudget = 80 * 1024;  // per workgroup: >= 2 per CU

// LDS budget per workgroup; NATTEN_AMD_LEAN_LDS_KB overrides it (tuning).
size_t lds_budget() {
  static const size_t b = [] {
    const char *e = std::getenv("NATTEN_AMD_LEAN_LDS_KB");
    const long v = e != nullptr ? std::atol(e) : 0;
    return v > 0 && v <= 160 ? (size_t)v * 1024 : kLdsBudget;
  }();
  return b;
}

// Largest number of waves per workgroup tried: 8 on rank 1, 4 otherwise
// (measured: eight-wave workgroups halve the workgroup count, and at
// config 2 size the CUs holding two of them set a longer tail than the 16
// CUs holding a fourth four-wave workgroup; on the 1-D config 4 they are
// faster).  NATTEN_AMD_LEAN_WAVES (1 to 8) overrides it (tuning).
int lean_waves_env() {
  static const int w = [] {
    const char *e = std::getenv("NATTEN_AMD_LEAN_WAVES");
    const int v = e != nullptr ? std::atoi(e) : 0;
    return v >= 1 && v <= 8 ? v : 0;
  }();
  return w;
}
bool lean_waves_forced() { return lean_waves_env() > 0; }
int lean_max_waves(int rank) {
  const int w = lean_waves_env();
  return w > 0 ? w : rank == 1 ? 8 : 4;
}

// Compute units of the gfx950 parts this library targets (MI350X, MI355X).
constexpr int kLeanCUs = 256;

struct LChoice {
  int T[3];      // wave tile (product 16 over the active axes)
  int W, sa;     // waves per workgroup and the axis they are stacked along
  int Em[3];     // workgroup key box (largest over tiles)
  int sl;        // rank 3: box layers staged at a time (Em[0]: all at once)
  bool cpr1;     // every wave sub-box row is at most 16 keys wide
  bool ok;
};

// Staged rows of a box layout (rank >= 2: rows padded to a power of two).
int lds_rows(int R, const int Em[3]) {
  if (R == 1) return Em[2];
  int p2 = 1;
  while (p2 < Em[2]) p2 <<= 1;
  return Em[0] * Em[1] * p2;
}

// LDS rows of the additional tokens (forward): n_extra rounded up to 16.
int lean_nxr(const Prob &P) { return (P.n_extra + 15) & ~15; }

// What a launch stages: the fused forward (K/V box, additional tokens),
// the fused backward (K/V box, then the query box with (lse, delta) per
// row), a query-centric split op (one tensor's key box plus 16 compact rows
// [kprod] per wave) or a key-centric one (one tensor's query box).
enum LMode { kLFwd, kLBwd, kLQK, kLInv };

__host__ __device__ constexpr int align16(int x) { return (x + 15) & ~15; }

// LDS bytes of a workgroup of W waves staging ebox box rows.
size_t lean_lds_bytes(const Prob &P, LMode mode, int ebox, int W) {
  const int D = P.D, kp = P.kprod;
  switch (mode) {
    case kLFwd:
      return (size_t)(lean_nxr(P) + ebox + kSlack) * lds_row(D) * 2;
    case kLBwd:  // the dQ pass stages the additional tokens before its box
      return (size_t)(lean_nxr(P) + ebox + kSlack) * lds_row(D) * 2;
    case kLQK:
      return (size_t)align16((ebox + kSlack) * lds_y(D) * 2) + (size_t)16 * W * kp * 2;
    default:
      return (size_t)(ebox + kSlack) * lds_y(D) * 2;
  }
}

// Host twins of the window rules.
int h_ws(const Axis &x, int i, int Lr) {
  return x.causal ? std::max(i - x.K + 1, 0)
                  : std::min(std::max(i - x.K / 2, 0), Lr - x.K);
}
int h_we(const Axis &x, int i, int Lr) {
  return x.causal ? i + 1 : h_ws(x, i, Lr) + x.K;
}
int h_iws(const Axis &x, int j, int Lr) {
  return x.causal ? j : (j <= x.K - 1 ? 0 : j - x.K / 2);
}
int h_iwe(const Axis &x, int j, int Lr) {
  return x.causal ? std::min(j + x.K, Lr) : (j >= Lr - x.K ? Lr : j + x.K / 2 + 1);
}

// Largest box (forward: keys of a tile's queries; inverse: queries of a
// tile's keys) over every tile of extent t on axis x, by enumeration.
int box_max(const Axis &x, int t, bool inverse) {
  int best = 1;
  for (int r = 0; r < x.d && r < x.L; ++r) {
    const int Lr = (x.L - 1 - r) / x.d + 1;
    for (int i0 = 0; i0 < Lr; i0 += t) {
      const int i1 = std::min(i0 + t, Lr) - 1;
      const int e = inverse ? h_iwe(x, i1, Lr) - h_iws(x, i0, Lr)
                            : h_we(x, i1, Lr) - h_ws(x, i0, Lr);
      best = std::max(best, e);
    }
  }
  return best;
}

// Wave tile: the power-of-two shape with the fewest (waves x chunks);
// workgroup: up to 8 waves stacked along the axis with the smallest staged
// box per wave whose box fits the LDS budget.  For the backward the boxes
// also cover the inverse windows (query boxes of key tiles) and the LDS
// holds a (lse, delta) pair per staged row.
LChoice lean_choice_compute(const Prob &P, LMode mode) {
  const int R = P.rank, lead = 3 - R;
  LChoice best{};
  best.ok = false;
  double best_cost = 1e300;
  auto ext = [&](int a, int t) {
    if (a < lead) return 1;
    const Axis &x = P.ax[a];
    if (P.sample_extent != nullptr) {
      // any sample (phase length >= K): a box of a tile of t points
      // spans at most t + K - 1 points of a phase no longer than the
      // tensor's.  An inverse box on a non-causal axis spans more where the
      // tile's keys are within K of an end of the sample (those keys are
      // in the windows of every query up to that end): with tiles starting
      // at multiples of t >= K, at most t + K - 1 + K / 2 (the last full
      // tile before the sample's end), else t + 2 (K - 1).  Both bounds
      // are attained.
      const bool inv = (mode == kLBwd || mode == kLInv) && !x.causal;
      const int e = !inv ? t + x.K - 1
                         : (t >= x.K ? t + x.K - 1 + x.K / 2 : t + 2 * (x.K - 1));
      return std::min((x.L + x.d - 1) / x.d, e);
    }
    if (mode == kLInv) return box_max(x, t, true);
    const int f = box_max(x, t, false);
    return mode == kLBwd ? std::max(f, box_max(x, t, true)) : f;
  };
  for (int l0 = 0; l0 <= 4; ++l0)
    for (int l1 = 0; l0 + l1 <= 4; ++l1) {
      const int Tt[3] = {1 << l0, 1 << l1, 1 << (4 - l0 - l1)};
      bool ok = true;
      for (int a = 0; a < lead; ++a)
        if (Tt[a] != 1) ok = false;
      if (!ok) continue;
      double waves = 1.0, rows = 1.0;
      for (int a = lead; a < 3; ++a) {
        const Axis &x = P.ax[a];
        const int Lr = (x.L + x.d - 1) / x.d;
        waves *= (double)x.d * ((Lr + Tt[a] - 1) / Tt[a]);
        if (a < 2) rows *= ext(a, Tt[a]);
      }
      const int e2 = ext(2, Tt[2]);
      const double cost = waves * rows * std::ceil(e2 / 16.0);
      if (cost < best_cost) {
        best_cost = cost;
        for (int a = 0; a < 3; ++a) best.T[a] = Tt[a];
        best.cpr1 = R > 1 && e2 <= 16;
      }
    }
  double best_per_wave = 1e300;
  // the largest wave count, then the powers of two below it
  int Ws[5], nW = 0;
  const int wmax = lean_max_waves(R);
  Ws[nW++] = wmax;
  for (int W = 8; W >= 1; W >>= 1)
    if (W < wmax) Ws[nW++] = W;
  for (int wi = 0; wi < nW; ++wi)
    for (int sa = lead; sa < 3; ++sa) {
      const int W = Ws[wi];
      const Axis &x = P.ax[sa];
      // every wave tile of a workgroup must start inside the phase
      if (W > 1 && best.T[sa] * (W - 1) >= (x.L + x.d - 1) / x.d) continue;
      int Em[3];
      for (int a = 0; a < 3; ++a) Em[a] = ext(a, best.T[a] * (a == sa ? W : 1));
      // rank 3 may stage the box a few layers (axis 0) at a time
      int sl = Em[0];
      while (sl > 1 && lean_lds_bytes(P, mode, lds_rows(R, Em) / Em[0] * sl, W) > lds_budget())
        --sl;
      const int ebox = lds_rows(R, Em) / Em[0] * sl;
      if (lean_lds_bytes(P, mode, ebox, W) > lds_budget()) continue;
      // staged rows per wave over all slabs, each extra slab (a restaging
      // round trip and barrier) counted as a quarter more
      const int nsl = (Em[0] + sl - 1) / sl;
      const double per_wave = (double)lds_rows(R, Em) / W * (1.0 + 0.25 * (nsl - 1));
      if (per_wave < best_per_wave * 0.999 ||
          (per_wave < best_per_wave * 1.001 && sl > best.sl)) {
        best_per_wave = per_wave;
        best.W = W;
        best.sa = sa;
        best.sl = sl;
        for (int a = 0; a < 3; ++a) best.Em[a] = Em[a];
        best.ok = true;
      }
    }
  // The rank-2 backward: a workgroup of 5 to 7 waves where its tile divides
  // every dilation phase exactly and fewer waves land on the busiest CU.
  // Every workgroup of such a launch is resident at once and the backward
  // is issue-bound, so the CU holding the most waves sets the time: at
  // 56 x 56 (config 2) 448 seven-wave workgroups put at most 14 waves on a
  // CU where 784 four-wave ones put 16 (13.9 vs 14.3 us; the forward,
  // lighter per wave, is not faster with them).  NATTEN_AMD_LEAN_WAVES
  // turns this off.
  if (best.ok && mode == kLBwd && R == 2 && !lean_waves_forced()) {
    auto tiles_of = [&](int W, int sa) {
      int64_t n = (int64_t)P.B * P.Hkv;
      for (int a = lead; a < 3; ++a) {
        const Axis &x = P.ax[a];
        const int tw = best.T[a] * (a == sa ? W : 1);
        n *= (int64_t)x.d * (((x.L + x.d - 1) / x.d + tw - 1) / tw);
      }
      return n;
    };
    auto busiest = [&](int W, int sa) {
      return (tiles_of(W, sa) + kLeanCUs - 1) / kLeanCUs * W;
    };
    int64_t cur = busiest(best.W, best.sa);
    for (int W = 7; W >= 5; --W)
      for (int sa = lead; sa < 3; ++sa) {
        const Axis &x = P.ax[sa];
        const int tw = best.T[sa] * W;
        if (x.L % x.d != 0 || (x.L / x.d) % tw != 0) continue;
        int Em[3];
        for (int a = 0; a < 3; ++a) Em[a] = ext(a, best.T[a] * (a == sa ? W : 1));
        const int ebox = lds_rows(R, Em);
        // resident two to a CU, no more staged rows per wave
        if (2 * lean_lds_bytes(P, mode, ebox, W) > (size_t)160 * 1024) continue;
        if ((double)ebox / W > best_per_wave) continue;
        const int64_t b = busiest(W, sa);
        if (b < cur) {
          cur = b;
          best.W = W;
          best.sa = sa;
          best.sl = Em[0];
          for (int a = 0; a < 3; ++a) best.Em[a] = Em[a];
        }
      }
  }
  return best;
}

// lean_choice, cached: a training loop plans the same few problems on every
// call, and the enumeration above costs microseconds of host time each time
// (several times per call: eligibility, workspace size, launch).  The key
// is every input the choice reads (the environment overrides it also reads
// are fixed for the process); the cache is per host thread, so it needs no
// lock, and keeps the last kPlanCache problems.
constexpr int kPlanCache = 8;
struct LChoiceKey {
  int32_t v[20];
};
LChoice lean_choice(const Prob &P, LMode mode) {
  LChoiceKey key{};
  int n = 0;
  key.v[n++] = (int32_t)mode;
  key.v[n++] = P.rank;
  key.v[n++] = P.D;
  key.v[n++] = P.kprod;
  key.v[n++] = P.n_extra;
  key.v[n++] = P.sample_extent != nullptr ? 1 : 0;
  key.v[n++] = P.B;
  key.v[n++] = P.Hkv;
  for (int a = 0; a < 3; ++a) {
    key.v[n++] = P.ax[a].L;
    key.v[n++] = P.ax[a].K;
    key.v[n++] = P.ax[a].d;
    key.v[n++] = P.ax[a].causal;
  }
  thread_local LChoiceKey keys[kPlanCache];
  thread_local LChoice vals[kPlanCache];
  thread_local int used = 0, next = 0;
  for (int i = 0; i < used; ++i)
    if (std::memcmp(&keys[i], &key, sizeof key) == 0) return vals[i];
  const LChoice c = lean_choice_compute(P, mode);
  keys[next] = key;
  vals[next] = c;
  next = (next + 1) % kPlanCache;
  used = std::min(used + 1, kPlanCache);
  return c;
}

LProb make_lprob(const Prob &P, const LChoice &C) {
  LProb L{};
  L.B = P.B;
  L.H = P.H;
  L.Hkv = P.Hkv;
  L.D = P.D;
  L.Ltot = P.ax[0].L * P.ax[1].L * P.ax[2].L;
  L.sl2 = P.scale * kLog2e;
  L.sa = C.sa;
  int tok = 1;
  int grid = 1;
  for (int a = 2; a >= 0; --a) {
    const Axis &x = P.ax[a];
    LAx &y = L.ax[a];
    y.L = x.L;
    y.K = x.K;
    y.d = x.d;
    y.causal = x.causal;
    y.nh = x.K / 2;
    y.Lq = x.L / x.d;
    y.Lrem = x.L % x.d;
    y.T = C.T[a];
    y.lgT = ilog2c(C.T[a]);
    y.TW = C.T[a] * (a == C.sa ? C.W : 1);
    y.lgTW = ilog2c(y.TW);
    y.Em = C.Em[a];
    const int Lr = (x.L + x.d - 1) / x.d;
    y.nt = (Lr + y.TW - 1) / y.TW;
    y.tok = tok;
    tok *= x.L;
    y.fG = make_fastdiv((uint32_t)(x.d * y.nt));
    y.fnt = make_fastdiv((uint32_t)y.nt);
    y.fd = make_fastdiv((uint32_t)x.d);
    grid *= x.d * y.nt;
  }
  L.ebox = lds_rows(P.rank, C.Em) / C.Em[0] * C.sl;
  L.sl = C.sl;
  L.hl = 0;
  L.fHg = make_fastdiv(1u);
  L.lgP2 = P.rank == 1 ? 0 : ilog2c(C.Em[2]);
  L.fGrid = make_fastdiv((uint32_t)grid);
  L.n_tiles = P.B * P.H * grid;
  L.n_launch = (L.n_tiles + 7) & ~7;
  L.fH = make_fastdiv((uint32_t)P.H);
  L.fRep = make_fastdiv((uint32_t)P.rep);
  L.fE1 = make_fastdiv((uint32_t)C.Em[1]);
  L.rep = P.rep;
  L.scale = P.scale;
  L.fHkv = make_fastdiv((uint32_t)P.Hkv);
  L.se = P.sample_extent;
  L.nx = P.n_extra;
  L.nxr = lean_nxr(P);
  L.kp = P.kprod;
  L.kst0 = P.ax[1].K * P.ax[2].K;
  L.kst1 = P.ax[2].K;
  return L;
}

bool lean_disabled();

// Dtype, head_dim, stride 1, the window rule of the lean kernels on every
// non-causal axis (odd K, d * K <= L) and the index arithmetic limits.
bool lean_shape_ok(const Prob &P, int dtype) {
  if (lean_disabled()) return false;
  if (dtype != NA_BF16 && dtype != NA_F16) return false;
  if (P.D != 32 && P.D != 64 && P.D != 128) return false;
  for (int a = 0; a < 3; ++a) {
    const Axis &x = P.ax[a];
    if (x.s != 1) return false;
    if (!x.causal && ((x.K % 2) == 0 || (int64_t)x.d * x.K > x.L)) return false;
  }
  // 32-bit element offsets
  const int64_t elems = (int64_t)P.B * P.ax[0].L * P.ax[1].L * P.ax[2].L *
                        std::max(P.H, P.Hkv) * P.D;
  if (elems >= (int64_t(1) << 31)) return false;
  // per-axis element strides fit the 24-bit multiplies of the staging code
  int64_t tok = 1;
  for (int a = 2; a >= 0; --a) {
    if ((int64_t)P.ax[a].d * tok * std::max(P.H, P.Hkv) * P.D >= (int64_t(1) << 24))
      return false;
    tok *= P.ax[a].L;
  }
  return true;
}

bool lean_disabled() {
  static const bool off = [] {
    const char *e = std::getenv("NATTEN_AMD_NO_LEAN");
    return e != nullptr && e[0] != '\0' && e[0] != '0';
  }();
  return off;
}

}  // namespace
}  // namespace na
