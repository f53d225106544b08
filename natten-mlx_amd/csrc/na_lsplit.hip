// na_lsplit.hip — lean matrix-core (gfx950) kernels for the split ops
// (na_qk_fwd / na_av_fwd and their backward) on the lean problem class
// (bf16/fp16, head_dim 32/64/128, stride 1, odd K with d*K <= L on every
// non-causal axis, no varlen, no additional tokens):
//
//   k_lqk  : out[q, slot] = scale * <x_q, y_key(slot)>, `fill` in the slots
//            outside the window (qk forward: x = q, y = k; av backward's
//            dattn: x = dO, y = v)
//   k_lav  : out_q = scale * sum over slots of a[q, slot] * y_key(slot)
//            (av forward: a = attn, y = v; qk backward's dq: a = dlogits,
//            y = k)
//   k_linv : z_key = scale * sum over the query heads of the key's group and
//            the queries q whose windows hold the key of
//            a[q, slot(q, key)] * x_q (qk backward's dk: a = dlogits,
//            x = q; av backward's dv: a = attn, x = dO)
//   k_lqh, k_lah : k_lqk and k_lav with every query head of a tile of 16
//            query positions in one workgroup (used where the heads fit)
//
// The tiling is the fused kernels' (na_lean.h): a wave owns 16 queries (or
// keys) of one dilation phase, W waves stacked along one axis form a
// workgroup, and the workgroup stages the box of rows its waves' windows
// cover in LDS once, here one tensor per row (row stride D + 8 elements).
// Each wave walks its sub-box in chunks of 16 rows through the MFMA; the
// compact rows [kprod] of the workgroup's queries pass through LDS and move
// to or from HBM a row at a time; k_linv gathers them from HBM instead
// (every element is used by exactly one key).
//
// Slot of key j in the window of query i: per axis (sub-grid coordinates)
// j - s(i) with s(i) = wend(i) - K, i.e. the window start on a non-causal
// axis and i - K + 1 on a causal one; slots are row-major over the axes
// (strides K1 K2, K2, 1), so slot = sum_a j_a st_a - sum_a s_a(i) st_a.
#include "na_lean.h"

namespace na {
namespace {

// An unsigned word of BYTES bytes (vector copies of 2-byte elements).
template <int BYTES>
struct RawWord;
template <>
struct RawWord<16> { typedef unsigned int type __attribute__((ext_vector_type(4))); };
template <>
struct RawWord<8> { typedef unsigned int type __attribute__((ext_vector_type(2))); };
template <>
struct RawWord<4> { typedef uint32_t type; };
template <>
struct RawWord<2> { typedef uint16_t type; };

// Stage a workgroup's box of rows of one tensor into LDS: box point (e0, e1,
// e2) at layout row ((e0 * Em1 + e1) << lgP2) + e2 (rank 1: e2), element
// row * (D + 8); layout points past the tile's true box are clamped onto it.
// The kSlack rows after the box are zeroed.
template <typename T, int D, int R>
__device__ __forceinline__ void stage_box1(const LProb &P, const LTile &t,
                                           const T *__restrict__ x,
                                           typename L16<T>::e *xs, int tid,
                                           int nthr, int s0) {
  typedef typename L16<T>::v8 v8;
  constexpr int OCT = D / 8;  // 16-byte units per row
  constexpr int RS = lds_y(D);
  const int nun = P.ebox * OCT;
  for (int u0 = 0; u0 < nun; u0 += 4 * nthr) {
    v8 xr[4];
    int g[4], la[4];
    unit_walk<R, OCT, RS>(P, t, u0, tid, nthr, s0, g, la);
#pragma unroll
    for (int j = 0; j < 4; ++j) xr[j] = ld8(x, g[j]);
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<v8 *>(xs + la[j]) = xr[j];
  }
  constexpr int SLU = kSlack * RS / 8;
  for (int u = tid; u < SLU; u += nthr) {
    v8 z;
#pragma unroll
    for (int i = 0; i < 8; ++i) z[i] = (typename L16<T>::e)0.f;
    *reinterpret_cast<v8 *>(xs + P.ebox * RS + 8 * u) = z;
  }
}

// The lane's row (query for k_lqk / k_lav, key for k_linv) of wave tile w:
// validity, element offset of the row (`heads` heads of head_dim D), its
// window (INV: inverse window) relative to the tile box, [wl, wl + ww) per
// axis (ww = 0 on every axis for rows outside the tensor), and its absolute
// sub-grid coordinates.
template <int R, bool INV>
__device__ __forceinline__ int lane_row(const LProb &P, const LTile &t,
                                        const WSub &ws, int n, int head,
                                        int heads, bool &valid, int wl[3],
                                        int ww[3], int idx[3]) {
  int u[3];
  const int lg2 = P.ax[2].lgT, lg1 = P.ax[1].lgT;
  u[2] = n & (P.ax[2].T - 1);
  u[1] = (n >> lg2) & (P.ax[1].T - 1);
  u[0] = n >> (lg2 + lg1);
  valid = ws.any;
  int tok = t.b * P.Ltot;
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    if (a < 3 - R) {
      wl[a] = 0;
      ww[a] = 1;
      idx[a] = 0;
      continue;
    }
    const LAx &x = P.ax[a];
    valid = valid && u[a] < ws.nv[a];
    // rows past the end take the tile's last row
    const int i = min(ws.i0[a] + min(u[a], max(ws.nv[a] - 1, 0)),
                      t.i0[a] + t.nv[a] - 1);
    tok += (t.r[a] + x.d * i) * x.tok;
    const int s0 = INV ? iwstart(x, i, t.Lr[a]) : wstart(x, i, t.Lr[a]);
    const int s1 = INV ? iwend(x, i, t.Lr[a]) : wend(x, i, t.Lr[a]);
    wl[a] = s0 - t.lo[a];
    ww[a] = s1 - s0;
    idx[a] = i;
  }
  if (!valid) ww[2] = 0;
  return tok * heads + head;
}

// Chunk j of a group: first LDS row, row test and the coordinates the slot
// arithmetic needs (box-relative e0, e1 and the first column).
struct ChunkPos {
  int kb;      // first LDS row
  bool rok;    // real chunk whose row lies in the lane's window
  int e0, e1;  // box coordinates of the chunk's row
  int e01;     // e0 * kst0 + e1 * kst1
  int col;     // box column of the chunk's first row
};

// Chunk ci of the walk; closed forms where the walk is one box row (rank 1)
// or one chunk per row (rank 2, CPR1), otherwise the cursor (chunks in
// order).
// LAYER3: the caller stages rank-3 boxes one layer (s0) per slab.
template <int R, bool CPR1, bool LAYER3 = false>
__device__ __forceinline__ ChunkPos chunk_pos(const LProb &P, const WSub &ws,
                                              Cursor &cc, int ci, int nch,
                                              int s0, int key0, const int wl[3],
                                              const int ww[3]) {
  ChunkPos c;
  const bool real = ci < nch;
  if (R == 1) {
    c.kb = key0 + (real ? 16 * ci : 0);
    c.rok = real;
    c.e0 = 0;
    c.e1 = 0;
    c.col = ws.ws[2] + 16 * ci;
  } else if (CPR1 && (R == 2 || LAYER3)) {
    // rank 2, or rank 3 whose slabs are one layer s0 (CPR1 rank-3 launches
    // use one-layer slabs only)
    c.kb = key0 + (real ? ci << P.lgP2 : 0);
    c.e0 = R == 3 ? s0 : 0;
    c.e1 = ws.ws[1] + ci;
    c.rok = real && (unsigned)(c.e1 - wl[1]) < (unsigned)ww[1];
    if (R == 3) c.rok = c.rok && (unsigned)(c.e0 - wl[0]) < (unsigned)ww[0];
    c.col = ws.ws[2];
  } else {
    c.kb = real ? (((cc.e0 - s0) * P.ax[1].Em + cc.e1) << P.lgP2) + ws.ws[2] + 16 * cc.cs
                : key0;
    bool ok = real;
    if (R > 1) ok = ok && (unsigned)(cc.e1 - wl[1]) < (unsigned)ww[1];
    if (R == 3) ok = ok && (unsigned)(cc.e0 - wl[0]) < (unsigned)ww[0];
    c.rok = ok;
    c.e0 = cc.e0;
    c.e1 = cc.e1;
    c.col = ws.ws[2] + 16 * cc.cs;
    advance(cc, ws);
  }
  c.e01 = c.e0 * P.kst0 + c.e1 * P.kst1;
  return c;
}

// ---------------------------------------------------------------------------
// k_lqk.  Per chunk S^T = Y_chunk . X^T (lane l: query l % 16, keys
// 4 (l / 16) + r), each in-window score to its slot of the query's row in
// LDS; then the rows to HBM.  FILL: some slots lie outside every window
// (a causal axis) and start as `fill`.
template <typename T, int D, int R, bool CPR1, bool CA>
__global__ void __launch_bounds__(512)
    k_lqk(LProb Pin, const T *__restrict__ x, const T *__restrict__ y,
          T *__restrict__ out, float scale, float fill, int prefill) {
  LProb P = Pin;  // without a causal axis the window rules fold to the clamped rule
  if constexpr (!CA) P.ax[0].causal = P.ax[1].causal = P.ax[2].causal = 0;
  typedef L16<T> M;
  typedef typename M::v8 v8;
  typedef typename M::e E;
  constexpr int NT = D / 32;
  constexpr int NB = 256 / D;  // chunks whose operands are read together
  constexpr int RS = lds_y(D);
  extern __shared__ __align__(16) char smem[];

  LTile t;
  const bool tile_any = decode_tile<R>(P, xcd_tile(blockIdx.x, P.n_launch), t);
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int n = lane & 15, gq = lane >> 4;
  const WSub ws = wave_sub<R>(P, t, w);
  bool qv;
  int wl[3], ww[3], qi[3];
  const int qrow = lane_row<R, false>(P, t, ws, n, t.head, P.H, qv, wl, ww, qi);
  // slot base of the lane's query (box-relative s_a = wl + ww - K)
  const int sq = (R == 3 ? (wl[0] + ww[0] - P.ax[0].K) * P.kst0 : 0) +
                 (R >= 2 ? (wl[1] + ww[1] - P.ax[1].K) * P.kst1 : 0) +
                 (wl[2] + (qv ? ww[2] : P.ax[2].K) - P.ax[2].K);
  if (!tile_any) return;  // uniform over the workgroup
  v8 qf[NT];
#pragma unroll
  for (int st = 0; st < NT; ++st) qf[st] = ld8(x, qrow * D + 32 * st + 8 * gq);

  E *ys = reinterpret_cast<E *>(smem);
  E *ob = ys + align16((P.ebox + kSlack) * RS * 2) / 2;
  const int kp = P.kp;
  if (prefill) {
    for (int i = tid; i < 16 * (nthr >> 6) * kp; i += nthr) ob[i] = (E)fill;
  }
  E *mine = ob + (16 * w + n) * kp;
  const int ka_off = n * RS + 8 * gq;
  const int nsl = R == 3 ? (t.E[0] + P.sl - 1) / P.sl : 1;
  const int rows1 = R > 1 ? ws.we[1] - ws.ws[1] : 1;
  for (int si = 0; si < nsl; ++si) {
    const int s0 = si * P.sl;
    if (si > 0) __syncthreads();  // the previous slab's reads are done
    stage_box1<T, D, R>(P, t, y, ys, tid, nthr, s0);
    __syncthreads();
    if (!ws.any) continue;
    const int a0 = R == 3 ? max(ws.ws[0], s0) : 0;
    const int b0 = R == 3 ? min(ws.we[0], s0 + P.sl) : 1;
    const int nch = b0 > a0 ? (b0 - a0) * rows1 * ws.cpr : 0;
    Cursor cc{a0, ws.ws[1], 0};
    const int key0 = (((a0 - s0) * P.ax[1].Em + ws.ws[1]) << P.lgP2) + ws.ws[2];
    for (int c0 = 0; c0 < nch; c0 += NB) {
      ChunkPos cp[NB];
#pragma unroll
      for (int j = 0; j < NB; ++j)
        cp[j] = chunk_pos<R, CPR1, true>(P, ws, cc, c0 + j, nch, s0, key0, wl, ww);
      v8 ka[NB][NT];
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int st = 0; st < NT; ++st)
          ka[j][st] = *reinterpret_cast<const v8 *>(ys + cp[j].kb * RS + ka_off + 32 * st);
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        f32x4 sv = zero4();
#pragma unroll
        for (int st = 0; st < NT; ++st) sv = M::mma(ka[j][st], qf[st], sv);
        const int xc = (CPR1 ? ws.ws[2] : cp[j].col) + 4 * gq;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool ok = cp[j].rok && (unsigned)(xc + r - wl[2]) < (unsigned)ww[2];
          if (ok) mine[cp[j].e01 + xc + r - sq] = (E)(sv[r] * scale);
        }
      }
    }
  }
  // the wave's 16 rows (written by this wave only) to HBM, four at a time
  wave_lds_sync();
  const uint64_t vb = __builtin_amdgcn_ballot_w64(qv);
  E *oe = reinterpret_cast<E *>(out);
  for (int p0 = 0; p0 < 16; p0 += 4) {
    for (int s = lane; s < kp; s += 64) {
      E vals[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) vals[j] = ob[(16 * w + p0 + j) * kp + s];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = __builtin_amdgcn_readlane(qrow, p0 + j);
        if ((vb >> (p0 + j)) & 1) oe[row * kp + s] = vals[j];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// k_lqh.  k_lqk with every query head of a tile of 16 query positions in one
// workgroup (wave w computes head w): the compact rows of one position are
// contiguous over the heads in memory ([.., position, H, kprod]), so the
// workgroup's output is 16 runs of H * kprod elements that go out as
// aligned vector stores.  The key rows of each chunk are read straight from
// memory as the MFMA's A operand (a wave's 16 queries have their own key
// sub-box, so nothing is shared through LDS and no barrier precedes the
// products); scores go to the LDS row buffer branch-free (out-of-window
// lanes write a per-lane spare slot past the rows).
template <typename T, int D, int R, bool CPR1, int VW, bool CA>
__device__ __forceinline__ void lqh_body(int bid, const LProb &Pin, const T *__restrict__ x,
                                         const T *__restrict__ y, T *__restrict__ out,
                                         float scale, float fill, int prefill, FastDiv fups) {
  LProb P = Pin;  // without a causal axis the window rules fold to the clamped rule
  if constexpr (!CA) P.ax[0].causal = P.ax[1].causal = P.ax[2].causal = 0;
  typedef L16<T> M;
  typedef typename M::v8 v8;
  typedef typename M::e E;
  constexpr int NT = D / 32;
  constexpr int NB = 256 / D;  // chunks whose operands are loaded together
  extern __shared__ __align__(16) char smem[];

  // tile: (sample, spatial tile of 16 queries); wave w: query head w
  const int tile = xcd_tile(bid, P.n_launch);
  const uint32_t bq = fdiv((uint32_t)tile, P.fGrid);
  const uint32_t sp = (uint32_t)tile - bq * P.fGrid.d;
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int n = lane & 15, gq = lane >> 4;
  LTile t;
  t.b = (int)bq;
  t.head = w;
  t.hk = (int)fdiv((uint32_t)w, P.fRep);
  const bool tile_any = tile_origin<R>(P, sp, t) & (t.b < P.B);
  if (!tile_any) return;  // uniform over the workgroup
  tile_box<R, false>(P, t, t.hk, P.Hkv);
  const WSub ws = wave_sub<R>(P, t, 0);
  bool qv;
  int wl[3], ww[3], qi[3];
  const int qrow = lane_row<R, false>(P, t, ws, n, t.head, P.H, qv, wl, ww, qi);
  const int sq = (R == 3 ? (wl[0] + ww[0] - P.ax[0].K) * P.kst0 : 0) +
                 (R >= 2 ? (wl[1] + ww[1] - P.ax[1].K) * P.kst1 : 0) +
                 (wl[2] + (qv ? ww[2] : P.ax[2].K) - P.ax[2].K);
  v8 qf[NT];
#pragma unroll
  for (int st = 0; st < NT; ++st) qf[st] = ld8(x, qrow * D + 32 * st + 8 * gq);

  const int kp = P.kp;
  const int rowlen = P.H * kp;  // one position: every head's compact row
  E *ob = reinterpret_cast<E *>(smem);
  E *mine = ob + n * rowlen + w * kp;
  const int spare = 16 * rowlen + lane - (n * rowlen + w * kp);  // from mine
  if (prefill) {
    for (int i = lane; i < 16 * kp; i += 64) {
      const int r = i / kp;  // small: division by the slot count
      ob[r * rowlen + w * kp + (i - r * kp)] = (E)fill;
    }
    wave_lds_sync();
  }
  const int rows1 = R > 1 ? ws.we[1] - ws.ws[1] : 1;
  const int nch = ws.any ? (R == 3 ? ws.we[0] - ws.ws[0] : 1) * rows1 * ws.cpr : 0;
  Cursor cc{R == 3 ? ws.ws[0] : 0, ws.ws[1], 0};
  // element offset of key column c of box row (e0, e1), clamped onto the box
  auto key_off = [&](int e0, int e1, int c) {
    int off = t.kbase + 8 * gq;
    if (R == 3) off += __umul24((unsigned)min(e0, t.E[0] - 1), (unsigned)t.SK[0]);
    if (R >= 2) off += __umul24((unsigned)min(e1, t.E[1] - 1), (unsigned)t.SK[1]);
    return off + __umul24((unsigned)min(c, t.E[2] - 1), (unsigned)t.SK[2]);
  };
  for (int c0 = 0; c0 < nch; c0 += NB) {
    ChunkPos cp[NB];
    v8 ka[NB][NT];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      cp[j] = chunk_pos<R, CPR1>(P, ws, cc, c0 + j, nch, 0, 0, wl, ww);
      const int off = key_off(cp[j].e0, cp[j].e1, cp[j].col + n);
#pragma unroll
      for (int st = 0; st < NT; ++st) ka[j][st] = ld8(y, off + 32 * st);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      f32x4 sv = zero4();
#pragma unroll
      for (int st = 0; st < NT; ++st) sv = M::mma(ka[j][st], qf[st], sv);
      const int xc = (CPR1 ? ws.ws[2] : cp[j].col) + 4 * gq;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = cp[j].rok && (unsigned)(xc + r - wl[2]) < (unsigned)ww[2];
        mine[ok ? cp[j].e01 + xc + r - sq : spare] = (E)(sv[r] * scale);
      }
    }
  }
  __syncthreads();  // every head's rows of the tile are in LDS

  // write-out: position p's run of rowlen elements goes to row
  // (token(p) * H) * kp, in units of VW elements (aligned: the host picks VW
  // so that rowlen is a multiple of it)
  typedef typename RawWord<VW * 2>::type VU;
  const int ups = rowlen / VW;  // units per position
  const int nun = 16 * ups;
  const int lg2 = P.ax[2].lgT, lg1 = P.ax[1].lgT;
  for (int u0 = 0; u0 < nun; u0 += 4 * nthr) {
    // four units per thread: their LDS reads together, then the stores
    VU val[4];
    size_t dst[4];
    bool ok[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int u = min(u0 + tid + j * nthr, nun - 1);
      const int p = (int)fdiv((uint32_t)u, fups);
      const int iu = u - p * ups;
      int uu[3];
      uu[2] = p & (P.ax[2].T - 1);
      uu[1] = (p >> lg2) & (P.ax[1].T - 1);
      uu[0] = p >> (lg2 + lg1);
      bool pv = u0 + tid + j * nthr < nun;
      int tok = t.b * P.Ltot;
#pragma unroll
      for (int a = 3 - R; a < 3; ++a) {
        const LAx &xa = P.ax[a];
        pv = pv && uu[a] < t.nv[a];
        tok += (t.r[a] + xa.d * (t.i0[a] + uu[a])) * xa.tok;
      }
      val[j] = *reinterpret_cast<const VU *>(ob + p * rowlen + iu * VW);
      dst[j] = (size_t)tok * rowlen + (size_t)iu * VW;
      ok[j] = pv;
    }
    // streaming stores: the compact rows are not read again here, and
    // they do not displace the inputs from the caches (qk 7.31 -> 7.0 us
    // at config 2)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (ok[j]) __builtin_nontemporal_store(val[j], reinterpret_cast<VU *>(out + dst[j]));
  }
}

// ---------------------------------------------------------------------------
// k_lah.  k_lav with every query head of a tile of 16 query positions in one
// workgroup (wave w computes head w): the tile's compact rows, contiguous
// over the heads per position, come in as aligned vector loads; each wave
// stages the Y rows of its own chunks (a group at a time) in a private LDS
// area for the transposing read, so only the compact rows pass a
// workgroup barrier.
template <typename T, int D, int R, bool CPR1, int VW, bool CA>
__device__ __forceinline__ void lah_body(int bid, const LProb &Pin, const T *__restrict__ a,
                                         const T *__restrict__ y, T *__restrict__ out,
                                         float scale, FastDiv fups) {
  LProb P = Pin;  // without a causal axis the window rules fold to the clamped rule
  if constexpr (!CA) P.ax[0].causal = P.ax[1].causal = P.ax[2].causal = 0;
  typedef L16<T> M;
  typedef typename M::v8 v8;
  typedef typename M::v4 v4;
  typedef typename M::e E;
  constexpr int NT = D / 32;
  constexpr int NB = D == 128 ? 2 : 4;  // chunks staged together (even)
  constexpr int NDB = D / 16;
  constexpr int RS = lds_y(D);
  extern __shared__ __align__(16) char smem[];

  const int tile = xcd_tile(bid, P.n_launch);
  const uint32_t bq = fdiv((uint32_t)tile, P.fGrid);
  const uint32_t sp = (uint32_t)tile - bq * P.fGrid.d;
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int n = lane & 15, gq = lane >> 4;
  LTile t;
  t.b = (int)bq;
  t.head = w;
  t.hk = (int)fdiv((uint32_t)w, P.fRep);
  const bool tile_any = tile_origin<R>(P, sp, t) & (t.b < P.B);
  if (!tile_any) return;  // uniform over the workgroup
  tile_box<R, false>(P, t, t.hk, P.Hkv);
  const WSub ws = wave_sub<R>(P, t, 0);
  bool qv;
  int wl[3], ww[3], qi[3];
  const int qrow = lane_row<R, false>(P, t, ws, n, t.head, P.H, qv, wl, ww, qi);
  const int sq = (R == 3 ? (wl[0] + ww[0] - P.ax[0].K) * P.kst0 : 0) +
                 (R >= 2 ? (wl[1] + ww[1] - P.ax[1].K) * P.kst1 : 0) +
                 (wl[2] + (qv ? ww[2] : P.ax[2].K) - P.ax[2].K);

  const int kp = P.kp;
  const int rowlen = P.H * kp;
  E *ab = reinterpret_cast<E *>(smem);  // [16 positions][H][kp]
  E *ys = ab + align16(16 * rowlen);     // per wave: NB chunks of 16 rows
  E *yw = ys + w * NB * 16 * RS;
  // the tile's compact rows, position by position (runs of rowlen), four
  // units per thread in flight at a time.  Positions past the tile's valid
  // extent load a valid position's row (clamped): only the rows of queries
  // that are not stored read them.  Indices past the end are clamped onto
  // the last unit, so neither the loads nor the stores branch.
  typedef typename RawWord<VW * 2>::type VU;
  const int ups = rowlen / VW;
  const int nun = 16 * ups;
  const int lg2 = P.ax[2].lgT, lg1 = P.ax[1].lgT;
  for (int u0 = 0; u0 < nun; u0 += 4 * nthr) {
    VU val[4];
    int dst[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int u = min(u0 + tid + j * nthr, nun - 1);
      const int p = (int)fdiv((uint32_t)u, fups);
      const int iu = u - p * ups;
      int uu[3];
      uu[2] = p & (P.ax[2].T - 1);
      uu[1] = (p >> lg2) & (P.ax[1].T - 1);
      uu[0] = p >> (lg2 + lg1);
      int tok = t.b * P.Ltot;
#pragma unroll
      for (int ax = 3 - R; ax < 3; ++ax) {
        const LAx &xa = P.ax[ax];
        tok += (t.r[ax] + xa.d * (t.i0[ax] + min(uu[ax], max(t.nv[ax] - 1, 0)))) * xa.tok;
      }
      val[j] = *reinterpret_cast<const VU *>(a + (size_t)tok * rowlen + (size_t)iu * VW);
      dst[j] = p * rowlen + iu * VW;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<VU *>(ab + dst[j]) = val[j];
  }
  __syncthreads();
  const E *mine = ab + n * rowlen + w * kp;

  f32x4 o[NDB];
#pragma unroll
  for (int j = 0; j < NDB; ++j) o[j] = zero4();
  const int tr_off = (4 * gq + (n >> 2)) * RS + 4 * (n & 3);
  const int rows1 = R > 1 ? ws.we[1] - ws.ws[1] : 1;
  const int nch = ws.any ? (R == 3 ? ws.we[0] - ws.ws[0] : 1) * rows1 * ws.cpr : 0;
  Cursor cc{R == 3 ? ws.ws[0] : 0, ws.ws[1], 0};
  auto row_off = [&](int e0, int e1, int c) {
    int off = t.kbase + 8 * gq;
    if (R == 3) off += __umul24((unsigned)min(e0, t.E[0] - 1), (unsigned)t.SK[0]);
    if (R >= 2) off += __umul24((unsigned)min(e1, t.E[1] - 1), (unsigned)t.SK[1]);
    return off + __umul24((unsigned)min(c, t.E[2] - 1), (unsigned)t.SK[2]);
  };
  for (int c0 = 0; c0 < nch; c0 += NB) {
    ChunkPos cp[NB];
    v8 yr[NB][NT];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      cp[j] = chunk_pos<R, CPR1>(P, ws, cc, c0 + j, nch, 0, 0, wl, ww);
      const int off = row_off(cp[j].e0, cp[j].e1, cp[j].col + n);
#pragma unroll
      for (int st = 0; st < NT; ++st) yr[j][st] = ld8(y, off + 32 * st);
    }
    // B operand: query n's weights of keys 4 (l / 16) + r of each chunk
    v8 bp[NB / 2];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int xc = (CPR1 ? ws.ws[2] : cp[j].col) + 4 * gq;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        // read unconditionally (slot 0 of the row outside the window), then
        // select: no branch per element
        const bool ok = cp[j].rok && (unsigned)(xc + r - wl[2]) < (unsigned)ww[2];
        const E av = mine[ok ? cp[j].e01 + xc + r - sq : 0];
        bp[j >> 1][4 * (j & 1) + r] = ok ? av : (E)0.f;
      }
    }
    wave_lds_sync();  // the previous group's transposing reads are done
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int st = 0; st < NT; ++st)
        *reinterpret_cast<v8 *>(yw + (16 * j + n) * RS + 32 * st + 8 * gq) = yr[j][st];
    wave_lds_sync();
#pragma unroll
    for (int jj = 0; jj < NB / 2; ++jj) {
      const E *ca = yw + 32 * jj * RS + tr_off;
      const E *cb = ca + 16 * RS;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const v4 lo4 = M::tr(ca + 16 * db);
        const v4 hi4 = M::tr(cb + 16 * db);
        const v8 av = __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
        o[db] = M::mma(av, bp[jj], o[db]);
      }
    }
  }
  if (!qv) return;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    v4 wv;
#pragma unroll
    for (int r = 0; r < 4; ++r) wv[r] = (E)(o[db][r] * scale);
    *reinterpret_cast<v4 *>(out + qrow * D + 16 * db + 4 * gq) = wv;
  }
}

// ---------------------------------------------------------------------------
// k_lav.  The wave's 16 compact rows to LDS; per pair of chunks the B
// operand (query n, keys 4 (l / 16) + r of each chunk) is gathered from them
// by slot (zero outside the window) and O^T += Y^T . A^T with Y^T through
// the transposing LDS read.
template <typename T, int D, int R, bool CPR1, bool CA>
__global__ void __launch_bounds__(512)
    k_lav(LProb Pin, const T *__restrict__ a, const T *__restrict__ y,
          T *__restrict__ out, float scale) {
  LProb P = Pin;  // without a causal axis the window rules fold to the clamped rule
  if constexpr (!CA) P.ax[0].causal = P.ax[1].causal = P.ax[2].causal = 0;
  typedef L16<T> M;
  typedef typename M::v8 v8;
  typedef typename M::v4 v4;
  typedef typename M::e E;
  constexpr int NB = D == 128 ? 2 : 4;  // chunks read together
  constexpr int NDB = D / 16;
  constexpr int RS = lds_y(D);
  extern __shared__ __align__(16) char smem[];

  LTile t;
  const bool tile_any = decode_tile<R>(P, xcd_tile(blockIdx.x, P.n_launch), t);
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int n = lane & 15, gq = lane >> 4;
  const WSub ws = wave_sub<R>(P, t, w);
  bool qv;
  int wl[3], ww[3], qi[3];
  const int qrow = lane_row<R, false>(P, t, ws, n, t.head, P.H, qv, wl, ww, qi);
  const int sq = (R == 3 ? (wl[0] + ww[0] - P.ax[0].K) * P.kst0 : 0) +
                 (R >= 2 ? (wl[1] + ww[1] - P.ax[1].K) * P.kst1 : 0) +
                 (wl[2] + (qv ? ww[2] : P.ax[2].K) - P.ax[2].K);
  if (!tile_any) return;  // uniform over the workgroup

  E *ys = reinterpret_cast<E *>(smem);
  E *ab = ys + align16((P.ebox + kSlack) * RS * 2) / 2;
  const int kp = P.kp;
  // the wave's 16 compact rows, all loads in flight together (issued
  // before the box staging)
  const uint64_t vb = __builtin_amdgcn_ballot_w64(qv);
  const E *ae = reinterpret_cast<const E *>(a);
  for (int s0 = 0; s0 < kp; s0 += 64) {
    const int s = s0 + lane;
    const bool in = s < kp;
    E vals[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int row = __builtin_amdgcn_readlane(qrow, j);
      vals[j] = in && ((vb >> j) & 1) ? ae[row * kp + s] : (E)0.f;
    }
    if (in) {
#pragma unroll
      for (int j = 0; j < 16; ++j) ab[(16 * w + j) * kp + s] = vals[j];
    }
  }
  const E *mine = ab + (16 * w + n) * kp;

  f32x4 o[NDB];
#pragma unroll
  for (int j = 0; j < NDB; ++j) o[j] = zero4();
  const int tr_off = (4 * gq + (n >> 2)) * RS + 4 * (n & 3);
  const int nsl = R == 3 ? (t.E[0] + P.sl - 1) / P.sl : 1;
  const int rows1 = R > 1 ? ws.we[1] - ws.ws[1] : 1;
  for (int si = 0; si < nsl; ++si) {
    const int s0 = si * P.sl;
    if (si > 0) __syncthreads();  // the previous slab's reads are done
    stage_box1<T, D, R>(P, t, y, ys, tid, nthr, s0);
    __syncthreads();
    if (!ws.any) continue;
    const int a0 = R == 3 ? max(ws.ws[0], s0) : 0;
    const int b0 = R == 3 ? min(ws.we[0], s0 + P.sl) : 1;
    const int nch = b0 > a0 ? (b0 - a0) * rows1 * ws.cpr : 0;
    Cursor cc{a0, ws.ws[1], 0};
    const int key0 = (((a0 - s0) * P.ax[1].Em + ws.ws[1]) << P.lgP2) + ws.ws[2];
    for (int c0 = 0; c0 < nch; c0 += NB) {
      ChunkPos cp[NB];
#pragma unroll
      for (int j = 0; j < NB; ++j)
        cp[j] = chunk_pos<R, CPR1, true>(P, ws, cc, c0 + j, nch, s0, key0, wl, ww);
      v8 bp[NB / 2];
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int xc = (CPR1 ? ws.ws[2] : cp[j].col) + 4 * gq;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool ok = cp[j].rok && (unsigned)(xc + r - wl[2]) < (unsigned)ww[2];
          bp[j >> 1][4 * (j & 1) + r] = ok ? mine[cp[j].e01 + xc + r - sq] : (E)0.f;
        }
      }
#pragma unroll
      for (int jj = 0; jj < NB / 2; ++jj) {
        const E *ca = ys + cp[2 * jj].kb * RS + tr_off;
        const E *cb = ys + cp[2 * jj + 1].kb * RS + tr_off;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const v4 lo4 = M::tr(ca + 16 * db);
          const v4 hi4 = M::tr(cb + 16 * db);
          const v8 av = __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
          o[db] = M::mma(av, bp[jj], o[db]);
        }
      }
    }
  }
  if (!qv) return;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    v4 wv;
#pragma unroll
    for (int r = 0; r < 4; ++r) wv[r] = (E)(o[db][r] * scale);
    *reinterpret_cast<v4 *>(out + qrow * D + 16 * db + 4 * gq) = wv;
  }
}

// ---------------------------------------------------------------------------
// k_linv.  A workgroup owns a tile of keys of one key/value head; per query
// head of the group it stages the X rows of the query box of the keys'
// inverse windows.  Per pair of chunks of 16 queries the B operand (queries
// 4 (l / 16) + r of each chunk, key l % 16) is a[q, J - S(q)] inside the
// key's inverse window, gathered from HBM (J = sum_a j_a st_a of the lane's
// key, S(q) = sum_a s_a(q) st_a), and Z^T += X^T . A with X^T through the
// transposing LDS read.  The gathers of a group of chunk pairs are issued
// together; every compact-row element is read by exactly one key.
template <typename T, int D, int R, bool CPR1, bool CA>
__device__ __forceinline__ void linv_body(int bid, const LProb &Pin, const T *__restrict__ a,
                                          const T *__restrict__ x, T *__restrict__ z,
                                          float scale) {
  LProb P = Pin;  // without a causal axis the window rules fold to the clamped rule
  if constexpr (!CA) P.ax[0].causal = P.ax[1].causal = P.ax[2].causal = 0;
  typedef L16<T> M;
  typedef typename M::v8 v8;
  typedef typename M::v4 v4;
  typedef typename M::e E;
  constexpr int NDB = D / 16;
  // chunk pairs whose gathers are issued together: one.  Each gathered
  // element carries its own address, so more pairs in flight cost
  // registers: at four the backward pairs (k_lqkb / k_lavb) took 108 VGPRs,
  // four waves per SIMD and 1.5 rounds of workgroups at config 2 (qk / av
  // backward 12.05 / 11.79 us), at two 76 (10.97 / 10.70 us), at one 60 /
  // 71 (10.74 / 10.13 us).
  constexpr int NP = 1;
  constexpr int RS = lds_y(D);
  extern __shared__ __align__(16) char smem[];

  // tile: (batch, key/value head, spatial tile)
  const int tile = xcd_tile(bid, P.n_launch);
  const uint32_t rest = fdiv((uint32_t)tile, P.fGrid);
  const uint32_t sp = (uint32_t)tile - rest * P.fGrid.d;
  const uint32_t bq = fdiv(rest, P.fHkv);
  LTile t;
  t.hk = (int)(rest - bq * P.fHkv.d);
  t.b = (int)bq;
  t.head = t.hk * P.rep;
  const bool tile_any = tile_origin<R>(P, sp, t) & (t.b < P.B);
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int n = lane & 15, gq = lane >> 4;
  if (!tile_any) return;  // uniform over the workgroup
  tile_box<R, true>(P, t, t.head, P.H);
  const WSub ws = wave_sub<R, true>(P, t, w);
  bool kv;
  int wl[3], ww[3], kj[3];
  const int krow = lane_row<R, true>(P, t, ws, n, t.hk, P.Hkv, kv, wl, ww, kj);
  const int J = (R == 3 ? kj[0] * P.kst0 : 0) + (R >= 2 ? kj[1] * P.kst1 : 0) + kj[2];

  E *xs = reinterpret_cast<E *>(smem);
  const E *ae = reinterpret_cast<const E *>(a);
  const int kp = P.kp;
  const LAx &x2 = P.ax[2];
  f32x4 acc[NDB];
#pragma unroll
  for (int j = 0; j < NDB; ++j) acc[j] = zero4();
  const int tr_off = (4 * gq + (n >> 2)) * RS + 4 * (n & 3);
  const int qbase0 = t.kbase;  // X rows of query head hk * rep
  const int nsl = R == 3 ? (t.E[0] + P.sl - 1) / P.sl : 1;
  const int rows1 = R > 1 ? ws.we[1] - ws.ws[1] : 1;
  const int Em1 = P.ax[1].Em;
  for (int hr = 0; hr < P.rep; ++hr) {
    t.kbase = qbase0 + hr * D;
    const int head = t.head + hr;
    for (int si = 0; si < nsl; ++si) {
      const int s0 = si * P.sl;
      __syncthreads();  // the LDS reads of the previous box or slab are done
      stage_box1<T, D, R>(P, t, x, xs, tid, nthr, s0);
      __syncthreads();
      if (!ws.any) continue;
      const int a0 = R == 3 ? max(ws.ws[0], s0) : 0;
      const int b0 = R == 3 ? min(ws.we[0], s0 + P.sl) : 1;
      const int nch = b0 > a0 ? (b0 - a0) * rows1 * ws.cpr : 0;
      Cursor cc{a0, ws.ws[1], 0};
      const int key0 = (((a0 - s0) * Em1 + ws.ws[1]) << P.lgP2) + ws.ws[2];
      for (int c0 = 0; c0 < nch; c0 += 2 * NP) {
        ChunkPos cp[2 * NP];
        v8 bp[NP];
#pragma unroll
        for (int j = 0; j < 2 * NP; ++j) {
          cp[j] = chunk_pos<R, CPR1, true>(P, ws, cc, c0 + j, nch, s0, key0, wl, ww);
          // the chunk's row: slot-base and token parts of axes 0 and 1
          int sb01 = 0, tok01 = t.b * P.Ltot + t.r[2];
          if (R == 3) {
            const int i0 = t.lo[0] + cp[j].e0;
            sb01 += (wend(P.ax[0], i0, t.Lr[0]) - P.ax[0].K) * P.kst0;
            tok01 += (t.r[0] + P.ax[0].d * i0) * P.ax[0].tok;
          }
          if (R >= 2) {
            const int i1 = t.lo[1] + cp[j].e1;
            sb01 += (wend(P.ax[1], i1, t.Lr[1]) - P.ax[1].K) * P.kst1;
            tok01 += (t.r[1] + P.ax[1].d * i1) * P.ax[1].tok;
          }
          const int xc = (CPR1 ? ws.ws[2] : cp[j].col) + 4 * gq;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const bool ok = cp[j].rok && (unsigned)(xc + r - wl[2]) < (unsigned)ww[2];
            const int i2 = t.lo[2] + xc + r;
            const int sq = sb01 + wend(x2, i2, t.Lr[2]) - x2.K;
            const int row = (tok01 + x2.d * i2) * P.H + head;
            bp[j >> 1][4 * (j & 1) + r] = ok ? ae[row * kp + J - sq] : (E)0.f;
          }
        }
#pragma unroll
        for (int jj = 0; jj < NP; ++jj) {
#pragma unroll
          for (int db = 0; db < NDB; ++db) {
            const v4 x0 = M::tr(xs + cp[2 * jj].kb * RS + tr_off + 16 * db);
            const v4 x1 = M::tr(xs + cp[2 * jj + 1].kb * RS + tr_off + 16 * db);
            const v8 xt = __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
            acc[db] = M::mma(xt, bp[jj], acc[db]);
          }
        }
      }
    }
  }
  if (!kv) return;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    v4 wv;
#pragma unroll
    for (int r = 0; r < 4; ++r) wv[r] = (E)(acc[db][r] * scale);
    *reinterpret_cast<v4 *>(z + krow * D + 16 * db + 4 * gq) = wv;
  }
}

template <typename T, int D, int R, bool CPR1, int VW, bool CA>
__global__ void __launch_bounds__(1024)
    k_lqh(LProb P, const T *__restrict__ x, const T *__restrict__ y, T *__restrict__ out,
          float scale, float fill, int prefill, FastDiv fups) {
  lqh_body<T, D, R, CPR1, VW, CA>((int)blockIdx.x, P, x, y, out, scale, fill, prefill, fups);
}

template <typename T, int D, int R, bool CPR1, int VW, bool CA>
__global__ void __launch_bounds__(1024)
    k_lah(LProb P, const T *__restrict__ a, const T *__restrict__ y, T *__restrict__ out,
          float scale, FastDiv fups) {
  lah_body<T, D, R, CPR1, VW, CA>((int)blockIdx.x, P, a, y, out, scale, fups);
}

template <typename T, int D, int R, bool CPR1, bool CA>
__global__ void __launch_bounds__(512)
    k_linv(LProb P, const T *__restrict__ a, const T *__restrict__ x, T *__restrict__ z,
           float scale) {
  linv_body<T, D, R, CPR1, CA>((int)blockIdx.x, P, a, x, z, scale);
}

// A backward's two passes in one launch (they are independent and their
// workgroups have the same size): n0 blocks of the all-heads pass (dq by
// k_lah over dlogits and the keys, or dattn by k_lqh over dout and the
// values), the rest the inverse pass (dk from dlogits and the queries, or
// dv from attn and dout) on their own problem description; k_lqkb puts the
// all-heads blocks first, k_lavb the inverse ones.
template <typename T, int D, int R, bool CPR1, int VW, bool CA>
__global__ void __launch_bounds__(1024)
    k_lqkb(LProb Pa, LProb Pi, const T *__restrict__ dl, const T *__restrict__ key,
           const T *__restrict__ q, T *__restrict__ dq, T *__restrict__ dk, float scale,
           FastDiv fups, int n0) {
  const int bid = (int)blockIdx.x;
  if (bid < n0)
    lah_body<T, D, R, CPR1, VW, CA>(bid, Pa, dl, key, dq, scale, fups);
  else
    linv_body<T, D, R, CPR1, CA>(bid - n0, Pi, dl, q, dk, scale);
}

template <typename T, int D, int R, bool CPR1, int VW, bool CA>
__global__ void __launch_bounds__(1024)
    k_lavb(LProb Pa, LProb Pi, const T *__restrict__ attn, const T *__restrict__ v,
           const T *__restrict__ dout, T *__restrict__ dattn, T *__restrict__ dv, int prefill,
           FastDiv fups, int n0) {
  // the inverse pass's blocks are dispatched first here (config 2 AV
  // backward 10.27 -> 9.87 us; the QK pair keeps the all-heads pass first,
  // 10.80 against 10.88 us)
  const int bid = (int)blockIdx.x;
  const int ni = (int)gridDim.x - n0;
  if (bid >= ni)
    lqh_body<T, D, R, CPR1, VW, CA>(bid - ni, Pa, dout, v, dattn, 1.f, 0.f, prefill, fups);
  else
    linv_body<T, D, R, CPR1, CA>(bid, Pi, attn, dout, dv, 1.f);
}

}  // namespace

bool lsplit_eligible(const Prob &P, int dtype) {
  if (!lean_shape_ok(P, dtype)) return false;
  if (P.dense || P.n_extra > 0 || P.sample_extent != nullptr) return false;
  // 32-bit offsets into the compact rows
  if ((int64_t)P.B * P.ax[0].L * P.ax[1].L * P.ax[2].L * P.H * P.kprod >=
      (int64_t(1) << 31))
    return false;
  return lean_choice(P, kLQK).ok && lean_choice(P, kLInv).ok;
}

#define LS_D(D_, BODY) \
  do {                 \
    if ((D_) == 32) {  \
      BODY(32);        \
    } else if ((D_) == 64) { \
      BODY(64);        \
    } else {           \
      BODY(128);       \
    }                  \
  } while (0)

// Launch KERNEL<T, D, R, CPR1> for the problem's dtype, head_dim and rank.
#define LS_DISPATCH(KERNEL, ARGS)                                               \
  do {                                                                          \
    auto go = [&](auto tt, auto dd, auto rr, auto cc) {                         \
      typedef decltype(tt) TT;                                                  \
      constexpr int DD = decltype(dd)::value, RR = decltype(rr)::value;         \
      constexpr bool CC = decltype(cc)::value;                                  \
      if (ca)                                                                   \
        hipLaunchKernelGGL((KERNEL<TT, DD, RR, CC, true>), grid, block, lds, st, L, \
                           ARGS);                                               \
      else                                                                      \
        hipLaunchKernelGGL((KERNEL<TT, DD, RR, CC, false>), grid, block, lds, st, L, \
                           ARGS);                                               \
    };                                                                          \
    auto by_r = [&](auto tt, auto dd) {                                         \
      if (P.rank == 1)                                                          \
        go(tt, dd, std::integral_constant<int, 1>(), std::false_type());        \
      else if (P.rank == 2) {                                                   \
        if (C.cpr1) go(tt, dd, std::integral_constant<int, 2>(), std::true_type()); \
        else go(tt, dd, std::integral_constant<int, 2>(), std::false_type());   \
      } else {                                                                  \
        if (C.cpr1 && C.sl == 1) go(tt, dd, std::integral_constant<int, 3>(), std::true_type()); \
        else go(tt, dd, std::integral_constant<int, 3>(), std::false_type());   \
      }                                                                         \
    };                                                                          \
    auto by_d = [&](auto tt) {                                                  \
      if (P.D == 32) by_r(tt, std::integral_constant<int, 32>());               \
      else if (P.D == 64) by_r(tt, std::integral_constant<int, 64>());          \
      else by_r(tt, std::integral_constant<int, 128>());                        \
    };                                                                          \
    if (dtype == NA_BF16) by_d(bf16_t());                                       \
    else by_d(f16_t());                                                         \
  } while (0)

// k_lqh's launch: every query head of a 16-query tile in one workgroup
// (at most 16 heads and 64 KB of rows), rows written in units of VW
// elements; false when it does not apply.
struct LqhPlan {
  int vw;
  size_t lds;
};
bool lqh_plan(const Prob &P, LqhPlan *pl) {
  if (P.H > 16) return false;
  const int rowlen = P.H * P.kprod;
  pl->lds = (size_t)16 * rowlen * 2 + 64 * 2;
  if (pl->lds > 65536) return false;
  pl->vw = rowlen % 8 == 0 ? 8 : rowlen % 4 == 0 ? 4 : rowlen % 2 == 0 ? 2 : 1;
  return true;
}

void lsplit_qk(const Prob &P, int dtype, const void *x, const void *y,
               void *out, float scale, float fill, hipStream_t st) {
  const bool ca = P.ax[0].causal || P.ax[1].causal || P.ax[2].causal;
  const LChoice C = lean_choice(P, kLQK);
  int prefill = 0;
  for (int a = 0; a < 3; ++a) prefill |= P.ax[a].causal;
  LqhPlan pl;
  if (lqh_plan(P, &pl)) {
    LChoice C1 = C;  // one wave tile per workgroup (waves are heads)
    C1.W = 1;
    LProb L = make_lprob(P, C1);
    L.n_tiles = P.B * (int)L.fGrid.d;
    L.n_launch = (L.n_tiles + 7) & ~7;
    if (L.n_tiles == 0) return;
    const FastDiv fups = make_fastdiv((uint32_t)(P.H * P.kprod / pl.vw));
    const dim3 grid(L.n_launch), block(64 * P.H);
    const size_t lds = pl.lds;
    auto go = [&](auto tt, auto dd, auto rr, auto cc, auto vv) {
      typedef decltype(tt) TT;
      constexpr int DD = decltype(dd)::value, RR = decltype(rr)::value;
      constexpr bool CC = decltype(cc)::value;
      constexpr int VV = decltype(vv)::value;
      if (ca)
        hipLaunchKernelGGL((k_lqh<TT, DD, RR, CC, VV, true>), grid, block, lds, st, L,
                           (const TT *)x, (const TT *)y, (TT *)out, scale, fill, prefill,
                           fups);
      else
        hipLaunchKernelGGL((k_lqh<TT, DD, RR, CC, VV, false>), grid, block, lds, st, L,
                           (const TT *)x, (const TT *)y, (TT *)out, scale, fill, prefill,
                           fups);
    };
    auto by_v = [&](auto tt, auto dd, auto rr, auto cc) {
      if (pl.vw == 8) go(tt, dd, rr, cc, std::integral_constant<int, 8>());
      else if (pl.vw == 4) go(tt, dd, rr, cc, std::integral_constant<int, 4>());
      else if (pl.vw == 2) go(tt, dd, rr, cc, std::integral_constant<int, 2>());
      else go(tt, dd, rr, cc, std::integral_constant<int, 1>());
    };
    auto by_r = [&](auto tt, auto dd) {
      if (P.rank == 1)
        by_v(tt, dd, std::integral_constant<int, 1>(), std::false_type());
      else if (P.rank == 2) {
        if (C.cpr1) by_v(tt, dd, std::integral_constant<int, 2>(), std::true_type());
        else by_v(tt, dd, std::integral_constant<int, 2>(), std::false_type());
      } else {
        if (C.cpr1 && C.sl == 1) by_v(tt, dd, std::integral_constant<int, 3>(), std::true_type());
        else by_v(tt, dd, std::integral_constant<int, 3>(), std::false_type());
      }
    };
    auto by_d = [&](auto tt) {
      if (P.D == 32) by_r(tt, std::integral_constant<int, 32>());
      else if (P.D == 64) by_r(tt, std::integral_constant<int, 64>());
      else by_r(tt, std::integral_constant<int, 128>());
    };
    if (dtype == NA_BF16) by_d(bf16_t());
    else by_d(f16_t());
    return;
  }
  const LProb L = make_lprob(P, C);
  if (L.n_tiles == 0) return;
  const size_t lds = lean_lds_bytes(P, kLQK, L.ebox, C.W);
  const dim3 grid(L.n_launch), block(64 * C.W);
#define LS_ARGS_QK(TT) (const TT *)x, (const TT *)y, (TT *)out, scale, fill, prefill
  LS_DISPATCH(k_lqk, LS_ARGS_QK(TT));
#undef LS_ARGS_QK
}

void lsplit_av(const Prob &P, int dtype, const void *a, const void *y,
               void *out, float scale, hipStream_t st) {
  const bool ca = P.ax[0].causal || P.ax[1].causal || P.ax[2].causal;
  const LChoice C = lean_choice(P, kLQK);
  LqhPlan pl;
  // k_lah's LDS: the tile's compact rows and, per wave, NB chunks of 16 rows
  const int nb = P.D == 128 ? 2 : 4;
  const size_t lah_lds = (size_t)align16(16 * P.H * P.kprod) * 2 +
                         (size_t)P.H * nb * 16 * lds_y(P.D) * 2;
  if (lqh_plan(P, &pl) && lah_lds <= 65536) {
    LChoice C1 = C;  // one wave tile per workgroup (waves are heads)
    C1.W = 1;
    LProb L = make_lprob(P, C1);
    L.n_tiles = P.B * (int)L.fGrid.d;
    L.n_launch = (L.n_tiles + 7) & ~7;
    if (L.n_tiles == 0) return;
    const FastDiv fups = make_fastdiv((uint32_t)(P.H * P.kprod / pl.vw));
    const dim3 grid(L.n_launch), block(64 * P.H);
    auto go = [&](auto tt, auto dd, auto rr, auto cc, auto vv) {
      typedef decltype(tt) TT;
      constexpr int DD = decltype(dd)::value, RR = decltype(rr)::value;
      constexpr bool CC = decltype(cc)::value;
      constexpr int VV = decltype(vv)::value;
      if (ca)
        hipLaunchKernelGGL((k_lah<TT, DD, RR, CC, VV, true>), grid, block, lah_lds, st, L,
                           (const TT *)a, (const TT *)y, (TT *)out, scale, fups);
      else
        hipLaunchKernelGGL((k_lah<TT, DD, RR, CC, VV, false>), grid, block, lah_lds, st, L,
                           (const TT *)a, (const TT *)y, (TT *)out, scale, fups);
    };
    auto by_v = [&](auto tt, auto dd, auto rr, auto cc) {
      if (pl.vw == 8) go(tt, dd, rr, cc, std::integral_constant<int, 8>());
      else if (pl.vw == 4) go(tt, dd, rr, cc, std::integral_constant<int, 4>());
      else if (pl.vw == 2) go(tt, dd, rr, cc, std::integral_constant<int, 2>());
      else go(tt, dd, rr, cc, std::integral_constant<int, 1>());
    };
    auto by_r = [&](auto tt, auto dd) {
      if (P.rank == 1)
        by_v(tt, dd, std::integral_constant<int, 1>(), std::false_type());
      else if (P.rank == 2) {
        if (C.cpr1) by_v(tt, dd, std::integral_constant<int, 2>(), std::true_type());
        else by_v(tt, dd, std::integral_constant<int, 2>(), std::false_type());
      } else {
        if (C.cpr1 && C.sl == 1) by_v(tt, dd, std::integral_constant<int, 3>(), std::true_type());
        else by_v(tt, dd, std::integral_constant<int, 3>(), std::false_type());
      }
    };
    auto by_d = [&](auto tt) {
      if (P.D == 32) by_r(tt, std::integral_constant<int, 32>());
      else if (P.D == 64) by_r(tt, std::integral_constant<int, 64>());
      else by_r(tt, std::integral_constant<int, 128>());
    };
    if (dtype == NA_BF16) by_d(bf16_t());
    else by_d(f16_t());
    return;
  }
  const LProb L = make_lprob(P, C);
  if (L.n_tiles == 0) return;
  const size_t lds = lean_lds_bytes(P, kLQK, L.ebox, C.W);
  const dim3 grid(L.n_launch), block(64 * C.W);
#define LS_ARGS_AV(TT) (const TT *)a, (const TT *)y, (TT *)out, scale
  LS_DISPATCH(k_lav, LS_ARGS_AV(TT));
#undef LS_ARGS_AV
}

void lsplit_inv(const Prob &P, int dtype, const void *a, const void *x,
                void *z, float scale, hipStream_t st) {
  const bool ca = P.ax[0].causal || P.ax[1].causal || P.ax[2].causal;
  const LChoice C = lean_choice(P, kLInv);
  LProb L = make_lprob(P, C);
  L.n_tiles = P.B * P.Hkv * (int)L.fGrid.d;
  L.n_launch = (L.n_tiles + 7) & ~7;
  if (L.n_tiles == 0) return;
  const size_t lds = lean_lds_bytes(P, kLInv, L.ebox, C.W);
  const dim3 grid(L.n_launch), block(64 * C.W);
#define LS_ARGS_INV(TT) (const TT *)a, (const TT *)x, (TT *)z, scale
  LS_DISPATCH(k_linv, LS_ARGS_INV(TT));
#undef LS_ARGS_INV
}

// NATTEN_AMD_SPLIT_PAIR=0 launches a split backward's two passes separately
// (A/B checks of the paired launch; read on every call, so a test can switch
// it within one process).
static bool split_pair_on() {
  const char *e = std::getenv("NATTEN_AMD_SPLIT_PAIR");
  return e == nullptr || e[0] != '0';
}

// A split backward's two passes in one launch (k_lqkb: dq + dk, k_lavb:
// dattn + dv) where the all-heads pass applies, its workgroups have the
// inverse pass's size and both take the same chunk walk; false otherwise
// (nothing launched).
static bool lsplit_pair(const Prob &P, int dtype, bool qk, const void *w, const void *y,
                        const void *xi, void *out_a, void *out_i, float scale,
                        hipStream_t st) {
  if (!split_pair_on()) return false;
  const LChoice C = lean_choice(P, kLQK);
  const LChoice Ci = lean_choice(P, kLInv);
  LqhPlan pl;
  if (!lqh_plan(P, &pl)) return false;
  const int nb = P.D == 128 ? 2 : 4;
  const size_t lah_lds = (size_t)align16(16 * P.H * P.kprod) * 2 +
                         (size_t)P.H * nb * 16 * lds_y(P.D) * 2;
  if (qk && lah_lds > 65536) return false;
  if (Ci.W != P.H) return false;
  const bool cp = P.rank == 3 ? C.cpr1 && C.sl == 1 : C.cpr1;
  const bool cpi = P.rank == 3 ? Ci.cpr1 && Ci.sl == 1 : Ci.cpr1;
  if (P.rank > 1 && cp != cpi) return false;
  LChoice C1 = C;  // one wave tile per workgroup (waves are heads)
  C1.W = 1;
  LProb La = make_lprob(P, C1);
  La.n_tiles = P.B * (int)La.fGrid.d;
  La.n_launch = (La.n_tiles + 7) & ~7;
  LProb Li = make_lprob(P, Ci);
  Li.n_tiles = P.B * P.Hkv * (int)Li.fGrid.d;
  Li.n_launch = (Li.n_tiles + 7) & ~7;
  if (La.n_tiles == 0 || Li.n_tiles == 0) return false;
  const size_t lds = std::max(qk ? lah_lds : pl.lds, lean_lds_bytes(P, kLInv, Li.ebox, Ci.W));
  int prefill = 0;
  for (int a = 0; a < 3; ++a) prefill |= P.ax[a].causal;
  const bool ca = prefill != 0;
  const FastDiv fups = make_fastdiv((uint32_t)(P.H * P.kprod / pl.vw));
  const int n0 = La.n_launch;
  const dim3 grid(La.n_launch + Li.n_launch), block(64 * P.H);
  auto go = [&](auto tt, auto dd, auto rr, auto cc, auto vv) {
    typedef decltype(tt) TT;
    constexpr int DD = decltype(dd)::value, RR = decltype(rr)::value;
    constexpr bool CC = decltype(cc)::value;
    constexpr int VV = decltype(vv)::value;
    if (qk) {
      // w = dlogits, y = keys, xi = queries; out_a = dq, out_i = dk
      if (ca)
        hipLaunchKernelGGL((k_lqkb<TT, DD, RR, CC, VV, true>), grid, block, lds, st, La, Li,
                           (const TT *)w, (const TT *)y, (const TT *)xi, (TT *)out_a,
                           (TT *)out_i, scale, fups, n0);
      else
        hipLaunchKernelGGL((k_lqkb<TT, DD, RR, CC, VV, false>), grid, block, lds, st, La, Li,
                           (const TT *)w, (const TT *)y, (const TT *)xi, (TT *)out_a,
                           (TT *)out_i, scale, fups, n0);
    } else {
      // w = attn, y = values, xi = dout; out_a = dattn, out_i = dv
      if (ca)
        hipLaunchKernelGGL((k_lavb<TT, DD, RR, CC, VV, true>), grid, block, lds, st, La, Li,
                           (const TT *)w, (const TT *)y, (const TT *)xi, (TT *)out_a,
                           (TT *)out_i, prefill, fups, n0);
      else
        hipLaunchKernelGGL((k_lavb<TT, DD, RR, CC, VV, false>), grid, block, lds, st, La, Li,
                           (const TT *)w, (const TT *)y, (const TT *)xi, (TT *)out_a,
                           (TT *)out_i, prefill, fups, n0);
    }
  };
  auto by_v = [&](auto tt, auto dd, auto rr, auto cc) {
    if (pl.vw == 8) go(tt, dd, rr, cc, std::integral_constant<int, 8>());
    else if (pl.vw == 4) go(tt, dd, rr, cc, std::integral_constant<int, 4>());
    else if (pl.vw == 2) go(tt, dd, rr, cc, std::integral_constant<int, 2>());
    else go(tt, dd, rr, cc, std::integral_constant<int, 1>());
  };
  auto by_r = [&](auto tt, auto dd) {
    if (P.rank == 1)
      by_v(tt, dd, std::integral_constant<int, 1>(), std::false_type());
    else if (P.rank == 2) {
      if (cp) by_v(tt, dd, std::integral_constant<int, 2>(), std::true_type());
      else by_v(tt, dd, std::integral_constant<int, 2>(), std::false_type());
    } else {
      if (cp) by_v(tt, dd, std::integral_constant<int, 3>(), std::true_type());
      else by_v(tt, dd, std::integral_constant<int, 3>(), std::false_type());
    }
  };
  auto by_d = [&](auto tt) {
    if (P.D == 32) by_r(tt, std::integral_constant<int, 32>());
    else if (P.D == 64) by_r(tt, std::integral_constant<int, 64>());
    else by_r(tt, std::integral_constant<int, 128>());
  };
  if (dtype == NA_BF16) by_d(bf16_t());
  else by_d(f16_t());
  return true;
}

void lsplit_qk_bwd(const Prob &P, int dtype, const void *q, const void *k,
                   const void *dlogits, void *dq, void *dk, hipStream_t st) {
  if (lsplit_pair(P, dtype, true, dlogits, k, q, dq, dk, P.scale, st)) return;
  lsplit_av(P, dtype, dlogits, k, dq, P.scale, st);
  lsplit_inv(P, dtype, dlogits, q, dk, P.scale, st);
}

void lsplit_av_bwd(const Prob &P, int dtype, const void *attn, const void *v,
                   const void *dout, void *dattn, void *dv, hipStream_t st) {
  if (lsplit_pair(P, dtype, false, attn, v, dout, dattn, dv, 1.f, st)) return;
  lsplit_qk(P, dtype, dout, v, dattn, 1.f, 0.f, st);
  lsplit_inv(P, dtype, attn, dout, dv, 1.f, st);
}

#undef LS_DISPATCH
#undef LS_D

}  // namespace na
