// na_lean.hip — lean matrix-core (gfx950) fused kernels for the common
// neighborhood problems.
//
// Problem class (lean_eligible): bf16/fp16, head_dim 32/64/128, stride 1,
// one extent for every sample, no additional tokens, not dense, and on every
// non-causal axis an odd K with d*K <= L.  On such an axis the window of the
// query at index i of its dilation phase (Lr points, sub-grid coordinates)
// is [clamp(i - K/2, 0, Lr - K), + K); on a causal axis [max(i - K + 1, 0),
// i].  Both are monotone in i, so the windows of a box of queries cover a
// box of keys and the queries whose windows hold a key form a box too.
//
// Tiling.  A wave owns 16 queries of one phase: a T0 x T1 x T2 box of
// powers of two (product 16); W waves stacked along one axis form a
// workgroup.  The workgroup stages the box of keys its queries' windows
// cover in LDS once (innermost extent padded to a power of two), and each
// wave walks the chunks of 16 keys of its own sub-box (one box row each when
// that row is at most 16 keys wide).  Per chunk:
//   S^T = K . Q^T            mfma_f32_16x16x32 (A = staged K rows, B = Q
//                            rows in registers); lane l holds the scores of
//                            query l%16 with keys 4(l/16) + r; the window
//                            mask is the accumulator's initial value
//   masked online softmax   over a group of 256/D chunks, max and sum over
//                            the query's four lanes by lane swaps
//   O^T += V^T . P^T         V^T from the staged V rows through the
//                            transposing LDS read (ds_read_tr16_b64); two
//                            chunks per MFMA, their probabilities packed as
//                            the B operand in the same k order.
// The backward (k_wbwd) runs dQ over the staged K/V box and then, in the
// same LDS, dK/dV over the staged query box of the tile's keys.
#include "na_lean.h"

namespace na {
namespace {

// ---------------------------------------------------------------------------
// Forward.  A workgroup of W waves owns W wave tiles stacked along the
// stack axis; its K/V box is staged in LDS once, then each wave runs the
// chunks of its own sub-box.

// One group of NB (even) chunks of 16 staged keys (first LDS rows kb[j]
// from the bases ks / vs; sv[j] holds the chunk's mask as the score
// accumulator's initial value): scores, online softmax update of (m, l, o)
// and O^T += V^T . P^T.  The row sums l come out of the matrix core too:
// `ones` is an A operand whose row 0 is all ones, so lacc[0] of lane n
// (lanes 0-15) accumulates the sum of query n's rounded probabilities (the
// same values that weight V) and the other lanes' lacc stay zero.
template <typename T, int D, int NB>
__device__ __forceinline__ void fwd_group(const typename L16<T>::e *ks,
                                          const typename L16<T>::e *vs,
                                          const int (&kb)[NB], f32x4 (&sv)[NB],
                                          const typename L16<T>::v8 (&qf)[D / 32],
                                          f32x4 (&o)[D / 16], float &m, f32x4 &lacc,
                                          const typename L16<T>::v8 &ones,
                                          float sl2, int ka_off, int tr_off,
                                          bool fresh) {
  typedef L16<T> M;
  typedef typename M::v8 v8;
  typedef typename M::v4 v4;
  typedef typename M::e E;
  constexpr int NT = D / 32;    // 32-wide k-steps over head_dim
  constexpr int NDB = D / 16;   // 16-row blocks of O^T
  constexpr int RSE = lds_row(D);
  v8 ka[NB][NT];
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int st = 0; st < NT; ++st)
      ka[j][st] = *reinterpret_cast<const v8 *>(ks + kb[j] * RSE + ka_off + 32 * st);
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int st = 0; st < NT; ++st) sv[j] = M::mma(ka[j][st], qf[st], sv[j]);
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sv[j][r]);
  // ---- online softmax ----
  mx = quad_max(mx) * sl2;
  // The reference point m may trail the running max by up to 8 (a factor
  // 2^8 in P): exact after the final division by l, and it spares the O
  // rescale on groups that do not raise any query's max by more.  The first
  // group of a query head finds O and l zero: it only sets m.
  if (fresh) {
    m = mx;
  } else if (__builtin_amdgcn_ballot_w64(mx > m + 8.f) != 0) {
    const float mn = fmaxf(m, mx);
    const float alpha = __builtin_amdgcn_exp2f(m - (mn == -INFINITY ? 0.f : mn));
    lacc *= alpha;
#pragma unroll
    for (int j = 0; j < NDB; ++j) o[j] *= alpha;
    m = mn;
  }
  const float mu = m == -INFINITY ? 0.f : m;
  v8 bp[NB / 2];
#pragma unroll
  for (int jj = 0; jj < NB / 2; ++jj)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = __builtin_amdgcn_exp2f(fmaf(sv[2 * jj + h][r], sl2, -mu));
        bp[jj][4 * h + r] = (E)p;
      }
  // ---- O^T += V^T . P^T, two chunks per MFMA ----
#pragma unroll
  for (int jj = 0; jj < NB / 2; ++jj) {
    const E *ca = vs + kb[2 * jj] * RSE + tr_off;
    const E *cb = vs + kb[2 * jj + 1] * RSE + tr_off;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const v4 lo4 = M::tr(ca + 16 * db);
      const v4 hi4 = M::tr(cb + 16 * db);
      const v8 a = __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
      o[db] = M::mma(a, bp[jj], o[db]);
    }
    lacc = M::mma(ones, bp[jj], lacc);
  }
}

// R: rank; CPR1: every wave sub-box row is one chunk (at most 16 keys wide),
// so the per-lane column tests are fixed.  VX: per-sample extents (P.se)
// and/or additional tokens (P.nx rows per sample of ek / ev, staged in LDS
// before the box and attended after it); query rows of the tensor outside
// their sample's extent get zero output and lse 0.
// CA: some axis is causal; without one the window rules are the clamped
// rule alone (the causal fields are known zero at compile time, so the
// setup's selects between the two rules fold away).
// PFS: the box is staged in several slabs and each slab's loads are issued
// while the previous slab is computed (SlabPrefetch).
template <typename T, int D, int R, bool CPR1, bool VX, bool CA, bool PFS>
__global__ void __launch_bounds__(512)
    k_wfwd(LProb Pin, const T *__restrict__ q, const T *__restrict__ k,
           const T *__restrict__ v, const T *__restrict__ ek,
           const T *__restrict__ ev, T *__restrict__ out,
           float *__restrict__ lse) {
  LProb P = Pin;
  if constexpr (!CA) P.ax[0].causal = P.ax[1].causal = P.ax[2].causal = 0;
  typedef L16<T> M;
  typedef typename M::v8 v8;
  typedef typename M::v4 v4;
  typedef typename M::e E;
  constexpr int NT = D / 32;    // 32-wide k-steps over head_dim
  constexpr int NB = 256 / D;   // chunks per softmax group
  constexpr int NDB = D / 16;   // 16-row blocks of O^T
  constexpr int RSE = lds_row(D);
  extern __shared__ __align__(16) char smem[];

  // setup is straight-line arithmetic on kernel arguments (so their loads
  // issue together); the exit test comes after it
  LTile t;
  bool hl = false;  // VX: every query head of the group over one box
  bool tile_any;
  if constexpr (VX) {
    hl = P.hl != 0;
    const int tile_id = xcd_tile(blockIdx.x, P.n_launch);
    tile_any = hl ? decode_tile_group<R>(P, tile_id, t) : decode_tile<R, VX>(P, tile_id, t);
  } else {
    tile_any = decode_tile<R, VX>(P, xcd_tile(blockIdx.x, P.n_launch), t);
  }
  const int nhl = hl ? P.hl : 1;
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int n = lane & 15, gq = lane >> 4;
  const WSub ws = wave_sub<R>(P, t, w);

  // ---- the lane's query (column n of the score tiles): qv, inside its
  // sample; qt, a row of the tensor (the two differ only when VX) ----
  int u[3];
  {
    const int lg2 = P.ax[2].lgT, lg1 = P.ax[1].lgT;
    u[2] = n & (P.ax[2].T - 1);
    u[1] = (n >> lg2) & (P.ax[1].T - 1);
    u[0] = n >> (lg2 + lg1);
  }
  bool qv = ws.any, qt = t.b < P.B;
  int qtok = t.b * P.Ltot;
  int wl[3], ww[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    if (a < 3 - R) {
      wl[a] = 0;
      ww[a] = 1;
      continue;
    }
    const LAx &x = P.ax[a];
    qv = qv && u[a] < ws.nv[a];
    qt = qt && u[a] < ws.nvt[a];
    // rows past the end (lanes of a partial wave tile, waves past the
    // tile) take the tile's last row
    const int i = min(ws.i0[a] + min(u[a], max(ws.nv[a] - 1, 0)),
                      t.i0[a] + t.nv[a] - 1);
    const int it = VX ? min(ws.i0[a] + min(u[a], max(ws.nvt[a] - 1, 0)),
                            t.i0[a] + t.nvt[a] - 1)
                      : i;
    qtok += (t.r[a] + x.d * it) * x.tok;
    const int s = wstart(x, i, t.Lr[a]);
    wl[a] = s - t.lo[a];
    ww[a] = wend(x, i, t.Lr[a]) - s;
  }
  if (!qv) ww[2] = 0;
  if (!tile_any) {  // uniform over the workgroup
    if (VX && qt) {  // rows of the tensor outside the sample: zeros
      v4 z;
#pragma unroll
      for (int r = 0; r < 4; ++r) z[r] = (E)0.f;
      for (int hr = 0; hr < nhl; ++hr) {
        const int zo = (qtok * P.H + t.head + hr) * D;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          *reinterpret_cast<v4 *>(out + zo + 16 * db + 4 * gq) = z;
        if (lse != nullptr && gq == 0) lse[(uint32_t)zo / D] = 0.f;
      }
    }
    return;
  }
  // the first head's query rows, issued before the staging
  v8 qf[NT];
#pragma unroll
  for (int st = 0; st < NT; ++st)
    qf[st] = ld8(q, (qtok * P.H + t.head) * D + 32 * st + 8 * gq);

  // ---- LDS: additional tokens (VX) in rows [0, nxr), then the K / V box,
  // staged in slabs of P.sl layers along axis 0 for rank 3 (one slab
  // otherwise) ----
  E *xk = reinterpret_cast<E *>(smem);
  E *xv = xk + lds_y(D);
  const int nxr = VX ? P.nxr : 0;
  E *ks = xk + nxr * RSE;
  E *vs = ks + lds_y(D);
  if (VX && nxr > 0) {
    // rows past nx repeat the last token (finite; masked below)
    constexpr int OCT = D / 8;
    const int xrow0 = (t.b * P.nx * P.Hkv + t.hk) * D;
    for (int uu = tid; uu < nxr * OCT; uu += nthr) {
      const int e = uu / OCT, oo = uu % OCT;
      const int g = xrow0 + min(e, P.nx - 1) * P.Hkv * D + 8 * oo;
      const v8 a = ld8(ek, g);
      const v8 b = ld8(ev, g);
      *reinterpret_cast<v8 *>(xk + e * RSE + 8 * oo) = a;
      *reinterpret_cast<v8 *>(xv + e * RSE + 8 * oo) = b;
    }
  }

  // column part of the mask of the lane's 4 keys per chunk (fixed when CPR1)
  float cb0[4];
  col_bias(ws.ws[2] + 4 * gq - wl[2], ww[2], cb0);

  for (int hr = 0; hr < nhl; ++hr) {  // query heads over the staged box (hl)
  const int qoff = (qtok * P.H + t.head + hr) * D;
  if (hr > 0) {
#pragma unroll
    for (int st = 0; st < NT; ++st) qf[st] = ld8(q, qoff + 32 * st + 8 * gq);
  }
  f32x4 o[NDB];
#pragma unroll
  for (int j = 0; j < NDB; ++j) o[j] = zero4();
  float m = -INFINITY;
  bool fresh = true;  // no softmax group of this query head run yet
  f32x4 lacc = zero4();
  v8 ones;
#pragma unroll
  for (int i = 0; i < 8; ++i) ones[i] = (E)(n == 0 ? 1.f : 0.f);
  const float sl2 = P.sl2;
  const int Em1 = P.ax[1].Em;
  // operand-read lane offsets inside a chunk: K rows (key n, 8 elements at
  // 8 gq) and the transposing read (row 4 gq + n / 4, column 4 (n % 4))
  const int ka_off = n * RSE + 8 * gq;
  const int tr_off = (4 * gq + (n >> 2)) * RSE + 4 * (n & 3);
  const int nsl = R == 3 ? (t.E[0] + P.sl - 1) / P.sl : 1;
  const int rows1 = R > 1 ? ws.we[1] - ws.ws[1] : 1;
  // additional-token chunks, run after the last slab's box chunks; their
  // rows sit before the box (LDS rows -nxr .. -1 from ks)
  const int nxc = VX ? nxr >> 4 : 0;
  SlabPrefetch<T, D, R> pf;
  if constexpr (PFS) {  // one query head (no hl): the first slab's loads
    pf.load(P, t, k, v, tid, nthr, 0);
    zero_slack<T, D>(P, ks, tid, nthr);
  }
  for (int si = 0; si < nsl; ++si) {
    const int s0 = si * P.sl;
    if (hr == 0) {  // with hl the whole box is one slab, staged once
      if (si > 0) __syncthreads();  // the previous slab's reads are done
      if constexpr (PFS) {
        pf.store(ks, vs);
        if (si + 1 < nsl) pf.load(P, t, k, v, tid, nthr, s0 + P.sl);
      } else {
        stage_box<T, D, R>(P, t, k, v, ks, vs, tid, nthr, s0);
      }
      __syncthreads();
    }
    if (!ws.any) continue;
    // the wave's box rows inside this slab
    const int a0 = R == 3 ? max(ws.ws[0], s0) : 0;
    const int b0 = R == 3 ? min(ws.we[0], s0 + P.sl) : 1;
    const int nchb = b0 > a0 ? (b0 - a0) * rows1 * ws.cpr : 0;
    const int nch = nchb + (si == nsl - 1 ? nxc : 0);
    Cursor cc{a0, ws.ws[1], 0};
    const int key0 = (((a0 - s0) * Em1 + ws.ws[1]) << P.lgP2) + ws.ws[2];
    // chunk rows and masks of a group of G chunks from chunk c0
    auto group = [&](int c0, auto g_) {
      constexpr int G = decltype(g_)::value;
      int kb[G];        // first LDS row of each chunk
      f32x4 sv[G];      // score accumulators, initialised with the mask
#pragma unroll
      for (int j = 0; j < G; ++j) {
        const int c = c0 + j;
        const bool box = c < nchb;
        const bool ext = VX && !box && c < nch;
        bool ok = box;
        // closed forms: one box row (rank 1) or one chunk per row (rank 2,
        // CPR1; rank 3, CPR1, whose slabs are one layer a0); otherwise the
        // cursor
        const int e1 = R >= 2 && CPR1 ? ws.ws[1] + c : cc.e1;
        const int cs = R == 1 ? c : CPR1 ? 0 : cc.cs;
        if (R > 1) ok = ok && (unsigned)(e1 - wl[1]) < (unsigned)ww[1];
        if (R == 3) ok = ok && (unsigned)((CPR1 ? a0 : cc.e0) - wl[0]) < (unsigned)ww[0];
        const int krow = R == 1 ? key0 + 16 * c
                         : CPR1 ? key0 + (c << P.lgP2)
                         : (((cc.e0 - s0) * Em1 + cc.e1) << P.lgP2) + ws.ws[2] + 16 * cc.cs;
        float cb[4];
        if (CPR1 && !VX) {
#pragma unroll
          for (int r = 0; r < 4; ++r) cb[r] = cb0[r];
          kb[j] = box ? krow : key0;
        } else {
          // extra chunk c - nchb: keys 16 (c - nchb) + 4 gq + r < nx
          const int xc = 16 * (c - nchb);
          col_bias(box ? ws.ws[2] + 16 * cs + 4 * gq - wl[2] : xc + 4 * gq,
                   box ? ww[2] : (qv ? P.nx : 0), cb);
          kb[j] = box ? krow : ext ? xc - nxr : key0;
          ok = ok || ext;
        }
        sv[j] = mask_init(ok, cb);
        if (R >= 2 && !CPR1) advance(cc, ws);
      }
      fwd_group<T, D, G>(ks, vs, kb, sv, qf, o, m, lacc, ones, sl2, ka_off, tr_off, fresh);
      fresh = false;
    };
    if constexpr (NB >= 4) {
      int c0 = 0;
      for (; c0 + NB / 2 < nch; c0 += NB) group(c0, std::integral_constant<int, NB>());
      // a tail of at most NB / 2 chunks runs as a half group
      if (c0 < nch) group(c0, std::integral_constant<int, NB / 2>());
    } else {
      for (int c0 = 0; c0 < nch; c0 += NB) group(c0, std::integral_constant<int, NB>());
    }
  }

  // ---- epilogue: sum l over the query's 4 lanes, normalise, store ----
  const float l = quad_sum(lacc[0]);
  if (VX ? qt : qv) {
    const float inv = qv && l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      v4 wv;
#pragma unroll
      for (int r = 0; r < 4; ++r) wv[r] = (E)(o[db][r] * inv);
      *reinterpret_cast<v4 *>(out + qoff + 16 * db + 4 * gq) = wv;
    }
    if (lse != nullptr && gq == 0)
      lse[(uint32_t)qoff / D] = !qv ? 0.f : l > 0.f ? (m + __log2f(l)) * kLn2 : -INFINITY;
  }
  }  // query heads
}

// ---------------------------------------------------------------------------
// Backward.

// One round of the dK/dV role's query-box staging: each lane's NU units of
// Q and dO rows (layout as stage_box) and per row the pair (lse * log2(e),
// rowsum(dO * O) - dlse), the row sum reduced over the D/8 consecutive
// lanes holding one row.  load() only reads memory into registers, so a
// wave may issue it before the barrier that ends the other waves' reads of
// the LDS it will overwrite; store() writes the LDS.  NU: units per lane
// in flight, by default two for the wider rank-1 heads, whose backward
// keeps four waves per SIMD (its dK / dV accumulators and the key's own
// rows stay live across the staging), else four.
template <typename T, int D, int R, int NU_ = (R == 1 && D >= 64 ? 2 : 4)>
struct QboxRound {
  typedef typename L16<T>::v8 v8;
  typedef typename L16<T>::e E;
  static constexpr int OCT = D / 8;
  static constexpr int RSE = lds_row(D);
  static constexpr int NU = NU_;
  v8 qr[NU], dr[NU], orr[NU];
  float lr[NU], dl[NU];
  int la[NU];
  __device__ __forceinline__ void load(const LProb &P, const LTile &t,
                                       const T *__restrict__ q, const T *__restrict__ dout,
                                       const T *__restrict__ out,
                                       const float *__restrict__ lse,
                                       const float *__restrict__ dlse, int u0, int tid,
                                       int nthr, int s0) {
    int g[NU];
    unit_walk<R, OCT, RSE, NU, false>(P, t, u0, tid, nthr, s0, g, la);
    const int o = tid % OCT;  // the lane's unit in each of its rows
#pragma unroll
    for (int j = 0; j < NU; ++j) {
      // element offsets are non-negative: an unsigned division is a shift
      const int row = (int)((uint32_t)(g[j] - 8 * o) / D);
      qr[j] = ld8(q, g[j]);
      dr[j] = ld8(dout, g[j]);
      orr[j] = ld8(out, g[j]);
      lr[j] = ldf(lse, row);
      dl[j] = dlse != nullptr ? ldf(dlse, row) : 0.f;
    }
  }
  __device__ __forceinline__ void store(E *qs, E *os, int tid) const {
    const int o = tid % OCT;
#pragma unroll
    for (int j = 0; j < NU; ++j) {
      *reinterpret_cast<v8 *>(qs + la[j]) = qr[j];
      *reinterpret_cast<v8 *>(os + la[j]) = dr[j];
      float part = 0.f;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        typename L16<T>::v2 a2, b2;
        a2[0] = dr[j][e];
        a2[1] = dr[j][e + 1];
        b2[0] = orr[j][e];
        b2[1] = orr[j][e + 1];
        part = L16<T>::dot2(a2, b2, part);
      }
      part = dpp_group_sum<OCT>(part);
      if (o == 0)
        *reinterpret_cast<float2 *>(qs + la[j] + D) =
            make_float2(lr[j] * kLog2e, dl[j] - part);
    }
  }
};

// Stage the dK/dV role's query box from unit u_begin on (the rounds before
// it staged by the caller), then clear the slack rows.
template <typename T, int D, int R>
__device__ __forceinline__ void stage_qbox(const LProb &P, const LTile &t,
                                           const T *__restrict__ q,
                                           const T *__restrict__ dout,
                                           const T *__restrict__ out,
                                           const float *__restrict__ lse,
                                           const float *__restrict__ dlse,
                                           typename L16<T>::e *qs,
                                           typename L16<T>::e *os, int tid,
                                           int nthr, int s0, int u_begin) {
  typedef QboxRound<T, D, R> QR;
  const int nun = P.ebox * QR::OCT;
  for (int u0 = u_begin; u0 < nun; u0 += QR::NU * nthr) {
    QR r;
    r.load(P, t, q, dout, out, lse, dlse, u0, tid, nthr, s0);
    r.store(qs, os, tid);
  }
  zero_slack<T, D>(P, qs, tid, nthr);
}

// Lane-window of a wave's 16 rows (queries in the dQ role, keys in the
// dK/dV role) inside the staged box: [wl, wl + ww) per axis, ww = 0 on
// every axis for rows outside the tensor.  Returns the row's element offset.
template <int R, bool INV>
__device__ __forceinline__ int lane_rows(const LProb &P, const LTile &t,
                                         const WSub &ws, int n, int head,
                                         int heads, bool &valid, int wl[3],
                                         int ww[3]) {
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
  }
  if (!valid) ww[2] = 0;
  return (tok * heads + head) * P.D;
}

// Rows of chunk pair (a, b) of a wave's sub-box: first LDS row, row test
// and column segment of each (padding chunks: row 0 of the sub-box, masked).
// Closed forms where the walk is one box row (rank 1: chunk c is columns
// 16 c..) or one chunk per row (rank 2, CPR1: chunk c is row ws1 + c; rank
// 3, CPR1, a slab of one layer a0: the same on that layer, whose row test
// l0ok is the caller's); otherwise the cursor walks rows and segments.
template <int R, bool CPR1>
__device__ __forceinline__ void pair_rows(const WSub &ws, Cursor &cc, int c0,
                                          int nch, int s0, int Em1, int lgP2,
                                          int key0,
                                          const int wl[3], const int ww[3],
                                          int kb[2], bool rok[2], int cs[2],
                                          bool layer = false, bool l0ok = false) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c = c0 + h;
    const bool real = c < nch;
    if (R == 1) {
      kb[h] = key0 + (real ? 16 * c : 0);
      cs[h] = c;
      rok[h] = real;
    } else if ((R == 2 || layer) && CPR1) {
      kb[h] = key0 + (real ? c << lgP2 : 0);
      cs[h] = 0;
      rok[h] = real && (unsigned)(ws.ws[1] + c - wl[1]) < (unsigned)ww[1] && (R == 2 || l0ok);
    } else {
      kb[h] = real ? (((cc.e0 - s0) * Em1 + cc.e1) << lgP2) + ws.ws[2] + 16 * cc.cs : key0;
      cs[h] = cc.cs;
      bool ok = real;
      if (R > 1) ok = ok && (unsigned)(cc.e1 - wl[1]) < (unsigned)ww[1];
      if (R == 3) ok = ok && (unsigned)(cc.e0 - wl[0]) < (unsigned)ww[0];
      rok[h] = ok;
      advance(cc, ws);
    }
  }
}

// A workgroup owns one spatial tile of one key/value head and runs both
// halves of the backward for it in sequence, in the same LDS: the K/V box
// of the tile's queries is staged and each wave computes dQ of its 16
// queries (per query head of the group); then, per query head, the query
// box of the tile's keys (Q, dO, lse, delta) is staged and each wave
// accumulates dK and dV of its 16 keys.  One workgroup per tile keeps the
// whole launch resident at once.
// PFS: the dQ half's K / V box is staged in several slabs, each slab's loads
// issued while the previous slab is computed (SlabPrefetch).
template <typename T, int D, int R, bool CPR1, bool VX, bool CA, bool PFS>
__global__ void __launch_bounds__(512)
    __attribute__((amdgpu_waves_per_eu(D == 64 && R == 1 ? 4 : 1)))
    k_wbwd(LProb Pin, const T *__restrict__ q, const T *__restrict__ k,
           const T *__restrict__ v, const T *__restrict__ ek,
           const T *__restrict__ ev, const T *__restrict__ out,
           const float *__restrict__ lse, const T *__restrict__ dout,
           const float *__restrict__ dlse, T *__restrict__ dq,
           T *__restrict__ dk, T *__restrict__ dv, float *__restrict__ dlt) {
  LProb P = Pin;
  if constexpr (!CA) P.ax[0].causal = P.ax[1].causal = P.ax[2].causal = 0;
  typedef L16<T> M;
  typedef typename M::v8 v8;
  typedef typename M::v4 v4;
  typedef typename M::e E;
  constexpr int NT = D / 32;
  constexpr int NDB = D / 16;
  constexpr int RSE = lds_row(D);
  extern __shared__ __align__(16) char smem[];

  const uint32_t tile = (uint32_t)xcd_tile(blockIdx.x, P.n_launch);
  const uint32_t rest = fdiv(tile, P.fGrid);
  const uint32_t sp = tile - rest * P.fGrid.d;
  const uint32_t bq = fdiv(rest, P.fHkv);
  LTile t;
  t.hk = (int)(rest - bq * P.fHkv.d);
  t.b = (int)bq;
  const bool tile_any = tile_origin<R, VX>(P, sp, t) & (t.b < P.B);
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int n = lane & 15, gq = lane >> 4;
  const float sl2 = P.sl2;
  const int Em1 = P.ax[1].Em;
  const int ka_off = n * RSE + 8 * gq;
  const int tr_off = (4 * gq + (n >> 2)) * RSE + 4 * (n & 3);
  // the (lse, -delta) pad of query row 4 gq of a chunk
  const int pad_off = 4 * gq * RSE + D;
  if (VX && t.b < P.B) {
    // the lane's row of the tensor (wave tile w, position n): rows of the
    // tensor outside the sample get zero dq (every head of the group), dk
    // and dv here; the passes below write the sample's rows only
    int u[3];
    const int lg2 = P.ax[2].lgT, lg1 = P.ax[1].lgT;
    u[2] = n & (P.ax[2].T - 1);
    u[1] = (n >> lg2) & (P.ax[1].T - 1);
    u[0] = n >> (lg2 + lg1);
    bool rin = true, rsm = true;
    int rtok = t.b * P.Ltot;
#pragma unroll
    for (int a = 3 - R; a < 3; ++a) {
      const LAx &x = P.ax[a];
      const int rel = (a == P.sa ? w * x.T : 0) + u[a];
      rin = rin && rel < t.nvt[a];
      rsm = rsm && rel < t.nv[a];
      rtok += (t.r[a] + x.d * (t.i0[a] + min(rel, max(t.nvt[a] - 1, 0)))) * x.tok;
    }
    if (rin && !rsm) {
      v4 z;
#pragma unroll
      for (int r = 0; r < 4; ++r) z[r] = (E)0.f;
      const int ko = (rtok * P.Hkv + t.hk) * D + 4 * gq;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        *reinterpret_cast<v4 *>(dk + ko + 16 * db) = z;
        *reinterpret_cast<v4 *>(dv + ko + 16 * db) = z;
      }
      for (int hr = 0; hr < P.rep; ++hr) {
        const int qo = (rtok * P.H + t.hk * P.rep + hr) * D + 4 * gq;
#pragma unroll
        for (int db = 0; db < NDB; ++db) *reinterpret_cast<v4 *>(dq + qo + 16 * db) = z;
      }
    }
  }
  if (!tile_any) return;  // uniform over the workgroup
  E *xs = reinterpret_cast<E *>(smem);
  E *ys = xs + lds_y(D);

  // =============================== dQ ===============================
  {
    tile_box<R, false>(P, t, t.hk, P.Hkv);
    const WSub ws = wave_sub<R, false>(P, t, w);
    // VX: the additional tokens in LDS rows [0, nxr) (rows past nx repeat
    // the last token: finite, masked), the K / V box after them; their
    // chunks run after the last slab's box chunks
    const int nxr = VX ? P.nxr : 0;
    const int nxc = nxr >> 4;
    E *ks = xs + nxr * RSE;
    E *vs = ys + nxr * RSE;
    if (VX && nxr > 0) {
      constexpr int OCT = D / 8;
      const int xrow0 = (t.b * P.nx * P.Hkv + t.hk) * D;
      for (int uu = tid; uu < nxr * OCT; uu += nthr) {
        const int e = uu / OCT, oo = uu % OCT;
        const int g = xrow0 + min(e, P.nx - 1) * P.Hkv * D + 8 * oo;
        *reinterpret_cast<v8 *>(xs + e * RSE + 8 * oo) = ld8(ek, g);
        *reinterpret_cast<v8 *>(ys + e * RSE + 8 * oo) = ld8(ev, g);
      }
    }
    // the K / V box in slabs of P.sl layers along axis 0 (rank 3); a single
    // slab is staged once for every query head of the group
    const int nsl = R == 3 ? (t.E[0] + P.sl - 1) / P.sl : 1;
    const int rows1 = R > 1 ? ws.we[1] - ws.ws[1] : 1;
    SlabPrefetch<T, D, R> pf;
    if constexpr (PFS) {
      pf.load(P, t, k, v, tid, nthr, 0);
      zero_slack<T, D>(P, ks, tid, nthr);
    }
    for (int hr = 0; hr < P.rep; ++hr) {
      const int hq = t.hk * P.rep + hr;
      bool qv;
      int wl[3], ww[3];
      const int qoff = lane_rows<R, false>(P, t, ws, n, hq, P.H, qv, wl, ww);
      v8 qf[NT], df[NT];
      float dsum = 0.f;
#pragma unroll
      for (int st = 0; st < NT; ++st) {
        qf[st] = ld8(q, qoff + 32 * st + 8 * gq);
        df[st] = ld8(dout, qoff + 32 * st + 8 * gq);
        const v8 of = ld8(out, qoff + 32 * st + 8 * gq);
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          typename M::v2 a2, b2;
          a2[0] = df[st][e];
          a2[1] = df[st][e + 1];
          b2[0] = of[e];
          b2[1] = of[e + 1];
          dsum = M::dot2(a2, b2, dsum);
        }
      }
      const int qrow = (int)((uint32_t)qoff / D);
      const float lse2 = ldf(lse, qrow) * kLog2e;
      const float dl = dlse != nullptr ? ldf(dlse, qrow) : 0.f;
      float delta = 0.f;
      float cb0[4];
      col_bias(ws.ws[2] + 4 * gq - wl[2], ww[2], cb0);
      f32x4 acc[NDB];
#pragma unroll
      for (int j = 0; j < NDB; ++j) acc[j] = zero4();
      for (int si = 0; si < nsl; ++si) {
      const int s0 = si * P.sl;
      if (nsl > 1 || hr == 0) {
        if (hr > 0 || si > 0) __syncthreads();  // the previous slab's reads are done
        if constexpr (PFS) {
          pf.store(ks, vs);
          // the next slab: of this head, else the first of the next head
          if (si + 1 < nsl)
            pf.load(P, t, k, v, tid, nthr, s0 + P.sl);
          else if (hr + 1 < P.rep)
            pf.load(P, t, k, v, tid, nthr, 0);
        } else {
          stage_box<T, D, R>(P, t, k, v, ks, vs, tid, nthr, s0);
        }
        __syncthreads();
      }
      if (!ws.any) continue;
      if (si == 0) delta = quad_sum(dsum) - dl;
      const int a0 = R == 3 ? max(ws.ws[0], s0) : 0;
      const int b0 = R == 3 ? min(ws.we[0], s0 + P.sl) : 1;
      const int nchb = b0 > a0 ? (b0 - a0) * rows1 * ws.cpr : 0;
      const int nch = nchb + (si == nsl - 1 ? nxc : 0);
      const int key0 = (((a0 - s0) * Em1 + ws.ws[1]) << P.lgP2) + ws.ws[2];
      // a slab of one layer (rank 3, CPR1: launched only with one-layer
      // slabs): its chunks are the rows of layer a0
      constexpr bool layer = R == 3 && CPR1;
      const bool l0ok = (unsigned)(a0 - wl[0]) < (unsigned)ww[0];
      Cursor cc{a0, ws.ws[1], 0};
      for (int c0 = 0; c0 < nch; c0 += 2) {
        int kb[2], cs[2];
        bool rok[2];
        pair_rows<R, CPR1>(ws, cc, c0, nchb, s0, Em1, P.lgP2, key0, wl, ww, kb, rok, cs,
                           layer, l0ok);
        bool ext[2] = {false, false};
        if (VX) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int c = c0 + h;
            ext[h] = c >= nchb && c < nch;
            if (ext[h]) {
              kb[h] = 16 * (c - nchb) - nxr;
              rok[h] = true;
            }
          }
        }
        v8 kr[2][NT], vr[2][NT];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int st = 0; st < NT; ++st) {
            kr[h][st] = *reinterpret_cast<const v8 *>(ks + kb[h] * RSE + ka_off + 32 * st);
            vr[h][st] = *reinterpret_cast<const v8 *>(vs + kb[h] * RSE + ka_off + 32 * st);
          }
        // K^T operands of dQ^T += K^T . dS^T: read now so their latency
        // overlaps the score MFMAs and exponentials, or after the scores
        // for the wider rank-1 heads (as in the dK / dV half)
        v8 kt[NDB];
        auto read_kt = [&]() {
#pragma unroll
          for (int db = 0; db < NDB; ++db) {
            const v4 lo4 = M::tr(ks + kb[0] * RSE + tr_off + 16 * db);
            const v4 hi4 = M::tr(ks + kb[1] * RSE + tr_off + 16 * db);
            kt[db] = __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
          }
        };
        constexpr bool EARLY_KT = D == 32 || R != 1;
        if (EARLY_KT) read_kt();
        __builtin_amdgcn_sched_barrier(0);  // keep every read of the pair ahead
        // S^T masked through its initial value, dP^T - delta through its
        f32x4 sc[2], dp[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float cb[4];
          if (VX && ext[h]) {  // keys 16 (c - nchb) + 4 gq + r < nx
            col_bias(16 * (c0 + h - nchb) + 4 * gq, qv ? P.nx : 0, cb);
          } else if (CPR1) {
#pragma unroll
            for (int r = 0; r < 4; ++r) cb[r] = cb0[r];
          } else {
            col_bias(ws.ws[2] + 16 * cs[h] + 4 * gq - wl[2], ww[2], cb);
          }
          sc[h] = mask_init(rok[h], cb);
#pragma unroll
          for (int r = 0; r < 4; ++r) dp[h][r] = -delta;
#pragma unroll
          for (int st = 0; st < NT; ++st) {
            sc[h] = M::mma(kr[h][st], qf[st], sc[h]);
            dp[h] = M::mma(vr[h][st], df[st], dp[h]);
          }
        }
        v8 bs;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float p = __builtin_amdgcn_exp2f(fmaf(sc[h][r], sl2, -lse2));
            bs[4 * h + r] = (E)(p * dp[h][r]);
          }
        if (!EARLY_KT) read_kt();
        // dQ^T += K^T . dS^T
#pragma unroll
        for (int db = 0; db < NDB; ++db) acc[db] = M::mma(kt[db], bs, acc[db]);
      }
      }  // slabs
      if (qv) {
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          v4 wv;
#pragma unroll
          for (int r = 0; r < 4; ++r) wv[r] = (E)(acc[db][r] * P.scale);
          *reinterpret_cast<v4 *>(dq + qoff + 16 * db + 4 * gq) = wv;
        }
        // VX: the row's delta, for the additional tokens' gradient pass
        if (VX && dlt != nullptr && gq == 0) dlt[(uint32_t)qoff / D] = delta;
      }
    }
  }

  // ============================= dK / dV =============================
  // keys of the tile (head hk); the query box of each query head of the group
  tile_box<R, true>(P, t, t.hk * P.rep, P.H);
  const WSub ws = wave_sub<R, true>(P, t, w);
  bool kv;
  int wl[3], ww[3];
  int koff;
  {
    int u[3];
    const int lg2 = P.ax[2].lgT, lg1 = P.ax[1].lgT;
    u[2] = n & (P.ax[2].T - 1);
    u[1] = (n >> lg2) & (P.ax[1].T - 1);
    u[0] = n >> (lg2 + lg1);
    kv = ws.any;
    int tok = t.b * P.Ltot;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      if (a < 3 - R) {
        wl[a] = 0;
        ww[a] = 1;
        continue;
      }
      const LAx &x = P.ax[a];
      kv = kv && u[a] < ws.nv[a];
      const int j = min(ws.i0[a] + min(u[a], max(ws.nv[a] - 1, 0)),
                        t.i0[a] + t.nv[a] - 1);
      tok += (t.r[a] + x.d * j) * x.tok;
      const int s0 = iwstart(x, j, t.Lr[a]);
      wl[a] = s0 - t.lo[a];
      ww[a] = iwend(x, j, t.Lr[a]) - s0;
    }
    if (!kv) ww[2] = 0;
    koff = (tok * P.Hkv + t.hk) * D;
  }
  v8 kf[NT], vf[NT];
#pragma unroll
  for (int st = 0; st < NT; ++st) {
    kf[st] = ld8(k, koff + 32 * st + 8 * gq);
    vf[st] = ld8(v, koff + 32 * st + 8 * gq);
  }
  float cb0[4];
  col_bias(ws.ws[2] + 4 * gq - wl[2], ww[2], cb0);
  f32x4 adk[NDB], adv[NDB];
#pragma unroll
  for (int j = 0; j < NDB; ++j) {
    adk[j] = zero4();
    adv[j] = zero4();
  }
  const int qbase0 = t.kbase;  // query box rows of head hk * rep
  const int nsl = R == 3 ? (t.E[0] + P.sl - 1) / P.sl : 1;
  const int rows1 = R > 1 ? ws.we[1] - ws.ws[1] : 1;
  // rank 1 and 2 (without the slab prefetch): each query box's first round
  // (three units per lane, two for the wider rank-1 heads) is loaded before
  // the barrier that ends the reads of the LDS it replaces (the dQ half's
  // K/V box, or the previous query head's box), so a wave that is done
  // with its chunks has those loads in flight while the others finish
  // (rank 3 keeps its registers for the slabs)
  constexpr bool PRE = R <= 2 && !PFS;
  typedef QboxRound<T, D, R, (R == 1 && D >= 64 ? 2 : 3)> QP;
  for (int hr = 0; hr < P.rep; ++hr) {
    t.kbase = qbase0 + hr * D;  // query head hk * rep + hr
    for (int si = 0; si < nsl; ++si) {
    const int s0 = si * P.sl;
    if (PRE) {
      QP pre;
      pre.load(P, t, q, dout, out, lse, dlse, 0, tid, nthr, s0);
      __syncthreads();
      pre.store(xs, ys, tid);
      stage_qbox<T, D, R>(P, t, q, dout, out, lse, dlse, xs, ys, tid, nthr, s0,
                          QP::NU * nthr);
    } else {
      __syncthreads();  // the LDS reads of the previous box or slab are done
      stage_qbox<T, D, R>(P, t, q, dout, out, lse, dlse, xs, ys, tid, nthr, s0, 0);
    }
    __syncthreads();
    if (!ws.any) continue;
    const int a0 = R == 3 ? max(ws.ws[0], s0) : 0;
    const int b0 = R == 3 ? min(ws.we[0], s0 + P.sl) : 1;
    const int nch = b0 > a0 ? (b0 - a0) * rows1 * ws.cpr : 0;
    const int key0 = (((a0 - s0) * Em1 + ws.ws[1]) << P.lgP2) + ws.ws[2];
    constexpr bool layer = R == 3 && CPR1;
    const bool l0ok = (unsigned)(a0 - wl[0]) < (unsigned)ww[0];
    Cursor cc{a0, ws.ws[1], 0};
    for (int c0 = 0; c0 < nch; c0 += 2) {
      int kb[2], cs[2];
      bool rok[2];
      pair_rows<R, CPR1>(ws, cc, c0, nch, s0, Em1, P.lgP2, key0, wl, ww, kb, rok, cs,
                         layer, l0ok);
      v8 qr[2][NT], orr[2][NT];
      float ls2[2][4];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int st = 0; st < NT; ++st) {
          qr[h][st] = *reinterpret_cast<const v8 *>(xs + kb[h] * RSE + ka_off + 32 * st);
          orr[h][st] = *reinterpret_cast<const v8 *>(ys + kb[h] * RSE + ka_off + 32 * st);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
          ls2[h][r] = *reinterpret_cast<const float *>(xs + kb[h] * RSE + pad_off + r * RSE);
      }
      // dO^T and Q^T operands of the dV / dK MFMAs.  Head_dim 32: read now
      // so their latency overlaps the score MFMAs and exponentials; wider
      // heads read them after the scores (the Q / dO rows are dead by
      // then), which keeps the rank-1 kernel within four waves per SIMD
      v8 ot[NDB], qt[NDB];
      auto read_t = [&]() {
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const v4 o0 = M::tr(ys + kb[0] * RSE + tr_off + 16 * db);
          const v4 o1 = M::tr(ys + kb[1] * RSE + tr_off + 16 * db);
          ot[db] = __builtin_shufflevector(o0, o1, 0, 1, 2, 3, 4, 5, 6, 7);
          const v4 q0 = M::tr(xs + kb[0] * RSE + tr_off + 16 * db);
          const v4 q1 = M::tr(xs + kb[1] * RSE + tr_off + 16 * db);
          qt[db] = __builtin_shufflevector(q0, q1, 0, 1, 2, 3, 4, 5, 6, 7);
        }
      };
      constexpr bool EARLY_T = D == 32 || R != 1;
      if (EARLY_T) read_t();
      __builtin_amdgcn_sched_barrier(0);  // keep every read of the pair ahead
      // S masked through its initial value, dP - delta through its
      f32x4 sc[2], dp[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float cb[4];
        if (CPR1) {
#pragma unroll
          for (int r = 0; r < 4; ++r) cb[r] = cb0[r];
        } else {
          col_bias(ws.ws[2] + 16 * cs[h] + 4 * gq - wl[2], ww[2], cb);
        }
        sc[h] = mask_init(rok[h], cb);
#pragma unroll
        for (int r = 0; r < 4; ++r)  // -delta of the row, read into the accumulator
          dp[h][r] = *reinterpret_cast<const float *>(xs + kb[h] * RSE + pad_off + r * RSE + 2);
#pragma unroll
        for (int st = 0; st < NT; ++st) {
          sc[h] = M::mma(qr[h][st], kf[st], sc[h]);
          dp[h] = M::mma(orr[h][st], vf[st], dp[h]);
        }
      }
      v8 bp, bs;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = __builtin_amdgcn_exp2f(fmaf(sc[h][r], sl2, -ls2[h][r]));
          bp[4 * h + r] = (E)p;
          bs[4 * h + r] = (E)(p * dp[h][r]);
        }
      if (!EARLY_T) read_t();
      // dV^T += dO^T . P, dK^T += Q^T . dS
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        adv[db] = M::mma(ot[db], bp, adv[db]);
        adk[db] = M::mma(qt[db], bs, adk[db]);
      }
    }
  }
  }  // slabs
  if (!kv) return;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    v4 wk, wv;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      wk[r] = (E)(adk[db][r] * P.scale);
      wv[r] = (E)adv[db][r];
    }
    *reinterpret_cast<v4 *>(dk + koff + 16 * db + 4 * gq) = wk;
    *reinterpret_cast<v4 *>(dv + koff + 16 * db + 4 * gq) = wv;
  }
}

}  // namespace

// NATTEN_AMD_NO_PFS=1 stages every slab after the previous one is computed
// (A/B checks of the slab prefetch).
bool slab_prefetch_off() {
  static const bool off = [] {
    const char *e = std::getenv("NATTEN_AMD_NO_PFS");
    return e != nullptr && e[0] != '\0' && e[0] != '0';
  }();
  return off;
}

bool lean_eligible(const Prob &P, int dtype) {
  if (!lean_shape_ok(P, dtype)) return false;
  if (P.dense) return false;
  // per-sample extents only when the caller states that every one of them
  // satisfies d * K <= L_b on each non-causal axis
  if (P.sample_extent != nullptr && !P.varlen_clamped) return false;
  if (!(P.scale > 0.f) || !std::isfinite(P.scale)) return false;
  if ((int64_t)P.B * P.n_extra * P.Hkv * P.D >= (int64_t(1) << 31)) return false;
  return lean_choice(P, kLFwd).ok;
}

bool lean_bwd_eligible(const Prob &P, int dtype) {
  return lean_eligible(P, dtype) && lean_choice(P, kLBwd).ok;
}

#define LEAN_D(D_, BODY) \
  do {                   \
    if ((D_) == 32) {    \
      BODY(32);          \
    } else if ((D_) == 64) { \
      BODY(64);          \
    } else {             \
      BODY(128);         \
    }                    \
  } while (0)

// The forward's launch: grouped query heads (one staged box for a group
// of query heads of one key/value head) for varlen / additional-token
// problems where the box is one slab and the grouped launch still gives at
// least 4 workgroups per CU; NATTEN_AMD_HL=0 / 1 turns the grouping off /
// on wherever it applies, NATTEN_AMD_HL_HEADS=h (a divisor of the group)
// runs h query heads per workgroup instead of all of them (both read per
// call).
LProb lean_fwd_lprob(const Prob &P, const LChoice &C) {
  LProb L = make_lprob(P, C);
  const bool vx = P.n_extra > 0 || P.sample_extent != nullptr;
  const char *hl_env = std::getenv("NATTEN_AMD_HL");
  const bool hl_auto = L.n_tiles / P.rep >= 1024;
  const bool hl_want = hl_env != nullptr ? hl_env[0] == '1' : hl_auto;
  if (vx && P.rep > 1 && (P.rank < 3 || L.sl >= L.ax[0].Em) && hl_want) {
    int hpw = P.rep;
    const char *hh = std::getenv("NATTEN_AMD_HL_HEADS");
    const int h = hh != nullptr ? std::atoi(hh) : 0;
    if (h >= 1 && h < P.rep && P.rep % h == 0) hpw = h;
    L.hl = hpw;
    L.fHg = make_fastdiv((uint32_t)(P.rep / hpw));
    L.n_tiles /= hpw;
    L.n_launch = (L.n_tiles + 7) & ~7;
  }
  return L;
}

// The backward's launch: one workgroup per (sample, key/value head, tile).
LProb lean_bwd_lprob(const Prob &P, const LChoice &C) {
  LProb L = make_lprob(P, C);
  L.n_tiles = P.B * P.Hkv * (int)L.fGrid.d;
  L.n_launch = (L.n_tiles + 7) & ~7;
  return L;
}

bool lean_plan(const Prob &P, int dtype, bool backward, LeanPlanInfo *o) {
  if (!(backward ? lean_bwd_eligible(P, dtype) : lean_eligible(P, dtype))) return false;
  const LMode mode = backward ? kLBwd : kLFwd;
  const LChoice C = lean_choice(P, mode);
  const LProb L = backward ? lean_bwd_lprob(P, C) : lean_fwd_lprob(P, C);
  for (int a = 0; a < 3; ++a) {
    o->T[a] = C.T[a];
    o->Em[a] = C.Em[a];
  }
  o->W = C.W;
  o->slabs = (C.Em[0] + C.sl - 1) / C.sl;
  o->hl = L.hl;
  o->workgroups = L.n_tiles;
  o->lds = (int)lean_lds_bytes(P, mode, L.ebox, C.W);
  return true;
}

void lean_fwd(const Prob &P, int dtype, const void *q, const void *k,
              const void *v, const void *ek, const void *ev, void *out,
              float *lse, hipStream_t st) {
  const LChoice C = lean_choice(P, kLFwd);
  const LProb L = lean_fwd_lprob(P, C);
  if (L.n_tiles == 0) return;
  const bool vx = P.n_extra > 0 || P.sample_extent != nullptr;
  const bool ca = P.ax[0].causal || P.ax[1].causal || P.ax[2].causal;
  // rank 3 staged in several slabs, one query head per box: each slab's
  // loads fly while the previous slab is computed (two rounds of four
  // units per lane must cover a slab)
  // The prefetched units take up to ~250 VGPRs (two waves per SIMD), so only
  // where the LDS already holds the launch to two workgroups per CU.
  const size_t lds_f = lean_lds_bytes(P, kLFwd, L.ebox, C.W);
  const bool pfs = P.rank == 3 && !vx && (C.Em[0] + C.sl - 1) / C.sl > 1 && !L.hl &&
                   (int64_t)L.ebox * (P.D / 8) <= (int64_t)8 * 64 * C.W &&
                   3 * lds_f > (size_t)160 * 1024 && C.W <= 4 && !slab_prefetch_off();
  const size_t lds = lean_lds_bytes(P, kLFwd, L.ebox, C.W);
  const dim3 grid(L.n_launch), block(64 * C.W);
#define LF_LAUNCH2(TT, DD, RR, CC, VV, AA, PP)                                  \
  hipLaunchKernelGGL((k_wfwd<TT, DD, RR, CC, VV, AA, PP>), grid, block, lds, st, L, \
                     (const TT *)q, (const TT *)k, (const TT *)v,              \
                     (const TT *)ek, (const TT *)ev, (TT *)out, lse)
#define LF_LAUNCH1(TT, DD, RR, CC, VV)                                          \
  do {                                                                        \
    if (RR == 3 && !VV && pfs) {                                              \
      if (ca) LF_LAUNCH2(TT, DD, RR, CC, VV, true, (RR == 3 && !VV));         \
      else LF_LAUNCH2(TT, DD, RR, CC, VV, false, (RR == 3 && !VV));           \
    } else {                                                                  \
      if (ca) LF_LAUNCH2(TT, DD, RR, CC, VV, true, false);                    \
      else LF_LAUNCH2(TT, DD, RR, CC, VV, false, false);                      \
    }                                                                         \
  } while (0)
#define LF_LAUNCH(TT, DD, RR, CC)                                              \
  do {                                                                        \
    if (vx) LF_LAUNCH1(TT, DD, RR, CC, true);                                 \
    else LF_LAUNCH1(TT, DD, RR, CC, false);                                   \
  } while (0)
#define LF_R(TT, DD)                                                          \
  do {                                                                        \
    if (P.rank == 1) LF_LAUNCH(TT, DD, 1, false);                             \
    else if (P.rank == 2) {                                                   \
      if (C.cpr1) LF_LAUNCH(TT, DD, 2, true); else LF_LAUNCH(TT, DD, 2, false); \
    } else {                                                                  \
      if (C.cpr1 && C.sl == 1) LF_LAUNCH(TT, DD, 3, true); else LF_LAUNCH(TT, DD, 3, false); \
    }                                                                         \
  } while (0)
#define LF_D(DD)                          \
  do {                                    \
    if (dtype == NA_BF16) LF_R(bf16_t, DD); \
    else LF_R(f16_t, DD);                 \
  } while (0)
  LEAN_D(P.D, LF_D);
#undef LF_D
#undef LF_R
#undef LF_LAUNCH
#undef LF_LAUNCH1
#undef LF_LAUNCH2
}

void lean_bwd(const Prob &P, int dtype, const void *q, const void *k,
              const void *v, const void *ek, const void *ev,
              const void *out, const float *lse,
              const void *dout, const float *dlse, void *dq, void *dk,
              void *dv, float *delta_out, hipStream_t st) {
  const LChoice C = lean_choice(P, kLBwd);
  const LProb L = lean_bwd_lprob(P, C);
  if (L.n_tiles == 0) return;
  const size_t lds = lean_lds_bytes(P, kLBwd, L.ebox, C.W);
  const dim3 grid(L.n_launch), block(64 * C.W);
  const bool vx = P.sample_extent != nullptr || P.n_extra > 0;
  const bool ca = P.ax[0].causal || P.ax[1].causal || P.ax[2].causal;
  // the dQ half's K / V slabs prefetched (as in lean_fwd)
  const bool pfs = P.rank == 3 && !vx && (C.Em[0] + C.sl - 1) / C.sl > 1 &&
                   (int64_t)L.ebox * (P.D / 8) <= (int64_t)8 * 64 * C.W &&
                   3 * lds > (size_t)160 * 1024 && C.W <= 4 && !slab_prefetch_off();
#define LB_LAUNCH2(TT, DD, RR, CC, VV, AA, PP)                                  \
  hipLaunchKernelGGL((k_wbwd<TT, DD, RR, CC, VV, AA, PP>), grid, block, lds, st, L, \
                     (const TT *)q, (const TT *)k, (const TT *)v,              \
                     (const TT *)ek, (const TT *)ev, (const TT *)out, lse,     \
                     (const TT *)dout, dlse, (TT *)dq, (TT *)dk, (TT *)dv, delta_out)
#define LB_LAUNCH1(TT, DD, RR, CC, VV)                                          \
  do {                                                                        \
    if (RR == 3 && !VV && pfs) {                                              \
      if (ca) LB_LAUNCH2(TT, DD, RR, CC, VV, true, (RR == 3 && !VV));         \
      else LB_LAUNCH2(TT, DD, RR, CC, VV, false, (RR == 3 && !VV));           \
    } else {                                                                  \
      if (ca) LB_LAUNCH2(TT, DD, RR, CC, VV, true, false);                    \
      else LB_LAUNCH2(TT, DD, RR, CC, VV, false, false);                      \
    }                                                                         \
  } while (0)
#define LB_LAUNCH(TT, DD, RR, CC)                                             \
  do {                                                                        \
    if (vx) LB_LAUNCH1(TT, DD, RR, CC, true);                                 \
    else LB_LAUNCH1(TT, DD, RR, CC, false);                                   \
  } while (0)
#define LB_R(TT, DD)                                                          \
  do {                                                                        \
    if (P.rank == 1) LB_LAUNCH(TT, DD, 1, false);                             \
    else if (P.rank == 2) {                                                   \
      if (C.cpr1) LB_LAUNCH(TT, DD, 2, true); else LB_LAUNCH(TT, DD, 2, false); \
    } else {                                                                  \
      if (C.cpr1 && C.sl == 1) LB_LAUNCH(TT, DD, 3, true); else LB_LAUNCH(TT, DD, 3, false); \
    }                                                                         \
  } while (0)
#define LB_D(DD)                          \
  do {                                    \
    if (dtype == NA_BF16) LB_R(bf16_t, DD); \
    else LB_R(f16_t, DD);                 \
  } while (0)
  LEAN_D(P.D, LB_D);
#undef LB_D
#undef LB_R
#undef LB_LAUNCH
#undef LB_LAUNCH1
#undef LB_LAUNCH2
}

}  // namespace na
