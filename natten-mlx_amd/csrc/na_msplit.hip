// na_msplit.hip — matrix-core (gfx950 MFMA) kernels for the split ops
// (na_qk_fwd / na_av_fwd and their backward), bf16/fp16, head_dim 32/64/128.
//
// They reuse the fused kernels' tiling (32-query tiles on one dilation
// phase, key boxes walked in 32-key chunks), with the attention matrix in
// its compact [query, kernel slot] form instead of an online softmax:
//
//   k_sqk  : S^T = Y_chunk . X^T, each in-window score scattered to its
//            slot of the query's row (qk forward: X = q, Y = k, times scale;
//            av backward's dattn: X = dO, Y = v)
//   k_sav  : O^T += Y^T . A^T with A gathered from the compact rows
//            (av forward: A = attn, Y = v; qk backward's dq: A = dlogits,
//            Y = k, times scale)
//   k_sinv : per 32-key tile, over the queries whose windows hold those
//            keys: Z^T += X^T . A with A gathered per (query, key)
//            (qk backward's dk: A = dlogits, X = q, times scale; av
//            backward's dv: A = attn, X = dO)
//
// A workgroup of k_sqk / k_sav owns one spatial tile for Hb consecutive
// query heads (one wave each), so the compact rows it reads or writes,
// [position][Hb heads][kprod], are contiguous per position: they pass
// through LDS once and move to or from HBM in whole 128-byte lines.
//
// Slot of a key in a query's window, per axis on the sub-grid: key minus
// the window start, where the start is clamp(i - K/2, 0, Lr - K) for a
// non-causal axis (d*K <= L) and i - K + 1 for a causal one.
#include "na_mfma.h"

namespace na {
namespace {

constexpr int kMaxHb = 8;  // query heads per k_sqk / k_sav workgroup

// Chunk mask (as chunk_mask) plus each element's kernel slot in the lane's
// query window: slot = sum over axes of (box coord - sb[a]) * ks[a], with
// sb the window's slot-0 coordinate relative to the box and ks the slot
// strides (K1*K2, K2, 1).
__device__ __forceinline__ void chunk_slots(const Box &bx, const ChunkRows &cr,
                                            int g0, int h, const int wlo[3],
                                            const int ww[3], const int sb[3],
                                            const int ks[3], bool ok[16],
                                            int slot[16]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int g = g0 + 8 * i;
    const int xb = g & ((1 << bx.lgP) - 1);
    int e0 = cr.e0, e1 = cr.e1;
    row_add(e0, e1, uni((g >> bx.lgP) - cr.R0), bx.E[1]);
    const bool rowok = ((unsigned)(e1 - wlo[1]) < (unsigned)ww[1]) &
                       ((unsigned)(e0 - wlo[0]) < (unsigned)ww[0]);
    const int rbase = (e0 - sb[0]) * ks[0] + (e1 - sb[1]) * ks[1];
    const int x0 = xb + 4 * h;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ok[4 * i + j] = rowok & ((unsigned)(x0 + j - wlo[2]) < (unsigned)ww[2]);
      slot[4 * i + j] = rbase + (x0 + j - sb[2]);
    }
  }
}

// Window start of sub-grid query i on axis a (see the file comment).
__device__ __forceinline__ int sub_start(const Axis &x, int i, int Lr) {
  if (x.causal) return i - x.K + 1;
  const int s = i - x.K / 2;
  return s < 0 ? 0 : (s > Lr - x.K ? Lr - x.K : s);
}

// Tile of a k_sqk / k_sav workgroup: wave w serves query head h0 + w.
struct SplitTile {
  QTile Q;
  int h0, head, hk;
  int sb[3], ks[3];
};

__device__ __forceinline__ SplitTile split_tile(const Prob &P, const Tiling &Tl,
                                                int tile, int Hb, int w, int n) {
  SplitTile S;
  TileCtx tc = decode_tile(P, Tl, tile, Tl.fH);
  S.h0 = tc.head * Hb;
  S.head = S.h0 + w;
  tc.head = S.head;
  S.Q = query_tile(P, Tl, tc, n);
  S.hk = S.head / P.rep;
  S.ks[2] = 1;
  S.ks[1] = P.ax[2].K;
  S.ks[0] = P.ax[1].K * P.ax[2].K;
#pragma unroll
  for (int a = 0; a < 3; ++a) S.sb[a] = S.Q.wlo[a] + S.Q.ww[a] - P.ax[a].K;
  return S;
}

// Token of tile position p, or -1 when p lies outside the tensor.
__device__ __forceinline__ int64_t tile_token(const Prob &P, const Tiling &Tl,
                                              const TileCtx &tc, int p) {
  int u[3];
  tile_slot(Tl, p, u);
  if (!((u[0] < tc.nt[0]) & (u[1] < tc.nt[1]) & (u[2] < tc.nt[2]))) return -1;
  int pos[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) pos[a] = tc.r[a] + P.ax[a].d * (tc.i0[a] + u[a]);
  return tok_in(P, tc.b, pos[0], pos[1], pos[2]);
}

// Chunks whose operand rows are loaded together before any is computed:
// the tiles hold few chunks (five for a 7x7 window), so issuing them all at
// once leaves one memory latency per tile instead of one per chunk.
constexpr int prefetch_depth(int D) { return D == 32 ? 8 : D == 64 ? 4 : 2; }

// Load the A-operand rows (lane (slot, h): elements 16t + 8h ..) of one chunk.
template <typename T, int D>
__device__ __forceinline__ void load_rows(const T *p, typename Mf<T>::v8 *f,
                                          int h) {
#pragma unroll
  for (int t = 0; t < D / 16; ++t) f[t] = ld8(p + 16 * t + 8 * h);
}

// ---------------------------------------------------------------------------
// k_sqk: compact scores out[q, slot] = scale * <x_q, y_key(slot)>; slots
// outside the window hold `fill`.
template <typename T, int D>
__global__ void __launch_bounds__(64 * kMaxHb)
    k_sqk(Prob P, Tiling Tl, const T *__restrict__ x, const T *__restrict__ y,
          T *__restrict__ out, float scale, float fill) {
  typedef Mf<T> M;
  typedef typename M::v8 v8;
  typedef typename M::e E;
  constexpr int NK = D / 16;
  extern __shared__ __align__(16) char smem[];

  const int tile = xcd_tile(blockIdx.x, Tl.n_launch);
  if (tile >= Tl.n_q) return;
  const int Hb = blockDim.x >> 6, w = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63, n = lane & 31, h = lane >> 5;
  const SplitTile S = split_tile(P, Tl, tile, Hb, w, n);
  const QTile &Q = S.Q;
  const int kp = P.kprod;
  E *stg = reinterpret_cast<E *>(smem);
  E *mine = stg + (n * Hb + w) * kp;
  const E fv = (E)fill;
  for (int s = h; s < kp; s += 2) mine[s] = fv;

  v8 qf[NK];
  const int64_t qrow = (Q.qtok * P.H + S.head) * D;
#pragma unroll
  for (int t = 0; t < NK; ++t)
    qf[t] = Q.q_valid ? ld8(x + qrow + 16 * t + 8 * h) : zero8<T>();

  // chunks in groups of NB: every load of a group is issued before the
  // first of its chunks is computed, so a group waits on memory once
  constexpr int NB = prefetch_depth(D);
  const BoxAddr ka = box_addr(P, Q.tc, Q.bx, S.hk, P.Hkv);
  RowCursor rc{0, 0, 0};
  for (int c0 = 0; c0 < Q.nbox; c0 += NB) {
    ChunkRows cr[NB];
    v8 kf[NB][NK];
#pragma unroll
    for (int j = 0; j < NB; ++j)
      if (c0 + j < Q.nbox) {
        cr[j] = chunk_rows(rc, Q.bx, 32 * (c0 + j));
        int e[3];
        box_point(Q.bx, cr[j], 32 * (c0 + j), n, e);
        load_rows<T, D>(y + ka.base + box_off(ka, e), kf[j], h);
      }
#pragma unroll
    for (int j = 0; j < NB; ++j)
      if (c0 + j < Q.nbox) {
        f32x16 s = zero16();
#pragma unroll
        for (int t = 0; t < NK; ++t) s = M::mma(kf[j][t], qf[t], s);
        bool ok[16];
        int slot[16];
        chunk_slots(Q.bx, cr[j], 32 * (c0 + j), h, Q.wlo, Q.ww, S.sb, S.ks, ok, slot);
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (ok[e]) mine[slot[e]] = (E)(s[e] * scale);
      }
  }
  __syncthreads();
  const int row = Hb * kp;
  E *dst0 = reinterpret_cast<E *>(out);
  for (int p = w; p < 32; p += Hb) {
    const int64_t tok = tile_token(P, Tl, Q.tc, p);
    if (tok < 0) continue;
    E *dst = dst0 + (tok * P.H + S.h0) * kp;
    const E *src = stg + p * row;
    for (int i = lane; i < row; i += 64) dst[i] = src[i];
  }
}

// ---------------------------------------------------------------------------
// k_sav: out_q = scale * sum over window slots of a[q, slot] * y_key(slot).
template <typename T, int D>
__global__ void __launch_bounds__(64 * kMaxHb)
    k_sav(Prob P, Tiling Tl, const T *__restrict__ a, const T *__restrict__ y,
          T *__restrict__ out, float scale) {
  typedef Mf<T> M;
  typedef typename M::v8 v8;
  typedef typename M::e E;
  constexpr int NK = D / 16, NC = D / 32;
  extern __shared__ __align__(16) char smem[];

  const int tile = xcd_tile(blockIdx.x, Tl.n_launch);
  if (tile >= Tl.n_q) return;
  const int Hb = blockDim.x >> 6, w = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63, n = lane & 31, h = lane >> 5;
  const SplitTile S = split_tile(P, Tl, tile, Hb, w, n);
  const QTile &Q = S.Q;
  const int kp = P.kprod;
  const int row = Hb * kp;
  E *stg = reinterpret_cast<E *>(smem);
  E *vt = stg + ((32 * row + 7) & ~7) + w * D * kRow;

  // the tile's compact rows, all Hb heads, into LDS
  const E *src0 = reinterpret_cast<const E *>(a);
  for (int p = w; p < 32; p += Hb) {
    const int64_t tok = tile_token(P, Tl, Q.tc, p);
    if (tok < 0) continue;
    const E *src = src0 + (tok * P.H + S.h0) * kp;
    E *dst = stg + p * row;
    for (int i = lane; i < row; i += 64) dst[i] = src[i];
  }
  __syncthreads();
  const E *mine = stg + (n * Hb + w) * kp;

  f32x16 acc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = zero16();
  constexpr int NB = prefetch_depth(D);
  const BoxAddr ka = box_addr(P, Q.tc, Q.bx, S.hk, P.Hkv);
  RowCursor rc{0, 0, 0};
  for (int c0 = 0; c0 < Q.nbox; c0 += NB) {
    ChunkRows cr[NB];
    v8 vf[NB][NK];
#pragma unroll
    for (int j = 0; j < NB; ++j)
      if (c0 + j < Q.nbox) {
        cr[j] = chunk_rows(rc, Q.bx, 32 * (c0 + j));
        int e[3];
        box_point(Q.bx, cr[j], 32 * (c0 + j), n, e);
        load_rows<T, D>(y + ka.base + box_off(ka, e), vf[j], h);
      }
#pragma unroll
    for (int j = 0; j < NB; ++j)
      if (c0 + j < Q.nbox) {
        bool ok[16];
        int slot[16];
        chunk_slots(Q.bx, cr[j], 32 * (c0 + j), h, Q.wlo, Q.ww, S.sb, S.ks, ok, slot);
        float pv[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) pv[e] = ok[e] ? (float)mine[slot[e]] : 0.f;
        wave_lds_sync();
#pragma unroll
        for (int t = 0; t < NK; ++t)
#pragma unroll
          for (int e = 0; e < 8; ++e)
            vt[(16 * t + 8 * h + e) * kRow + n] = vf[j][t][e];
        wave_lds_sync();
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const v8 bp = pack8<T>(pv + 8 * kb);
#pragma unroll
          for (int cc = 0; cc < NC; ++cc)
            acc[cc] = M::mma(lds_a<T>(vt + (32 * cc + n) * kRow + 16 * kb, h), bp,
                             acc[cc]);
        }
      }
  }
  if (Q.q_tensor) {
    const int64_t orow = (Q.qtok * P.H + S.head) * D;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        typename M::v4 wv;
#pragma unroll
        for (int j = 0; j < 4; ++j) wv[j] = (E)(acc[cc][4 * i + j] * scale);
        *reinterpret_cast<typename M::v4 *>(out + orow + 32 * cc + 8 * i + 4 * h) = wv;
      }
  }
}

// ---------------------------------------------------------------------------
// k_sinv: z_key = scale * sum over query heads of the key's group and the
// queries i whose windows hold the key, of a[i, slot(i, key)] * x_i.
template <typename T, int D>
__global__ void __launch_bounds__(64)
    k_sinv(Prob P, Tiling Tl, const T *__restrict__ a, const T *__restrict__ x,
           T *__restrict__ out, float scale) {
  typedef Mf<T> M;
  typedef typename M::v8 v8;
  typedef typename M::e E;
  constexpr int NK = D / 16, NC = D / 32;
  extern __shared__ __align__(16) char smem[];

  const int tile = xcd_tile(blockIdx.x, Tl.n_launch);
  if (tile >= Tl.n_k) return;
  const int lane = threadIdx.x & 63, n = lane & 31, h = lane >> 5;
  E *ta = reinterpret_cast<E *>(smem);
  const TileCtx tc = decode_tile(P, Tl, tile, Tl.fHk);
  const int hk = tc.head;
  const int kp = P.kprod;
  int u[3];
  tile_slot(Tl, n, u);
  const bool k_tensor = (u[0] < tc.nt[0]) & (u[1] < tc.nt[1]) & (u[2] < tc.nt[2]);
  const bool k_valid = (u[0] < tc.nv[0]) & (u[1] < tc.nv[1]) & (u[2] < tc.nv[2]);
  const bool any = (tc.nv[0] > 0) & (tc.nv[1] > 0) & (tc.nv[2] > 0);
  int pos[3], Lr[3], kj[3];
#pragma unroll
  for (int ax = 0; ax < 3; ++ax) {
    kj[ax] = tc.i0[ax] + u[ax];
    pos[ax] = tc.r[ax] + P.ax[ax].d * kj[ax];
    Lr[ax] = P.ax[ax].d == 1 ? tc.L[ax]
             : tc.L[ax] > tc.r[ax]
                 ? (int)fdiv((uint32_t)(tc.L[ax] - 1 - tc.r[ax]), Tl.fd[ax]) + 1
                 : 0;
  }
  const int64_t krow = (tok_in(P, tc.b, pos[0], pos[1], pos[2]) * P.Hkv + hk) * D;

  // query box = union of the tile keys' inverse neighborhoods
  Box bx;
#pragma unroll
  for (int ax = 0; ax < 3; ++ax) {
    int lo0 = 0, hi0 = 0, lo1 = 0, hi1 = 0;
    if (any) {
      sub_inverse(P, Tl, ax, tc.L[ax], tc.r[ax], Lr[ax], tc.i0[ax], lo0, hi0);
      sub_inverse(P, Tl, ax, tc.L[ax], tc.r[ax], Lr[ax], tc.i0[ax] + tc.nv[ax] - 1,
                  lo1, hi1);
    }
    bx.lo[ax] = uni(lo0);
    bx.E[ax] = uni(any ? max(hi1 - lo0 + 1, 1) : 1);
  }
  box_init(bx);
  bx.lgP = uni(bx.lgP);
  const int nchunk = uni(any ? (bx.slots + 31) >> 5 : 0);
  const int K0 = P.ax[0].K, K1 = P.ax[1].K, K2 = P.ax[2].K;
  constexpr int NB = prefetch_depth(D) / 2;

  f32x16 acc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = zero16();

  for (int hq = hk * P.rep; hq < (hk + 1) * P.rep; ++hq) {
    const BoxAddr xa = box_addr(P, tc, bx, hq, P.H);
    // the same box addressed in compact rows (element (tok*H + hq)*kp)
    BoxAddr aa;
    aa.base = xa.base / D * kp;
#pragma unroll
    for (int ax = 0; ax < 3; ++ax) aa.S[ax] = uni(xa.S[ax] / D * kp);
    RowCursor rc{0, 0, 0};
    for (int c0 = 0; c0 < nchunk; c0 += NB) {
      // issue the group's query-row loads and A gathers, then compute
      v8 xf[NB][NK];
      float pv[NB][16];
#pragma unroll
      for (int jc = 0; jc < NB; ++jc) {
        if (c0 + jc >= nchunk) break;
        const int c = c0 + jc;
        const ChunkRows cr = chunk_rows(rc, bx, 32 * c);
        int e[3];
        box_point(bx, cr, 32 * c, n, e);
        load_rows<T, D>(x + xa.base + box_off(xa, e), xf[jc], h);
        // A of (query element, this lane's key): element 4i + j is chunk
        // slot 8i + 4h + j; its row (e0, e1) is wave-uniform per i
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int g = 32 * c + 8 * i;
          const int xb = g & ((1 << bx.lgP) - 1);
          int e0 = cr.e0, e1 = cr.e1;
          row_add(e0, e1, uni((g >> bx.lgP) - cr.R0), bx.E[1]);
          const int s0 = kj[0] - sub_start(P.ax[0], bx.lo[0] + e0, Lr[0]);
          const int s1 = kj[1] - sub_start(P.ax[1], bx.lo[1] + e1, Lr[1]);
          const bool rowok = (e0 < bx.E[0]) & ((unsigned)s0 < (unsigned)K0) &
                             ((unsigned)s1 < (unsigned)K1) & k_valid;
          const int64_t rbase = aa.base + e0 * aa.S[0] + e1 * aa.S[1] +
                                (s0 * K1 + s1) * K2;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int xe = xb + 4 * h + j;
            const int s2 = kj[2] - sub_start(P.ax[2], bx.lo[2] + xe, Lr[2]);
            const bool ok = rowok & (xe < bx.E[2]) & ((unsigned)s2 < (unsigned)K2);
            pv[jc][4 * i + j] =
                ok ? (float)reinterpret_cast<const E *>(a)[rbase + xe * aa.S[2] + s2]
                   : 0.f;
          }
        }
      }
#pragma unroll
      for (int jc = 0; jc < NB; ++jc) {
        if (c0 + jc >= nchunk) break;
        wave_lds_sync();
#pragma unroll
        for (int t = 0; t < NK; ++t)
#pragma unroll
          for (int e = 0; e < 8; ++e) ta[(16 * t + 8 * h + e) * kRow + n] = xf[jc][t][e];
        wave_lds_sync();
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const v8 bp = pack8<T>(pv[jc] + 8 * kb);
#pragma unroll
          for (int cc = 0; cc < NC; ++cc)
            acc[cc] = M::mma(lds_a<T>(ta + (32 * cc + n) * kRow + 16 * kb, h), bp,
                             acc[cc]);
        }
      }
    }
  }
  if (k_tensor) {
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        typename M::v4 wv;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          wv[j] = (E)(k_valid ? acc[cc][4 * i + j] * scale : 0.f);
        *reinterpret_cast<typename M::v4 *>(out + krow + 32 * cc + 8 * i + 4 * h) = wv;
      }
  }
}

// ---------------------------------------------------------------------------
// Host side.

// Query heads per k_sqk / k_sav workgroup: the largest divisor of H up to
// kMaxHb whose compact rows (32 positions x Hb x kprod) fit in 32 KB.
int split_heads(const Prob &P) {
  for (int hb = kMaxHb; hb >= 1; --hb)
    if (P.H % hb == 0 && (size_t)32 * hb * P.kprod * 2 <= 32768) return hb;
  return 1;
}

Tiling split_tiling(const Prob &P, int Hb) {
  double chunks = 1.0;
  Tiling Tl = choose_tiling(P, P.H / Hb, P.Hkv, &chunks);
  return Tl;
}

size_t stage_bytes(const Prob &P, int Hb) {
  return (((size_t)32 * Hb * P.kprod + 7) & ~(size_t)7) * 2;
}

#define NA_MS_D(D_, BODY) \
  do {                    \
    if ((D_) == 32) {     \
      BODY(32);           \
    } else if ((D_) == 64) { \
      BODY(64);           \
    } else {              \
      BODY(128);          \
    }                     \
  } while (0)

}  // namespace

bool msplit_eligible(const Prob &P, int dtype) {
  if (!mfma_eligible(P, dtype) || P.dense || P.sample_extent != nullptr)
    return false;
  for (int a = 0; a < 3; ++a) {
    const Axis &x = P.ax[a];
    if (!x.causal && x.d * x.K > x.L) return false;
  }
  return (size_t)32 * P.kprod * 2 <= 32768;
}

void msplit_qk(const Prob &P, int dtype, const void *x, const void *y,
               void *out, float scale, float fill, hipStream_t st) {
  const int Hb = split_heads(P);
  Tiling Tl = split_tiling(P, Hb);
  Tl.n_launch = (Tl.n_q + 7) & ~7;
  if (Tl.n_q == 0) return;
  const size_t lds = stage_bytes(P, Hb);
#define QK_(DD)                                                               \
  if (dtype == NA_BF16)                                                       \
    hipLaunchKernelGGL((k_sqk<bf16_t, DD>), dim3(Tl.n_launch), dim3(64 * Hb), \
                       lds, st, P, Tl, (const bf16_t *)x, (const bf16_t *)y,  \
                       (bf16_t *)out, scale, fill);                           \
  else                                                                        \
    hipLaunchKernelGGL((k_sqk<f16_t, DD>), dim3(Tl.n_launch), dim3(64 * Hb),  \
                       lds, st, P, Tl, (const f16_t *)x, (const f16_t *)y,    \
                       (f16_t *)out, scale, fill)
  NA_MS_D(P.D, QK_);
#undef QK_
}

void msplit_av(const Prob &P, int dtype, const void *a, const void *y,
               void *out, float scale, hipStream_t st) {
  const int Hb = split_heads(P);
  Tiling Tl = split_tiling(P, Hb);
  Tl.n_launch = (Tl.n_q + 7) & ~7;
  if (Tl.n_q == 0) return;
  const size_t lds = stage_bytes(P, Hb) + (size_t)Hb * P.D * kRow * 2;
#define AV_(DD)                                                               \
  if (dtype == NA_BF16)                                                       \
    hipLaunchKernelGGL((k_sav<bf16_t, DD>), dim3(Tl.n_launch), dim3(64 * Hb), \
                       lds, st, P, Tl, (const bf16_t *)a, (const bf16_t *)y,  \
                       (bf16_t *)out, scale);                                 \
  else                                                                        \
    hipLaunchKernelGGL((k_sav<f16_t, DD>), dim3(Tl.n_launch), dim3(64 * Hb),  \
                       lds, st, P, Tl, (const f16_t *)a, (const f16_t *)y,    \
                       (f16_t *)out, scale)
  NA_MS_D(P.D, AV_);
#undef AV_
}

void msplit_inv(const Prob &P, int dtype, const void *a, const void *x,
                void *out, float scale, hipStream_t st) {
  double chunks = 1.0;
  Tiling Tl = choose_tiling(P, P.H, P.Hkv, &chunks);
  Tl.n_launch = (Tl.n_k + 7) & ~7;
  if (Tl.n_k == 0) return;
  const size_t lds = (size_t)P.D * kRow * 2;
#define INV_(DD)                                                              \
  if (dtype == NA_BF16)                                                       \
    hipLaunchKernelGGL((k_sinv<bf16_t, DD>), dim3(Tl.n_launch), dim3(64), lds, \
                       st, P, Tl, (const bf16_t *)a, (const bf16_t *)x,       \
                       (bf16_t *)out, scale);                                 \
  else                                                                        \
    hipLaunchKernelGGL((k_sinv<f16_t, DD>), dim3(Tl.n_launch), dim3(64), lds,  \
                       st, P, Tl, (const f16_t *)a, (const f16_t *)x,         \
                       (f16_t *)out, scale)
  NA_MS_D(P.D, INV_);
#undef INV_
}

}  // namespace na
