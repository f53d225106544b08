// na_dense.hip — dense (FMHA) forward on gfx950 matrix cores: every query
// attends to every key of its sample and to the sample's additional tokens.
// This is the reference's dense-attention route for kernel_size >= extent on
// every axis (functional.py:141-187, which calls the framework's scaled dot
// product attention); a query's window is the whole sample, so the spatial
// structure drops out and a sample is a sequence of Ltot tokens.
//
// Workgroup: 4 waves over 64 NQ consecutive queries of one (sample, head);
// each wave holds NQ sub-tiles of 16 queries.  The keys run in tiles of 64
// (four 16-key chunks), staged once per workgroup into one of two LDS
// buffers, K and V rows interleaved as in the lean kernels, while the tile
// before it is computed; one barrier per tile.  Per tile and sub-tile:
// S^T = K Q^T on 16x16x32 MFMAs (K rows from LDS as the A operand, shared by
// the NQ sub-tiles; Q in registers), the online softmax of the lean forward
// (lazy rescale, row sums on the matrix core), then O^T += V^T P^T with V^T
// read by transposing LDS reads, also shared by the sub-tiles.

#include "na_launch.h"
#include "na_lean.h"

namespace na {
namespace {

constexpr int kDTileKeys = 64;  // keys per staged tile
constexpr int kDThreads = 256;  // 4 waves

struct DProb {
  int32_t L;         // tokens per sample (query and key positions)
  int32_t Lk;        // keys per sample: L + nx
  int32_t nx;        // additional tokens per sample
  int32_t H, Hkv, nqb, n_tiles, n_launch;
  float sl2;         // scale * log2(e)
  float scale;
  FastDiv fnqb;      // query blocks per (sample, head)
  FastDiv fH;        // query heads
  FastDiv fRep;      // query heads per key/value head
  FastDiv fHkv;      // key/value heads
};

template <typename T, int D, int NQ>
__global__ void __launch_bounds__(kDThreads)
    k_dfwd(DProb P, const T *__restrict__ q, const T *__restrict__ k,
           const T *__restrict__ v, const T *__restrict__ ek,
           const T *__restrict__ ev, T *__restrict__ out,
           float *__restrict__ lse) {
  typedef L16<T> M;
  typedef typename M::v8 v8;
  typedef typename M::v4 v4;
  typedef typename M::e E;
  constexpr int NT = D / 32;   // 32-wide k-steps over head_dim
  constexpr int NDB = D / 16;  // 16-row blocks of O^T
  constexpr int RSE = lds_row(D);
  constexpr int UPR = D / 4;                       // 16-byte units per staged row (K, V)
  constexpr int RPP = kDThreads / UPR;             // rows per pass of the workgroup
  constexpr int NU = kDTileKeys / RPP;             // units per thread per tile
  extern __shared__ __align__(16) char smem[];
  E *const buf0 = reinterpret_cast<E *>(smem);

  const int tile = xcd_tile(blockIdx.x, P.n_launch);
  if (tile >= P.n_tiles) return;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int n = lane & 15, gq = lane >> 4;
  const int bh = (int)fdiv((uint32_t)tile, P.fnqb);
  const int qb = tile - bh * P.nqb;
  const int b = (int)fdiv((uint32_t)bh, P.fH);
  const int h = bh - b * P.H;
  const int hk = (int)fdiv((uint32_t)h, P.fRep);

  // ---- staging: this thread's fixed column unit c and rows r0 + RPP i ----
  const int c = tid % UPR, r0 = tid / UPR;
  const bool isv = c >= D / 8;
  const int col = 8 * (isv ? c - D / 8 : c);
  const T *const src = isv ? v : k;
  const T *const xsrc = isv ? ev : ek;
  const int lds_unit = r0 * RSE + 8 * c + (isv ? 8 : 0);
  v8 pre[NU];
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int i = 0; i < NU; ++i) {
      const int kk = min(t0 + r0 + RPP * i, P.Lk - 1);
      const bool box = kk < P.L;
      const int off = box ? ((b * P.L + kk) * P.Hkv + hk) * D + col
                          : ((b * P.nx + kk - P.L) * P.Hkv + hk) * D + col;
      pre[i] = ld8(box ? src : xsrc, off);
    }
  };
  auto store_tile = [&](E *dst) {
#pragma unroll
    for (int i = 0; i < NU; ++i)
      *reinterpret_cast<v8 *>(dst + lds_unit + RPP * i * RSE) = pre[i];
  };

  // ---- the wave's query rows (clamped loads; rows past L are not stored) ----
  const int qbase = qb * (64 * NQ) + w * (16 * NQ);
  v8 qf[NQ][NT];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
    const int qq = min(qbase + 16 * qi + n, P.L - 1);
#pragma unroll
    for (int st = 0; st < NT; ++st)
      qf[qi][st] = ld8(q, ((b * P.L + qq) * P.H + h) * D + 32 * st + 8 * gq);
  }
  load_tile(0);

  f32x4 o[NQ][NDB], lacc[NQ];
  float m[NQ];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[qi][db] = zero4();
    lacc[qi] = zero4();
    m[qi] = -INFINITY;
  }
  v8 ones;
#pragma unroll
  for (int i = 0; i < 8; ++i) ones[i] = (E)(n == 0 ? 1.f : 0.f);
  const float sl2 = P.sl2;
  // operand-read lane offsets inside a chunk: K rows (key n, 8 elements at
  // 8 gq) and the transposing read of V (row 4 gq + n / 4, column 4 (n % 4))
  const int ka_off = n * RSE + 8 * gq;
  const int tr_off = (4 * gq + (n >> 2)) * RSE + 4 * (n & 3);

  store_tile(buf0);
  __syncthreads();
  const int nkt = (P.Lk + kDTileKeys - 1) / kDTileKeys;
  // One 64-key tile.  Only the last tile can hold keys past the sample's
  // last token: its scores start at 0 or -inf per key, every other tile's
  // at zero (the MFMA's zero accumulator operand, no per-element setup).
  auto run_tile = [&](const int j, auto last_tile) {
    constexpr bool LAST = decltype(last_tile)::value;
    const int t0 = j * kDTileKeys;
    if (!LAST) load_tile(t0 + kDTileKeys);  // in flight during this tile
    const E *ks = buf0 + (j & 1) * (kDTileKeys * RSE);
    const E *vs = ks + lds_y(D);
    v8 ka[4][NT];
#pragma unroll
    for (int ch = 0; ch < 4; ++ch)
#pragma unroll
      for (int st = 0; st < NT; ++st)
        ka[ch][st] = *reinterpret_cast<const v8 *>(ks + 16 * ch * RSE + ka_off + 32 * st);
    float cb[4][4];
#pragma unroll
    for (int ch = 0; ch < 4; ++ch)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        cb[ch][r] = !LAST || t0 + 16 * ch + 4 * gq + r < P.Lk ? 0.f : -INFINITY;
    v8 bp[NQ][2];
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) {
      f32x4 sv[4];
#pragma unroll
      for (int ch = 0; ch < 4; ++ch) {
#pragma unroll
        for (int r = 0; r < 4; ++r) sv[ch][r] = cb[ch][r];
#pragma unroll
        for (int st = 0; st < NT; ++st) sv[ch] = M::mma(ka[ch][st], qf[qi][st], sv[ch]);
      }
      float mx = -INFINITY;
#pragma unroll
      for (int ch = 0; ch < 4; ++ch)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sv[ch][r]);
      mx = quad_max(mx) * sl2;
      // the reference point may trail the running max by up to 8 (a factor
      // 2^8 in P): exact after the final division by l
      if (__builtin_amdgcn_ballot_w64(mx > m[qi] + 8.f) != 0) {
        const float mn = fmaxf(m[qi], mx);
        const float alpha = __builtin_amdgcn_exp2f(m[qi] - (mn == -INFINITY ? 0.f : mn));
        lacc[qi] *= alpha;
#pragma unroll
        for (int db = 0; db < NDB; ++db) o[qi][db] *= alpha;
        m[qi] = mn;
      }
      const float mu = m[qi] == -INFINITY ? 0.f : m[qi];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            bp[qi][jj][4 * hh + r] =
                (E)__builtin_amdgcn_exp2f(fmaf(sv[2 * jj + hh][r], sl2, -mu));
    }
    // O^T += V^T . P^T, two chunks per MFMA, the V^T operand shared by the
    // sub-tiles
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const E *ca = vs + 32 * jj * RSE + tr_off;
      const E *cb2 = ca + 16 * RSE;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const v4 lo4 = M::tr(ca + 16 * db);
        const v4 hi4 = M::tr(cb2 + 16 * db);
        const v8 a = __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int qi = 0; qi < NQ; ++qi) o[qi][db] = M::mma(a, bp[qi][jj], o[qi][db]);
      }
#pragma unroll
      for (int qi = 0; qi < NQ; ++qi) lacc[qi] = M::mma(ones, bp[qi][jj], lacc[qi]);
    }
    if (!LAST) store_tile(buf0 + ((j + 1) & 1) * (kDTileKeys * RSE));
    __syncthreads();
  };
  for (int j = 0; j + 1 < nkt; ++j) run_tile(j, std::false_type{});
  run_tile(nkt - 1, std::true_type{});

  // ---- epilogue: l over the query's 4 lanes, normalise, store ----
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
    const float l = quad_sum(lacc[qi][0]);
    const int qq = qbase + 16 * qi + n;
    if (qq < P.L) {
      const int qoff = ((b * P.L + qq) * P.H + h) * D;
      const float inv = 1.f / l;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        v4 wv;
#pragma unroll
        for (int r = 0; r < 4; ++r) wv[r] = (E)(o[qi][db][r] * inv);
        *reinterpret_cast<v4 *>(out + qoff + 16 * db + 4 * gq) = wv;
      }
      if (lse != nullptr && gq == 0) lse[qoff / D] = (m[qi] + __log2f(l)) * kLn2;
    }
  }
}

// ---------------------------------------------------------------------------
// Backward: delta = rowsum(dO * O) - dLSE per query row comes from the delta
// pass; then two kernels, each deterministic (no atomics):
//  * k_ddkv: a workgroup per (sample, key/value head, block of 64 NK keys,
//    the additional tokens being keys L .. L + nx - 1); each wave holds NK
//    sub-tiles of 16 keys (K, V rows in registers) and the query rows of
//    every query head of the group stream through LDS in tiles of 64 (Q and
//    dO rows interleaved, with lse * log2(e) and delta per row): S = Q K^T,
//    dP - delta = dO V^T - delta, P = exp2(S scale log2(e) - lse log2(e)),
//    dS = P (dP - delta); dV^T += dO^T P and dK^T += Q^T dS with the
//    transposed operands read once per chunk pair for the NK sub-tiles.
//  * k_ddq: a workgroup per (sample, head, block of 64 NQ queries); Q and dO
//    rows in registers, K / V tiles of 64 keys through LDS as in the
//    forward: S^T, dP^T - delta, dS^T, then dQ^T += K^T dS^T.

template <typename T, int D, int NK>
__global__ void __launch_bounds__(kDThreads)
    k_ddkv(DProb P, const T *__restrict__ q, const T *__restrict__ k,
           const T *__restrict__ v, const T *__restrict__ ek,
           const T *__restrict__ ev, const T *__restrict__ dout,
           const float *__restrict__ lse, const float *__restrict__ delta,
           T *__restrict__ dk, T *__restrict__ dv, T *__restrict__ dek,
           T *__restrict__ dev) {
  typedef L16<T> M;
  typedef typename M::v8 v8;
  typedef typename M::v4 v4;
  typedef typename M::e E;
  constexpr int NT = D / 32, NDB = D / 16;
  constexpr int RSE = lds_row(D);
  constexpr int UPR = D / 4, RPP = kDThreads / UPR, NU = kDTileKeys / RPP;
  constexpr int TILE = kDTileKeys * RSE;  // elements of one row buffer
  extern __shared__ __align__(16) char smem[];
  E *const buf0 = reinterpret_cast<E *>(smem);
  float *const fl0 = reinterpret_cast<float *>(buf0 + 2 * TILE);  // [2][lse2 64, delta 64]

  const int tile = xcd_tile(blockIdx.x, P.n_launch);
  if (tile >= P.n_tiles) return;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int n = lane & 15, gq = lane >> 4;
  const int bh = (int)fdiv((uint32_t)tile, P.fnqb);  // key blocks per (sample, kv head)
  const int kb = tile - bh * P.nqb;
  const int b = (int)fdiv((uint32_t)bh, P.fHkv);
  const int hk = bh - b * P.Hkv;
  const int rep = P.H / P.Hkv;

  // the wave's keys: sub-tile ki holds keys kbase + 16 ki + n (clamped loads)
  const int kbase = kb * (64 * NK) + w * (16 * NK);
  v8 kf[NK][NT], vf[NK][NT];
#pragma unroll
  for (int ki = 0; ki < NK; ++ki) {
    const int kk = min(kbase + 16 * ki + n, P.Lk - 1);
    const bool box = kk < P.L;
    const int off = box ? ((b * P.L + kk) * P.Hkv + hk) * D
                        : ((b * P.nx + kk - P.L) * P.Hkv + hk) * D;
#pragma unroll
    for (int st = 0; st < NT; ++st) {
      kf[ki][st] = ld8(box ? k : ek, off + 32 * st + 8 * gq);
      vf[ki][st] = ld8(box ? v : ev, off + 32 * st + 8 * gq);
    }
  }

  // ---- staging of query tile it = (head hr of the group, tile t) ----
  const int c = tid % UPR, r0 = tid / UPR;
  const bool isd = c >= D / 8;
  const int col = 8 * (isd ? c - D / 8 : c);
  const T *const src = isd ? dout : q;
  const int lds_unit = r0 * RSE + 8 * c + (isd ? 8 : 0);
  const int nqt = (P.L + kDTileKeys - 1) / kDTileKeys;
  v8 pre[NU];
  float pre_l = 0.f, pre_d = 0.f;
  // query tile (head hk rep + hr, rows t0 ..): unit i reads row t0 + r0 + RPP i
  const int qstep = P.H * D;
  auto load_tile = [&](int hr, int t0) {
    const int h = hk * rep + hr;
    if (t0 + kDTileKeys <= P.L) {  // wave-uniform
      const int o0 = ((b * P.L + t0 + r0) * P.H + h) * D + col;
#pragma unroll
      for (int i = 0; i < NU; ++i) pre[i] = ld8(src, o0 + RPP * i * qstep);
    } else {
#pragma unroll
      for (int i = 0; i < NU; ++i) {
        const int qq = min(t0 + r0 + RPP * i, P.L - 1);
        pre[i] = ld8(src, ((b * P.L + qq) * P.H + h) * D + col);
      }
    }
    if (tid < kDTileKeys) {
      const int qq = t0 + tid;
      const int row = (b * P.L + min(qq, P.L - 1)) * P.H + h;
      // rows past the sample: lse +inf gives P = 0, delta 0 keeps dS = 0
      pre_l = qq < P.L ? ldf(lse, row) * kLog2e : INFINITY;
      pre_d = qq < P.L ? ldf(delta, row) : 0.f;
    }
  };
  auto store_tile = [&](int slot) {
    E *dst = buf0 + slot * TILE;
#pragma unroll
    for (int i = 0; i < NU; ++i)
      *reinterpret_cast<v8 *>(dst + lds_unit + RPP * i * RSE) = pre[i];
    if (tid < kDTileKeys) {
      fl0[slot * 128 + tid] = pre_l;
      fl0[slot * 128 + 64 + tid] = pre_d;
    }
  };

  f32x4 adk[NK][NDB], adv[NK][NDB];
#pragma unroll
  for (int ki = 0; ki < NK; ++ki)
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      adk[ki][db] = zero4();
      adv[ki][db] = zero4();
    }
  const float sl2 = P.sl2;
  const int ka_off = n * RSE + 8 * gq;
  const int tr_off = (4 * gq + (n >> 2)) * RSE + 4 * (n & 3);

  const int nit = rep * nqt;
  load_tile(0, 0);
  store_tile(0);
  __syncthreads();
  int nhr = 0, nt0 = 0;  // the next tile's head of the group and first row
  for (int it = 0; it < nit; ++it) {
    const bool more = it + 1 < nit;
    nt0 += kDTileKeys;
    if (nt0 >= P.L) {
      nt0 = 0;
      ++nhr;
    }
    if (more) load_tile(nhr, nt0);
    const E *qs = buf0 + (it & 1) * TILE;
    const E *ds = qs + lds_y(D);
    const float *fl = fl0 + (it & 1) * 128;
#pragma unroll
    for (int cp = 0; cp < 2; ++cp) {
      v8 qa[2][NT], da[2][NT];
      f32x4 l2[2], dl[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int rb = (32 * cp + 16 * hh) * RSE + ka_off;
#pragma unroll
        for (int st = 0; st < NT; ++st) {
          qa[hh][st] = *reinterpret_cast<const v8 *>(qs + rb + 32 * st);
          da[hh][st] = *reinterpret_cast<const v8 *>(ds + rb + 32 * st);
        }
        l2[hh] = *reinterpret_cast<const f32x4 *>(fl + 32 * cp + 16 * hh + 4 * gq);
        dl[hh] = *reinterpret_cast<const f32x4 *>(fl + 64 + 32 * cp + 16 * hh + 4 * gq);
      }
      // dO^T and Q^T operands (dims x 32 queries), shared by the sub-tiles
      v8 ot[NDB], qt[NDB];
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const int o0 = 32 * cp * RSE + tr_off + 16 * db;
        const v4 a0 = M::tr(ds + o0), a1 = M::tr(ds + o0 + 16 * RSE);
        ot[db] = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
        const v4 b0 = M::tr(qs + o0), b1 = M::tr(qs + o0 + 16 * RSE);
        qt[db] = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int ki = 0; ki < NK; ++ki) {
        f32x4 sc[2], dp[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          sc[hh] = zero4();
          dp[hh] = -dl[hh];
#pragma unroll
          for (int st = 0; st < NT; ++st) {
            sc[hh] = M::mma(qa[hh][st], kf[ki][st], sc[hh]);
            dp[hh] = M::mma(da[hh][st], vf[ki][st], dp[hh]);
          }
        }
        v8 bp, bs;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float p = __builtin_amdgcn_exp2f(fmaf(sc[hh][r], sl2, -l2[hh][r]));
            bp[4 * hh + r] = (E)p;
            bs[4 * hh + r] = (E)(p * dp[hh][r]);
          }
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          adv[ki][db] = M::mma(ot[db], bp, adv[ki][db]);
          adk[ki][db] = M::mma(qt[db], bs, adk[ki][db]);
        }
      }
    }
    if (more) store_tile((it + 1) & 1);
    __syncthreads();
  }

  // ---- store: key rows of the sample to dk / dv, additional tokens to
  // dek / dev (when requested) ----
#pragma unroll
  for (int ki = 0; ki < NK; ++ki) {
    const int kk = kbase + 16 * ki + n;
    if (kk >= P.Lk) continue;
    const bool box = kk < P.L;
    if (!box && dek == nullptr) continue;
    const int off = box ? ((b * P.L + kk) * P.Hkv + hk) * D
                        : ((b * P.nx + kk - P.L) * P.Hkv + hk) * D;
    T *const wk = box ? dk : dek;
    T *const wv = box ? dv : dev;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      v4 a, bb;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        a[r] = (E)(adk[ki][db][r] * P.scale);
        bb[r] = (E)adv[ki][db][r];
      }
      *reinterpret_cast<v4 *>(wk + off + 16 * db + 4 * gq) = a;
      *reinterpret_cast<v4 *>(wv + off + 16 * db + 4 * gq) = bb;
    }
  }
}

template <typename T, int D, int NQ>
__global__ void __launch_bounds__(kDThreads)
    k_ddq(DProb P, const T *__restrict__ q, const T *__restrict__ k,
          const T *__restrict__ v, const T *__restrict__ ek,
          const T *__restrict__ ev, const T *__restrict__ dout,
          const float *__restrict__ lse, const float *__restrict__ delta,
          T *__restrict__ dq) {
  typedef L16<T> M;
  typedef typename M::v8 v8;
  typedef typename M::v4 v4;
  typedef typename M::e E;
  constexpr int NT = D / 32, NDB = D / 16;
  constexpr int RSE = lds_row(D);
  constexpr int UPR = D / 4, RPP = kDThreads / UPR, NU = kDTileKeys / RPP;
  constexpr int TILE = kDTileKeys * RSE;
  extern __shared__ __align__(16) char smem[];
  E *const buf0 = reinterpret_cast<E *>(smem);

  const int tile = xcd_tile(blockIdx.x, P.n_launch);
  if (tile >= P.n_tiles) return;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int n = lane & 15, gq = lane >> 4;
  const int bh = (int)fdiv((uint32_t)tile, P.fnqb);
  const int qb = tile - bh * P.nqb;
  const int b = (int)fdiv((uint32_t)bh, P.fH);
  const int h = bh - b * P.H;
  const int hk = (int)fdiv((uint32_t)h, P.fRep);

  const int c = tid % UPR, r0 = tid / UPR;
  const bool isv = c >= D / 8;
  const int col = 8 * (isv ? c - D / 8 : c);
  const T *const src = isv ? v : k;
  const T *const xsrc = isv ? ev : ek;
  const int lds_unit = r0 * RSE + 8 * c + (isv ? 8 : 0);
  v8 pre[NU];
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int i = 0; i < NU; ++i) {
      const int kk = min(t0 + r0 + RPP * i, P.Lk - 1);
      const bool box = kk < P.L;
      const int off = box ? ((b * P.L + kk) * P.Hkv + hk) * D + col
                          : ((b * P.nx + kk - P.L) * P.Hkv + hk) * D + col;
      pre[i] = ld8(box ? src : xsrc, off);
    }
  };
  auto store_tile = [&](int slot) {
#pragma unroll
    for (int i = 0; i < NU; ++i)
      *reinterpret_cast<v8 *>(buf0 + slot * TILE + lds_unit + RPP * i * RSE) = pre[i];
  };

  // the wave's query rows (B operands), lse * log2(e) and delta per lane
  const int qbase = qb * (64 * NQ) + w * (16 * NQ);
  v8 qf[NQ][NT], df[NQ][NT];
  float l2[NQ], dl[NQ];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
    const int row = (b * P.L + min(qbase + 16 * qi + n, P.L - 1)) * P.H + h;
#pragma unroll
    for (int st = 0; st < NT; ++st) {
      qf[qi][st] = ld8(q, row * D + 32 * st + 8 * gq);
      df[qi][st] = ld8(dout, row * D + 32 * st + 8 * gq);
    }
    l2[qi] = ldf(lse, row) * kLog2e;
    dl[qi] = ldf(delta, row);
  }
  load_tile(0);

  f32x4 acc[NQ][NDB];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi)
#pragma unroll
    for (int db = 0; db < NDB; ++db) acc[qi][db] = zero4();
  const float sl2 = P.sl2;
  const int ka_off = n * RSE + 8 * gq;
  const int tr_off = (4 * gq + (n >> 2)) * RSE + 4 * (n & 3);

  store_tile(0);
  __syncthreads();
  const int nkt = (P.Lk + kDTileKeys - 1) / kDTileKeys;
  // only the last tile can hold keys past the sample's last token (scores
  // start at -inf there); every other tile's scores start at zero
  auto run_tile = [&](const int j, auto last_tile) {
    constexpr bool LAST = decltype(last_tile)::value;
    const int t0 = j * kDTileKeys;
    if (!LAST) load_tile(t0 + kDTileKeys);
    const E *ks = buf0 + (j & 1) * TILE;
    const E *vs = ks + lds_y(D);
#pragma unroll
    for (int cp = 0; cp < 2; ++cp) {
      v8 ka[2][NT], va[2][NT];
      float cb[2][4];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int rb = (32 * cp + 16 * hh) * RSE + ka_off;
#pragma unroll
        for (int st = 0; st < NT; ++st) {
          ka[hh][st] = *reinterpret_cast<const v8 *>(ks + rb + 32 * st);
          va[hh][st] = *reinterpret_cast<const v8 *>(vs + rb + 32 * st);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
          cb[hh][r] = !LAST || t0 + 32 * cp + 16 * hh + 4 * gq + r < P.Lk ? 0.f : -INFINITY;
      }
      // K^T operand (dims x 32 keys), shared by the sub-tiles
      v8 kt[NDB];
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const int o0 = 32 * cp * RSE + tr_off + 16 * db;
        const v4 a0 = M::tr(ks + o0), a1 = M::tr(ks + o0 + 16 * RSE);
        kt[db] = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int qi = 0; qi < NQ; ++qi) {
        f32x4 sc[2], dp[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            sc[hh][r] = cb[hh][r];
            dp[hh][r] = -dl[qi];
          }
#pragma unroll
          for (int st = 0; st < NT; ++st) {
            sc[hh] = M::mma(ka[hh][st], qf[qi][st], sc[hh]);
            dp[hh] = M::mma(va[hh][st], df[qi][st], dp[hh]);
          }
        }
        v8 bs;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float p = __builtin_amdgcn_exp2f(fmaf(sc[hh][r], sl2, -l2[qi]));
            bs[4 * hh + r] = (E)(p * dp[hh][r]);
          }
#pragma unroll
        for (int db = 0; db < NDB; ++db) acc[qi][db] = M::mma(kt[db], bs, acc[qi][db]);
      }
    }
    if (!LAST) store_tile((j + 1) & 1);
    __syncthreads();
  };
  for (int j = 0; j + 1 < nkt; ++j) run_tile(j, std::false_type{});
  run_tile(nkt - 1, std::true_type{});

#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
    const int qq = qbase + 16 * qi + n;
    if (qq >= P.L) continue;
    const int qoff = ((b * P.L + qq) * P.H + h) * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      v4 wv;
#pragma unroll
      for (int r = 0; r < 4; ++r) wv[r] = (E)(acc[qi][db][r] * P.scale);
      *reinterpret_cast<v4 *>(dq + qoff + 16 * db + 4 * gq) = wv;
    }
  }
}

template <int D>
constexpr int dense_nq() {
  return D == 128 ? 2 : 4;
}
template <int D>
constexpr int dense_nk() {
  return D == 128 ? 1 : 2;
}
template <int D>
constexpr int dense_nq_bwd() {
  return D == 128 ? 1 : 4;  // head_dim 128: 208 VGPRs, two waves per SIMD
}

DProb make_dprob(const Prob &P, int nq) {
  DProb A{};
  A.L = P.ax[0].L * P.ax[1].L * P.ax[2].L;
  A.nx = P.n_extra;
  A.Lk = A.L + A.nx;
  A.H = P.H;
  A.Hkv = P.Hkv;
  A.nqb = (A.L + 64 * nq - 1) / (64 * nq);
  A.n_tiles = P.B * P.H * A.nqb;
  A.n_launch = (A.n_tiles + 7) & ~7;
  A.sl2 = P.scale * kLog2e;
  A.scale = P.scale;
  A.fnqb = make_fastdiv((uint32_t)A.nqb);
  A.fH = make_fastdiv((uint32_t)P.H);
  A.fRep = make_fastdiv((uint32_t)P.rep);
  A.fHkv = make_fastdiv((uint32_t)P.Hkv);
  return A;
}

// The key-side backward grid: blocks of 64 nk keys (of L + nx) per
// (sample, key/value head); nqb / fnqb hold the key blocks.
DProb make_dprob_keys(const Prob &P, int nk) {
  DProb A = make_dprob(P, 1);
  A.nqb = (A.Lk + 64 * nk - 1) / (64 * nk);
  A.n_tiles = P.B * P.Hkv * A.nqb;
  A.n_launch = (A.n_tiles + 7) & ~7;
  A.fnqb = make_fastdiv((uint32_t)A.nqb);
  return A;
}

}  // namespace

bool dense_fwd_eligible(const Prob &P, int dtype) {
  if (!P.dense || P.sample_extent != nullptr) return false;
  if (dtype != NA_BF16 && dtype != NA_F16) return false;
  if (P.D != 32 && P.D != 64 && P.D != 128) return false;
  if (!(P.scale > 0.f) || !std::isfinite(P.scale)) return false;
  const int64_t L = (int64_t)P.ax[0].L * P.ax[1].L * P.ax[2].L;
  // 32-bit element offsets in every tensor, 32-bit tile indices
  if ((int64_t)P.B * L * P.H * P.D >= (int64_t(1) << 31)) return false;
  if ((int64_t)P.B * P.n_extra * P.Hkv * P.D >= (int64_t(1) << 31)) return false;
  if ((int64_t)P.B * P.H * (L + 63) / 64 >= (int64_t(1) << 31)) return false;
  return L + P.n_extra < (int64_t(1) << 30);
}

void dense_fwd(const Prob &P, int dtype, const void *q, const void *k,
               const void *v, const void *ek, const void *ev, void *out,
               float *lse, hipStream_t st) {
#define DF_LAUNCH(TT, DD)                                                          \
  do {                                                                             \
    constexpr int NQ = dense_nq<DD>();                                             \
    const DProb A = make_dprob(P, NQ);                                             \
    if (A.n_tiles == 0) return;                                                    \
    const size_t lds = (size_t)2 * kDTileKeys * lds_row(DD) * 2;                    \
    hipLaunchKernelGGL((k_dfwd<TT, DD, NQ>), dim3(A.n_launch), dim3(kDThreads), lds, \
                       st, A, (const TT *)q, (const TT *)k, (const TT *)v,         \
                       (const TT *)ek, (const TT *)ev, (TT *)out, lse);            \
  } while (0)
#define DF_D(DD)                                   \
  do {                                             \
    if (dtype == NA_BF16) DF_LAUNCH(bf16_t, DD);   \
    else DF_LAUNCH(f16_t, DD);                     \
  } while (0)
  if (P.D == 32) DF_D(32);
  else if (P.D == 64) DF_D(64);
  else DF_D(128);
#undef DF_D
#undef DF_LAUNCH
}

void dense_bwd(const Prob &P, int dtype, const void *q, const void *k,
               const void *v, const void *ek, const void *ev, const void *dout,
               const float *lse, const float *delta, void *dq, void *dk, void *dv,
               void *dek, void *dev, hipStream_t st) {
#define DB_LAUNCH(TT, DD)                                                          \
  do {                                                                             \
    constexpr int NK = dense_nk<DD>(), NQ = dense_nq_bwd<DD>();                    \
    const size_t rows = (size_t)2 * kDTileKeys * lds_row(DD) * 2;                  \
    const DProb AK = make_dprob_keys(P, NK);                                       \
    if (AK.n_tiles > 0)                                                            \
      hipLaunchKernelGGL((k_ddkv<TT, DD, NK>), dim3(AK.n_launch), dim3(kDThreads), \
                         rows + 2 * 128 * sizeof(float), st, AK, (const TT *)q,    \
                         (const TT *)k, (const TT *)v, (const TT *)ek,             \
                         (const TT *)ev, (const TT *)dout, lse, delta, (TT *)dk,   \
                         (TT *)dv, (TT *)dek, (TT *)dev);                          \
    const DProb AQ = make_dprob(P, NQ);                                            \
    if (AQ.n_tiles > 0)                                                            \
      hipLaunchKernelGGL((k_ddq<TT, DD, NQ>), dim3(AQ.n_launch), dim3(kDThreads),  \
                         rows, st, AQ, (const TT *)q, (const TT *)k, (const TT *)v, \
                         (const TT *)ek, (const TT *)ev, (const TT *)dout, lse,    \
                         delta, (TT *)dq);                                         \
  } while (0)
#define DB_D(DD)                                   \
  do {                                             \
    if (dtype == NA_BF16) DB_LAUNCH(bf16_t, DD);   \
    else DB_LAUNCH(f16_t, DD);                     \
  } while (0)
  if (P.D == 32) DB_D(32);
  else if (P.D == 64) DB_D(64);
  else DB_D(128);
#undef DB_D
#undef DB_LAUNCH
}

}  // namespace na
