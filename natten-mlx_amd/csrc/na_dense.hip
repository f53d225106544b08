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
  FastDiv fnqb;      // query blocks per (sample, head)
  FastDiv fH;        // query heads
  FastDiv fRep;      // query heads per key/value head
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
  for (int j = 0; j < nkt; ++j) {
    const int t0 = j * kDTileKeys;
    const bool more = j + 1 < nkt;
    if (more) load_tile(t0 + kDTileKeys);  // in flight during this tile
    const E *ks = buf0 + (j & 1) * (kDTileKeys * RSE);
    const E *vs = ks + lds_y(D);
    v8 ka[4][NT];
#pragma unroll
    for (int ch = 0; ch < 4; ++ch)
#pragma unroll
      for (int st = 0; st < NT; ++st)
        ka[ch][st] = *reinterpret_cast<const v8 *>(ks + 16 * ch * RSE + ka_off + 32 * st);
    // keys past the sample's last token (last tile only): -inf scores
    float cb[4][4];
#pragma unroll
    for (int ch = 0; ch < 4; ++ch)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        cb[ch][r] = t0 + 16 * ch + 4 * gq + r < P.Lk ? 0.f : -INFINITY;
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
    if (more) store_tile(buf0 + ((j + 1) & 1) * (kDTileKeys * RSE));
    __syncthreads();
  }

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

template <int D>
constexpr int dense_nq() {
  return D == 128 ? 2 : 4;
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
  A.fnqb = make_fastdiv((uint32_t)A.nqb);
  A.fH = make_fastdiv((uint32_t)P.H);
  A.fRep = make_fastdiv((uint32_t)P.rep);
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

}  // namespace na
