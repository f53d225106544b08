// na_vsplit.hip — vector-ALU gather kernel for the split QK product
// (na_qk_fwd, and the AV backward's dattn) on rank-2 problems:
//
//   out[q, slot] = scale * <x_q, y_key(slot)>
//
// with one thread per (query, head, window row): the workgroup stages its
// tile's key box and query rows in LDS, each thread reads its query row
// once and then the K key rows of its window row, one packed dot2 product
// per pair of elements, and the compact rows [H, K*K] of the tile leave
// through LDS as whole runs.  A measured alternative to the matrix-core
// k_lqh; selected with NATTEN_AMD_VSPLIT=1 (A/B checks).
//
// Problem class: rank 2, bf16/fp16, head_dim 32 or 64, stride 1, the same
// odd K on both axes with d K <= L, non-causal, no varlen, no additional
// tokens.  Window of the query at index i of its dilation phase (Lr
// points): [clamp(i - K/2, 0, Lr - K), + K) on each axis.
#include "na_lean.h"

namespace na {
namespace {

// An unsigned word of BYTES bytes (copies of 2-byte elements).
template <int BYTES>
struct VqWord;
template <>
struct VqWord<16> { typedef unsigned int type __attribute__((ext_vector_type(4))); };
template <>
struct VqWord<8> { typedef unsigned int type __attribute__((ext_vector_type(2))); };
template <>
struct VqWord<4> { typedef uint32_t type; };
template <>
struct VqWord<2> { typedef uint16_t type; };

struct VqProb {
  int32_t B, H, L0, L1, d0, d1;
  int32_t TY, TX;    // query tile (phase coordinates)
  int32_t nty, ntx;  // tiles per phase per axis (of the longest phase)
  int32_t BW;        // LDS key-box row stride in positions (TX + K - 1)
  int32_t kprod;     // K * K
  float scale;
};

__device__ __forceinline__ int vq_ws(int i, int Lr, int K) {
  return min(max(i - K / 2, 0), Lr - K);
}

// LDS row stride (elements) of one (position, head) row: D plus 16 bytes
template <int D>
constexpr int vq_rs() { return D + 8; }

template <typename T, int D, int K, int VW>
__global__ void __launch_bounds__(1024)
    k_vqk(VqProb P, const T *__restrict__ x, const T *__restrict__ y,
          T *__restrict__ out) {
  typedef L16<T> M;
  typedef typename M::v8 v8;
  typedef typename M::v2 v2;
  typedef typename M::e E;
  constexpr int RS = vq_rs<D>();
  constexpr int OCT = D / 8;
  extern __shared__ __align__(16) char smem[];

  int bid = (int)blockIdx.x;
  const int tx = bid % P.ntx;
  bid /= P.ntx;
  const int ty = bid % P.nty;
  bid /= P.nty;
  const int rx = bid % P.d1;
  bid /= P.d1;
  const int ry = bid % P.d0;
  const int b = bid / P.d0;
  const int Ly = (P.L0 - ry + P.d0 - 1) / P.d0, Lx = (P.L1 - rx + P.d1 - 1) / P.d1;
  const int y0 = ty * P.TY, x0 = tx * P.TX;
  if (b >= P.B || y0 >= Ly || x0 >= Lx) return;  // uniform over the workgroup
  const int ny = min(P.TY, Ly - y0), nx = min(P.TX, Lx - x0);
  const int by0 = vq_ws(y0, Ly, K), bh = vq_ws(y0 + ny - 1, Ly, K) + K - by0;
  const int bx0 = vq_ws(x0, Lx, K), bw = vq_ws(x0 + nx - 1, Lx, K) + K - bx0;
  const int H = P.H, tid = (int)threadIdx.x, nthr = (int)blockDim.x;

  E *ks = reinterpret_cast<E *>(smem);                   // [bh * BW][H][RS]
  E *qs = ks + (size_t)(P.TY + K - 1) * P.BW * H * RS;   // [TY * TX][H][RS]
  E *os = qs + (size_t)P.TY * P.TX * H * RS;             // [TY * TX][H * kprod]

  // stage the key box and the query rows: 16-byte units, OCT per head row
  const int upos = H * OCT;
  const int nku = bh * bw * upos, nqu = ny * nx * upos;
  for (int u = tid; u < nku + nqu; u += nthr) {
    const bool key = u < nku;
    const int uu = key ? u : u - nku;
    const int pos = uu / upos, rem = uu - pos * upos;
    const int h = rem / OCT, o = rem - h * OCT;
    const int w = key ? bw : nx;
    const int ey = pos / w, ex = pos - ey * w;
    const int py = (key ? by0 : y0) + ey, px = (key ? bx0 : x0) + ex;
    const int tok = (b * P.L0 + ry + P.d0 * py) * P.L1 + rx + P.d1 * px;
    const v8 val = ld8(key ? y : x, (tok * H + h) * D + 8 * o);
    E *dst = key ? ks + ((ey * P.BW + ex) * H + h) * RS : qs + ((ey * P.TX + ex) * H + h) * RS;
    *reinterpret_cast<v8 *>(dst + 8 * o) = val;
  }
  __syncthreads();

  // thread (window row r, tile position p, head h)
  const int tpos = P.TY * P.TX;
  const int h = tid % H;
  const int p = (tid / H) % tpos;
  const int r = tid / (H * tpos);
  const int py = p / P.TX, px = p - py * P.TX;
  if (r < K && py < ny && px < nx) {
    v8 qv[OCT];
    const E *qrow = qs + (p * H + h) * RS;
#pragma unroll
    for (int o = 0; o < OCT; ++o) qv[o] = *reinterpret_cast<const v8 *>(qrow + 8 * o);
    const int ky = vq_ws(y0 + py, Ly, K) - by0 + r;
    const int kx = vq_ws(x0 + px, Lx, K) - bx0;
    const E *krow = ks + ((ky * P.BW + kx) * H + h) * RS;
    E *orow = os + (p * H + h) * P.kprod + r * K;
#pragma unroll
    for (int c = 0; c < K; ++c) {
      float acc = 0.f;
#pragma unroll
      for (int o = 0; o < OCT; ++o) {
        const v8 kv = *reinterpret_cast<const v8 *>(krow + c * H * RS + 8 * o);
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          v2 a2, b2;
          a2[0] = qv[o][e];
          a2[1] = qv[o][e + 1];
          b2[0] = kv[e];
          b2[1] = kv[e + 1];
          acc = M::dot2(a2, b2, acc);
        }
      }
      orow[c] = (E)(acc * P.scale);
    }
  }
  __syncthreads();

  // the tile's compact rows: each position's H * kprod run is contiguous
  typedef typename VqWord<VW * 2>::type W;
  const int run = H * P.kprod / VW;  // words per position
  for (int u = tid; u < ny * nx * run; u += nthr) {
    const int pos = u / run, o = u - pos * run;
    const int ey = pos / nx, ex = pos - ey * nx;
    const int tok = (b * P.L0 + ry + P.d0 * (y0 + ey)) * P.L1 + rx + P.d1 * (x0 + ex);
    const W val = *reinterpret_cast<const W *>(os + (ey * P.TX + ex) * H * P.kprod + VW * o);
    __builtin_nontemporal_store(
        val, reinterpret_cast<W *>(out + (size_t)tok * H * P.kprod) + o);
  }
}

struct VqPlan {
  VqProb P;
  size_t lds;
  int nthr, nblk, vw;
};

bool vq_plan(const Prob &Pr, float scale, VqPlan *pl) {
  if (Pr.rank != 2 || Pr.sample_extent != nullptr || Pr.n_extra > 0 || Pr.dense) return false;
  if (Pr.D != 32 && Pr.D != 64) return false;
  const Axis &a = Pr.ax[1], &c = Pr.ax[2];
  if (a.causal || c.causal || a.s != 1 || c.s != 1 || a.K != c.K) return false;
  const int K = a.K;
  if (K != 3 && K != 5 && K != 7) return false;
  if ((int64_t)a.d * K > a.L || (int64_t)c.d * K > c.L) return false;
  if (Pr.H != Pr.Hkv) return false;
  VqProb &P = pl->P;
  P.B = Pr.B;
  P.H = Pr.H;
  P.L0 = a.L;
  P.L1 = c.L;
  P.d0 = a.d;
  P.d1 = c.d;
  P.kprod = K * K;
  P.scale = scale;
  // the largest tile of TY x TX positions (TX = 8, else 4) with one thread
  // per (position, head, window row) in a workgroup of at most 1024
  const int per = Pr.H * K;
  if (per > 1024 / 4) return false;
  P.TX = per * 8 * 2 <= 1024 ? 8 : 4;
  P.TY = std::max(1, std::min(8, 1024 / (per * P.TX)));
  const int Lqy = (a.L + a.d - 1) / a.d, Lqx = (c.L + c.d - 1) / c.d;
  P.nty = (Lqy + P.TY - 1) / P.TY;
  P.ntx = (Lqx + P.TX - 1) / P.TX;
  P.BW = P.TX + K - 1;
  const int RS = Pr.D + 8;
  pl->lds = ((size_t)(P.TY + K - 1) * P.BW * Pr.H * RS + (size_t)P.TY * P.TX * Pr.H * RS) * 2 +
            (size_t)P.TY * P.TX * Pr.H * P.kprod * 2;
  if (pl->lds > 80 * 1024) return false;
  pl->nthr = P.TY * P.TX * Pr.H * K;
  pl->nthr = (pl->nthr + 63) & ~63;
  const int64_t nb = (int64_t)Pr.B * a.d * c.d * P.nty * P.ntx;
  if (nb <= 0 || nb >= (int64_t)1 << 31) return false;
  pl->nblk = (int)nb;
  const int rowlen = Pr.H * P.kprod;
  pl->vw = rowlen % 8 == 0 ? 8 : rowlen % 4 == 0 ? 4 : rowlen % 2 == 0 ? 2 : 1;
  // token offsets stay 32-bit
  if ((int64_t)Pr.B * a.L * c.L * Pr.H * std::max(Pr.D, P.kprod) >= (int64_t)1 << 31)
    return false;
  return true;
}

}  // namespace

bool vsplit_on() {
  const char *e = std::getenv("NATTEN_AMD_VSPLIT");
  return e != nullptr && e[0] == '1';
}

bool vsplit_qk(const Prob &Pr, int dtype, const void *x, const void *y, void *out,
               float scale, hipStream_t st) {
  VqPlan pl;
  if (!vq_plan(Pr, scale, &pl)) return false;
  const int K = Pr.ax[1].K;
  auto go = [&](auto tt, auto dd, auto kk, auto vv) {
    typedef decltype(tt) TT;
    constexpr int DD = decltype(dd)::value, KK = decltype(kk)::value,
                  VV = decltype(vv)::value;
    hipLaunchKernelGGL((k_vqk<TT, DD, KK, VV>), dim3(pl.nblk), dim3(pl.nthr), pl.lds, st,
                       pl.P, (const TT *)x, (const TT *)y, (TT *)out);
  };
  auto by_v = [&](auto tt, auto dd, auto kk) {
    if (pl.vw == 8) go(tt, dd, kk, std::integral_constant<int, 8>());
    else if (pl.vw == 4) go(tt, dd, kk, std::integral_constant<int, 4>());
    else if (pl.vw == 2) go(tt, dd, kk, std::integral_constant<int, 2>());
    else go(tt, dd, kk, std::integral_constant<int, 1>());
  };
  auto by_k = [&](auto tt, auto dd) {
    if (K == 3) by_v(tt, dd, std::integral_constant<int, 3>());
    else if (K == 5) by_v(tt, dd, std::integral_constant<int, 5>());
    else by_v(tt, dd, std::integral_constant<int, 7>());
  };
  auto by_d = [&](auto tt) {
    if (Pr.D == 32) by_k(tt, std::integral_constant<int, 32>());
    else by_k(tt, std::integral_constant<int, 64>());
  };
  if (dtype == NA_BF16) by_d(bf16_t());
  else by_d(f16_t());
  return true;
}

}  // namespace na
