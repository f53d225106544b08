// na_dextra.hip — gradients of the additional (global) key/value tokens:
//
//   dek[b, e, hk] = scale * sum over the sample's output positions o and the
//                   query heads h of group hk of dS[o, h, e] * q[o, h]
//   dev[b, e, hk] = sum of P[o, h, e] * dO[o, h]
//
// with P = exp(scale * <q, ek_e> - lse) and dS = P * (<dO, ev_e> - delta),
// the extra tokens' part of the reference's merged attention
// (functional.py:71-138 + merge.py:20-68).  Every dtype and head_dim.
//
// A segment reduction in two passes.  Pass 1 (k_xpart): a workgroup owns
// (sample, key/value head, tile of up to 16 tokens, segment of rows); it
// walks its segment in chunks of RW rows (row = (output position, query head
// of the group)), stages each chunk's q and dO rows in LDS as float, computes
// P and dS of every (row, token) pair, and accumulates the 16 x D dek / dev
// sums of its segment in registers; the segment's sums go to a float
// workspace.  Pass 2 (k_xreduce) adds the segments of each output in a fixed
// order, so the result is deterministic.
#include <algorithm>
#include <cmath>

#include "na_common.h"
#include "na_launch.h"
#include "na_lean.h"

namespace na {
namespace {

constexpr int kXThreads = 256;

// Tokens per tile: 16, fewer for head_dim > 256 so that the tile's output
// sums (XT x D per pass) stay at four 4-column groups per thread.
int xtile(int D) { return D <= 256 ? 16 : D <= 512 ? 8 : 4; }

// Rows of a chunk: the largest power of two <= 4096 / D (LDS for the
// chunk's q and dO rows: 2 * RW * D floats <= 32 KB), between 8 and 64.
int xrows(int D) {
  int r = 64;
  while (r > 8 && r * D > 4096) r >>= 1;
  return r;
}

struct XPlan {
  int xt, rw, ntt, nsg, nper;
  int64_t nrows;  // rows of one (sample, key/value head): positions x rep
  size_t part_floats;
};

XPlan xplan(const Prob &P) {
  XPlan x;
  x.xt = xtile(P.D);
  x.rw = xrows(P.D);
  x.ntt = (P.n_extra + x.xt - 1) / x.xt;
  x.nrows = (int64_t)P.ax[0].O * P.ax[1].O * P.ax[2].O * P.rep;
  const int64_t nchunk = (x.nrows + x.rw - 1) / x.rw;
  const int64_t base = (int64_t)P.B * P.Hkv * x.ntt;
  // about four workgroups per CU over the whole launch
  int64_t nsg = base > 0 ? (1024 + base - 1) / base : 1;
  nsg = std::max<int64_t>(1, std::min<int64_t>(nsg, nchunk));
  x.nper = (int)((nchunk + nsg - 1) / nsg);
  x.nsg = (int)((nchunk + x.nper - 1) / x.nper);
  x.part_floats = (size_t)base * x.nsg * 2 * x.xt * P.D;
  return x;
}

// Pass 1.  LDS (floats): q and dO rows [RW][DR] (DR = D rounded up to 4,
// zero padded, so rows are read as float4), the token tile's ek and ev rows
// [XT][DR + 4] (padded against bank conflicts), P and dS [RW][XT], and per
// row lse * log2(e) (+inf for rows outside the sample: P = 0) and delta.
// Scores: each thread a 2 x 2 block of (row, token) pairs; sums: each thread
// the columns 4c..4c+3 of one token (XT * DR / 4 <= 4 * 256 groups).
template <typename T, int kXT>
__global__ void __launch_bounds__(kXThreads)
    k_xpart(Prob P, const T *__restrict__ q, const T *__restrict__ ek,
            const T *__restrict__ ev, const float *__restrict__ lse,
            const float *__restrict__ delta, const T *__restrict__ dout,
            float *__restrict__ part, int rw, int ntt, int nsg, int nper,
            int64_t nrows) {
  extern __shared__ __align__(16) float sm[];
  const int D = P.D, DR = (D + 3) & ~3, DK = DR + 4;
  float *sq = sm;
  float *sd = sq + rw * DR;
  float *sk = sd + rw * DR;
  float *sv = sk + kXT * DK;
  float *sp = sv + kXT * DK;
  float *ss = sp + rw * kXT;
  float *sl = ss + rw * kXT;
  float *sdl = sl + rw;
  // q / dO row element offsets (-1: row outside the sample)
  int64_t *sqo = reinterpret_cast<int64_t *>(sdl + rw);
  int64_t *sdo = sqo + rw;

  int wg = blockIdx.x;
  const int sg = wg % nsg;
  wg /= nsg;
  const int tt = wg % ntt;
  wg /= ntt;
  const int hk = wg % P.Hkv;
  const int b = wg / P.Hkv;
  const int tid = threadIdx.x;
  int32_t L[3], O[3];
  sample_extents(P, b, L, O);
  const int e0 = tt * kXT;
  const int ne = min(kXT, P.n_extra - e0);
  const float sl2 = P.scale * kLog2e;

  // the tile's extra-token rows (zero past the tile and past D)
  for (int i = tid; i < kXT * DK; i += kXThreads) {
    const int e = i / DK, dd = i - e * DK;
    const bool ok = e < ne && dd < D;
    const int64_t row = (((int64_t)b * P.n_extra + e0 + e) * P.Hkv + hk) * D + dd;
    sk[i] = ok ? to_f32(ek[row]) : 0.f;
    sv[i] = ok ? to_f32(ev[row]) : 0.f;
  }
  // output groups (token, 4 columns) of this thread: g = tid + 256 j
  constexpr int kMaxG = 4;  // XT * DR / 4 <= 4 * 256 (xtile)
  const int ngrp = kXT * DR / 4;
  float4 adk[kMaxG], adv[kMaxG];
#pragma unroll
  for (int j = 0; j < kMaxG; ++j) {
    adk[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    adv[j] = adk[j];
  }
  // score block of this thread: rows 2 (t / TP) + {0, 1}, tokens
  // 2 (t % TP) + {0, 1}, with TP = XT / 2 token pairs
  constexpr int TP = kXT / 2;
  const int br = 2 * (tid / TP), be = 2 * (tid % TP);

  const int O12 = P.ax[1].O * P.ax[2].O;
  // rows past the sample's extent on the first axis are all outside it
  nrows = min(nrows, (int64_t)O[0] * O12 * P.rep);
  for (int ci = 0; ci < nper; ++ci) {
    const int64_t r0 = ((int64_t)sg * nper + ci) * rw;
    if (r0 >= nrows) break;  // uniform
    __syncthreads();  // the previous chunk's reads are done (first: ek/ev)
    // per row: validity (inside the sample), q / dO offsets, lse, delta
    for (int r = tid; r < rw; r += kXThreads) {
      const int64_t ri = r0 + r;
      bool ok = ri < nrows;
      const int64_t of = ok ? ri / P.rep : 0;
      const int hr = (int)(ri - of * P.rep);
      const int o0 = (int)(of / O12);
      const int rem = (int)(of - (int64_t)o0 * O12);
      const int o1 = rem / P.ax[2].O;
      const int o2 = rem - o1 * P.ax[2].O;
      ok = ok && o0 < O[0] && o1 < O[1] && o2 < O[2];
      const int h = hk * P.rep + hr;
      const int64_t qt = tok_in(P, b, o0 * P.ax[0].s, o1 * P.ax[1].s, o2 * P.ax[2].s);
      const int64_t ot = tok_out(P, b, o0, o1, o2);
      sqo[r] = ok ? (qt * P.H + h) * D : -1;
      sdo[r] = ok ? (ot * P.H + h) * D : -1;
      sl[r] = ok ? lse[ot * P.H + h] * kLog2e : INFINITY;
      sdl[r] = ok ? delta[ot * P.H + h] : 0.f;
    }
    __syncthreads();
    // the chunk's q and dO rows, eight elements of each in flight per thread
    for (int i0 = 0; i0 < rw * DR; i0 += 8 * kXThreads) {
      float a[8], c[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = i0 + j * kXThreads + tid;
        const int r = i / DR, dd = i - r * DR;
        const bool in = i < rw * DR && dd < D;
        const int64_t qo = in ? sqo[r] : -1, dof = in ? sdo[r] : -1;
        a[j] = qo >= 0 ? to_f32(q[qo + dd]) : 0.f;
        c[j] = dof >= 0 ? to_f32(dout[dof + dd]) : 0.f;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = i0 + j * kXThreads + tid;
        if (i < rw * DR) {
          sq[i] = a[j];
          sd[i] = c[j];
        }
      }
    }
    __syncthreads();
    // P and dS: this thread's 2 x 2 (row, token) blocks (rw is even)
    for (int rb = br; rb < rw; rb += 2 * (kXThreads / TP)) {
      float s[2][2] = {{0.f, 0.f}, {0.f, 0.f}}, dp[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
      for (int dd = 0; dd < DR; dd += 4) {
        float4 qv[2], dv[2], kv[2], vv[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          qv[u] = *reinterpret_cast<const float4 *>(sq + (rb + u) * DR + dd);
          dv[u] = *reinterpret_cast<const float4 *>(sd + (rb + u) * DR + dd);
          kv[u] = *reinterpret_cast<const float4 *>(sk + (be + u) * DK + dd);
          vv[u] = *reinterpret_cast<const float4 *>(sv + (be + u) * DK + dd);
        }
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int y = 0; y < 2; ++y) {
            s[x][y] = fmaf(qv[x].x, kv[y].x, s[x][y]);
            s[x][y] = fmaf(qv[x].y, kv[y].y, s[x][y]);
            s[x][y] = fmaf(qv[x].z, kv[y].z, s[x][y]);
            s[x][y] = fmaf(qv[x].w, kv[y].w, s[x][y]);
            dp[x][y] = fmaf(dv[x].x, vv[y].x, dp[x][y]);
            dp[x][y] = fmaf(dv[x].y, vv[y].y, dp[x][y]);
            dp[x][y] = fmaf(dv[x].z, vv[y].z, dp[x][y]);
            dp[x][y] = fmaf(dv[x].w, vv[y].w, dp[x][y]);
          }
      }
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y) {
          const int r = rb + x, e = be + y;
          const float p = e < ne ? exp2f(fmaf(s[x][y], sl2, -sl[r])) : 0.f;
          sp[r * kXT + e] = p;
          ss[r * kXT + e] = p * (dp[x][y] - sdl[r]);
        }
    }
    __syncthreads();
    // this thread's (token, 4 columns) groups over the chunk's rows
#pragma unroll
    for (int j = 0; j < kMaxG; ++j) {
      const int g = tid + j * kXThreads;
      if (g >= ngrp) break;
      const int e = g / (DR / 4), c4 = 4 * (g - e * (DR / 4));
      float4 a = adk[j], v = adv[j];
      for (int r = 0; r < rw; ++r) {
        const float ds = ss[r * kXT + e], p = sp[r * kXT + e];
        const float4 qq = *reinterpret_cast<const float4 *>(sq + r * DR + c4);
        const float4 oo = *reinterpret_cast<const float4 *>(sd + r * DR + c4);
        a.x = fmaf(ds, qq.x, a.x);
        a.y = fmaf(ds, qq.y, a.y);
        a.z = fmaf(ds, qq.z, a.z);
        a.w = fmaf(ds, qq.w, a.w);
        v.x = fmaf(p, oo.x, v.x);
        v.y = fmaf(p, oo.y, v.y);
        v.z = fmaf(p, oo.z, v.z);
        v.w = fmaf(p, oo.w, v.w);
      }
      adk[j] = a;
      adv[j] = v;
    }
  }
  // the segment's sums: [2][16][D] floats (dek, then dev)
  float *dst = part + (((int64_t)(b * P.Hkv + hk) * ntt + tt) * nsg + sg) * 2 * kXT * D;
#pragma unroll
  for (int j = 0; j < kMaxG; ++j) {
    const int g = tid + j * kXThreads;
    if (g >= ngrp) break;
    const int e = g / (DR / 4), c4 = 4 * (g - e * (DR / 4));
    const float a4[4] = {adk[j].x, adk[j].y, adk[j].z, adk[j].w};
    const float v4[4] = {adv[j].x, adv[j].y, adv[j].z, adv[j].w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (c4 + u < D) {
        dst[e * D + c4 + u] = a4[u];
        dst[kXT * D + e * D + c4 + u] = v4[u];
      }
    }
  }
}

// Pass 2: one thread per (sample, token, key/value head, column) sums the
// segments in order.
template <typename T, int kXT>
__global__ void __launch_bounds__(kXThreads)
    k_xreduce(Prob P, const float *__restrict__ part, T *__restrict__ dek,
              T *__restrict__ dev, int ntt, int nsg) {
  const int64_t n = (int64_t)P.B * P.n_extra * P.Hkv * P.D;
  const int64_t i = (int64_t)blockIdx.x * kXThreads + threadIdx.x;
  if (i >= n) return;
  const int D = P.D;
  int64_t r = i / D;
  const int dd = (int)(i - r * D);
  const int hk = (int)(r % P.Hkv);
  r /= P.Hkv;
  const int e = (int)(r % P.n_extra);
  const int b = (int)(r / P.n_extra);
  const int tt = e / kXT, el = e - tt * kXT;
  const float *src = part + (((int64_t)(b * P.Hkv + hk) * ntt + tt) * nsg) * 2 * kXT * D +
                     el * D + dd;
  // in segment order, eight segments' loads in flight at a time
  const int64_t sst = (int64_t)2 * kXT * D;
  float a = 0.f, v = 0.f;
  int sg = 0;
  for (; sg + 8 <= nsg; sg += 8) {
    float ta[8], tv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ta[j] = src[(sg + j) * sst];
      tv[j] = src[(sg + j) * sst + kXT * D];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      a += ta[j];
      v += tv[j];
    }
  }
  for (; sg < nsg; ++sg) {
    a += src[sg * sst];
    v += src[sg * sst + kXT * D];
  }
  dek[i] = from_f32<T>(a * P.scale);
  dev[i] = from_f32<T>(v);
}

// Matrix-core variant (bf16 / fp16, head_dim 32, 64 or 128; 16 tokens per
// tile).  Each wave takes 32 rows at a time: it gathers their q and dO rows
// into its own LDS slice ([32][D + 8]), computes S = q ek^T and dP = dO ev^T
// for two 16-row blocks on mfma_f32_16x16x32 (ek / ev of the tile live in
// registers as the B operand), forms P and dS in the accumulator layout
// (lane: token l % 16, rows 4 (l / 16) + r) and packs them, as a rounded
// part plus the rounded remainder in the input type, as the B operands of
// dek^T += q^T dS and dev^T += dO^T P, whose
// A operand is read from the staged rows with the transposing LDS read.  The
// four waves' sums are added in LDS in wave order at the end.
constexpr int kXMRows = 128;  // rows per workgroup step (4 waves x 32)

// Row decode divisors of k_xmfma (row = ((o0 O1 + o1) O2 + o2) rep + head):
// query heads per key/value head, O1 O2 and O2 of the output grid.
struct XDiv {
  FastDiv rep, o12, o2;
};

// delta: rowsum(dO * O) - dlse per row, written by the backward kernel that
// runs before this one (or a delta pass).
template <typename T, int D>
__global__ void __launch_bounds__(256)
    k_xmfma(Prob P, const T *__restrict__ q, const T *__restrict__ ek,
            const T *__restrict__ ev, const float *__restrict__ lse,
            const float *__restrict__ delta, const T *__restrict__ dout,
            float *__restrict__ part, int ntt, int nsg, int nper, int64_t nrows,
            XDiv xd) {
  typedef L16<T> M;
  typedef typename M::v8 v8;
  typedef typename M::v4 v4;
  typedef typename M::e E;
  constexpr int RS = D + 8, NKB = D / 32, NDB = D / 16, UPL = D / 16, C8 = D / 8;
  extern __shared__ __align__(16) char xsm[];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
  E *sq = reinterpret_cast<E *>(xsm) + w * 2 * 32 * RS;
  E *sd = sq + 32 * RS;

  int wg = blockIdx.x;
  const int sg = wg % nsg;
  wg /= nsg;
  const int tt = wg % ntt;
  wg /= ntt;
  const int hk = wg % P.Hkv;
  const int b = wg / P.Hkv;
  int32_t L[3], O[3];
  sample_extents(P, b, L, O);
  const int O12 = P.ax[1].O * P.ax[2].O;
  nrows = min(nrows, (int64_t)O[0] * O12 * P.rep);
  const int e0 = tt * 16;
  const int ne = min(16, P.n_extra - e0);
  const float sl2 = P.scale * kLog2e;
  v8 zero;
#pragma unroll
  for (int i = 0; i < 8; ++i) zero[i] = (E)0.f;
  // the tile's ek / ev as the B operand: token n, columns 32 kb + 8 g + i
  v8 bk[NKB], bv[NKB];
  {
    const int64_t row = (((int64_t)b * P.n_extra + e0 + n) * P.Hkv + hk) * D + 8 * g;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      bk[kb] = n < ne ? *reinterpret_cast<const v8 *>(ek + row + 32 * kb) : zero;
      bv[kb] = n < ne ? *reinterpret_cast<const v8 *>(ev + row + 32 * kb) : zero;
    }
  }
  f32x4 adk[NDB], adv[NDB];
#pragma unroll
  for (int j = 0; j < NDB; ++j) {
    adk[j] = zero4();
    adv[j] = zero4();
  }
  const int tr_off = (4 * g + (n >> 2)) * RS + 4 * (n & 3);

  // One step's rows: lanes 0..31 decode the wave's 32 rows (q / dO
  // offsets, lse * log2(e): +inf outside the sample, P = 0; delta), then
  // the 16-byte units u = lane + 64 j of the q and dO rows are loaded.
  // Steps are software-pipelined: the next step's loads are issued before
  // this step's matrix work.
  struct Step {
    int32_t qo, dof;  // element offsets (tensors below 2^31 elements)
    float l2, dl;
    v8 xq[UPL], xd[UPL];
  };
  auto fetch = [&](int ci, Step &st) -> bool {
    const int64_t r0 = ((int64_t)sg * nper + ci) * kXMRows + 32 * w;
    if (ci >= nper || r0 >= nrows) return false;  // wave-uniform
    st.qo = -1;
    st.dof = -1;
    st.l2 = INFINITY;
    st.dl = 0.f;
    if (lane < 32) {
      // rows are below 2^31 (xmfma_ok): 32-bit decode by multiply-shift
      const uint32_t ri = (uint32_t)(r0 + lane);
      bool ok = ri < (uint64_t)nrows;
      const uint32_t of = ok ? fdiv(ri, xd.rep) : 0u;
      const int hr = (int)(ri - of * (uint32_t)P.rep);
      const int o0 = (int)fdiv(of, xd.o12);
      const int rem = (int)(of - (uint32_t)o0 * (uint32_t)O12);
      const int o1 = (int)fdiv((uint32_t)rem, xd.o2);
      const int o2 = rem - o1 * P.ax[2].O;
      ok = ok && o0 < O[0] && o1 < O[1] && o2 < O[2];
      const int h = hk * P.rep + hr;
      if (ok) {
        const int64_t qt = tok_in(P, b, o0 * P.ax[0].s, o1 * P.ax[1].s, o2 * P.ax[2].s);
        const int64_t ot = tok_out(P, b, o0, o1, o2);
        st.qo = (int32_t)((qt * P.H + h) * D);
        st.dof = (int32_t)((ot * P.H + h) * D);
        st.l2 = lse[ot * P.H + h] * kLog2e;
        st.dl = delta[ot * P.H + h];
      }
    }
#pragma unroll
    for (int j = 0; j < UPL; ++j) {
      const int u = lane + 64 * j, row = u / C8, c8 = u - row * C8;
      const int32_t a = __shfl(st.qo, row), c = __shfl(st.dof, row);
      st.xq[j] = a >= 0 ? ld8(q, a + 8 * c8) : zero;
      st.xd[j] = c >= 0 ? ld8(dout, c + 8 * c8) : zero;
    }
    return true;
  };

  Step cur;
  bool have = fetch(0, cur);
  for (int ci = 0; have; ++ci) {
    const float dl = cur.dl;
    const float l2 = cur.l2;
    wave_lds_sync();  // the previous step's reads of the slice are done
#pragma unroll
    for (int j = 0; j < UPL; ++j) {
      const int u = lane + 64 * j, row = u / C8, c8 = u - row * C8;
      *reinterpret_cast<v8 *>(sq + row * RS + 8 * c8) = cur.xq[j];
      *reinterpret_cast<v8 *>(sd + row * RS + 8 * c8) = cur.xd[j];
    }
    Step nxt;
    const bool hn = fetch(ci + 1, nxt);
    wave_lds_sync();
    // P and dS as B operands, each split into a rounded part and the
    // rounded remainder (two products: the sums keep float accuracy over
    // the thousands of rows a token's gradient adds)
    v8 bp, bds, bpl, bdsl;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      f32x4 s = zero4(), dp = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const int off = (16 * h + n) * RS + 32 * kb + 8 * g;
        s = M::mma(*reinterpret_cast<const v8 *>(sq + off), bk[kb], s);
        dp = M::mma(*reinterpret_cast<const v8 *>(sd + off), bv[kb], dp);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * h + 4 * g + r;
        const float l2r = __shfl(l2, row), dlr = __shfl(dl, row);
        const float p = n < ne ? exp2f(fmaf(s[r], sl2, -l2r)) : 0.f;
        const float ds = p * (dp[r] - dlr);
        const E ph = (E)p, dh = (E)ds;
        bp[4 * h + r] = ph;
        bpl[4 * h + r] = (E)(p - (float)ph);
        bds[4 * h + r] = dh;
        bdsl[4 * h + r] = (E)(ds - (float)dh);
      }
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const v4 q0 = M::tr(sq + tr_off + 16 * db), q1 = M::tr(sq + 16 * RS + tr_off + 16 * db);
      const v4 o0 = M::tr(sd + tr_off + 16 * db), o1 = M::tr(sd + 16 * RS + tr_off + 16 * db);
      const v8 aq = __builtin_shufflevector(q0, q1, 0, 1, 2, 3, 4, 5, 6, 7);
      const v8 ao = __builtin_shufflevector(o0, o1, 0, 1, 2, 3, 4, 5, 6, 7);
      adk[db] = M::mma(aq, bdsl, M::mma(aq, bds, adk[db]));
      adv[db] = M::mma(ao, bpl, M::mma(ao, bp, adv[db]));
    }
    if (hn) cur = nxt;
    have = hn;
  }
  // the four waves' sums, added in wave order: red[w][2][16][D + 1] (the
  // odd row stride spreads a write's 16 rows over distinct banks)
  constexpr int RR = D + 1;
  __syncthreads();
  float *red = reinterpret_cast<float *>(xsm);
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c = 16 * db + 4 * g + r;
      red[(w * 2 * 16 + n) * RR + c] = adk[db][r];
      red[(w * 2 * 16 + 16 + n) * RR + c] = adv[db][r];
    }
  __syncthreads();
  float *dst = part + (((int64_t)(b * P.Hkv + hk) * ntt + tt) * nsg + sg) * 2 * 16 * D;
  for (int i = threadIdx.x; i < 2 * 16 * D; i += 256) {
    const int ri = i / D, ci = i % D;  // D is a power of two
    float acc = red[ri * RR + ci];
#pragma unroll
    for (int ww = 1; ww < 4; ++ww) acc += red[(ww * 2 * 16 + ri) * RR + ci];
    dst[i] = acc;
  }
}

bool xmfma_ok(const Prob &P, int dtype) {
  // 32-bit element offsets into q, out and dout
  const int64_t rows_in = (int64_t)P.B * P.ax[0].L * P.ax[1].L * P.ax[2].L * P.H;
  const int64_t rows_out = (int64_t)P.B * P.ax[0].O * P.ax[1].O * P.ax[2].O * P.H;
  return dtype != NA_F32 && (P.D == 32 || P.D == 64 || P.D == 128) &&
         std::max(rows_in, rows_out) * P.D < (int64_t(1) << 31);
}

}  // namespace

bool dextra_uses_matrix(const Prob &P, int dtype, bool matrix) {
  return matrix && xmfma_ok(P, dtype);
}

namespace {

XPlan xplan_mfma(const Prob &P) {
  XPlan x;
  x.xt = 16;
  x.rw = kXMRows;
  x.ntt = (P.n_extra + 15) / 16;
  x.nrows = (int64_t)P.ax[0].O * P.ax[1].O * P.ax[2].O * P.rep;
  const int64_t nchunk = (x.nrows + kXMRows - 1) / kXMRows;
  const int64_t base = (int64_t)P.B * P.Hkv * x.ntt;
  int64_t nsg = base > 0 ? (1024 + base - 1) / base : 1;
  nsg = std::max<int64_t>(1, std::min<int64_t>(nsg, nchunk));
  x.nper = (int)((nchunk + nsg - 1) / nsg);
  x.nsg = (int)((nchunk + x.nper - 1) / x.nper);
  x.part_floats = (size_t)base * x.nsg * 2 * 16 * P.D;
  return x;
}

}  // namespace

size_t dextra_workspace_bytes(const Prob &P) {
  if (P.n_extra <= 0) return 0;
  // either variant (the choice depends on the dtype)
  return std::max(xplan(P).part_floats, xplan_mfma(P).part_floats) * sizeof(float);
}

void dextra(const Prob &P, int dtype, const void *q, const void *ek,
            const void *ev, const float *lse, const float *delta,
            const void *dout, void *dek, void *dev, float *part, bool matrix,
            hipStream_t st) {
  if (P.n_extra <= 0 || P.B == 0) return;
  if (matrix && xmfma_ok(P, dtype)) {
    const XPlan x = xplan_mfma(P);
    const size_t lds = (size_t)4 * 2 * 32 * (P.D + 8) * 2;
    const unsigned g1 = (unsigned)((int64_t)P.B * P.Hkv * x.ntt * x.nsg);
    const int64_t n2 = (int64_t)P.B * P.n_extra * P.Hkv * P.D;
    const unsigned g2 = (unsigned)((n2 + kXThreads - 1) / kXThreads);
    const XDiv xd{make_fastdiv((uint32_t)P.rep),
                  make_fastdiv((uint32_t)(P.ax[1].O * P.ax[2].O)),
                  make_fastdiv((uint32_t)P.ax[2].O)};
#define XM_(TT, DD)                                                              \
  hipLaunchKernelGGL((k_xmfma<TT, DD>), dim3(g1), dim3(256), lds, st, P,         \
                     (const TT *)q, (const TT *)ek, (const TT *)ev, lse, delta,  \
                     (const TT *)dout, part, x.ntt, x.nsg, x.nper, x.nrows, xd)
#define XMD_(TT)          \
  do {                    \
    if (P.D == 32)        \
      XM_(TT, 32);        \
    else if (P.D == 64)   \
      XM_(TT, 64);        \
    else                  \
      XM_(TT, 128);       \
    hipLaunchKernelGGL((k_xreduce<TT, 16>), dim3(g2), dim3(kXThreads), 0, st, P, \
                       (const float *)part, (TT *)dek, (TT *)dev, x.ntt, x.nsg); \
  } while (0)
    if (dtype == NA_F16)
      XMD_(f16_t);
    else
      XMD_(bf16_t);
#undef XMD_
#undef XM_
    return;
  }
  const XPlan x = xplan(P);
  const int DR = (P.D + 3) & ~3;
  const size_t lds = sizeof(float) * ((size_t)2 * x.rw * DR + (size_t)2 * x.xt * (DR + 4) +
                                      (size_t)2 * x.rw * x.xt + 2 * x.rw) +
                     sizeof(int64_t) * 2 * x.rw;
  const unsigned g1 = (unsigned)((int64_t)P.B * P.Hkv * x.ntt * x.nsg);
  const int64_t n2 = (int64_t)P.B * P.n_extra * P.Hkv * P.D;
  const unsigned g2 = (unsigned)((n2 + kXThreads - 1) / kXThreads);
#define XL_(TT, XT)                                                            \
  do {                                                                         \
    hipLaunchKernelGGL((k_xpart<TT, XT>), dim3(g1), dim3(kXThreads), lds, st,  \
                       P, (const TT *)q, (const TT *)ek, (const TT *)ev, lse,  \
                       delta, (const TT *)dout, part, x.rw, x.ntt, x.nsg,      \
                       x.nper, x.nrows);                                       \
    hipLaunchKernelGGL((k_xreduce<TT, XT>), dim3(g2), dim3(kXThreads), 0, st,  \
                       P, (const float *)part, (TT *)dek, (TT *)dev, x.ntt,    \
                       x.nsg);                                                 \
  } while (0)
#define XT_(TT)         \
  do {                  \
    if (x.xt == 16)     \
      XL_(TT, 16);      \
    else if (x.xt == 8) \
      XL_(TT, 8);       \
    else                \
      XL_(TT, 4);       \
  } while (0)
  if (dtype == NA_F32)
    XT_(float);
  else if (dtype == NA_F16)
    XT_(f16_t);
  else
    XT_(bf16_t);
#undef XT_
#undef XL_
}

}  // namespace na
