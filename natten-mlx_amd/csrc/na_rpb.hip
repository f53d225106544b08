// na_rpb.hip — DiNAT all-in-one operators: QK with relative position bias
// and AV over a window of side K_a and dilation d_a per axis on one or two
// spatial axes, forward and backward (reference extras/allin1 and the
// NATTEN 0.14 compat functions).
//
// Window of a query on an axis: slot k holds key s + k*d with s the
// dilation-partition start, valid iff 0 <= key < end; its bias row is
// clip(pb + k, 0, 2K-2) (reference extras/allin1/reference_impl.py:13-45,
// compat/v014.py:18-23).  Invalid slots produce -inf logits (zero dattn)
// and contribute nothing to any gradient.
//
// Rows are (b, h, position) triples of either layout, [B, *L, H, X]
// (spatial-first) or [B, H, *L, X] (heads-first); threads are enumerated in
// memory order, so a wavefront touches consecutive rows with 16-byte
// accesses.  One aligned group of G lanes owns one row (G = 1 for the
// DiNAT head_dim of 12 in fp32).  Every kernel is a gather: dK/dV walk each
// key's inverse neighborhood and the bias gradient is a fixed-order
// two-pass reduction, so results are deterministic (no atomics).
#include "na_common.h"
#include "na_launch.h"
#include "na_row.h"
#include "na_window.h"

namespace na {
namespace {

constexpr int kNT = 4;         // element chunks per lane
constexpr int kBiasChunk = 16;  // queries per bias-gradient partial

struct RPos {
  int32_t b, h, i0, i1;
};

__device__ __forceinline__ RPos rpos(const RpbProb &A, uint32_t r) {
  RPos p;
  uint32_t q;
  if (A.heads_first) {
    q = fdiv(r, A.fL1);
    p.i1 = (int32_t)(r - q * (uint32_t)A.L1);
    r = q;
    q = fdiv(r, A.fL0);
    p.i0 = (int32_t)(r - q * (uint32_t)A.L0);
    r = q;
    q = fdiv(r, A.fH);
    p.h = (int32_t)(r - q * (uint32_t)A.H);
    p.b = (int32_t)q;
  } else {
    q = fdiv(r, A.fH);
    p.h = (int32_t)(r - q * (uint32_t)A.H);
    r = q;
    q = fdiv(r, A.fL1);
    p.i1 = (int32_t)(r - q * (uint32_t)A.L1);
    r = q;
    q = fdiv(r, A.fL0);
    p.i0 = (int32_t)(r - q * (uint32_t)A.L0);
    p.b = (int32_t)q;
  }
  return p;
}

__device__ __forceinline__ int64_t rrow(const RpbProb &A, int32_t b, int32_t h,
                                        int32_t i0, int32_t i1) {
  return A.heads_first
             ? (((int64_t)b * A.H + h) * A.L0 + i0) * A.L1 + i1
             : (((int64_t)b * A.L0 + i0) * A.L1 + i1) * A.H + h;
}

struct RWin {
  int32_t s;   // position of slot 0
  int32_t e;   // keys must be below this
  int32_t pb;  // bias row of slot 0 (before clipping)
};

// Window of position i on an axis of length L, side K and dilation d:
// window_start_partition, window_end and pb_start (na_window.h) with the
// divisions by the dilation done by multiply-shift (fd divides by d).
__device__ __forceinline__ RWin rwin_axis(int32_t K, int32_t d, FastDiv fd,
                                          int32_t i, int32_t L) {
  const int32_t nh = K / 2;
  RWin w;
  if (d == 1) {
    int32_t s = i > nh ? i - nh : 0;
    if (i + nh >= L) s += L - i - nh - 1;
    w.s = s;
    w.e = min(s + K, L);
    int32_t pb = nh;
    if (i < nh) pb += nh - i;
    if (i + nh >= L) pb += L - i - 1 - nh;
    w.pb = pb;
    return w;
  }
  const int32_t slot = (int32_t)fdiv((uint32_t)i, fd);
  const int32_t phase = i - slot * d;
  const int32_t plen = (int32_t)fdiv((uint32_t)(L - 1 - phase), fd) + 1;
  int32_t s = slot > nh ? slot - nh : 0;
  if (slot + nh >= plen) s += plen - slot - nh - 1;
  w.s = s * d + phase;
  w.e = min(w.s + K * d, L);
  if (i < nh * d)
    w.pb = K - 1 - slot;
  else if (i + nh * d >= L)
    w.pb = (int32_t)fdiv((uint32_t)(L - i - 1), fd);
  else
    w.pb = nh;
  return w;
}

__device__ __forceinline__ RWin rwin0(const RpbProb &A, int32_t i0) {
  return rwin_axis(A.K0, A.d0, A.fd0, i0, A.L0);
}

// Axis-1 window (a single always-valid slot for rank 1).
__device__ __forceinline__ RWin rwin1(const RpbProb &A, int32_t i1) {
  if (A.rank == 2) return rwin_axis(A.K1, A.d1, A.fd1, i1, A.L1);
  return RWin{0, 1, 0};
}

__device__ __forceinline__ int32_t clampi(int32_t x, int32_t lo, int32_t hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}

__device__ __forceinline__ int32_t bias_index(const RpbProb &A, int32_t h,
                                              int32_t r0, int32_t r1) {
  const int32_t a = h * A.R0 + clampi(r0, 0, A.R0 - 1);
  return A.rank == 2 ? a * A.R1 + clampi(r1, 0, A.R1 - 1) : a;
}

// ---- row helpers (lane-local part of a D-row; element type per call) ------
template <typename T, int VEC>
__device__ __forceinline__ void ld_row(float (&v)[kNT][VEC], const T *row,
                                       int lane, int G, int D) {
#pragma unroll
  for (int t = 0; t < kNT; ++t) {
    const int d0 = (t * G + lane) * VEC;
    if (d0 < D) {
      VecIO<T, VEC>::load(row + d0, v[t]);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[t][e] = 0.f;
    }
  }
}

template <typename T, int VEC>
__device__ __forceinline__ float dot_row(const float (&v)[kNT][VEC],
                                         const T *row, int lane, int G, int D) {
  float acc = 0.f;
#pragma unroll
  for (int t = 0; t < kNT; ++t) {
    const int d0 = (t * G + lane) * VEC;
    if (d0 < D) {
      float x[VEC];
      VecIO<T, VEC>::load(row + d0, x);
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc = fmaf(v[t][e], x[e], acc);
    }
  }
  return acc;
}

template <typename T, int VEC>
__device__ __forceinline__ void axpy_row(float (&acc)[kNT][VEC], float w,
                                         const T *row, int lane, int G, int D) {
#pragma unroll
  for (int t = 0; t < kNT; ++t) {
    const int d0 = (t * G + lane) * VEC;
    if (d0 < D) {
      float x[VEC];
      VecIO<T, VEC>::load(row + d0, x);
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[t][e] = fmaf(w, x[e], acc[t][e]);
    }
  }
}

template <typename T, int VEC>
__device__ __forceinline__ void st_row(T *row, float (&v)[kNT][VEC], float s,
                                       int lane, int G, int D) {
#pragma unroll
  for (int t = 0; t < kNT; ++t) {
    const int d0 = (t * G + lane) * VEC;
    if (d0 < D) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[t][e] *= s;
      VecIO<T, VEC>::store(row + d0, v[t]);
    }
  }
}

// x <- round_to_TX(x * scale): the query scaling the reference applies in
// the query's dtype before the dot (extras/allin1/__init__.py:61-62).
template <typename TX, int VEC>
__device__ __forceinline__ void scale_round(float (&v)[kNT][VEC], float s) {
#pragma unroll
  for (int t = 0; t < kNT; ++t)
#pragma unroll
    for (int e = 0; e < VEC; ++e) v[t][e] = round_to<TX>(v[t][e] * s);
}


// Block-wide copy of n 16-byte units, four per thread in flight at a time
// (every load of a batch is issued before its stores), so a copy of a few
// units per thread costs one memory latency rather than one per unit.  The
// trip count is uniform and indices past the end are clamped onto the last
// unit (its copies write the same value), so nothing branches per lane.
// NT: the stores are nontemporal (streaming), for a kernel's output rows
// that this kernel does not read again: they do not displace the inputs
// from the caches (config 5, K=7 d=1: qk 5.18 -> 4.86 us, av 5.52 -> 4.76).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
template <bool NT = false>
__device__ __forceinline__ void block_copy16(uint4 *dst, const uint4 *src,
                                             int64_t n) {
  constexpr int kB = 4;
  if (n <= 0) return;
  const int nn = (int)n, nt = (int)blockDim.x, tid = (int)threadIdx.x;
  u32x4 *d = reinterpret_cast<u32x4 *>(dst);
  const u32x4 *s = reinterpret_cast<const u32x4 *>(src);
  for (int base = 0; base < nn; base += kB * nt) {
    u32x4 r[kB];
    int ix[kB];
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      ix[j] = min(base + j * nt + tid, nn - 1);
      r[j] = s[ix[j]];
    }
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      if (NT)
        __builtin_nontemporal_store(r[j], d + ix[j]);
      else
        d[ix[j]] = r[j];
    }
  }
}

// Block-wide copy of n floats between 16-byte aligned ranges: 16-byte
// units through block_copy16, then the tail.
template <bool NT = false>
__device__ __forceinline__ void block_copy_f32(float *dst, const float *src,
                                               int64_t n) {
  const int64_t n4 = n >> 2;
  block_copy16<NT>(reinterpret_cast<uint4 *>(dst), reinterpret_cast<const uint4 *>(src), n4);
  for (int64_t i = 4 * n4 + threadIdx.x; i < n; i += blockDim.x) {
    if (NT)
      __builtin_nontemporal_store(src[i], dst + i);
    else
      dst[i] = src[i];
  }
}

// Rank 1: the keys (or values) of every row of a block lie within K*d
// positions of the block's rows, i.e. in the row range [lo, hi) below;
// the block copies that range into LDS with contiguous 16-byte loads
// (`ystage`) so the per-slot row reads hit LDS.  Returns lo.
template <typename T>
__device__ __forceinline__ int64_t stage_window(const RpbProb &A, const T *y,
                                                T *ystage, int lgG) {
  const int64_t step = A.heads_first ? 1 : A.H;
  const int64_t row0 = ((int64_t)blockIdx.x * blockDim.x) >> lgG;
  const int64_t rows = min((int64_t)(blockDim.x >> lgG), (int64_t)A.n_rows - row0);
  const int64_t reach = (int64_t)A.K0 * A.d0 * step;
  const int64_t lo = max((int64_t)0, row0 - reach);
  const int64_t hi = min((int64_t)A.n_rows, row0 + rows + reach);
  const int64_t n16 = (hi - lo) * A.D * (int64_t)sizeof(T) / 16;
  block_copy16(reinterpret_cast<uint4 *>(ystage),
               reinterpret_cast<const uint4 *>(y + lo * A.D), n16);
  __syncthreads();
  return lo;
}

// Rows of the staged window per block of rb threads (bounds its LDS).
inline int64_t window_rows(const RpbProb &A, int lgG, int rb) {
  const int64_t step = A.heads_first ? 1 : A.H;
  return (rb >> lgG) + 2 * (int64_t)A.K0 * A.d0 * step;
}

// ---- kernels ---------------------------------------------------------------

// out[r, n] = <x'[r], y[nbr(r, n)]> (+ bias) for valid slots, `fill` for
// invalid ones; x' = round(x * scale) when scale_x.  QK+RPB forward
// (x = q, y = key, fill = -inf) and the AV backward's dattn (x = dout,
// y = value, no bias, fill = 0).
template <typename TX, typename TY, int VEC, bool YS>
__global__ void __launch_bounds__(512)
    k_rpb_dot(RpbProb A, const TX *__restrict__ x, const TY *__restrict__ y,
              const float *__restrict__ rpb, float *__restrict__ out,
              int scale_x, float fill, int staged, int G, int lgG,
              int bias_lds) {
  const Group g = make_group(lgG, A.n_rows);
  const RPos p = rpos(A, (uint32_t)g.id);
  float xv[kNT][VEC];
  ld_row<TX, VEC>(xv, x + g.id * A.D, g.lane, G, A.D);
  if (scale_x) scale_round<TX, VEC>(xv, A.scale);
  const RWin w0 = rwin0(A, p.i0);
  const RWin w1 = rwin1(A, p.i1);
  // rows of this block are consecutive in memory: stage them in LDS and
  // write the block's slot values as one contiguous range
  extern __shared__ __align__(16) float stage[];
  const int lrow = (int)(threadIdx.x >> lgG);
  float *dst = staged ? stage + lrow * A.KK : out + g.id * A.KK;
  // bias_lds: the bias table [H, R0 (, R1)] is copied to LDS (after the
  // slot rows and the staged window) with the window's loads, so the slot
  // loop's bias reads do not each wait on a memory round trip
  const float *bias = rpb;
  if (bias_lds) {
    float *bs = stage + bias_lds;
    const int nb = A.H * A.R0 * A.R1;
    for (int i = (int)threadIdx.x; i < nb; i += (int)blockDim.x) bs[i] = rpb[i];
    bias = bs;
    if (A.rank != 1 || !YS) __syncthreads();  // else stage_window's barrier
  }
  if (A.rank == 1) {
    // one axis: the row of key position j is this row + (j - i) * step
    const int64_t step = A.heads_first ? 1 : A.H;
    const float *rb = rpb != nullptr ? bias + p.h * A.R0 : nullptr;
    const TY *ybase = y;
    int64_t ylo = 0;
    if constexpr (YS) {
      TY *ys = reinterpret_cast<TY *>(stage + (staged ? (blockDim.x >> lgG) * A.KK : 0));
      ylo = stage_window<TY>(A, y, ys, lgG);
      ybase = ys;
    }
    for (int k0 = 0; k0 < A.K0; ++k0) {
      const int32_t j0 = w0.s + k0 * A.d0;
      float s = fill;
      if (j0 >= 0 && j0 < w0.e) {
        const TY *yr = ybase + (g.id - ylo + (int64_t)(j0 - p.i0) * step) * A.D;
        s = group_sum(dot_row<TY, VEC>(xv, yr, g.lane, G, A.D), G);
        if (rb != nullptr) s += rb[clampi(w0.pb + k0, 0, A.R0 - 1)];
      }
      if (g.live && g.lane == 0) dst[k0] = s;
    }
  } else {
    int n = 0;
    for (int k0 = 0; k0 < A.K0; ++k0) {
      const int32_t j0 = w0.s + k0 * A.d0;
      const bool v0 = j0 >= 0 && j0 < w0.e;
      for (int k1 = 0; k1 < A.K1; ++k1, ++n) {
        const int32_t j1 = w1.s + k1 * A.d1;
        float s = fill;
        if (v0 && j1 >= 0 && j1 < w1.e) {
          const TY *yr = y + rrow(A, p.b, p.h, j0, j1) * A.D;
          s = group_sum(dot_row<TY, VEC>(xv, yr, g.lane, G, A.D), G);
          if (rpb != nullptr) s += bias[bias_index(A, p.h, w0.pb + k0, w1.pb + k1)];
        }
        if (g.live && g.lane == 0) dst[n] = s;
      }
    }
  }
  if (staged) {
    __syncthreads();
    const int64_t row0 = ((int64_t)blockIdx.x * blockDim.x) >> lgG;
    const int64_t rows = min((int64_t)(blockDim.x >> lgG), (int64_t)A.n_rows - row0);
    const int64_t nv = rows * A.KK;
    block_copy_f32<true>(out + row0 * A.KK, stage, nv);
  }
}

// out[r] = post * sum_n w[r, n] * y[nbr(r, n)] over valid slots.  AV
// forward (w = attn, y = value) and the QK backward's dq (w = dlogits,
// y = key, post = the query scale).
template <typename TY, typename TO, int VEC, bool YS>
__global__ void __launch_bounds__(512)
    k_rpb_gather(RpbProb A, const float *__restrict__ w,
                 const TY *__restrict__ y, TO *__restrict__ out, float post,
                 int staged, int G, int lgG) {
  const Group g = make_group(lgG, A.n_rows);
  const RPos p = rpos(A, (uint32_t)g.id);
  const RWin w0 = rwin0(A, p.i0);
  const RWin w1 = rwin1(A, p.i1);
  // the block's weight rows are one contiguous range: read it coalesced
  extern __shared__ __align__(16) float stage[];
  const float *wr = w + g.id * A.KK;
  if (staged) {
    const int64_t row0 = ((int64_t)blockIdx.x * blockDim.x) >> lgG;
    const int64_t rows = min((int64_t)(blockDim.x >> lgG), (int64_t)A.n_rows - row0);
    const int64_t nv = rows * A.KK;
    block_copy_f32(stage, w + row0 * A.KK, nv);
    __syncthreads();
    wr = stage + (int)(threadIdx.x >> lgG) * A.KK;
  }
  float acc[kNT][VEC];
#pragma unroll
  for (int t = 0; t < kNT; ++t)
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[t][e] = 0.f;
  if (A.rank == 1) {
    const int64_t step = A.heads_first ? 1 : A.H;
    const TY *ybase = y;
    int64_t ylo = 0;
    if constexpr (YS) {
      TY *ys = reinterpret_cast<TY *>(stage + (staged ? (blockDim.x >> lgG) * A.KK : 0));
      ylo = stage_window<TY>(A, y, ys, lgG);
      ybase = ys;
    }
    for (int k0 = 0; k0 < A.K0; ++k0) {
      const int32_t j0 = w0.s + k0 * A.d0;
      if (j0 >= 0 && j0 < w0.e)
        axpy_row<TY, VEC>(acc, wr[k0],
                          ybase + (g.id - ylo + (int64_t)(j0 - p.i0) * step) * A.D,
                          g.lane, G, A.D);
    }
  } else {
    int n = 0;
    for (int k0 = 0; k0 < A.K0; ++k0) {
      const int32_t j0 = w0.s + k0 * A.d0;
      const bool v0 = j0 >= 0 && j0 < w0.e;
      for (int k1 = 0; k1 < A.K1; ++k1, ++n) {
        const int32_t j1 = w1.s + k1 * A.d1;
        if (v0 && j1 >= 0 && j1 < w1.e)
          axpy_row<TY, VEC>(acc, wr[n], y + rrow(A, p.b, p.h, j0, j1) * A.D,
                            g.lane, G, A.D);
      }
    }
  }
  if (g.live) st_row<TO, VEC>(out + g.id * A.D, acc, post, g.lane, G, A.D);
}

// ---- rank 1, fp32, head_dim 4 NC <= 16, window side K fixed ----------------
// Row block of dispatch index bid in a launch of nb blocks.  Workgroups are
// dealt to the 8 XCDs in turn (bid mod 8), each XCD with its own L2: here
// XCD x runs one contiguous run of row blocks, so the halo rows that a
// block stages with its neighbours are mostly fetched once per run.
__device__ __forceinline__ int xcd_block(int bid, int nb) {
  const int x = bid & 7, s = bid >> 3, per = nb >> 3, rem = nb & 7;
  return x * per + min(x, rem) + s;
}

// The DiNAT 1-D shapes (fp32 rows of a few 16-byte units, K in 3..13) with
// the neighbor window staged: one thread per row, the slot loop unrolled
// over K with each slot row read from LDS at a constant stride from the
// first.  LDS layout per block of nthr rows: the block's slot rows
// (nthr * K floats, rounded to 16 bytes), the window of rows
// [row0 - K d step, row0 + nthr + K d step) clamped to the tensor, then
// (k_r1_dot) the bias table [H, 2K-1].

// Window row range of the block and its first slot row / slot stride.
struct R1Rows {
  int lo, hi;  // staged rows [lo, hi)
  int rows;    // live rows of the block
  int r;       // this thread's row (clamped to the block's last live row)
};

// Rows a block stages beyond its own on each side, at most: a window holds
// its query and spans (K - 1) d positions, and a block's range is widened
// to whole positions (spatial-first rows hold the heads of a position).
__host__ __device__ __forceinline__ int r1_halo(int K, int d, int step) {
  return ((K - 1) * d + 1) * step;
}

// The staged key rows of a block.  With d = 1 the window start and end are
// non-decreasing along a sequence (and later sequences lie at later rows),
// so the first row's window start and the last row's window end bound the
// range, taken over every head of those positions in the spatial-first
// layout (a row of a lower position may carry a higher head).  Otherwise
// the rows widened by (K - 1) d positions per side (same head).
template <int K>
__device__ __forceinline__ R1Rows r1_rows(const RpbProb &A, int step, int bid) {
  R1Rows o;
  const int nthr = (int)blockDim.x;
  const int row0 = bid * nthr;
  o.rows = min(nthr, A.n_rows - row0);
  o.r = row0 + min((int)threadIdx.x, o.rows - 1);
  if (A.d0 == 1) {
    const int rl = row0 + o.rows - 1;
    const RPos pf = rpos(A, (uint32_t)row0), pl = rpos(A, (uint32_t)rl);
    const RWin wf = rwin_axis(K, 1, A.fd0, pf.i0, A.L0);
    const RWin wl = rwin_axis(K, 1, A.fd0, pl.i0, A.L0);
    const int hf = A.heads_first ? 0 : pf.h, hl = A.heads_first ? 0 : pl.h;
    o.lo = row0 - hf + (wf.s - pf.i0) * step;
    o.hi = rl - hl + (wl.s + K - 1 - pl.i0) * step + step;
  } else {
    // a block of one sequence whose first and last positions have centred
    // windows (K/2 d <= i < L - K/2 d, the interval where no window is
    // pinned) covers [first - K/2 d, last + K/2 d]; other blocks take
    // their rows widened by (K - 1) d positions per side
    const int rl = row0 + o.rows - 1;
    const RPos pf = rpos(A, (uint32_t)row0), pl = rpos(A, (uint32_t)rl);
    const int nhd = (K / 2) * A.d0;
    const bool inner = !A.heads_first && pf.b == pl.b && pf.i0 >= nhd && pl.i0 + nhd < A.L0;
    const int reach = (K - 1) * A.d0 * step;
    o.lo = inner ? row0 - pf.h - nhd * step : max(0, row0 - reach);
    o.hi = inner ? rl - pl.h + (nhd + 1) * step : min(A.n_rows, row0 + o.rows + reach);
  }
  return o;
}

// A block copy of n >= 1 16-byte units in two steps: load() issues the
// first four units of each thread (indices clamped onto the last unit), so
// a kernel can issue its other loads beside them before any is waited on;
// store() writes them to LDS (clamped indices rewrite the last unit with its
// own value: no branch for the loads to sink into) and copies any further
// units.
struct R1Copy {
  uint4 r[4];
  __device__ __forceinline__ void load(const uint4 *src, int n, int tid, int nthr) {
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = src[min(tid + j * nthr, n - 1)];
  }
  __device__ __forceinline__ void store(uint4 *dst, const uint4 *src, int n, int tid,
                                        int nthr) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) dst[min(tid + j * nthr, n - 1)] = r[j];
    block_copy16(dst + 4 * nthr, src + 4 * nthr, (int64_t)n - 4 * nthr);
  }
};

// logits / dattn: out[r, k] = <x'[r], y[nbr(r, k)]> (+ bias); every slot is
// inside its window here, so no slot takes the `fill` value.
template <int K, int NC>
__device__ __forceinline__ void r1_dot_body(int bid, const RpbProb &A,
                                            const float *__restrict__ x,
                                            const float *__restrict__ y,
                                            const float *__restrict__ rpb,
                                            float *__restrict__ out, int scale_x) {
  extern __shared__ __align__(16) float4 sm4[];
  const int nthr = (int)blockDim.x, tid = (int)threadIdx.x;
  const int step = A.heads_first ? 1 : A.H;
  const R1Rows b = r1_rows<K>(A, step, bid);
  float *so = reinterpret_cast<float *>(sm4);
  float4 *win = sm4 + (nthr * K + 3) / 4;
  constexpr int R0 = 2 * K - 1;
  float *bs = reinterpret_cast<float *>(win + (nthr + 2 * r1_halo(K, A.d0, step)) * NC);
  // every load of the prologue is issued before any is waited on: the query
  // row, one bias entry per thread (H (2K - 1) <= nthr; without a bias table
  // a harmless read of x into the spare slot), the window's first units
  float4 xv[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) xv[c] = reinterpret_cast<const float4 *>(x)[(int64_t)b.r * NC + c];
  const int nb = rpb != nullptr ? A.H * R0 : 1;
  const float bv = (rpb != nullptr ? rpb : x)[min(tid, nb - 1)];
  const uint4 *ysrc = reinterpret_cast<const uint4 *>(y) + (int64_t)b.lo * NC;
  const int nwin = (b.hi - b.lo) * NC;
  R1Copy cw;
  cw.load(ysrc, nwin, tid, nthr);
  bs[min(tid, nb - 1)] = bv;
  cw.store(reinterpret_cast<uint4 *>(win), ysrc, nwin, tid, nthr);
  const RPos p = rpos(A, (uint32_t)b.r);
  const RWin w = rwin_axis(K, A.d0, A.fd0, p.i0, A.L0);
  if (scale_x) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      xv[c].x *= A.scale;
      xv[c].y *= A.scale;
      xv[c].z *= A.scale;
      xv[c].w *= A.scale;
    }
  }
  __syncthreads();
  // slot k reads window row r - lo + (s + k d - i0) step.  With K d <= L
  // (r1_lds) every window lies inside its sequence: all K slots are valid
  // and their rows lie in the staged range
  const float4 *yb = win + (b.r - b.lo + (w.s - p.i0) * step) * NC;
  const int ys = A.d0 * step * NC;
  const float *br = bs + p.h * R0;
  float *sr = so + tid * K;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float4 t = yb[k * ys + c];
      acc = fmaf(xv[c].x, t.x, acc);
      acc = fmaf(xv[c].y, t.y, acc);
      acc = fmaf(xv[c].z, t.z, acc);
      acc = fmaf(xv[c].w, t.w, acc);
    }
    if (rpb != nullptr) acc += br[clampi(w.pb + k, 0, R0 - 1)];
    sr[k] = acc;
  }
  __syncthreads();
  block_copy_f32<true>(out + (int64_t)bid * nthr * K, so, (int64_t)b.rows * K);
}

template <int K, int NC>
__global__ void __launch_bounds__(512)
    k_r1_dot(RpbProb A, const float *__restrict__ x, const float *__restrict__ y,
             const float *__restrict__ rpb, float *__restrict__ out,
             int scale_x) {
  r1_dot_body<K, NC>(xcd_block((int)blockIdx.x, (int)gridDim.x), A, x, y, rpb, out, scale_x);
}

// AV / dq: out[r] = post * sum_k w[r, k] * y[nbr(r, k)] over valid slots.
// nblk: blocks of this pass (the bias partials' stride).
template <int K, int NC>
__device__ __forceinline__ void r1_gather_body(int bid, int nblk, const RpbProb &A,
                                               const float *__restrict__ wgt,
                                               const float *__restrict__ y,
                                               float *__restrict__ out, float post,
                                               double *__restrict__ bpart) {
  extern __shared__ __align__(16) float4 sm4[];
  const int nthr = (int)blockDim.x, tid = (int)threadIdx.x;
  const int step = A.heads_first ? 1 : A.H;
  const R1Rows b = r1_rows<K>(A, step, bid);
  float *sw = reinterpret_cast<float *>(sm4);
  float4 *win = sm4 + (nthr * K + 3) / 4;
  // every load of the prologue is issued before any is waited on: the
  // block's weight rows (16-byte aligned: row0 K is a multiple of 4) as
  // units plus a tail of floats, and the window's first units
  constexpr int JW = (K + 3) / 4;  // weight units per thread (rows <= nthr)
  const int nwf = b.rows * K, nw4 = nwf >> 2;
  const float *wg = wgt + (int64_t)bid * nthr * K;
  const uint4 *ysrc = reinterpret_cast<const uint4 *>(y) + (int64_t)b.lo * NC;
  const int nwin = (b.hi - b.lo) * NC;
  // without a whole weight unit the unit loads read the window instead and
  // their stores go to the spare unit after the window
  const uint4 *wsrc = nw4 > 0 ? reinterpret_cast<const uint4 *>(wg) : ysrc;
  uint4 *wdst = nw4 > 0 ? reinterpret_cast<uint4 *>(sw)
                        : reinterpret_cast<uint4 *>(win + (nthr + 2 * r1_halo(K, A.d0, step)) * NC);
  uint4 wu[JW];
#pragma unroll
  for (int j = 0; j < JW; ++j) wu[j] = wsrc[min(tid + j * nthr, max(nw4, 1) - 1)];
  const int ti = min(4 * nw4 + tid, nwf - 1);  // the tail floats (clamped)
  const float wt = wg[ti];
  R1Copy cw;
  cw.load(ysrc, nwin, tid, nthr);
#pragma unroll
  for (int j = 0; j < JW; ++j) wdst[min(tid + j * nthr, max(nw4, 1) - 1)] = wu[j];
  sw[ti] = wt;
  cw.store(reinterpret_cast<uint4 *>(win), ysrc, nwin, tid, nthr);
  const RPos p = rpos(A, (uint32_t)b.r);
  const RWin w = rwin_axis(K, A.d0, A.fd0, p.i0, A.L0);
  // bias-gradient partials (QK backward's dq pass): each row's first bias
  // cell, after the window and its spare unit
  int *spb = reinterpret_cast<int *>(win + (nthr + 2 * r1_halo(K, A.d0, step)) * NC + 1);
  if (bpart != nullptr) spb[tid] = w.pb;
  __syncthreads();
  const float4 *yb = win + (b.r - b.lo + (w.s - p.i0) * step) * NC;
  const int ys = A.d0 * step * NC;
  const float *wr = sw + tid * K;
  float4 acc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const float wk = wr[k];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float4 t = yb[k * ys + c];
      acc[c].x = fmaf(wk, t.x, acc[c].x);
      acc[c].y = fmaf(wk, t.y, acc[c].y);
      acc[c].z = fmaf(wk, t.z, acc[c].z);
      acc[c].w = fmaf(wk, t.w, acc[c].w);
    }
  }
  // the block's output rows are one contiguous range: write them through
  // LDS (over the window, once every thread has read its rows) as
  // consecutive 16-byte units rather than one strided row per lane; the
  // bias partials run after, with the accumulators already stored
  __syncthreads();
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float4 o = acc[c];
    o.x *= post;
    o.y *= post;
    o.z *= post;
    o.w *= post;
    win[tid * NC + c] = o;
  }
  if (bpart != nullptr) {
    // thread (h, c) of the H (2K - 1) bias cells adds, in row order and in
    // float64, the block's weights w[r, k] of head h with pb(r) + k = c
    // (spatial-first rows: head = row mod H; pb + k never needs clamping
    // here, pb lies in [0, K - 1]); one partial per (cell, block)
    constexpr int R0 = 2 * K - 1;
    if (tid < A.H * R0) {
      const int h = tid / R0, c = tid - h * R0;
      const int row0 = bid * nthr;
      const int h0 = row0 - (int)fdiv((uint32_t)row0, A.fH) * A.H;
      // a block of one sequence whose first and last positions have
      // unclamped windows (pb = K/2, which holds exactly on the interior
      // interval) has pb = K/2 on every row: slot c - K/2 of each row, no
      // per-row test (the same terms in the same order as the general loop)
      const RPos pf = rpos(A, (uint32_t)row0), pl = rpos(A, (uint32_t)(row0 + b.rows - 1));
      const int nh = K / 2;
      const bool inner = pf.b == pl.b && pf.i0 >= nh * A.d0 && pl.i0 + nh * A.d0 < A.L0;
      double acc_b = 0.0;
      int j = h >= h0 ? h - h0 : h - h0 + A.H;
      if (inner) {
        const int k = c - nh;
        if ((unsigned)k < (unsigned)K) {
          for (; j + 3 * A.H < b.rows; j += 4 * A.H) {
            const float t0 = sw[j * K + k], t1 = sw[(j + A.H) * K + k];
            const float t2 = sw[(j + 2 * A.H) * K + k], t3 = sw[(j + 3 * A.H) * K + k];
            acc_b += (double)t0;
            acc_b += (double)t1;
            acc_b += (double)t2;
            acc_b += (double)t3;
          }
          for (; j < b.rows; j += A.H) acc_b += (double)sw[j * K + k];
        }
      } else {
        for (; j < b.rows; j += A.H) {
          const int k = c - spb[j];
          if ((unsigned)k < (unsigned)K) acc_b += (double)sw[j * K + k];
        }
      }
      bpart[(int64_t)tid * nblk + bid] = acc_b;
    }
  }
  __syncthreads();
  block_copy16<true>(reinterpret_cast<uint4 *>(out) + (int64_t)bid * nthr * NC,
               reinterpret_cast<const uint4 *>(win), (int64_t)b.rows * NC);
}

template <int K, int NC>
__global__ void __launch_bounds__(512)
    k_r1_gather(RpbProb A, const float *__restrict__ wgt,
                const float *__restrict__ y, float *__restrict__ out,
                float post, double *__restrict__ bpart) {
  r1_gather_body<K, NC>(xcd_block((int)blockIdx.x, (int)gridDim.x), (int)gridDim.x, A, wgt, y,
                        out, post, bpart);
}

// ---- rank 1, spatial-first, dilation d > 1: rows in phase-major order ----
// A block takes rows in the order (sample, phase r, index m in the phase,
// head): phase r of a sample is an undilated sequence of plen(r) positions
// i = r + d m whose windows stay in the phase (the partition rule: in phase
// units the window of m starts at clamp(m - K/2, 0, plen - K)), so a block
// stages exactly the positions its windows reach, as at d = 1, instead of
// (K - 1) d positions on each side.  Memory keeps the [B, L, H, ...] order:
// the copies map each virtual position (b L + pstart(r) + m) to its memory
// position (b L + r + d m), whose rows of all heads form one run.
struct PhMap {
  int32_t q, rem;      // L / d and L % d: phase r holds q + (r < rem) positions
  FastDiv fq, fq1;     // q, q + 1
};

struct PhPos {
  int b, r, m, plen, pstart;
};

__device__ __forceinline__ PhPos ph_pos(const RpbProb &A, const PhMap &M, int pos) {
  PhPos o;
  o.b = (int)fdiv((uint32_t)pos, A.fL0);
  const int p = pos - o.b * A.L0;
  const int c1 = M.rem * (M.q + 1);
  if (p < c1) {
    o.r = (int)fdiv((uint32_t)p, M.fq1);
    o.m = p - o.r * (M.q + 1);
  } else {
    const int r2 = (int)fdiv((uint32_t)(p - c1), M.fq);
    o.r = M.rem + r2;
    o.m = p - c1 - r2 * M.q;
  }
  o.plen = M.q + (o.r < M.rem ? 1 : 0);
  o.pstart = o.r * M.q + min(o.r, M.rem);
  return o;
}

// Copy n 16-byte units of the virtual range starting at unit g0 (ru units per
// position) between memory and LDS, four per thread in flight.  LOAD: memory
// to LDS; else LDS to memory with streaming stores.
template <bool LOAD, bool NT = true>
__device__ __forceinline__ void ph_copy(const RpbProb &A, const PhMap &M, int ru,
                                        FastDiv fru, const uint4 *gsrc, uint4 *gdst,
                                        uint4 *lds, int g0, int n) {
  constexpr int kB = 4;
  if (n <= 0) return;
  const int nt = (int)blockDim.x, tid = (int)threadIdx.x;
  for (int base = 0; base < n; base += kB * nt) {
    u32x4 r[kB];
    int ix[kB], mu[kB];
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      ix[j] = min(base + j * nt + tid, n - 1);
      const int g = g0 + ix[j];
      const int pos = (int)fdiv((uint32_t)g, fru);
      const PhPos o = ph_pos(A, M, pos);
      mu[j] = (o.b * A.L0 + o.r + A.d0 * o.m) * ru + (g - pos * ru);
      r[j] = LOAD ? reinterpret_cast<const u32x4 *>(gsrc)[mu[j]]
                  : reinterpret_cast<const u32x4 *>(lds)[ix[j]];
    }
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      if (LOAD)
        reinterpret_cast<u32x4 *>(lds)[ix[j]] = r[j];
      else if (NT)
        __builtin_nontemporal_store(r[j], reinterpret_cast<u32x4 *>(gdst) + mu[j]);
      else
        reinterpret_cast<u32x4 *>(gdst)[mu[j]] = r[j];
    }
  }
}

// The first round of a LOAD ph_copy (four units per thread) split into its
// loads and its LDS stores, so that a kernel staging two ranges issues both
// ranges' first loads before it waits on either (one load round trip for
// the common block instead of two); ph_copy stages any units past the first
// round (units [4 nthr, n), copied by the caller).
struct PhRound {
  u32x4 r[4];
  int ix[4];
  __device__ __forceinline__ void load(const RpbProb &A, const PhMap &M, int ru, FastDiv fru,
                                       const uint4 *gsrc, int g0, int n) {
    const int nt = (int)blockDim.x, tid = (int)threadIdx.x;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ix[j] = min(j * nt + tid, n - 1);
      const int g = g0 + ix[j];
      const int pos = (int)fdiv((uint32_t)g, fru);
      const PhPos o = ph_pos(A, M, pos);
      const int mu = (o.b * A.L0 + o.r + A.d0 * o.m) * ru + (g - pos * ru);
      r[j] = reinterpret_cast<const u32x4 *>(gsrc)[mu];
    }
  }
  __device__ __forceinline__ void store(uint4 *lds) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) reinterpret_cast<u32x4 *>(lds)[ix[j]] = r[j];
  }
};

// Two LOAD copies (n0, n1 >= 1 units) with their first rounds' loads in
// flight together.
__device__ __forceinline__ void ph_copy2(const RpbProb &A, const PhMap &M, int ru0,
                                         FastDiv fru0, const uint4 *src0, uint4 *lds0,
                                         int g0, int n0, int ru1, FastDiv fru1,
                                         const uint4 *src1, uint4 *lds1, int g1, int n1) {
  const int kr = 4 * (int)blockDim.x;
  PhRound a, b;
  a.load(A, M, ru0, fru0, src0, g0, n0);
  b.load(A, M, ru1, fru1, src1, g1, n1);
  a.store(lds0);
  b.store(lds1);
  ph_copy<true>(A, M, ru0, fru0, src0, nullptr, lds0 + kr, g0 + kr, n0 - kr);
  ph_copy<true>(A, M, ru1, fru1, src1, nullptr, lds1 + kr, g1 + kr, n1 - kr);
}

// The block's rows [row0, row0 + rows) and the virtual positions [lo, hi)
// of their windows; the thread's row: virtual position, head, phase place.
struct PhRows {
  int row0, rows, lo, hi;
  int h, mrow;  // the thread's head and memory row
  PhPos o;      // the thread's phase place
  int wsm;      // its window start in phase units
};

template <int K>
__device__ __forceinline__ PhRows ph_rows(const RpbProb &A, const PhMap &M, int bid) {
  PhRows R;
  const int nthr = (int)blockDim.x;
  R.row0 = bid * nthr;
  R.rows = min(nthr, A.n_rows - R.row0);
  const PhPos f = ph_pos(A, M, (int)fdiv((uint32_t)R.row0, A.fH));
  const PhPos l = ph_pos(A, M, (int)fdiv((uint32_t)(R.row0 + R.rows - 1), A.fH));
  R.lo = f.b * A.L0 + f.pstart + min(max(f.m - K / 2, 0), f.plen - K);
  R.hi = l.b * A.L0 + l.pstart + min(max(l.m - K / 2, 0), l.plen - K) + K;
  const int v = R.row0 + min((int)threadIdx.x, R.rows - 1);
  const int vpos = (int)fdiv((uint32_t)v, A.fH);
  R.h = v - vpos * A.H;
  R.o = ph_pos(A, M, vpos);
  R.mrow = (R.o.b * A.L0 + R.o.r + A.d0 * R.o.m) * A.H + R.h;
  R.wsm = min(max(R.o.m - K / 2, 0), R.o.plen - K);
  return R;
}

// Unit counts and their divisors for the phase-major copies: key / value
// rows (H NC units per position), slot rows (H K / 4 units per position).
struct PhUnits {
  int ry, rk;
  FastDiv fry, frk;
};

template <int K, int NC>
__device__ __forceinline__ void r1p_dot_body(int bid, const RpbProb &A, const PhMap &M,
                                             const PhUnits &U, const float *__restrict__ x,
                                             const float *__restrict__ y,
                                             const float *__restrict__ rpb,
                                             float *__restrict__ out, int scale_x) {
  extern __shared__ __align__(16) float4 sm4[];
  const int nthr = (int)blockDim.x, tid = (int)threadIdx.x;
  const PhRows R = ph_rows<K>(A, M, bid);
  float *so = reinterpret_cast<float *>(sm4);
  float4 *win = sm4 + (nthr * K + 3) / 4;
  constexpr int R0 = 2 * K - 1;
  float *bs = reinterpret_cast<float *>(win + (nthr + 2 * r1_halo(K, 1, A.H)) * NC);
  float4 xv[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) xv[c] = reinterpret_cast<const float4 *>(x)[(int64_t)R.mrow * NC + c];
  const int nb = rpb != nullptr ? A.H * R0 : 1;
  const float bv = (rpb != nullptr ? rpb : x)[min(tid, nb - 1)];
  ph_copy<true>(A, M, U.ry, U.fry, reinterpret_cast<const uint4 *>(y), nullptr,
                reinterpret_cast<uint4 *>(win), R.lo * U.ry, (R.hi - R.lo) * U.ry);
  bs[min(tid, nb - 1)] = bv;
  const RWin w = rwin_axis(K, A.d0, A.fd0, R.o.r + A.d0 * R.o.m, A.L0);
  if (scale_x) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      xv[c].x *= A.scale;
      xv[c].y *= A.scale;
      xv[c].z *= A.scale;
      xv[c].w *= A.scale;
    }
  }
  __syncthreads();
  const float4 *yb =
      win + ((R.o.b * A.L0 + R.o.pstart + R.wsm - R.lo) * A.H + R.h) * NC;
  const int ys = A.H * NC;
  const float *br = bs + R.h * R0;
  float *sr = so + tid * K;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float4 t = yb[k * ys + c];
      acc = fmaf(xv[c].x, t.x, acc);
      acc = fmaf(xv[c].y, t.y, acc);
      acc = fmaf(xv[c].z, t.z, acc);
      acc = fmaf(xv[c].w, t.w, acc);
    }
    if (rpb != nullptr) acc += br[clampi(w.pb + k, 0, R0 - 1)];
    sr[k] = acc;
  }
  __syncthreads();
  ph_copy<false>(A, M, U.rk, U.frk, nullptr, reinterpret_cast<uint4 *>(out),
                 reinterpret_cast<uint4 *>(so), R.row0 * K / 4, R.rows * K / 4);
}

template <int K, int NC>
__global__ void __launch_bounds__(512)
    k_r1p_dot(RpbProb A, PhMap M, PhUnits U, const float *__restrict__ x,
              const float *__restrict__ y, const float *__restrict__ rpb,
              float *__restrict__ out, int scale_x) {
  r1p_dot_body<K, NC>(xcd_block((int)blockIdx.x, (int)gridDim.x), A, M, U, x, y, rpb, out,
                      scale_x);
}

// bpart (the QK backward's dq pass): also the bias gradient's float64
// partials, one per (cell, block), as the contiguous staged gather forms
// them (the block's rows are (position, head) rows, heads innermost, in
// phase-major order; the reduction adds blocks in order).
template <int K, int NC>
__device__ __forceinline__ void r1p_gather_body(int bid, int nblk, const RpbProb &A,
                                                const PhMap &M, const PhUnits &U,
                                                const float *__restrict__ wgt,
                                                const float *__restrict__ y,
                                                float *__restrict__ out, float post,
                                                double *__restrict__ bpart) {
  extern __shared__ __align__(16) float4 sm4[];
  const int nthr = (int)blockDim.x, tid = (int)threadIdx.x;
  const PhRows R = ph_rows<K>(A, M, bid);
  float *sw = reinterpret_cast<float *>(sm4);
  float4 *win = sm4 + (nthr * K + 3) / 4;
  int *spb = reinterpret_cast<int *>(win + (nthr + 2 * r1_halo(K, 1, A.H)) * NC);
  ph_copy2(A, M, U.rk, U.frk, reinterpret_cast<const uint4 *>(wgt),
           reinterpret_cast<uint4 *>(sw), R.row0 * K / 4, R.rows * K / 4, U.ry, U.fry,
           reinterpret_cast<const uint4 *>(y), reinterpret_cast<uint4 *>(win), R.lo * U.ry,
           (R.hi - R.lo) * U.ry);
  if (bpart != nullptr)
    spb[tid] = rwin_axis(K, A.d0, A.fd0, R.o.r + A.d0 * R.o.m, A.L0).pb;
  __syncthreads();
  const float4 *yb =
      win + ((R.o.b * A.L0 + R.o.pstart + R.wsm - R.lo) * A.H + R.h) * NC;
  const int ys = A.H * NC;
  const float *wr = sw + tid * K;
  float4 acc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const float wk = wr[k];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float4 t = yb[k * ys + c];
      acc[c].x = fmaf(wk, t.x, acc[c].x);
      acc[c].y = fmaf(wk, t.y, acc[c].y);
      acc[c].z = fmaf(wk, t.z, acc[c].z);
      acc[c].w = fmaf(wk, t.w, acc[c].w);
    }
  }
  // the output rows over the window (once every thread has read its
  // rows), then the bias partials with the accumulators already stored
  __syncthreads();
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float4 o = acc[c];
    o.x *= post;
    o.y *= post;
    o.z *= post;
    o.w *= post;
    win[tid * NC + c] = o;
  }
  if (bpart != nullptr) {
    // thread (h, c) of the H (2K - 1) bias cells adds, in row order and in
    // float64, the block's weights w[r, k] of head h with pb(r) + k = c
    constexpr int R0 = 2 * K - 1;
    if (tid < A.H * R0) {
      const int h = tid / R0, c = tid - h * R0;
      const int h0 = R.row0 - (int)fdiv((uint32_t)R.row0, A.fH) * A.H;
      // a block inside one phase of one sample whose first and last indices
      // have unclamped windows (K/2 <= m <= plen - 1 - K/2, where pb = K/2)
      // has pb = K/2 on every row, as in the staged gather
      const int nh = K / 2;
      const PhPos f = ph_pos(A, M, (int)fdiv((uint32_t)R.row0, A.fH));
      const PhPos l = ph_pos(A, M, (int)fdiv((uint32_t)(R.row0 + R.rows - 1), A.fH));
      const bool inner = f.b == l.b && f.r == l.r && f.m >= nh && l.m + nh < l.plen;
      double acc_b = 0.0;
      int j = h >= h0 ? h - h0 : h - h0 + A.H;
      if (inner) {
        const int k = c - nh;
        if ((unsigned)k < (unsigned)K) {
          for (; j + 3 * A.H < R.rows; j += 4 * A.H) {
            const float t0 = sw[j * K + k], t1 = sw[(j + A.H) * K + k];
            const float t2 = sw[(j + 2 * A.H) * K + k], t3 = sw[(j + 3 * A.H) * K + k];
            acc_b += (double)t0;
            acc_b += (double)t1;
            acc_b += (double)t2;
            acc_b += (double)t3;
          }
          for (; j < R.rows; j += A.H) acc_b += (double)sw[j * K + k];
        }
      } else {
        for (; j < R.rows; j += A.H) {
          const int k = c - spb[j];
          if ((unsigned)k < (unsigned)K) acc_b += (double)sw[j * K + k];
        }
      }
      bpart[(int64_t)tid * nblk + bid] = acc_b;
    }
  }
  __syncthreads();
  ph_copy<false>(A, M, U.ry, U.fry, nullptr, reinterpret_cast<uint4 *>(out),
                 reinterpret_cast<uint4 *>(win), R.row0 * NC, R.rows * NC);
}

template <int K, int NC>
__global__ void __launch_bounds__(512)
    k_r1p_gather(RpbProb A, PhMap M, PhUnits U, const float *__restrict__ wgt,
                 const float *__restrict__ y, float *__restrict__ out, float post,
                 double *__restrict__ bpart) {
  r1p_gather_body<K, NC>(xcd_block((int)blockIdx.x, (int)gridDim.x), (int)gridDim.x, A, M, U,
                         wgt, y, out, post, bpart);
}

// dk / dv on the phase-major rows (d > 1): one thread per key row in the
// order (sample, phase, index m, head).  In phase units the queries whose
// windows hold key m are [m <= K-1 ? 0 : m - K/2, m >= plen-K ? plen-1 :
// m + K/2] (K d <= L), at slot m - clamp(mq - K/2, 0, plen - K); the
// block stages the query rows and weight rows of the virtual positions from
// its first key's first query to its last key's last query (at most K - 1
// positions of halo per side, where the contiguous inverse needs (K - 1) d).
// Where every key of the block lies at a phase index in [K, plen - K - 1]
// of one phase the K candidates m + t, |t| <= K/2, take slot K/2 - t with no
// window test (the interior rule of the contiguous inverse in phase units).
template <int K, int NC>
__device__ __forceinline__ void r1p_inverse_body(int bid, const RpbProb &A, const PhMap &M,
                                                 const PhUnits &U, const float *__restrict__ w,
                                                 const float *__restrict__ x,
                                                 float *__restrict__ out, float post, int cap) {
  extern __shared__ __align__(16) float4 sm4[];
  const int nthr = (int)blockDim.x, tid = (int)threadIdx.x;
  const int row0 = bid * nthr;
  const int rows = min(nthr, A.n_rows - row0);
  const PhPos f = ph_pos(A, M, (int)fdiv((uint32_t)row0, A.fH));
  const PhPos l = ph_pos(A, M, (int)fdiv((uint32_t)(row0 + rows - 1), A.fH));
  const int lo = f.b * A.L0 + f.pstart + (f.m <= K - 1 ? 0 : f.m - K / 2);
  const int hi = l.b * A.L0 + l.pstart + (l.m >= l.plen - K ? l.plen - 1 : l.m + K / 2) + 1;
  float4 *xs = sm4;                                     // cap rows of NC units
  float *ws = reinterpret_cast<float *>(sm4 + cap * NC);  // cap rows of K floats
  ph_copy2(A, M, U.ry, U.fry, reinterpret_cast<const uint4 *>(x),
           reinterpret_cast<uint4 *>(xs), lo * U.ry, (hi - lo) * U.ry, U.rk, U.frk,
           reinterpret_cast<const uint4 *>(w), reinterpret_cast<uint4 *>(ws), lo * U.rk,
           (hi - lo) * U.rk);
  const int v = row0 + min(tid, rows - 1);
  const int vpos = (int)fdiv((uint32_t)v, A.fH);
  const int h = v - vpos * A.H;
  const PhPos o = ph_pos(A, M, vpos);
  // staged row of the phase's index 0, head h
  const int rb0 = (o.b * A.L0 + o.pstart - lo) * A.H + h;
  __syncthreads();
  float4 acc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = make_float4(0.f, 0.f, 0.f, 0.f);
  auto add = [&](float wk, int sr) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float4 t = xs[sr * NC + c];
      acc[c].x = fmaf(wk, t.x, acc[c].x);
      acc[c].y = fmaf(wk, t.y, acc[c].y);
      acc[c].z = fmaf(wk, t.z, acc[c].z);
      acc[c].w = fmaf(wk, t.w, acc[c].w);
    }
  };
  const bool interior = f.b == l.b && f.r == l.r && f.m >= K && l.m <= l.plen - K - 1;
  if (interior) {
#pragma unroll
    for (int t = -(K / 2); t <= K / 2; ++t) {
      const int sr = rb0 + (o.m + t) * A.H;
      add(ws[sr * K + (K / 2 - t)], sr);
    }
  } else {
#pragma unroll 4
    for (int t = -(K - 1); t <= K - 1; ++t) {
      const int mq = o.m + t;
      const int sl = o.m - min(max(mq - K / 2, 0), o.plen - K);
      const bool ok = mq >= 0 && mq < o.plen && sl >= 0 && sl < K;
      const int sr = ok ? rb0 + mq * A.H : rb0 + o.m * A.H;
      add(ok ? ws[sr * K + sl] : 0.f, sr);
    }
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float4 r = acc[c];
    r.x *= post;
    r.y *= post;
    r.z *= post;
    r.w *= post;
    sm4[tid * NC + c] = r;
  }
  __syncthreads();
  ph_copy<false, false>(A, M, U.ry, U.fry, nullptr, reinterpret_cast<uint4 *>(out),
                        reinterpret_cast<uint4 *>(sm4), row0 * NC, rows * NC);
}

template <int K, int NC>
__global__ void __launch_bounds__(512)
    k_r1p_inverse(RpbProb A, PhMap M, PhUnits U, const float *__restrict__ w,
                  const float *__restrict__ x, float *__restrict__ out, float post,
                  int cap) {
  r1p_inverse_body<K, NC>(xcd_block((int)blockIdx.x, (int)gridDim.x), A, M, U, w, x, out, post,
                          cap);
}

// A backward's two passes on the phase-major rows in one launch, n0 blocks
// each: QK, dq by the gather over dlogits (with the bias partials when
// bpart is set) in blocks [0, n0), then dk; AV, dv first, then dattn by the
// dot of dout with the values; each pass's row blocks in contiguous runs
// per XCD as in k_r1_qkb.
template <int K, int NC>
__global__ void __launch_bounds__(512)
    k_r1p_qkb(RpbProb A, PhMap M, PhUnits U, const float *__restrict__ dl,
              const float *__restrict__ q, const float *__restrict__ key,
              float *__restrict__ dq, float *__restrict__ dk, float post,
              double *__restrict__ bpart, int n0, int cap) {
  const int bid = (int)blockIdx.x;
  if (bid < n0)
    r1p_gather_body<K, NC>(xcd_block(bid, n0), n0, A, M, U, dl, key, dq, post, bpart);
  else
    r1p_inverse_body<K, NC>(xcd_block(bid - n0, n0), A, M, U, dl, q, dk, post, cap);
}

template <int K, int NC>
__global__ void __launch_bounds__(512)
    k_r1p_avb(RpbProb A, PhMap M, PhUnits U, const float *__restrict__ attn,
              const float *__restrict__ v, const float *__restrict__ dout,
              float *__restrict__ dattn, float *__restrict__ dv, int n0, int cap) {
  // the dv pass's blocks first, as in k_r1_avb
  const int bid = (int)blockIdx.x;
  if (bid >= n0)
    r1p_dot_body<K, NC>(xcd_block(bid - n0, n0), A, M, U, dout, v, nullptr, dattn, 0);
  else
    r1p_inverse_body<K, NC>(xcd_block(bid, n0), A, M, U, attn, dout, dv, 1.f, cap);
}

// dk / dv: out[j] = post * sum over the queries i whose window holds key j
// of w[i, slot of j] * x[i] (the transpose of k_r1_gather), for the shapes
// of k_r1_dot / k_r1_gather.  One thread per key row; the block stages the
// query rows and weight rows within (K - 1) d positions of its keys (same
// head), tests the 2K - 1 candidates i = j + t d, |t| < K, against the
// window rule, and writes its output rows through LDS as consecutive
// 16-byte units (streaming stores).
template <int K, int NC, bool D1>
__device__ __forceinline__ void r1_inverse_body(int bid, const RpbProb &A,
                                                const float *__restrict__ w,
                                                const float *__restrict__ x,
                                                float *__restrict__ out, float post) {
  extern __shared__ __align__(16) float4 sm4[];
  const int nthr = (int)blockDim.x, tid = (int)threadIdx.x;
  const int step = A.heads_first ? 1 : A.H;
  const int row0 = bid * nthr;
  const int rows = min(nthr, A.n_rows - row0);
  const int r = row0 + min(tid, rows - 1);
  // every key of the block at a position j in [K d, L - 1 - K d] of one
  // sequence (block-uniform): j's phase index m and the phase indices m + t,
  // |t| <= K/2, of the queries j + t d lie at least K from both ends of the
  // phase, so those queries' windows are unclamped ([m + t - K/2, m + t +
  // K/2], holding j at slot K/2 - t) and every other query's window (of the
  // same phase: unclamped and more than K/2 away, or clamped to the first
  // or last K indices) misses j; the K candidates need no window test, and
  // the block stages only the rows K/2 d positions either side of its own
  bool interior;
  {
    const RPos pf = rpos(A, (uint32_t)row0), pl = rpos(A, (uint32_t)(row0 + rows - 1));
    const int kd = K * A.d0;
    interior = pf.b == pl.b && pf.h == (A.heads_first ? pl.h : pf.h) && pf.i0 >= kd &&
               pl.i0 <= A.L0 - 1 - kd;
  }
  const int reach = (interior ? K / 2 : K - 1) * A.d0 * step;
  const int lo = max(0, row0 - reach), hi = min(A.n_rows, row0 + rows + reach);
  const int cap = nthr + 2 * r1_halo(K, A.d0, step);  // staged rows, at most
  float4 *xs = sm4;
  float *ws = reinterpret_cast<float *>(sm4 + cap * NC);
  // every load of the prologue is issued before any is waited on
  const uint4 *xsrc = reinterpret_cast<const uint4 *>(x) + (int64_t)lo * NC;
  const int nx = (hi - lo) * NC;
  // weight floats [f0, f1) at ws[f - base], base = f0 rounded down to a
  // 16-byte unit: whole units [u0, u1) as float4, the few floats before u0
  // and after u1 one by one (no read past the tensor)
  const int f0 = lo * K, f1 = hi * K;
  const int base = f0 & ~3, u0 = (f0 + 3) & ~3, u1 = f1 & ~3;
  const int nu = u1 > u0 ? (u1 - u0) >> 2 : 0;
  R1Copy cx;
  cx.load(xsrc, nx, tid, nthr);
  const float4 *wu = reinterpret_cast<const float4 *>(w + u0);
  float4 *wd = reinterpret_cast<float4 *>(ws + (u0 - base));
  float4 wr0 = make_float4(0.f, 0.f, 0.f, 0.f), wr1 = wr0;
  if (nu > 0) {
    wr0 = wu[min(tid, nu - 1)];
    wr1 = wu[min(tid + nthr, nu - 1)];
  }
  const int nh = min(u0, f1) - f0, nt = u1 >= u0 ? f1 - u1 : 0;
  const float hv = tid < nh ? w[f0 + tid] : 0.f;
  const float tv = tid < nt ? w[u1 + tid] : 0.f;
  cx.store(reinterpret_cast<uint4 *>(xs), xsrc, nx, tid, nthr);
  if (nu > 0) {
    wd[min(tid, nu - 1)] = wr0;
    wd[min(tid + nthr, nu - 1)] = wr1;
    for (int i = tid + 2 * nthr; i < nu; i += nthr) wd[i] = wu[i];
  }
  if (tid < nh) ws[f0 - base + tid] = hv;
  if (tid < nt) ws[u1 - base + tid] = tv;
  const RPos p = rpos(A, (uint32_t)r);
  const int wrow0 = f0 - base;  // ws offset of staged row 0
  __syncthreads();
  float4 acc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = make_float4(0.f, 0.f, 0.f, 0.f);
  auto add = [&](float wk, const float4 *xr) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float4 v = xr[c];
      acc[c].x = fmaf(wk, v.x, acc[c].x);
      acc[c].y = fmaf(wk, v.y, acc[c].y);
      acc[c].z = fmaf(wk, v.z, acc[c].z);
      acc[c].w = fmaf(wk, v.w, acc[c].w);
    }
  };
  if (interior) {
#pragma unroll
    for (int t = -(K / 2); t <= K / 2; ++t) {
      const int sr = r - lo + t * A.d0 * step;
      add(ws[wrow0 + sr * K + (K / 2 - t)], xs + sr * NC);
    }
  } else {
  // four candidates per step keep the loads in flight without holding all
  // 2K - 1 candidates' rows in registers
#pragma unroll 4
  for (int t = -(K - 1); t <= K - 1; ++t) {
    const int i = p.i0 + t * A.d0;
    bool ok = i >= 0 && i < A.L0;
    int k = 0;
    if (D1) {
      // d = 1 (K <= L): window start clamp(i - K / 2, 0, L - K)
      k = p.i0 - min(max(i - K / 2, 0), A.L0 - K);
      ok = ok && k >= 0 && k < K;
    } else if (ok) {
      const RWin wi = rwin_axis(K, A.d0, A.fd0, i, A.L0);
      const int off = p.i0 - wi.s;  // a multiple of d (same phase)
      k = (int)fdiv((uint32_t)max(off, 0), A.fd0);
      ok = off >= 0 && k < K;
    }
    const int sr = r - lo + t * A.d0 * step;  // the candidate's staged row
    const float wk = ok ? ws[wrow0 + sr * K + k] : 0.f;
    add(wk, xs + (ok ? sr : r - lo) * NC);
  }
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float4 o = acc[c];
    o.x *= post;
    o.y *= post;
    o.z *= post;
    o.w *= post;
    sm4[tid * NC + c] = o;
  }
  __syncthreads();
  block_copy16<true>(reinterpret_cast<uint4 *>(out) + (int64_t)row0 * NC,
                     reinterpret_cast<const uint4 *>(sm4), (int64_t)rows * NC);
}

template <int K, int NC, bool D1>
__global__ void __launch_bounds__(512)
    k_r1_inverse(RpbProb A, const float *__restrict__ w,
                 const float *__restrict__ x, float *__restrict__ out, float post) {
  r1_inverse_body<K, NC, D1>(xcd_block((int)blockIdx.x, (int)gridDim.x), A, w, x, out, post);
}

// The two passes of a backward in one launch (they are independent), n0
// blocks each.  QK backward: dq by the gather over dlogits (with the bias
// partials when bpart is set), blocks [0, n0), then dk; AV backward: dv
// first, then dattn by the dot of dout with the values.  Each pass deals
// its row blocks to the XCDs in contiguous runs (xcd_block), the two
// passes' dispatch ranges kept apart: interleaving the
// passes block by block in one run per XCD was slower (config 5 K=7 d=1
// QK backward 13.0 -> 13.8 us; the passes apart 12.7 us).
template <int K, int NC, bool D1>
__global__ void __launch_bounds__(512)
    k_r1_qkb(RpbProb A, const float *__restrict__ dl, const float *__restrict__ q,
             const float *__restrict__ key, float *__restrict__ dq,
             float *__restrict__ dk, float post, double *__restrict__ bpart, int n0) {
  const int bid = (int)blockIdx.x;
  if (bid < n0)
    r1_gather_body<K, NC>(xcd_block(bid, n0), n0, A, dl, key, dq, post, bpart);
  else
    r1_inverse_body<K, NC, D1>(xcd_block(bid - n0, n0), A, dl, q, dk, post);
}

template <int K, int NC, bool D1>
__global__ void __launch_bounds__(512)
    k_r1_avb(RpbProb A, const float *__restrict__ attn, const float *__restrict__ v,
             const float *__restrict__ dout, float *__restrict__ dattn,
             float *__restrict__ dv, int n0) {
  // the dv pass's blocks are dispatched first here, the dq pass's in
  // k_r1_qkb (config 5 AV backward, dattn pass first -> dv pass first:
  // K=7 d=1 7.12 -> 6.77 us, K=3 d=8 7.62 -> 6.53, K=5 d=1 6.31 -> 5.60;
  // the QK pairs the other way round: K=7 d=1 12.7 -> 13.5 us)
  const int bid = (int)blockIdx.x;
  if (bid >= n0)
    r1_dot_body<K, NC>(xcd_block(bid - n0, n0), A, dout, v, nullptr, dattn, 0);
  else
    r1_inverse_body<K, NC, D1>(xcd_block(bid, n0), A, attn, dout, dv, 1.f);
}

// out[j] = sum over (r, n) with nbr(r, n) == j of w[r, n] * x'[r]: the
// transpose of k_rpb_gather, evaluated per key row.  A query i can hold key
// j only on j's dilation phase and within K*d of it, so the candidates
// are i = j + t*d, |t| <= K, per axis, kept when j lies in
// [start(i), end(i)).
// QK backward's dk (w = dlogits, x = q scaled as in the forward) and AV
// backward's dv (w = attn, x = dout).
template <typename TX, typename TO, int VEC>
__global__ void __launch_bounds__(256)
    k_rpb_inverse(RpbProb A, const float *__restrict__ w,
                  const TX *__restrict__ x, TO *__restrict__ out, int scale_x,
                  int G, int lgG) {
  const Group g = make_group(lgG, A.n_rows);
  const RPos p = rpos(A, (uint32_t)g.id);
  float acc[kNT][VEC];
#pragma unroll
  for (int t = 0; t < kNT; ++t)
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[t][e] = 0.f;
  if (A.rank == 1) {
    // candidates i0 = i + t d, |t| <= K, in batches of four: the batch's
    // window tests first, then every load of the batch, then the FMAs
    const int64_t step = A.heads_first ? 1 : A.H;
    for (int32_t tb = -A.K0; tb <= A.K0; tb += 4) {
      float wt[4];
      float xv[4][kNT][VEC];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int32_t t0 = tb + u;
        const int32_t i0 = p.i0 + t0 * A.d0;
        bool ok = t0 <= A.K0 && i0 >= 0 && i0 < A.L0;
        int32_t k0 = 0;
        if (ok) {
          const RWin w0 = rwin0(A, i0);
          ok = p.i0 >= w0.s && p.i0 < w0.e;
          k0 = (int32_t)fdiv((uint32_t)(p.i0 - w0.s), A.fd0);
        }
        const int64_t r = g.id + (int64_t)t0 * A.d0 * step;
        wt[u] = ok ? w[r * A.KK + k0] : 0.f;
        if (ok) {
          ld_row<TX, VEC>(xv[u], x + r * A.D, g.lane, G, A.D);
        } else {
#pragma unroll
          for (int t = 0; t < kNT; ++t)
#pragma unroll
            for (int e = 0; e < VEC; ++e) xv[u][t][e] = 0.f;
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (scale_x) scale_round<TX, VEC>(xv[u], A.scale);
#pragma unroll
        for (int t = 0; t < kNT; ++t)
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[t][e] = fmaf(wt[u], xv[u][t][e], acc[t][e]);
      }
    }
    if (g.live) st_row<TO, VEC>(out + g.id * A.D, acc, 1.f, g.lane, G, A.D);
    return;
  }
  const int32_t t1max = A.rank == 2 ? A.K1 : 0;
  for (int32_t t0 = -A.K0; t0 <= A.K0; ++t0) {
    const int32_t i0 = p.i0 + t0 * A.d0;
    if (i0 < 0 || i0 >= A.L0) continue;
    const RWin w0 = rwin0(A, i0);
    if (p.i0 < w0.s || p.i0 >= w0.e) continue;
    const int32_t k0 = (p.i0 - w0.s) / A.d0;
    for (int32_t t1 = -t1max; t1 <= t1max; ++t1) {
      const int32_t i1 = p.i1 + t1 * A.d1;
      if (i1 < 0 || i1 >= A.L1) continue;
      const RWin w1 = rwin1(A, i1);
      if (p.i1 < w1.s || p.i1 >= w1.e) continue;
      const int32_t k1 = (p.i1 - w1.s) / A.d1;
      const int64_t r = rrow(A, p.b, p.h, i0, i1);
      const float wt = w[r * A.KK + k0 * A.K1 + k1];
      float xv[kNT][VEC];
      ld_row<TX, VEC>(xv, x + r * A.D, g.lane, G, A.D);
      if (scale_x) scale_round<TX, VEC>(xv, A.scale);
#pragma unroll
      for (int t = 0; t < kNT; ++t)
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[t][e] = fmaf(wt, xv[t][e], acc[t][e]);
    }
  }
  if (g.live) st_row<TO, VEC>(out + g.id * A.D, acc, 1.f, g.lane, G, A.D);
}

// Slots k in [0, K) whose clipped bias row clip(pb + k, 0, R-1) equals r:
// one slot in the interior, a run at either clipped end.
__device__ __forceinline__ void slots_of_bias_row(int32_t r, int32_t pb,
                                                  int32_t K, int32_t R,
                                                  int32_t *lo, int32_t *hi) {
  int32_t a = r - pb, b = r - pb;
  if (r == 0) a = -pb - 2 * K;        // everything at or below row 0
  if (r == R - 1) b = R - 1 - pb + 2 * K;  // everything at or above R-1
  *lo = a < 0 ? 0 : a;
  *hi = b > K - 1 ? K - 1 : b;
}

// Bias gradient, pass 1: one block per chunk of `chunk` (<= kBiasChunk)
// queries (rows in (b, i0, i1) order); partial[bin * n_chunks + c] is the
// chunk's float64 sum for bin = (h, r0[, r1]), output-major so pass 2 reads each
// bin's partials contiguously.  `scatter` (the chunk's [query][head][bin]
// sums fit 32 KB of LDS): thread (t, h) adds its row's valid slots into
// its own LDS cells [t][h][clipped bias row] (slot order), then thread
// `bin` sums the chunk's cells in query order.  Otherwise thread `bin` walks
// the queries and reads the slots whose clipped bias row is the bin.
// Either way the order of every sum is fixed.
__global__ void __launch_bounds__(256)
    k_rpb_bias_partial(RpbProb A, const float *__restrict__ dl,
                       double *__restrict__ partial, int32_t chunk,
                       int32_t n_chunks, int scatter) {
  extern __shared__ float sacc[];
  __shared__ RWin sw0[kBiasChunk], sw1[kBiasChunk];
  __shared__ int32_t sb[kBiasChunk], si0[kBiasChunk], si1[kBiasChunk];
  const int32_t c = blockIdx.x;
  const int32_t nq = A.B * A.L0 * A.L1;
  const int32_t q0 = c * chunk;
  const int32_t nqc = min(chunk, nq - q0);
  const int tid = threadIdx.x;
  const int32_t per_h = A.R0 * A.R1;
  const int32_t nb = A.H * per_h;
  if (tid < nqc) {
    const int32_t qi = q0 + tid;
    const int32_t rest = (int32_t)fdiv((uint32_t)qi, A.fL1);
    const int32_t i1 = qi - rest * A.L1;
    const int32_t b = (int32_t)fdiv((uint32_t)rest, A.fL0);
    const int32_t i0 = rest - b * A.L0;
    sw0[tid] = rwin0(A, i0);
    sw1[tid] = rwin1(A, i1);
    sb[tid] = b;
    si0[tid] = i0;
    si1[tid] = i1;
  }
  if (scatter) {
    for (int32_t i = tid; i < nqc * nb; i += blockDim.x) sacc[i] = 0.f;
    __syncthreads();
    for (int32_t th = tid; th < nqc * A.H; th += blockDim.x) {
      const int32_t t = th / A.H;
      const int32_t h = th - t * A.H;
      const RWin w0 = sw0[t];
      const RWin w1 = sw1[t];
      const float *row = dl + rrow(A, sb[t], h, si0[t], si1[t]) * A.KK;
      float *cell = sacc + th * per_h;
      for (int32_t k0 = 0; k0 < A.K0; ++k0) {
        const int32_t j0 = w0.s + k0 * A.d0;
        if (j0 < 0 || j0 >= w0.e) continue;
        const int32_t r0 = clampi(w0.pb + k0, 0, A.R0 - 1);
        if (A.rank == 1) {
          cell[r0] += row[k0];
          continue;
        }
        for (int32_t k1 = 0; k1 < A.K1; ++k1) {
          const int32_t j1 = w1.s + k1 * A.d1;
          if (j1 < 0 || j1 >= w1.e) continue;
          cell[r0 * A.R1 + clampi(w1.pb + k1, 0, A.R1 - 1)] += row[k0 * A.K1 + k1];
        }
      }
    }
    __syncthreads();
    for (int32_t bin = tid; bin < nb; bin += blockDim.x) {
      const int32_t h = bin / per_h;
      const int32_t rb = bin - h * per_h;
      double acc = 0.0;
      for (int32_t t = 0; t < nqc; ++t) acc += (double)sacc[(t * A.H + h) * per_h + rb];
      partial[(int64_t)bin * n_chunks + c] = acc;
    }
    return;
  }
  __syncthreads();
  for (int32_t bin = tid; bin < nb; bin += blockDim.x) {
    const int32_t h = bin / per_h;
    const int32_t rb = bin - h * per_h;
    const int32_t r0 = rb / A.R1;
    const int32_t r1 = rb - r0 * A.R1;
    double acc = 0.0;
    for (int32_t t = 0; t < nqc; ++t) {
      const RWin w0 = sw0[t];
      int32_t a0, b0;
      slots_of_bias_row(r0, w0.pb, A.K0, A.R0, &a0, &b0);
      if (a0 > b0) continue;
      const RWin w1 = sw1[t];
      int32_t a1 = 0, b1 = 0;
      if (A.rank == 2) slots_of_bias_row(r1, w1.pb, A.K1, A.R1, &a1, &b1);
      const float *row = dl + rrow(A, sb[t], h, si0[t], si1[t]) * A.KK;
      for (int32_t k0 = a0; k0 <= b0; ++k0) {
        const int32_t j0 = w0.s + k0 * A.d0;
        if (j0 < 0 || j0 >= w0.e) continue;
        for (int32_t k1 = a1; k1 <= b1; ++k1) {
          const int32_t j1 = w1.s + k1 * A.d1;
          if (j1 < 0 || j1 >= w1.e) continue;
          acc += (double)row[k0 * A.K1 + k1];
        }
      }
    }
    partial[(int64_t)bin * n_chunks + c] = acc;
  }
}

// Bias gradient, pass 2: one wavefront per bin sums its chunk partials,
// lane l taking chunks l, l+64, ... and a fixed xor tree after.  Both
// passes accumulate in float64 (a bin adds one float32 term per query of
// the whole problem, and such sums can cancel to far below their terms), so
// the only float32 rounding is that of the result.
__global__ void __launch_bounds__(64)
    k_rpb_bias_reduce(const double *__restrict__ partial, int32_t n_chunks,
                      float *__restrict__ drpb) {
  const int32_t o = blockIdx.x;
  const int lane = threadIdx.x;
  const double *src = partial + (int64_t)o * n_chunks;
  // eight loads in flight per lane, summed in a fixed order
  double acc = 0.0;
  for (int32_t c0 = 0; c0 < n_chunks; c0 += 8 * 64) {
    double v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int32_t c = c0 + j * 64 + lane;
      v[j] = c < n_chunks ? src[c] : 0.0;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += v[j];
  }
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) drpb[o] = (float)acc;
}

// ---- host launchers --------------------------------------------------------

struct RShape {
  int vec, G, lgG;
};

// Widest access both element types allow (16 bytes of the wider one) when
// D divides into it, then the fewest lanes per row with kNT chunks each.
RShape rshape(int D, int vmax) {
  RShape s;
  s.vec = (D % vmax == 0) ? vmax : 1;
  const int chunks = (D + s.vec - 1) / s.vec;
  const int per = (chunks + kNT - 1) / kNT;
  s.G = 1;
  s.lgG = 0;
  while (s.G < per) {
    s.G <<= 1;
    ++s.lgG;
  }
  return s;
}

dim3 rgrid(const RpbProb &A, int lgG, int rb = 256) {
  const int64_t threads = (int64_t)A.n_rows << lgG;
  return dim3((unsigned)((threads + rb - 1) / rb));
}

size_t r1_lds(const RpbProb &A, int rb, bool bias);

// Threads per block of the forward gathers (k_rpb_dot / k_rpb_gather and
// the staged rank-1 kernels).  Rank 1 with a window reach K0 * d0 of at
// least 7: 256 rows for d0 = 1 (a block stages exactly its windows' rows);
// for larger dilations 256 where a window reaches (K0/2) d0 >= 6 positions
// either side and the staged kernels take that block (with a bias table),
// else 384 where they take it, else 512; everything else 256.  Measured at
// D = 12, K in {3, 5, 7}, d in {1..8}, with each launch's row blocks in
// contiguous runs per XCD: K=7 d=1 qk / av 4.99 / 5.25 us at 512 rows,
// 4.64 / 4.69 at 256; K=7 d=2 5.31 / 5.36 at 384, 5.08 / 5.09 at 256; K=5
// d=4 4.95 / 5.17 at 384, 4.84 / 4.91 at 256; K=3 d=4 4.30 / 4.79 at 384,
// 4.43 / 4.69 at 256.
// NATTEN_AMD_RPB_BLOCK overrides it (tuning).
// NATTEN_AMD_RPB_BLOCK (64 to 512) forces the rows per block (tuning).
int block_forced() {
  static const int forced = [] {
    const char *e = std::getenv("NATTEN_AMD_RPB_BLOCK");
    const int v = e != nullptr ? std::atoi(e) : 0;
    return v == 64 || v == 128 || v == 256 || v == 384 || v == 512 ? v : 0;
  }();
  return forced;
}

int rpb_block(const RpbProb &A) {
  const int forced = block_forced();
  if (forced > 0) return forced;
  if (A.rank != 1 || A.K0 * A.d0 < 7) return 256;
  if (A.d0 == 1 || ((A.K0 / 2) * A.d0 >= 6 && r1_lds(A, 256, true) != 0))
    return r1_lds(A, 256, true) != 0 ? 256 : 512;
  return r1_lds(A, 384, true) != 0 ? 384 : 512;
}

template <typename A_, typename B_>
constexpr int vmax_of() {
  return 16 / (int)(sizeof(A_) > sizeof(B_) ? sizeof(A_) : sizeof(B_));
}

// LDS for a block's slot rows (rb / G rows of KK floats), or 0 when that
// exceeds 32 KB and the rows go straight to memory.
size_t stage_bytes(const RpbProb &A, int lgG, int rb) {
  const size_t b = (size_t)(rb >> lgG) * A.KK * sizeof(float);
  return b <= 32768 ? b : 0;
}

// LDS of the staged neighbor window (rank 1), or 0 when it is not used:
// rows must be whole 16-byte units, the halo at most the block's rows and
// the window must fit with the slot staging in 64 KB.
template <typename TY>
size_t window_bytes(const RpbProb &A, int lgG, size_t slot_bytes, int rb) {
  if (A.rank != 1 || (A.D * sizeof(TY)) % 16 != 0) return 0;
  // only worth it while the halo is no larger than the block's own rows
  // (large dilations would mostly copy other phases' rows)
  if (window_rows(A, lgG, rb) > 2 * (int64_t)(rb >> lgG)) return 0;
  const size_t b = (size_t)window_rows(A, lgG, rb) * A.D * sizeof(TY);
  return slot_bytes + b <= 65536 ? b : 0;
}

// LDS of the rank-1 fp32 kernels (k_r1_dot / k_r1_gather) for blocks of rb
// rows, or 0 where they do not apply: rank 2, head_dim not a multiple of 4
// or above 16, K outside {3, 5, .., 13}, K d > L (windows with slots before
// the sequence), or halos more than the block's rows on each side (large
// dilations: the generic kernels read those rows directly; staging up to
// three times the block's rows still beats them: config 5 K=7 d=4 qk / av
// 9.08 / 10.5 -> 6.08 / 5.68 us).  With K d <= L every window lies inside
// the sequence, so each slot row is in the staged range.
// The staged and phase-major kernels index rows, slot rows and 16-byte units
// with 32-bit integers: a row index times K or head_dim must stay below
// 2^31 (larger problems take the generic kernels, whose row offsets are
// 64-bit).
// NATTEN_AMD_RPB_PAIR=0 keeps the backward's two passes in two launches
// (A/B checks of k_r1_qkb / k_r1_avb / k_r1p_qkb / k_r1p_avb; read per
// call).
bool pair_launch_off() {
  const char *e = std::getenv("NATTEN_AMD_RPB_PAIR");
  return e != nullptr && e[0] == '0';
}

// Whether dk (qk: the QK backward) or dv, as a launch of its own (the
// paired launches off or not applicable), takes the phase-major inverse
// before the contiguous staged inverse, where both apply (d > 1).  The QK
// backward's dk does where the contiguous inverse's halo is wide,
// (K - 1) d >= 12 with K >= 5 (config 5, dq a launch of its own: K=7 d=2
// 23.7 -> 21.1 us, K=7 d=4 25.5 -> 22.0, K=5 d=4 20.5 -> 19.9); the AV
// backward's dv and K = 3 keep the staged inverse.  NATTEN_AMD_RPB_PHINV=1
// / 0 forces / forbids it (A/B checks; read per call).
bool phase_inverse_first(const RpbProb &A, bool qk) {
  if (A.d0 < 2) return false;
  const char *e = std::getenv("NATTEN_AMD_RPB_PHINV");
  if (e != nullptr && (e[0] == '1' || e[0] == '0')) return e[0] == '1';
  return qk && A.K0 >= 5 && (A.K0 - 1) * A.d0 >= 12;
}

// Whether the backward's phase-major pair (k_r1p_qkb / k_r1p_avb) goes
// before the staged kernels where both apply: where K >= 5 and
// (K - 1) d >= 12, for both backward calls (config 5, phase-major pair
// against the staged one: qk K=5 d=4 13.7 vs 15.1 us, K=7 d=2 15.7 vs 16.8,
// av K=7 d=4 10.0 vs 11.7; the staged pair is faster at K=3 d=4 / 8 (12.6 /
// 13.2 vs 13.0 / 13.6 us) and K=5 d=2 (13.0 vs 13.7)).
// NATTEN_AMD_RPB_PHPAIR=1 / 0 forces / forbids it (A/B checks; read per
// call).
bool phase_pair_first(const RpbProb &A, bool qk) {
  if (A.d0 < 2) return false;
  const char *e = std::getenv("NATTEN_AMD_RPB_PHPAIR");
  if (e != nullptr && (e[0] == '1' || e[0] == '0')) return e[0] == '1';
  (void)qk;
  return A.K0 >= 5 && (A.K0 - 1) * A.d0 >= 12;
}

bool r1_offsets_fit(const RpbProb &A) {
  return (int64_t)A.n_rows * std::max(A.K0, A.D) < ((int64_t)1 << 31);
}

size_t r1_lds(const RpbProb &A, int rb, bool bias) {
  if (A.rank != 1 || A.D % 4 != 0 || A.D > 16) return 0;
  if (!r1_offsets_fit(A)) return 0;
  if ((int64_t)A.K0 * A.d0 > A.L0) return 0;
  if (A.K0 < 3 || A.K0 > 13 || (A.K0 & 1) == 0 || A.R0 != 2 * A.K0 - 1) return 0;
  if (bias && A.H * A.R0 > rb) return 0;  // one bias entry per thread
  const int64_t step = A.heads_first ? 1 : A.H;
  const int64_t wrows = rb + 2 * (int64_t)r1_halo(A.K0, A.d0, (int)step);
  if (wrows > 3 * (int64_t)rb) return 0;
  const size_t b = ((size_t)rb * A.K0 * 4 + 15) / 16 * 16 + (size_t)wrows * A.D * 4 +
                   (bias ? (size_t)A.H * A.R0 * 4 : 16);  // the bias table or a spare unit
  return b <= 65536 ? b : 0;
}

#define R1_K(KK_, BODY)           \
  switch (KK_) {                  \
    case 3: BODY(3, NC_); break;  \
    case 5: BODY(5, NC_); break;  \
    case 7: BODY(7, NC_); break;  \
    case 9: BODY(9, NC_); break;  \
    case 11: BODY(11, NC_); break; \
    default: BODY(13, NC_); break; \
  }

// The rank-1 fp32 dot / gather when r1_lds applies; false otherwise (no
// slot of these shapes is outside its window, so `fill` is never written).
// The phase-major kernels (k_r1p_*), where the contiguous staged kernels do
// not apply (halos above twice the block's rows: large dilations):
// spatial-first rows, d > 1, the staged shapes of r1_lds, and runs of H K
// slot floats that are whole 16-byte units.  Blocks of 256 rows; LDS as
// r1_lds with a halo of K positions of H rows per side.  Config 5: K=5 d=8
// qk / av 8.15 / 9.31 -> 5.6 / 6.2 us, K=7 d=8 10.2 / 10.9 -> 5.9 / 5.95 us
// (where the contiguous kernels apply they are faster: the phase-major
// copies map every 16-byte unit to its memory position).
constexpr int kPhBlock = 256;
size_t ph_lds(const RpbProb &A, bool bias) {
  if (A.heads_first || A.rank != 1 || A.d0 < 2 || (A.H * A.K0) % 4 != 0) return 0;
  if (!r1_offsets_fit(A)) return 0;
  if (A.D % 4 != 0 || A.D > 16) return 0;
  if ((int64_t)A.K0 * A.d0 > A.L0) return 0;
  if (A.K0 < 3 || A.K0 > 13 || (A.K0 & 1) == 0 || A.R0 != 2 * A.K0 - 1) return 0;
  if (bias && A.H * A.R0 > kPhBlock) return 0;
  const int64_t wrows = kPhBlock + 2 * (int64_t)r1_halo(A.K0, 1, A.H);
  if (wrows > 3 * (int64_t)kPhBlock) return 0;
  const size_t b = ((size_t)kPhBlock * A.K0 * 4 + 15) / 16 * 16 + (size_t)wrows * A.D * 4 +
                   (bias ? (size_t)A.H * A.R0 * 4 : 16);
  return b <= 65536 ? b : 0;
}

// The phase-major gather that also forms the bias partials: one bias cell
// per thread, each row's first cell in LDS after the window.
size_t ph_bias_gather_lds(const RpbProb &A) {
  const size_t l = ph_lds(A, false);
  if (l == 0 || A.H * A.R0 > kPhBlock) return 0;
  const size_t b = l + (size_t)kPhBlock * sizeof(int);
  return b <= 65536 ? b : 0;
}

void ph_maps(const RpbProb &A, PhMap *M, PhUnits *U) {
  M->q = A.L0 / A.d0;
  M->rem = A.L0 % A.d0;
  M->fq = make_fastdiv((uint32_t)M->q);
  M->fq1 = make_fastdiv((uint32_t)(M->q + 1));
  U->ry = A.H * (A.D / 4);
  U->rk = A.H * A.K0 / 4;
  U->fry = make_fastdiv((uint32_t)U->ry);
  U->frk = make_fastdiv((uint32_t)U->rk);
}

// LDS of the phase-major inverse (rows of the staged query positions: x
// rows and weight rows), or 0 where it does not apply; *cap: its rows.
size_t ph_inverse_lds(const RpbProb &A, int *cap) {
  if (ph_lds(A, false) == 0) return 0;
  const int64_t pos = kPhBlock / A.H + 2 + 2 * (int64_t)(A.K0 - 1);
  const int64_t rows = pos * A.H;
  const size_t b = (size_t)rows * (A.D / 4) * 16 + (size_t)rows * A.K0 * 4;
  if (cap != nullptr) *cap = (int)rows;
  return b <= 65536 ? b : 0;
}

// Which rank-1 fp32 kernels apply (the launchers below and rpb_plan share
// these): the staged contiguous ones, the phase-major ones, or neither.
enum R1Kind { kR1None = 0, kR1Staged = 1, kR1Phase = 2 };
R1Kind r1_kind(const RpbProb &A, bool bias) {
  if (r1_lds(A, rpb_block(A), bias) != 0) return kR1Staged;
  if (ph_lds(A, bias) != 0) return kR1Phase;
  return kR1None;
}
// The staged gather that also forms the bias gradient's partials:
// spatial-first rows, one thread per bias cell, each row's first bias cell
// in LDS.
size_t r1_bias_gather_lds(const RpbProb &A, int rb) {
  const size_t lds = r1_lds(A, rb, false);
  if (lds == 0 || A.heads_first || A.H * A.R0 > rb) return 0;
  const size_t b = lds + (size_t)rb * sizeof(int);
  return b <= 65536 ? b : 0;
}
size_t r1_bias_gather_lds(const RpbProb &A) { return r1_bias_gather_lds(A, rpb_block(A)); }
// LDS of the staged inverse (dk / dv), or 0 where it does not apply.  Up
// to 80 KB (two blocks per CU): the candidate queries' rows of dilated
// windows (K = 7 at d = 4 takes 73 KB for 384 keys).
constexpr size_t kR1InvLds = 80 * 1024;
size_t r1_inverse_lds(const RpbProb &A, int rb) {
  if (r1_lds(A, rb, false) == 0) return 0;
  const int step = A.heads_first ? 1 : A.H;
  const size_t cap = (size_t)rb + 2 * (size_t)r1_halo(A.K0, A.d0, step);
  const size_t lds = cap * (A.D / 4) * 16 + (cap * A.K0 + 4) * sizeof(float);
  return lds <= kR1InvLds ? lds : 0;
}
size_t r1_inverse_lds(const RpbProb &A) { return r1_inverse_lds(A, rpb_block(A)); }

// Rows per block of the AV backward's staged pair (k_r1_avb), with the dv
// blocks dispatched first: 512 at d = 1 from K = 7, 256 at larger
// dilations, where the staged kernels take them (config 5 av backward:
// K=7 d=1 6.80 at 256 rows, 6.64 at 512; K=5 d=1 5.53 / 6.03; K=3 d=2
// 5.54 / 5.89; K=3 d=4 6.12 at 256, 6.28 at 384, 6.52 at 512; K=5 d=2
// 6.77 / 6.88 / 7.36 us).
int avb_block(const RpbProb &A) {
  const int rb = rpb_block(A);
  if (block_forced()) return rb;
  const int want = A.d0 == 1 && A.K0 >= 7 ? 512 : A.d0 > 1 ? 256 : rb;
  if (want == rb) return rb;
  const size_t li = r1_inverse_lds(A, want);
  return r1_lds(A, want, false) != 0 && li != 0 && li <= 65536 ? want : rb;
}

// Rows per block of the QK backward's staged pair (k_r1_qkb): 512 where
// K >= 5, (K - 1) d >= 6 and its LDS fits, else the forward's (config 5 qk
// backward, 256 -> 512 rows: K=7 d=1 15.1 -> 13.1 us before the XCD runs,
// 12.6 either way after; K=3 d=1 10.1 -> 11.8, K=5 d=1 11.5 -> 12.8 and
// K=3 d=2 11.1 -> 11.6 keep 256; K=3 d=4 11.5 at 384 rows, 12.4 at 512,
// and K=3 d=8 11.6 at 256, 12.4 at 512, keep the forward's).
int qkb_block(const RpbProb &A) {
  const int rb = rpb_block(A);
  if (block_forced() || A.K0 < 5 || (A.K0 - 1) * A.d0 < 6 || rb >= 512) return rb;
  const size_t li = r1_inverse_lds(A, 512);
  return r1_bias_gather_lds(A, 512) != 0 && li != 0 && li <= 65536 ? 512 : rb;
}

bool r1_dot(const RpbProb &A, const float *x, const float *y, const float *rpb,
            float *out, int scale_x, hipStream_t st) {
  const int rb = rpb_block(A);
  const size_t lds = r1_lds(A, rb, rpb != nullptr);
  if (lds == 0) {
    const size_t pl = ph_lds(A, rpb != nullptr);
    if (pl == 0) return false;
    PhMap M;
    PhUnits U;
    ph_maps(A, &M, &U);
    const dim3 pg((unsigned)((A.n_rows + kPhBlock - 1) / kPhBlock));
#define R1PD_(KK, NC)                                                                \
  hipLaunchKernelGGL((k_r1p_dot<KK, NC>), pg, dim3(kPhBlock), pl, st, A, M, U, x, y, \
                     rpb, out, scale_x)
    switch (A.D / 4) {
#define NC_ 1
      case 1: R1_K(A.K0, R1PD_) break;
#undef NC_
#define NC_ 2
      case 2: R1_K(A.K0, R1PD_) break;
#undef NC_
#define NC_ 3
      case 3: R1_K(A.K0, R1PD_) break;
#undef NC_
#define NC_ 4
      default: R1_K(A.K0, R1PD_) break;
#undef NC_
    }
#undef R1PD_
    return true;
  }
  const dim3 grid((unsigned)((A.n_rows + rb - 1) / rb));
#define R1D_(KK, NC)                                                           \
  hipLaunchKernelGGL((k_r1_dot<KK, NC>), grid, dim3(rb), lds, st, A, x, y, rpb, \
                     out, scale_x)
  switch (A.D / 4) {
#define NC_ 1
    case 1: R1_K(A.K0, R1D_) break;
#undef NC_
#define NC_ 2
    case 2: R1_K(A.K0, R1D_) break;
#undef NC_
#define NC_ 3
    case 3: R1_K(A.K0, R1D_) break;
#undef NC_
#define NC_ 4
    default: R1_K(A.K0, R1D_) break;
#undef NC_
  }
#undef R1D_
  return true;
}

// The rank-1 fp32 gather: the staged contiguous kernel, else the
// phase-major one; with bpart also the bias gradient's partials (*nblk: the
// blocks, one partial each).  False where neither applies.
bool r1_gather(const RpbProb &A, const float *w, const float *y, float *out,
               float post, hipStream_t st, double *bpart = nullptr, int *nblk = nullptr) {
  const int rb = rpb_block(A);
  size_t lds = r1_lds(A, rb, false);
  if (bpart != nullptr) lds = r1_bias_gather_lds(A);
  if (lds == 0) {
    const size_t pl = bpart != nullptr ? ph_bias_gather_lds(A) : ph_lds(A, false);
    if (pl == 0) return false;
    PhMap M;
    PhUnits U;
    ph_maps(A, &M, &U);
    const dim3 pg((unsigned)((A.n_rows + kPhBlock - 1) / kPhBlock));
    if (nblk != nullptr) *nblk = (int)pg.x;
#define R1PG_(KK, NC)                                                                \
  hipLaunchKernelGGL((k_r1p_gather<KK, NC>), pg, dim3(kPhBlock), pl, st, A, M, U, w, \
                     y, out, post, bpart)
    switch (A.D / 4) {
#define NC_ 1
      case 1: R1_K(A.K0, R1PG_) break;
#undef NC_
#define NC_ 2
      case 2: R1_K(A.K0, R1PG_) break;
#undef NC_
#define NC_ 3
      case 3: R1_K(A.K0, R1PG_) break;
#undef NC_
#define NC_ 4
      default: R1_K(A.K0, R1PG_) break;
#undef NC_
    }
#undef R1PG_
    return true;
  }
  const dim3 grid((unsigned)((A.n_rows + rb - 1) / rb));
  if (nblk != nullptr) *nblk = (int)grid.x;
#define R1G_(KK, NC)                                                              \
  hipLaunchKernelGGL((k_r1_gather<KK, NC>), grid, dim3(rb), lds, st, A, w, y, out, post, \
                     bpart)
  switch (A.D / 4) {
#define NC_ 1
    case 1: R1_K(A.K0, R1G_) break;
#undef NC_
#define NC_ 2
    case 2: R1_K(A.K0, R1G_) break;
#undef NC_
#define NC_ 3
    case 3: R1_K(A.K0, R1G_) break;
#undef NC_
#define NC_ 4
    default: R1_K(A.K0, R1G_) break;
#undef NC_
  }
#undef R1G_
  return true;
}

// The rank-1 fp32 inverse (dk / dv) where the staged dot / gather apply.
bool r1p_inverse(const RpbProb &A, const float *w, const float *x, float *out,
                 float post, hipStream_t st) {
  int cap = 0;
  const size_t lds = ph_inverse_lds(A, &cap);
  if (lds == 0) return false;
  PhMap M;
  PhUnits U;
  ph_maps(A, &M, &U);
  const dim3 pg((unsigned)((A.n_rows + kPhBlock - 1) / kPhBlock));
#define R1PI_(KK, NC)                                                                  \
  hipLaunchKernelGGL((k_r1p_inverse<KK, NC>), pg, dim3(kPhBlock), lds, st, A, M, U, w, \
                     x, out, post, cap)
  switch (A.D / 4) {
#define NC_ 1
    case 1: R1_K(A.K0, R1PI_) break;
#undef NC_
#define NC_ 2
    case 2: R1_K(A.K0, R1PI_) break;
#undef NC_
#define NC_ 3
    case 3: R1_K(A.K0, R1PI_) break;
#undef NC_
#define NC_ 4
    default: R1_K(A.K0, R1PI_) break;
#undef NC_
  }
#undef R1PI_
  return true;
}

bool r1_inverse(const RpbProb &A, const float *w, const float *x, float *out,
                float post, hipStream_t st) {
  const int rb = rpb_block(A);
  const size_t lds = r1_inverse_lds(A);
  if (lds == 0) return false;
  const dim3 grid((unsigned)((A.n_rows + rb - 1) / rb));
#define R1I_(KK, NC)                                                              \
  do {                                                                            \
    if (A.d0 == 1)                                                                \
      hipLaunchKernelGGL((k_r1_inverse<KK, NC, true>), grid, dim3(rb), lds, st, A, \
                         w, x, out, post);                                        \
    else                                                                          \
      hipLaunchKernelGGL((k_r1_inverse<KK, NC, false>), grid, dim3(rb), lds, st,   \
                         A, w, x, out, post);                                     \
  } while (0)
  switch (A.D / 4) {
#define NC_ 1
    case 1: R1_K(A.K0, R1I_) break;
#undef NC_
#define NC_ 2
    case 2: R1_K(A.K0, R1I_) break;
#undef NC_
#define NC_ 3
    case 3: R1_K(A.K0, R1I_) break;
#undef NC_
#define NC_ 4
    default: R1_K(A.K0, R1I_) break;
#undef NC_
  }
#undef R1I_
  return true;
}
#undef R1_K

// The QK / AV backward's two passes in one launch (k_r1_qkb / k_r1_avb)
// where both run on the staged rank-1 fp32 kernels; false otherwise.
#define R1_KD(KK_, BODY)                 \
  switch (KK_) {                         \
    case 3: BODY(3); break;              \
    case 5: BODY(5); break;              \
    case 7: BODY(7); break;              \
    case 9: BODY(9); break;              \
    case 11: BODY(11); break;            \
    default: BODY(13); break;            \
  }
size_t ph_inverse_lds(const RpbProb &A, int *cap);

bool r1_qk_bwd_fused(const RpbProb &A, const float *dl, const float *q, const float *key,
                     float *dq, float *dk, double *bpart, hipStream_t st) {
  if (pair_launch_off()) return false;
  if ((phase_inverse_first(A, true) || phase_pair_first(A, true)) &&
      ph_inverse_lds(A, nullptr) != 0)
    return false;
  const int rb = qkb_block(A);
  const size_t lg = bpart != nullptr ? r1_bias_gather_lds(A, rb) : r1_lds(A, rb, false);
  const size_t li = r1_inverse_lds(A, rb);
  // the pair shares one LDS size: an inverse above 64 KB would hold the
  // gather's blocks to two per CU too (K = 7, d = 4: 26.4 us as two
  // launches, 29.9 us as one)
  if (lg == 0 || li == 0 || li > 65536) return false;
  const int n0 = (A.n_rows + rb - 1) / rb;
  const dim3 grid((unsigned)(2 * n0)), block(rb);
  const size_t lds = std::max(lg, li);
  const float post = A.has_scale ? A.scale : 1.f;
#define QKB_(KK, NC)                                                                   \
  do {                                                                                 \
    if (A.d0 == 1)                                                                     \
      hipLaunchKernelGGL((k_r1_qkb<KK, NC, true>), grid, block, lds, st, A, dl, q, key, \
                         dq, dk, post, bpart, n0);                                     \
    else                                                                               \
      hipLaunchKernelGGL((k_r1_qkb<KK, NC, false>), grid, block, lds, st, A, dl, q, key, \
                         dq, dk, post, bpart, n0);                                     \
  } while (0)
#define QKB_NC(KK)                                  \
  do {                                              \
    if (A.D == 4) QKB_(KK, 1);                      \
    else if (A.D == 8) QKB_(KK, 2);                 \
    else if (A.D == 12) QKB_(KK, 3);                \
    else QKB_(KK, 4);                               \
  } while (0)
  R1_KD(A.K0, QKB_NC);
#undef QKB_NC
#undef QKB_
  return true;
}

bool r1_av_bwd_fused(const RpbProb &A, const float *attn, const float *v, const float *dout,
                     float *dattn, float *dv, hipStream_t st) {
  if ((phase_inverse_first(A, false) || phase_pair_first(A, false)) &&
      ph_inverse_lds(A, nullptr) != 0)
    return false;
  if (pair_launch_off()) return false;
  const int rb = avb_block(A);
  const size_t ld = r1_lds(A, rb, false);
  const size_t li = r1_inverse_lds(A, rb);
  if (ld == 0 || li == 0) return false;
  const int n0 = (A.n_rows + rb - 1) / rb;
  const dim3 grid((unsigned)(2 * n0)), block(rb);
  const size_t lds = std::max(ld, li);
#define AVB_(KK, NC)                                                                   \
  do {                                                                                 \
    if (A.d0 == 1)                                                                     \
      hipLaunchKernelGGL((k_r1_avb<KK, NC, true>), grid, block, lds, st, A, attn, v,    \
                         dout, dattn, dv, n0);                                         \
    else                                                                               \
      hipLaunchKernelGGL((k_r1_avb<KK, NC, false>), grid, block, lds, st, A, attn, v,   \
                         dout, dattn, dv, n0);                                         \
  } while (0)
#define AVB_NC(KK)                                  \
  do {                                              \
    if (A.D == 4) AVB_(KK, 1);                      \
    else if (A.D == 8) AVB_(KK, 2);                 \
    else if (A.D == 12) AVB_(KK, 3);                \
    else AVB_(KK, 4);                               \
  } while (0)
  R1_KD(A.K0, AVB_NC);
#undef AVB_NC
#undef AVB_
  return true;
}

// The same pairs on the phase-major kernels (k_r1p_qkb / k_r1p_avb): where
// the first pass (dq's gather, dattn's dot) is phase-major, because the
// staged one does not apply, and the inverse is phase-major too.  Both
// halves run kPhBlock-row blocks, so the launch is two equal halves.
bool r1p_pair_lds(const RpbProb &A, bool qk, size_t first, size_t *lds, int *cap) {
  if (pair_launch_off() || first == 0) return false;
  const bool phase_inv =
      phase_pair_first(A, qk) || phase_inverse_first(A, qk) || r1_inverse_lds(A) == 0;
  const size_t li = ph_inverse_lds(A, cap);
  if (!phase_inv || li == 0) return false;
  *lds = std::max(first, li);
  return true;
}

bool r1p_qk_bwd_pair(const RpbProb &A, const float *dl, const float *q, const float *key,
                     float *dq, float *dk, double *bpart, hipStream_t st) {
  const bool staged = bpart != nullptr ? r1_bias_gather_lds(A) != 0
                                       : r1_lds(A, rpb_block(A), false) != 0;
  if (staged && !phase_pair_first(A, true)) return false;
  size_t lds = 0;
  int cap = 0;
  if (!r1p_pair_lds(A, true, bpart != nullptr ? ph_bias_gather_lds(A) : ph_lds(A, false),
                    &lds, &cap))
    return false;
  PhMap M;
  PhUnits U;
  ph_maps(A, &M, &U);
  const int n0 = (A.n_rows + kPhBlock - 1) / kPhBlock;
  const float post = A.has_scale ? A.scale : 1.f;
#define QKP_(KK, NC)                                                                    \
  hipLaunchKernelGGL((k_r1p_qkb<KK, NC>), dim3((unsigned)(2 * n0)), dim3(kPhBlock), lds, \
                     st, A, M, U, dl, q, key, dq, dk, post, bpart, n0, cap)
#define QKP_NC(KK)                \
  do {                            \
    if (A.D == 4) QKP_(KK, 1);    \
    else if (A.D == 8) QKP_(KK, 2); \
    else if (A.D == 12) QKP_(KK, 3); \
    else QKP_(KK, 4);             \
  } while (0)
  R1_KD(A.K0, QKP_NC);
#undef QKP_NC
#undef QKP_
  return true;
}

bool r1p_av_bwd_pair(const RpbProb &A, const float *attn, const float *v, const float *dout,
                     float *dattn, float *dv, hipStream_t st) {
  if (r1_lds(A, rpb_block(A), false) != 0 && !phase_pair_first(A, false)) return false;
  size_t lds = 0;
  int cap = 0;
  if (!r1p_pair_lds(A, false, ph_lds(A, false), &lds, &cap)) return false;
  PhMap M;
  PhUnits U;
  ph_maps(A, &M, &U);
  const int n0 = (A.n_rows + kPhBlock - 1) / kPhBlock;
#define AVP_(KK, NC)                                                                    \
  hipLaunchKernelGGL((k_r1p_avb<KK, NC>), dim3((unsigned)(2 * n0)), dim3(kPhBlock), lds, \
                     st, A, M, U, attn, v, dout, dattn, dv, n0, cap)
#define AVP_NC(KK)                \
  do {                            \
    if (A.D == 4) AVP_(KK, 1);    \
    else if (A.D == 8) AVP_(KK, 2); \
    else if (A.D == 12) AVP_(KK, 3); \
    else AVP_(KK, 4);             \
  } while (0)
  R1_KD(A.K0, AVP_NC);
#undef AVP_NC
#undef AVP_
  return true;
}
#undef R1_KD

template <typename TX, typename TY>
void launch_dot(const RpbProb &A, const void *x, const void *y,
                const float *rpb, float *out, int scale_x, float fill,
                hipStream_t st) {
  if constexpr (sizeof(TX) == 4 && sizeof(TY) == 4) {
    if (r1_dot(A, (const float *)x, (const float *)y, rpb, out, scale_x, st)) return;
  }
  constexpr int V = vmax_of<TX, TY>();
  const RShape s = rshape(A.D, V);
  const int rb = rpb_block(A);
  const size_t lds = stage_bytes(A, s.lgG, rb);
  const int staged = lds > 0;
  const size_t wb = window_bytes<TY>(A, s.lgG, lds, rb);
  // the bias table in LDS after the slot rows and the window (float index)
  const size_t nbias = rpb != nullptr ? (size_t)A.H * A.R0 * A.R1 : 0;
  const size_t bb = nbias > 0 && nbias * 4 <= 16384 ? nbias * 4 : 0;
  const int bias_lds = bb > 0 ? (int)((lds + wb + 15) / 16 * 4) : 0;
  const size_t total = bb > 0 ? (size_t)bias_lds * 4 + bb : lds + wb;
#define DOT_(VV, YS)                                                          \
  hipLaunchKernelGGL((k_rpb_dot<TX, TY, VV, YS>), rgrid(A, s.lgG, rb), dim3(rb), \
                     total, st, A, (const TX *)x, (const TY *)y, rpb, out,     \
                     scale_x, fill, staged, s.G, s.lgG, bias_lds)
  if (s.vec == V) {
    if (wb > 0) DOT_(V, true); else DOT_(V, false);
  } else {
    if (wb > 0) DOT_(1, true); else DOT_(1, false);
  }
#undef DOT_
}

template <typename TY, typename TO>
void launch_gather(const RpbProb &A, const float *w, const void *y, void *out,
                   float post, hipStream_t st) {
  if constexpr (sizeof(TY) == 4 && sizeof(TO) == 4) {
    if (r1_gather(A, w, (const float *)y, (float *)out, post, st)) return;
  }
  constexpr int V = vmax_of<TY, TO>();
  const RShape s = rshape(A.D, V);
  const int rb = rpb_block(A);
  const size_t lds = stage_bytes(A, s.lgG, rb);
  const int staged = lds > 0;
  const size_t wb = window_bytes<TY>(A, s.lgG, lds, rb);
#define GAT_(VV, YS)                                                          \
  hipLaunchKernelGGL((k_rpb_gather<TY, TO, VV, YS>), rgrid(A, s.lgG, rb),     \
                     dim3(rb), lds + wb, st, A, w, (const TY *)y, (TO *)out,   \
                     post, staged, s.G, s.lgG)
  if (s.vec == V) {
    if (wb > 0) GAT_(V, true); else GAT_(V, false);
  } else {
    if (wb > 0) GAT_(1, true); else GAT_(1, false);
  }
#undef GAT_
}

template <typename TX, typename TO>
void launch_inverse(const RpbProb &A, const float *w, const void *x, void *out,
                    int scale_x, hipStream_t st, bool qk) {
  if constexpr (sizeof(TX) == 4 && sizeof(TO) == 4) {
    // fp32 x: x scale is exact up to rounding, so the scale is applied to
    // the sums instead
    const float post = scale_x ? A.scale : 1.f;
    if (phase_inverse_first(A, qk) && r1p_inverse(A, w, (const float *)x, (float *)out, post, st))
      return;
    if (r1_inverse(A, w, (const float *)x, (float *)out, post, st)) return;
    if (r1p_inverse(A, w, (const float *)x, (float *)out, post, st)) return;
  }
  constexpr int V = vmax_of<TX, TO>();
  const RShape s = rshape(A.D, V);
  if (s.vec == V)
    hipLaunchKernelGGL((k_rpb_inverse<TX, TO, V>), rgrid(A, s.lgG), dim3(256),
                       0, st, A, w, (const TX *)x, (TO *)out, scale_x, s.G,
                       s.lgG);
  else
    hipLaunchKernelGGL((k_rpb_inverse<TX, TO, 1>), rgrid(A, s.lgG), dim3(256),
                       0, st, A, w, (const TX *)x, (TO *)out, scale_x, s.G,
                       s.lgG);
}

// Calls f(T{}) with the storage type of dtype code dt.
template <typename F>
void with_dtype(int dt, F &&f) {
  if (dt == NA_F32)
    f(float{});
  else if (dt == NA_F16)
    f(f16_t{});
  else
    f(bf16_t{});
}

// Queries per bias-gradient partial (one pass-1 block each).
void bias_chunking(const RpbProb &A, int32_t *chunk, int32_t *n_chunks) {
  const int64_t nq = (int64_t)A.B * A.L0 * A.L1;
  *chunk = kBiasChunk;
  *n_chunks = (int32_t)((nq + kBiasChunk - 1) / kBiasChunk);
}

}  // namespace

void rpb_qk_fwd(const RpbProb &A, int dtype, const void *q, const void *key,
                const float *rpb, float *logits, hipStream_t st) {
  with_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    launch_dot<T, T>(A, q, key, rpb, logits, A.has_scale, -INFINITY, st);
  });
}

void rpb_av_fwd(const RpbProb &A, int dtype, int out_dtype, const float *attn,
                const void *value, void *out, hipStream_t st) {
  with_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    if (out_dtype == NA_F32)
      launch_gather<T, float>(A, attn, value, out, 1.f, st);
    else
      launch_gather<T, T>(A, attn, value, out, 1.f, st);
  });
}

size_t rpb_bias_workspace_bytes(const RpbProb &A) {
  int32_t chunk, n_chunks;
  bias_chunking(A, &chunk, &n_chunks);
  const size_t nb = (size_t)A.H * A.R0 * A.R1;
  return (size_t)n_chunks * nb * sizeof(double);
}

void rpb_qk_bwd(const RpbProb &A, int dtype, const void *q, const void *key,
                const float *dlogits, void *dq, void *dk, float *drpb,
                void *workspace, hipStream_t st) {
  int32_t chunk, n_chunks;
  bias_chunking(A, &chunk, &n_chunks);
  // fp32 rank 1 on the staged kernels: the dq pass also writes the bias
  // gradient's partials, one per block (when they fit the workspace)
  int32_t n_fused = 0;
  bool pair = false;  // dq and dk in one launch
  if (dq != nullptr && dk != nullptr && dtype == NA_F32 && A.n_rows > 0) {
    const int32_t nblk = (A.n_rows + qkb_block(A) - 1) / qkb_block(A);
    const bool bias = drpb != nullptr && nblk <= n_chunks;
    if ((drpb == nullptr || bias) &&
        r1_qk_bwd_fused(A, dlogits, (const float *)q, (const float *)key, (float *)dq,
                        (float *)dk, bias ? (double *)workspace : nullptr, st)) {
      pair = true;
      if (bias) n_fused = nblk;
    }
    const int32_t nph = (A.n_rows + kPhBlock - 1) / kPhBlock;
    const bool pbias = drpb != nullptr && nph <= n_chunks;
    if (!pair && (drpb == nullptr || pbias) &&
        r1p_qk_bwd_pair(A, dlogits, (const float *)q, (const float *)key, (float *)dq,
                        (float *)dk, pbias ? (double *)workspace : nullptr, st)) {
      pair = true;
      if (pbias) n_fused = nph;
    }
  }
  if (!pair && drpb != nullptr && dq != nullptr && dtype == NA_F32 && A.n_rows > 0) {
    // the staged gather's blocks, or the phase-major one's
    const int32_t nblk = r1_bias_gather_lds(A) != 0
                             ? (A.n_rows + rpb_block(A) - 1) / rpb_block(A)
                             : (A.n_rows + kPhBlock - 1) / kPhBlock;
    int used = 0;
    if (nblk <= n_chunks &&
        r1_gather(A, dlogits, (const float *)key, (float *)dq, A.has_scale ? A.scale : 1.f,
                  st, (double *)workspace, &used))
      n_fused = used;
  }
  with_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    if (A.n_rows == 0 || pair) return;
    if (dq != nullptr && n_fused == 0)
      launch_gather<T, T>(A, dlogits, key, dq, A.has_scale ? A.scale : 1.f,
                          st);
    if (dk != nullptr) launch_inverse<T, T>(A, dlogits, q, dk, A.has_scale, st, true);
  });
  if (drpb != nullptr && n_fused > 0) {
    hipLaunchKernelGGL(k_rpb_bias_reduce, dim3((unsigned)(A.H * A.R0 * A.R1)), dim3(64), 0,
                       st, (const double *)workspace, n_fused, drpb);
  } else if (drpb != nullptr) {
    const int32_t nb = A.H * A.R0 * A.R1;
    // per-(query, head) bin cells in LDS when they fit 32 KB
    const size_t sbytes = (size_t)chunk * nb * sizeof(float);
    const int scatter = sbytes <= 32768;
    if (n_chunks > 0)
      hipLaunchKernelGGL(k_rpb_bias_partial, dim3((unsigned)n_chunks), dim3(256),
                         scatter ? sbytes : 0, st, A, dlogits, (double *)workspace, chunk,
                         n_chunks, scatter);
    hipLaunchKernelGGL(k_rpb_bias_reduce, dim3((unsigned)nb), dim3(64), 0, st,
                       (const double *)workspace, n_chunks, drpb);
  }
}

void rpb_plan(const RpbProb &A, int dtype, RpbPlanInfo *o) {
  // the rank-1 fp32 kernels take float inputs and outputs only
  const bool f32 = dtype == NA_F32;
  auto kind = [&](bool bias) { return f32 ? (int)r1_kind(A, bias) : 0; };
  o->qk = kind(true);
  o->av = kind(false);
  o->dattn = kind(false);
  const bool phinv = f32 && ph_inverse_lds(A, nullptr) != 0;
  const bool pairs = !pair_launch_off();
  auto inv_kind = [&](bool qk) {
    return phinv && (phase_inverse_first(A, qk) || (pairs && phase_pair_first(A, qk)))
               ? (int)kR1Phase
           : f32 && r1_inverse_lds(A) != 0     ? (int)kR1Staged
           : phinv                             ? (int)kR1Phase
                                               : 0;
  };
  o->dk = inv_kind(true);
  o->dv = inv_kind(false);
  int32_t chunk, n_chunks;
  bias_chunking(A, &chunk, &n_chunks);
  const int rb = rpb_block(A);
  const int64_t nblk = ((int64_t)A.n_rows + rb - 1) / rb;
  const int64_t nph = ((int64_t)A.n_rows + kPhBlock - 1) / kPhBlock;
  // the QK backward's phase-major pair takes dq (and the partials) where it
  // goes first
  const bool ppair = f32 && phinv && pairs && phase_pair_first(A, true) &&
                     ph_bias_gather_lds(A) != 0 && nph <= n_chunks;
  if (f32 && phinv && pairs && phase_pair_first(A, false) && ph_lds(A, false) != 0)
    o->dattn = (int)kR1Phase;  // the AV backward's phase-major pair
  const bool staged_bias = !ppair && r1_bias_gather_lds(A) != 0;
  const bool phase_bias = !staged_bias && ph_bias_gather_lds(A) != 0;
  o->fused_bias = f32 && A.n_rows > 0 &&
                  ((staged_bias && nblk <= n_chunks) || (phase_bias && nph <= n_chunks));
  o->dq = o->fused_bias ? (staged_bias ? (int)kR1Staged : (int)kR1Phase) : kind(false);
  o->block = o->qk == kR1Phase ? kPhBlock : rb;
}

void rpb_av_bwd(const RpbProb &A, int dtype, int out_dtype, const float *attn,
                const void *value, const void *dout, float *dattn, void *dvalue,
                hipStream_t st) {
  // fp32 (dout fp32 whatever out_dtype): dattn and dv in one launch
  if (dtype == NA_F32 && dattn != nullptr && dvalue != nullptr && A.n_rows > 0 &&
      (r1_av_bwd_fused(A, attn, (const float *)value, (const float *)dout, dattn,
                       (float *)dvalue, st) ||
       r1p_av_bwd_pair(A, attn, (const float *)value, (const float *)dout, dattn,
                       (float *)dvalue, st)))
    return;
  with_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    if (out_dtype == NA_F32) {
      if (dattn != nullptr)
        launch_dot<float, T>(A, dout, value, nullptr, dattn, 0, 0.f, st);
      if (dvalue != nullptr)
        launch_inverse<float, T>(A, attn, dout, dvalue, 0, st, false);
    } else {
      if (dattn != nullptr)
        launch_dot<T, T>(A, dout, value, nullptr, dattn, 0, 0.f, st);
      if (dvalue != nullptr) launch_inverse<T, T>(A, attn, dout, dvalue, 0, st, false);
    }
  });
}

}  // namespace na
