// na_rpb.hip — DiNAT all-in-one operators: QK with relative position bias
// and AV over a square window (side K, uniform dilation) on one or two
// spatial axes, forward and backward (reference extras/allin1).
//
// Window of a query on an axis: slot k holds key s + k*dil with s the
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

constexpr int kNT = 4;  // element chunks per lane

struct RPos {
  int32_t b, h, i0, i1;
};

__device__ __forceinline__ RPos rpos(const RpbProb &A, uint32_t r) {
  RPos p;
  if (A.heads_first) {
    p.i1 = (int32_t)(r % (uint32_t)A.L1);
    r /= (uint32_t)A.L1;
    p.i0 = (int32_t)(r % (uint32_t)A.L0);
    r /= (uint32_t)A.L0;
    p.h = (int32_t)(r % (uint32_t)A.H);
    p.b = (int32_t)(r / (uint32_t)A.H);
  } else {
    p.h = (int32_t)(r % (uint32_t)A.H);
    r /= (uint32_t)A.H;
    p.i1 = (int32_t)(r % (uint32_t)A.L1);
    r /= (uint32_t)A.L1;
    p.i0 = (int32_t)(r % (uint32_t)A.L0);
    p.b = (int32_t)(r / (uint32_t)A.L0);
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

__device__ __forceinline__ RWin rwin(int32_t i, int32_t L, int32_t K,
                                     int32_t dil) {
  RWin w;
  w.s = window_start_partition(i, L, K, K / 2, dil);
  w.e = window_end(w.s, L, K, dil);
  w.pb = pb_start(i, L, K, K / 2, dil);
  return w;
}

// Axis-1 window (a single always-valid slot for rank 1).
__device__ __forceinline__ RWin rwin1(const RpbProb &A, int32_t i1) {
  if (A.rank == 2) return rwin(i1, A.L1, A.K, A.dil);
  return RWin{0, 1, 0};
}

__device__ __forceinline__ int32_t clampi(int32_t x, int32_t lo, int32_t hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}

__device__ __forceinline__ int32_t bias_index(const RpbProb &A, int32_t h,
                                              int32_t r0, int32_t r1) {
  const int32_t a = h * A.R + clampi(r0, 0, A.R - 1);
  return A.rank == 2 ? a * A.R + clampi(r1, 0, A.R - 1) : a;
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

// ---- kernels ---------------------------------------------------------------

// out[r, n] = <x'[r], y[nbr(r, n)]> (+ bias) for valid slots, `fill` for
// invalid ones; x' = round(x * scale) when scale_x.  QK+RPB forward
// (x = q, y = key, fill = -inf) and the AV backward's dattn (x = dout,
// y = value, no bias, fill = 0).
template <typename TX, typename TY, int VEC>
__global__ void __launch_bounds__(256)
    k_rpb_dot(RpbProb A, const TX *__restrict__ x, const TY *__restrict__ y,
              const float *__restrict__ rpb, float *__restrict__ out,
              int scale_x, float fill, int G, int lgG) {
  const Group g = make_group(lgG, A.n_rows);
  const RPos p = rpos(A, (uint32_t)g.id);
  float xv[kNT][VEC];
  ld_row<TX, VEC>(xv, x + g.id * A.D, g.lane, G, A.D);
  if (scale_x) scale_round<TX, VEC>(xv, A.scale);
  const RWin w0 = rwin(p.i0, A.L0, A.K, A.dil);
  const RWin w1 = rwin1(A, p.i1);
  float *dst = out + g.id * A.KK;
  int n = 0;
  for (int k0 = 0; k0 < A.K; ++k0) {
    const int32_t j0 = w0.s + k0 * A.dil;
    const bool v0 = j0 >= 0 && j0 < w0.e;
    for (int k1 = 0; k1 < A.K1; ++k1, ++n) {
      const int32_t j1 = w1.s + k1 * A.dil;
      float s = fill;
      if (v0 && j1 >= 0 && j1 < w1.e) {
        const TY *yr = y + rrow(A, p.b, p.h, j0, j1) * A.D;
        s = group_sum(dot_row<TY, VEC>(xv, yr, g.lane, G, A.D), G);
        if (rpb != nullptr) s += rpb[bias_index(A, p.h, w0.pb + k0, w1.pb + k1)];
      }
      if (g.live && g.lane == 0) dst[n] = s;
    }
  }
}

// out[r] = post * sum_n w[r, n] * y[nbr(r, n)] over valid slots.  AV
// forward (w = attn, y = value) and the QK backward's dq (w = dlogits,
// y = key, post = the query scale).
template <typename TY, typename TO, int VEC>
__global__ void __launch_bounds__(256)
    k_rpb_gather(RpbProb A, const float *__restrict__ w,
                 const TY *__restrict__ y, TO *__restrict__ out, float post,
                 int G, int lgG) {
  const Group g = make_group(lgG, A.n_rows);
  const RPos p = rpos(A, (uint32_t)g.id);
  const RWin w0 = rwin(p.i0, A.L0, A.K, A.dil);
  const RWin w1 = rwin1(A, p.i1);
  const float *wr = w + g.id * A.KK;
  float acc[kNT][VEC];
#pragma unroll
  for (int t = 0; t < kNT; ++t)
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[t][e] = 0.f;
  int n = 0;
  for (int k0 = 0; k0 < A.K; ++k0) {
    const int32_t j0 = w0.s + k0 * A.dil;
    const bool v0 = j0 >= 0 && j0 < w0.e;
    for (int k1 = 0; k1 < A.K1; ++k1, ++n) {
      const int32_t j1 = w1.s + k1 * A.dil;
      if (v0 && j1 >= 0 && j1 < w1.e)
        axpy_row<TY, VEC>(acc, wr[n], y + rrow(A, p.b, p.h, j0, j1) * A.D,
                          g.lane, G, A.D);
    }
  }
  if (g.live) st_row<TO, VEC>(out + g.id * A.D, acc, post, g.lane, G, A.D);
}

// out[j] = sum over (r, n) with nbr(r, n) == j of w[r, n] * x'[r]: the
// transpose of k_rpb_gather, evaluated per key row.  A query i can hold key
// j only on j's dilation phase and within K*dil of it, so the candidates
// are i = j + t*dil, |t| <= K, kept when j lies in [start(i), end(i)).
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
  const int32_t t1max = A.rank == 2 ? A.K : 0;
  for (int32_t t0 = -A.K; t0 <= A.K; ++t0) {
    const int32_t i0 = p.i0 + t0 * A.dil;
    if (i0 < 0 || i0 >= A.L0) continue;
    const RWin w0 = rwin(i0, A.L0, A.K, A.dil);
    if (p.i0 < w0.s || p.i0 >= w0.e) continue;
    const int32_t k0 = (p.i0 - w0.s) / A.dil;
    for (int32_t t1 = -t1max; t1 <= t1max; ++t1) {
      const int32_t i1 = p.i1 + t1 * A.dil;
      if (i1 < 0 || i1 >= A.L1) continue;
      const RWin w1 = rwin1(A, i1);
      if (p.i1 < w1.s || p.i1 >= w1.e) continue;
      const int32_t k1 = (p.i1 - w1.s) / A.dil;
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

// Bias gradient, pass 1: partial[c, h, bin] = sum of dlogits over the
// queries of chunk c (rows in (b, i0, i1) order) and the slots whose
// clipped bias row is `bin`.  One thread per (c, h, bin), fixed order.
__global__ void __launch_bounds__(256)
    k_rpb_bias_partial(RpbProb A, const float *__restrict__ dl,
                       float *__restrict__ partial, int32_t chunk,
                       int32_t n_chunks) {
  const int32_t nb = A.rank == 2 ? A.R * A.R : A.R;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (int64_t)n_chunks * A.H * nb) return;
  const int32_t bin = (int32_t)(id % nb);
  const int32_t h = (int32_t)((id / nb) % A.H);
  const int32_t c = (int32_t)(id / ((int64_t)nb * A.H));
  const int32_t r0 = A.rank == 2 ? bin / A.R : bin;
  const int32_t r1 = A.rank == 2 ? bin % A.R : 0;
  const int32_t nq = A.B * A.L0 * A.L1;
  const int32_t q0 = c * chunk;
  const int32_t q1 = q0 + chunk < nq ? q0 + chunk : nq;
  float acc = 0.f;
  for (int32_t qi = q0; qi < q1; ++qi) {
    const int32_t i1 = qi % A.L1;
    const int32_t rest = qi / A.L1;
    const int32_t i0 = rest % A.L0;
    const int32_t b = rest / A.L0;
    const RWin w0 = rwin(i0, A.L0, A.K, A.dil);
    int32_t a0, b0;
    slots_of_bias_row(r0, w0.pb, A.K, A.R, &a0, &b0);
    if (a0 > b0) continue;
    const RWin w1 = rwin1(A, i1);
    int32_t a1 = 0, b1 = 0;
    if (A.rank == 2) slots_of_bias_row(r1, w1.pb, A.K, A.R, &a1, &b1);
    const float *row = dl + rrow(A, b, h, i0, i1) * A.KK;
    for (int32_t k0 = a0; k0 <= b0; ++k0) {
      const int32_t j0 = w0.s + k0 * A.dil;
      if (j0 < 0 || j0 >= w0.e) continue;
      for (int32_t k1 = a1; k1 <= b1; ++k1) {
        const int32_t j1 = w1.s + k1 * A.dil;
        if (j1 < 0 || j1 >= w1.e) continue;
        acc += row[k0 * A.K1 + k1];
      }
    }
  }
  partial[id] = acc;
}

// Bias gradient, pass 2: one wavefront per (h, bin) sums the chunk
// partials, lane l taking chunks l, l+64, ... and a fixed xor tree after.
__global__ void __launch_bounds__(64)
    k_rpb_bias_reduce(const float *__restrict__ partial, int32_t n_chunks,
                      int32_t n_out, float *__restrict__ drpb) {
  const int32_t o = blockIdx.x;
  const int lane = threadIdx.x;
  float acc = 0.f;
  for (int32_t c = lane; c < n_chunks; c += 64)
    acc += partial[(int64_t)c * n_out + o];
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) drpb[o] = acc;
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

dim3 rgrid(const RpbProb &A, int lgG) {
  const int64_t threads = (int64_t)A.n_rows << lgG;
  return dim3((unsigned)((threads + 255) / 256));
}

template <typename A_, typename B_>
constexpr int vmax_of() {
  return 16 / (int)(sizeof(A_) > sizeof(B_) ? sizeof(A_) : sizeof(B_));
}

template <typename TX, typename TY>
void launch_dot(const RpbProb &A, const void *x, const void *y,
                const float *rpb, float *out, int scale_x, float fill,
                hipStream_t st) {
  constexpr int V = vmax_of<TX, TY>();
  const RShape s = rshape(A.D, V);
  if (s.vec == V)
    hipLaunchKernelGGL((k_rpb_dot<TX, TY, V>), rgrid(A, s.lgG), dim3(256), 0,
                       st, A, (const TX *)x, (const TY *)y, rpb, out, scale_x,
                       fill, s.G, s.lgG);
  else
    hipLaunchKernelGGL((k_rpb_dot<TX, TY, 1>), rgrid(A, s.lgG), dim3(256), 0,
                       st, A, (const TX *)x, (const TY *)y, rpb, out, scale_x,
                       fill, s.G, s.lgG);
}

template <typename TY, typename TO>
void launch_gather(const RpbProb &A, const float *w, const void *y, void *out,
                   float post, hipStream_t st) {
  constexpr int V = vmax_of<TY, TO>();
  const RShape s = rshape(A.D, V);
  if (s.vec == V)
    hipLaunchKernelGGL((k_rpb_gather<TY, TO, V>), rgrid(A, s.lgG), dim3(256),
                       0, st, A, w, (const TY *)y, (TO *)out, post, s.G, s.lgG);
  else
    hipLaunchKernelGGL((k_rpb_gather<TY, TO, 1>), rgrid(A, s.lgG), dim3(256),
                       0, st, A, w, (const TY *)y, (TO *)out, post, s.G, s.lgG);
}

template <typename TX, typename TO>
void launch_inverse(const RpbProb &A, const float *w, const void *x, void *out,
                    int scale_x, hipStream_t st) {
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

// Chunk of queries per bias-gradient partial: about 2^18 threads in pass 1.
void bias_chunking(const RpbProb &A, int32_t *chunk, int32_t *n_chunks) {
  const int64_t nb = (int64_t)A.H * (A.rank == 2 ? A.R * A.R : A.R);
  const int64_t nq = (int64_t)A.B * A.L0 * A.L1;
  int64_t want = ((int64_t)1 << 18) / (nb > 0 ? nb : 1);
  if (want < 1) want = 1;
  int64_t c = (nq + want - 1) / want;
  if (c < 16) c = 16;
  *chunk = (int32_t)c;
  *n_chunks = (int32_t)((nq + c - 1) / c);
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
  const size_t nb = (size_t)A.H * (A.rank == 2 ? A.R * A.R : A.R);
  return (size_t)n_chunks * nb * sizeof(float);
}

void rpb_qk_bwd(const RpbProb &A, int dtype, const void *q, const void *key,
                const float *dlogits, void *dq, void *dk, float *drpb,
                float *workspace, hipStream_t st) {
  with_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    if (A.n_rows == 0) return;
    if (dq != nullptr)
      launch_gather<T, T>(A, dlogits, key, dq, A.has_scale ? A.scale : 1.f,
                          st);
    if (dk != nullptr) launch_inverse<T, T>(A, dlogits, q, dk, A.has_scale, st);
  });
  if (drpb != nullptr) {
    int32_t chunk, n_chunks;
    bias_chunking(A, &chunk, &n_chunks);
    const int32_t nb = A.H * (A.rank == 2 ? A.R * A.R : A.R);
    const int64_t n1 = (int64_t)n_chunks * nb;
    if (n1 > 0)
      hipLaunchKernelGGL(k_rpb_bias_partial,
                         dim3((unsigned)((n1 + 255) / 256)), dim3(256), 0, st,
                         A, dlogits, workspace, chunk, n_chunks);
    hipLaunchKernelGGL(k_rpb_bias_reduce, dim3((unsigned)nb), dim3(64), 0, st,
                       (const float *)workspace, n_chunks, nb, drpb);
  }
}

void rpb_av_bwd(const RpbProb &A, int dtype, int out_dtype, const float *attn,
                const void *value, const void *dout, float *dattn, void *dvalue,
                hipStream_t st) {
  with_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    if (out_dtype == NA_F32) {
      if (dattn != nullptr)
        launch_dot<float, T>(A, dout, value, nullptr, dattn, 0, 0.f, st);
      if (dvalue != nullptr)
        launch_inverse<float, T>(A, attn, dout, dvalue, 0, st);
    } else {
      if (dattn != nullptr)
        launch_dot<T, T>(A, dout, value, nullptr, dattn, 0, 0.f, st);
      if (dvalue != nullptr) launch_inverse<T, T>(A, attn, dout, dvalue, 0, st);
    }
  });
}

}  // namespace na
