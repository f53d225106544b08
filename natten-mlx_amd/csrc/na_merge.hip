// na_merge.hip — merge of attention outputs that share their queries, as if
// their key/value sets had been concatenated (reference merge.py:20-68).
//
// Per row r (every leading index of [..., D]) with part LSEs l_i:
//   L = logsumexp_i l_i,  w_i = exp(l_i - L),  out = sum_i w_i * out_i.
// This is the closed form of the reference's sequential sigmoid merge
// (out <- out - sigmoid(l_i - L)(out - out_i), L <- L - logsigmoid(L - l_i)),
// evaluated as max-shifted exponentials in fp32.  Backward, with
// p_i = <dOut, out_i> and dL the LSE cotangent:
//   dout_i = w_i * dOut,  dl_i = w_i * (p_i - sum_j w_j p_j + dL).
//
// Forward is one elementwise pass (16-byte accesses, every input read once,
// HBM-bound); backward is one pass with a lane group per row (the p_i are
// row dot products).  Part pointers travel in the kernel arguments.
#include "na_common.h"
#include "na_launch.h"
#include "na_row.h"

namespace na {
namespace {

struct MergeIn {
  const void *out[kMergeMaxParts];
  const float *lse[kMergeMaxParts];
};

struct MergeGrad {
  void *dout[kMergeMaxParts];
  float *dlse[kMergeMaxParts];
};

// w_i and L of row r over the first n parts (the loops are unrolled to the
// maximum so w stays in registers).
__device__ __forceinline__ float merge_weights(const MergeIn &S, int n,
                                               int64_t r,
                                               float (&w)[kMergeMaxParts]) {
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < kMergeMaxParts; ++i) {
    w[i] = i < n ? S.lse[i][r] : -INFINITY;
    m = fmaxf(m, w[i]);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kMergeMaxParts; ++i)
    if (i < n) s += exp2f((w[i] - m) * kLog2e);
  const float L = m + __log2f(s) * kLn2;
#pragma unroll
  for (int i = 0; i < kMergeMaxParts; ++i)
    w[i] = i < n ? exp2f((w[i] - L) * kLog2e) : 0.f;
  return L;
}

// One thread per VEC consecutive elements of a row (VEC divides D).  P2:
// D / VEC is 2^lg and the whole tensor has fewer than 2^31 such units, so
// the row index is a 32-bit shift (a 64-bit division by a runtime value is
// a long instruction sequence here, most of the kernel's work).
template <typename T, int VEC, bool P2>
__global__ void __launch_bounds__(256)
    k_merge_fwd(MergeIn S, int n, int64_t rows, int D, int lg, T *__restrict__ out,
                float *__restrict__ lse) {
  int64_t idx, r, per_row;
  if constexpr (P2) {
    const uint32_t i32 = blockIdx.x * blockDim.x + threadIdx.x;
    if ((int64_t)i32 >= (rows << lg)) return;
    idx = i32;
    r = i32 >> lg;
    per_row = (int64_t)1 << lg;
  } else {
    per_row = D / VEC;
    idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * per_row) return;
    r = idx / per_row;
  }
  const int64_t e0 = idx * VEC;  // == r * D + (idx - r * per_row) * VEC
  float w[kMergeMaxParts];
  const float L = merge_weights(S, n, r, w);
  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
#pragma unroll
  for (int i = 0; i < kMergeMaxParts; ++i) {
    if (i < n) {
      float x[VEC];
      VecIO<T, VEC>::load(static_cast<const T *>(S.out[i]) + e0, x);
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = fmaf(w[i], x[e], acc[e]);
    }
  }
  VecIO<T, VEC>::store_nt(out + e0, acc);
  if (idx == r * per_row) lse[r] = L;
}

// One lane group per row.
template <typename T, int VEC, int NT>
__global__ void __launch_bounds__(256)
    k_merge_bwd(MergeIn S, MergeGrad Gd, int n, int64_t rows, int D,
                const T *__restrict__ dout, const float *__restrict__ dlse,
                int G, int lgG) {
  const Group g = make_group(lgG, rows);
  const int64_t r = g.id;
  float w[kMergeMaxParts];
  merge_weights(S, n, r, w);
  Row<T, VEC, NT> d;
  d.load(dout + r * D, g.lane, G, D);
  float p[kMergeMaxParts];
  float pw = 0.f;
#pragma unroll
  for (int i = 0; i < kMergeMaxParts; ++i) {
    p[i] = 0.f;
    if (i < n) {
      p[i] = group_sum(
          d.dot_mem(static_cast<const T *>(S.out[i]) + r * D, g.lane, G, D), G);
      pw = fmaf(w[i], p[i], pw);
    }
  }
  const float dl = dlse != nullptr ? dlse[r] : 0.f;
  if (!g.live) return;
#pragma unroll
  for (int i = 0; i < kMergeMaxParts; ++i) {
    if (i >= n) continue;
    if (Gd.dout[i] != nullptr) {
      Row<T, VEC, NT> t = d;
      t.mul(w[i]);
      t.store_nt(static_cast<T *>(Gd.dout[i]) + r * D, g.lane, G, D);
    }
    if (Gd.dlse[i] != nullptr && g.lane == 0)
      Gd.dlse[i][r] = w[i] * (p[i] - pw + dl);
  }
}

template <typename T>
void merge_fwd_t(const MergeIn &S, int n, int64_t rows, int D, void *out,
                 float *lse, hipStream_t st) {
  constexpr int V = 16 / (int)sizeof(T);
  if (D % V == 0) {
    const int pr = D / V;
    const int64_t threads = rows * pr;
    int lg = 0;
    while ((1 << lg) < pr) ++lg;
    const dim3 grid((unsigned)((threads + 255) / 256));
    if ((1 << lg) == pr && threads + 255 < ((int64_t)1 << 31))
      hipLaunchKernelGGL((k_merge_fwd<T, V, true>), grid, dim3(256), 0, st, S, n, rows, D,
                         lg, (T *)out, lse);
    else
      hipLaunchKernelGGL((k_merge_fwd<T, V, false>), grid, dim3(256), 0, st, S, n, rows, D,
                         0, (T *)out, lse);
  } else {
    const int64_t threads = rows * D;
    hipLaunchKernelGGL((k_merge_fwd<T, 1, false>), dim3((unsigned)((threads + 255) / 256)),
                       dim3(256), 0, st, S, n, rows, D, 0, (T *)out, lse);
  }
}

template <typename T>
void merge_bwd_t(const MergeIn &S, const MergeGrad &Gd, int n, int64_t rows,
                 int D, const void *dout, const float *dlse, hipStream_t st) {
  const Shape s = pick_shape<T>(D);
#define L_(TT, V, N)                                                          \
  hipLaunchKernelGGL((k_merge_bwd<TT, V, N>), grid_for(rows, s.lgG),          \
                     dim3(256), 0, st, S, Gd, n, rows, D, (const TT *)dout,   \
                     dlse, s.G, s.lgG)
  NA_VALU_DISPATCH(T, s, L_);
#undef L_
}

}  // namespace

void merge_fwd(int dtype, int n, int64_t rows, int D, const void *const *outs,
               const float *const *lses, void *out, float *lse,
               hipStream_t st) {
  MergeIn S{};
  for (int i = 0; i < n; ++i) {
    S.out[i] = outs[i];
    S.lse[i] = lses[i];
  }
  NA_BY_DTYPE(dtype, merge_fwd_t, S, n, rows, D, out, lse, st);
}

void merge_bwd(int dtype, int n, int64_t rows, int D, const void *const *outs,
               const float *const *lses, const void *dout, const float *dlse,
               void *const *d_outs, float *const *d_lses, hipStream_t st) {
  MergeIn S{};
  MergeGrad Gd{};
  for (int i = 0; i < n; ++i) {
    S.out[i] = outs[i];
    S.lse[i] = lses[i];
    Gd.dout[i] = d_outs != nullptr ? d_outs[i] : nullptr;
    Gd.dlse[i] = d_lses != nullptr ? d_lses[i] : nullptr;
  }
  NA_BY_DTYPE(dtype, merge_bwd_t, S, Gd, n, rows, D, dout, dlse, st);
}

}  // namespace na
