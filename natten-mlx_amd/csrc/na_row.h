// na_row.h — lane-group row helpers shared by the vector-ALU kernels.
//
// One aligned group of G lanes (a power of two) owns one token row of D
// elements; each lane holds NT chunks of VEC consecutive elements, so a row
// is read with 16-byte accesses and dot products finish with a log2(G)-step
// xor shuffle (group_sum).  All arithmetic is fp32.
#pragma once
#include "na_common.h"

namespace na {

template <typename T, int VEC, int NT>
struct Row {
  float v[NT][VEC];

  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[t][e] = 0.f;
  }
  __device__ __forceinline__ void load(const T *row, int lane, int G, int D) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int d0 = (t * G + lane) * VEC;
      if (d0 < D) {
        VecIO<T, VEC>::load(row + d0, v[t]);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[t][e] = 0.f;
      }
    }
  }
  __device__ __forceinline__ void store(T *row, int lane, int G, int D) const {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int d0 = (t * G + lane) * VEC;
      if (d0 < D) VecIO<T, VEC>::store(row + d0, v[t]);
    }
  }
  __device__ __forceinline__ void store_nt(T *row, int lane, int G, int D) const {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int d0 = (t * G + lane) * VEC;
      if (d0 < D) VecIO<T, VEC>::store_nt(row + d0, v[t]);
    }
  }
  // load() without a branch: chunks past D read the row's last chunk and
  // are zeroed by selection, so a load issued ahead of its use stays where
  // it is issued (no branch for it to sink into).
  __device__ __forceinline__ void load_nb(const T *row, int lane, int G, int D) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int d0 = (t * G + lane) * VEC;
      float x[VEC];
      VecIO<T, VEC>::load(row + min(d0, D - VEC), x);
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[t][e] = d0 < D ? x[e] : 0.f;
    }
  }
  // this = this * a + w * o
  __device__ __forceinline__ void scale_add(float a, float w, const Row &o) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[t][e] = fmaf(v[t][e], a, w * o.v[t][e]);
  }
  // Partial dot product with a row in memory (lane-local part).
  __device__ __forceinline__ float dot_mem(const T *row, int lane, int G,
                                           int D) const {
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
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
  __device__ __forceinline__ float dot(const Row &o) const {
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc = fmaf(v[t][e], o.v[t][e], acc);
    return acc;
  }
  // this = this * a + w * row
  __device__ __forceinline__ void scale_add_mem(float a, float w, const T *row,
                                                int lane, int G, int D) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int d0 = (t * G + lane) * VEC;
      if (d0 < D) {
        float x[VEC];
        VecIO<T, VEC>::load(row + d0, x);
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[t][e] = fmaf(v[t][e], a, w * x[e]);
      }
    }
  }
  __device__ __forceinline__ void add_scaled(float w, const Row &o) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[t][e] = fmaf(w, o.v[t][e], v[t][e]);
  }
  __device__ __forceinline__ void mul(float a) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[t][e] *= a;
  }
};

struct Group {
  int64_t id;  // group index (clamped to a live group for idle lanes)
  int lane;
  bool live;
};

__device__ __forceinline__ Group make_group(int lgG, int64_t n_groups) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  Group g;
  g.id = gid >> lgG;
  g.lane = (int)(gid & ((1 << lgG) - 1));
  g.live = g.id < n_groups;
  if (!g.live) g.id = 0;  // idle lanes shadow group 0 and never store
  return g;
}

// ---- launch shape ----------------------------------------------------------
// 16-byte accesses when D allows, NT = 4 chunks per lane past 32 chunks, and
// the fewest lanes per row (a power of two) that cover D.
struct Shape {
  int vec, nt, G, lgG;
};

template <typename T>
Shape pick_shape(int D) {
  Shape s;
  const int vmax = 16 / (int)sizeof(T);
  s.vec = (D % vmax == 0) ? vmax : 1;
  const int chunks = (D + s.vec - 1) / s.vec;
  s.nt = chunks > 32 ? 4 : 1;
  const int per = (chunks + s.nt - 1) / s.nt;
  s.G = 1;
  s.lgG = 0;
  while (s.G < per) {
    s.G <<= 1;
    ++s.lgG;
  }
  return s;
}

inline dim3 grid_for(int64_t n_groups, int lgG) {
  const int64_t threads = n_groups << lgG;
  return dim3((unsigned)((threads + 255) / 256));
}

// Expands `body` with the compile-time (VEC, NT) matching shape s.
#define NA_VALU_DISPATCH(T, s, LAUNCH)                                  \
  do {                                                                  \
    constexpr int VMAX = 16 / (int)sizeof(T);                           \
    if ((s).vec == VMAX && (s).nt == 1) {                               \
      LAUNCH(T, VMAX, 1);                                               \
    } else if ((s).vec == VMAX) {                                       \
      LAUNCH(T, VMAX, 4);                                               \
    } else if ((s).nt == 1) {                                           \
      LAUNCH(T, 1, 1);                                                  \
    } else {                                                            \
      LAUNCH(T, 1, 4);                                                  \
    }                                                                   \
  } while (0)

// Calls FN<storage type of dtype code dt>(...).
#define NA_BY_DTYPE(dt, FN, ...)             \
  do {                                       \
    if ((dt) == NA_F32) {                    \
      FN<float>(__VA_ARGS__);                \
    } else if ((dt) == NA_F16) {             \
      FN<f16_t>(__VA_ARGS__);                \
    } else {                                 \
      FN<bf16_t>(__VA_ARGS__);               \
    }                                        \
  } while (0)

}  // namespace na
