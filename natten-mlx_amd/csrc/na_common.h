// na_common.h — problem descriptor, dtype conversion and vector I/O shared
// by every kernel of libnatten_amd.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "natten_amd.h"
#include "na_window.h"

namespace na {

// ---- storage types ---------------------------------------------------------
// bf16 is kept as raw 16-bit words; conversion is round-to-nearest-even.
struct bf16_t {
  uint16_t bits;
};
typedef _Float16 f16_t;

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(f16_t x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16_t x) {
  return __uint_as_float(((uint32_t)x.bits) << 16);
}

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) {
  return x;
}
template <>
__device__ __forceinline__ f16_t from_f32<f16_t>(float x) {
  return (f16_t)x;
}
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) {
  uint32_t u = __float_as_uint(x);
  bf16_t r;
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    r.bits = 0x7fc0;  // quiet NaN
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
    r.bits = (uint16_t)(u >> 16);
  }
  return r;
}

// Round a float to the storage precision of T and back.
template <typename T>
__device__ __forceinline__ float round_to(float x) {
  return to_f32(from_f32<T>(x));
}

// ---- vector I/O: VEC consecutive elements as one wide access ---------------
// store_nt: the same store, nontemporal (streaming) where the access is 16
// bytes, for output rows written in long contiguous runs (the merge
// kernels: two bf16 parts at config-3 size, forward 11.4 -> 10.7 us,
// backward 19.1 -> 17.4 us).  Scattered per-row stores stay ordinary: the
// allin1 backward's dk / dv rows ran 15.1 -> 17.1 us with them streaming.
template <typename T, int VEC>
struct VecIO;

template <typename T>
struct VecIO<T, 1> {
  static __device__ __forceinline__ void load(const T *p, float *o) {
    o[0] = to_f32(p[0]);
  }
  static __device__ __forceinline__ void store(T *p, const float *x) {
    p[0] = from_f32<T>(x[0]);
  }
  static __device__ __forceinline__ void store_nt(T *p, const float *x) { store(p, x); }
};

template <>
struct VecIO<float, 4> {
  static __device__ __forceinline__ void load(const float *p, float *o) {
    const float4 t = *reinterpret_cast<const float4 *>(p);
    o[0] = t.x;
    o[1] = t.y;
    o[2] = t.z;
    o[3] = t.w;
  }
  static __device__ __forceinline__ void store(float *p, const float *x) {
    *reinterpret_cast<float4 *>(p) = make_float4(x[0], x[1], x[2], x[3]);
  }
  static __device__ __forceinline__ void store_nt(float *p, const float *x) {
    typedef float f32v4 __attribute__((ext_vector_type(4)));
    const f32v4 v = {x[0], x[1], x[2], x[3]};
    __builtin_nontemporal_store(v, reinterpret_cast<f32v4 *>(p));
  }
};

template <typename T>
struct VecIO16x8 {  // 8 x 16-bit elements = one 16-byte access
  static __device__ __forceinline__ void load(const T *p, float *o) {
    const uint4 t = *reinterpret_cast<const uint4 *>(p);
    const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      T lo, hi;
      __builtin_memcpy(&lo, reinterpret_cast<const char *>(&w[i]), 2);
      __builtin_memcpy(&hi, reinterpret_cast<const char *>(&w[i]) + 2, 2);
      o[2 * i] = to_f32(lo);
      o[2 * i + 1] = to_f32(hi);
    }
  }
  static __device__ __forceinline__ void store(T *p, const float *x) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const T lo = from_f32<T>(x[2 * i]);
      const T hi = from_f32<T>(x[2 * i + 1]);
      uint16_t a, b;
      __builtin_memcpy(&a, &lo, 2);
      __builtin_memcpy(&b, &hi, 2);
      w[i] = (uint32_t)a | ((uint32_t)b << 16);
    }
    *reinterpret_cast<uint4 *>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  static __device__ __forceinline__ void store_nt(T *p, const float *x) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const T lo = from_f32<T>(x[2 * i]);
      const T hi = from_f32<T>(x[2 * i + 1]);
      uint16_t a, b;
      __builtin_memcpy(&a, &lo, 2);
      __builtin_memcpy(&b, &hi, 2);
      w[i] = (uint32_t)a | ((uint32_t)b << 16);
    }
    typedef unsigned int u32v4 __attribute__((ext_vector_type(4)));
    const u32v4 wv = {w[0], w[1], w[2], w[3]};
    __builtin_nontemporal_store(wv, reinterpret_cast<u32v4 *>(p));
  }
};
template <>
struct VecIO<bf16_t, 8> : VecIO16x8<bf16_t> {};
template <>
struct VecIO<f16_t, 8> : VecIO16x8<f16_t> {};

template <typename T>
struct VecIO16x4 {  // 4 x 16-bit elements = one 8-byte access
  static __device__ __forceinline__ void load(const T *p, float *o) {
    const uint2 t = *reinterpret_cast<const uint2 *>(p);
    const uint32_t w[2] = {t.x, t.y};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      T lo, hi;
      __builtin_memcpy(&lo, reinterpret_cast<const char *>(&w[i]), 2);
      __builtin_memcpy(&hi, reinterpret_cast<const char *>(&w[i]) + 2, 2);
      o[2 * i] = to_f32(lo);
      o[2 * i + 1] = to_f32(hi);
    }
  }
  static __device__ __forceinline__ void store(T *p, const float *x) {
    uint32_t w[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const T lo = from_f32<T>(x[2 * i]);
      const T hi = from_f32<T>(x[2 * i + 1]);
      uint16_t a, b;
      __builtin_memcpy(&a, &lo, 2);
      __builtin_memcpy(&b, &hi, 2);
      w[i] = (uint32_t)a | ((uint32_t)b << 16);
    }
    *reinterpret_cast<uint2 *>(p) = make_uint2(w[0], w[1]);
  }
  static __device__ __forceinline__ void store_nt(T *p, const float *x) { store(p, x); }
};
template <>
struct VecIO<bf16_t, 4> : VecIO16x4<bf16_t> {};
template <>
struct VecIO<f16_t, 4> : VecIO16x4<f16_t> {};

// ---- problem descriptor (kernel argument, passed by value) ------------------
struct Axis {
  int32_t L;       // tensor extent (maximum over samples for varlen)
  int32_t K;       // kernel size
  int32_t d;       // dilation
  int32_t s;       // stride
  int32_t causal;  // 0 / 1
  int32_t O;       // output extent ceil(L / s)
};

struct Prob {
  Axis ax[3];      // axis 0 outermost; unit axes pad rank < 3
  int32_t B, H, Hkv, D, rep;  // rep = H / Hkv
  int32_t rank;
  int32_t kprod;   // K0 * K1 * K2
  int32_t n_extra;
  int32_t dense;   // every query sees every key of its sample
  float scale;
  const int32_t *sample_extent;  // [B, rank] or nullptr
  int32_t varlen_clamped;  // caller: d * K <= sample extent, non-causal axes
};

// Division by a divisor fixed at launch (round-up multiply method of
// Granlund and Montgomery): q = (mulhi(n, mul) + n) >> shift, exact for
// 0 <= n < 2^31 and 1 <= d < 2^31.
struct FastDiv {
  uint32_t d, mul, shift;
};

inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  FastDiv f;
  f.d = d;
  f.shift = l;
  f.mul = (uint32_t)(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1);
  return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv &f) {
  return (__umulhi(n, f.mul) + n) >> f.shift;
}

// Tiling of the MFMA kernels: 32-query (or 32-key) tiles of T0 x T1 x T2
// sub-grid points (powers of two), nt[a] tiles per dilation phase.
struct Tiling {
  int32_t T[3], lgT[3], nt[3];
  int32_t n_q, n_k;   // query tiles, key tiles
  int32_t n_launch;   // workgroups launched (multiple of 8)
  FastDiv fG[3];      // per-axis tile-grid extent d * nt
  FastDiv fnt[3];     // per-axis tiles per phase
  FastDiv fd[3];      // per-axis dilation
  FastDiv fH, fHk;    // query heads, key/value heads
  FastDiv fRep1;      // query heads per key/value head, plus one
};

// Extents of sample b (varlen aware).
__device__ __forceinline__ void sample_extents(const Prob &P, int32_t b,
                                               int32_t L[3], int32_t O[3]) {
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    L[a] = P.ax[a].L;
    if (P.sample_extent != nullptr && a >= 3 - P.rank)
      L[a] = P.sample_extent[b * P.rank + (a - (3 - P.rank))];
    O[a] = (L[a] + P.ax[a].s - 1) / P.ax[a].s;
  }
}

// Window of output index o on axis a for a sample whose extent is L
// (dense problems span the whole sample).
__device__ __forceinline__ AxisWin prob_window(const Prob &P, int a, int32_t o,
                                               int32_t L) {
  if (P.dense) {
    AxisWin w;
    w.raw = 0;
    w.lo = 0;
    w.hi = L;
    return w;
  }
  const Axis &x = P.ax[a];
  return axis_window(o * x.s, L, x.K, x.d, x.causal);
}

// Step between consecutive neighbors on axis a.
__device__ __forceinline__ int32_t prob_step(const Prob &P, int a) {
  return P.dense ? 1 : P.ax[a].d;
}

// Linear token index of spatial position (x0, x1, x2) of sample b.
__device__ __forceinline__ int64_t tok_in(const Prob &P, int32_t b, int32_t x0,
                                          int32_t x1, int32_t x2) {
  return (((int64_t)b * P.ax[0].L + x0) * P.ax[1].L + x1) * P.ax[2].L + x2;
}
__device__ __forceinline__ int64_t tok_out(const Prob &P, int32_t b, int32_t o0,
                                           int32_t o1, int32_t o2) {
  return (((int64_t)b * P.ax[0].O + o0) * P.ax[1].O + o1) * P.ax[2].O + o2;
}

// Sum over an aligned group of G lanes (G a power of two, <= 64).
__device__ __forceinline__ float group_sum(float x, int G) {
  for (int off = G >> 1; off > 0; off >>= 1) x += __shfl_xor(x, off, G);
  return x;
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

}  // namespace na
