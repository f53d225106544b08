// na_window.h — neighborhood window arithmetic shared by host and device.
//
// Positions are integers on one spatial axis of length L.  A query at
// position i attends to the K keys start + k*dilation (k = 0..K-1) that pass
// the validity rule below; every kernel and the exported host twins use
// these functions, so device and host agree bit for bit.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define NA_HD __host__ __device__ __forceinline__
#else
#define NA_HD static inline
#endif

namespace na {

// Non-causal window start with the NATTEN 0.14 boundary rule
// (reference utils/window.py:8-34).  The window is centred on the query
// and pinned against either edge; with dilation it stays on the query's
// phase (start == index mod dilation).
NA_HD int32_t window_start(int32_t index, int32_t length, int32_t K,
                           int32_t nh, int32_t dil) {
  if (dil <= 1) {
    int32_t s = index > nh ? index - nh : 0;
    if (index + nh >= length) s += length - index - nh - 1;
    return s;
  }
  if (index < nh * dil) return index % dil;                  // pinned left
  if (index + nh * dil < length) return index - nh * dil;    // centred
  // Pinned right: `whole` positions form complete dilation groups and the
  // first `rem` phases own one extra trailing point.
  const int32_t phase = index % dil;
  const int32_t whole = (length / dil) * dil;
  const int32_t rem = length - whole;
  return phase < rem ? whole + phase - 2 * nh * dil : whole + phase - K * dil;
}

// Half-open window end (reference utils/window.py:37-39).
NA_HD int32_t window_end(int32_t start, int32_t length, int32_t K,
                         int32_t dil) {
  const int32_t e = start + K * dil;
  return e < length ? e : length;
}

// First relative-position-bias row used by the query's window
// (reference utils/window.py:42-62).  For slot k the bias index is
// pb_start + k, which equals (key - index) / dilation + K - 1.
NA_HD int32_t pb_start(int32_t index, int32_t length, int32_t K, int32_t nh,
                       int32_t dil) {
  if (dil <= 1) {
    int32_t pb = nh;
    if (index < nh) pb += nh - index;
    if (index + nh >= length) pb += length - index - 1 - nh;
    return pb;
  }
  if (index < nh * dil) return K - 1 - index / dil;
  if (index + nh * dil >= length) return (length - index - 1) / dil;
  return nh;
}

// Window start computed on the query's dilation phase as an undilated
// problem (reference extras/allin1/reference_impl.py:13-25): the phase
// holds `phase_len` positions, the query is the `slot`-th of them.
NA_HD int32_t window_start_partition(int32_t index, int32_t length, int32_t K,
                                     int32_t nh, int32_t dil) {
  const int32_t phase = index % dil;
  const int32_t slot = index / dil;
  const int32_t phase_len = (length - 1 - phase) / dil + 1;
  int32_t s = slot > nh ? slot - nh : 0;
  if (slot + nh >= phase_len) s += phase_len - slot - nh - 1;
  return s * dil + phase;
}

// One spatial axis of a problem, with the per-query window bounds:
// a key position j is a neighbor of the query at position p iff
// lo <= j < hi and j == lo (mod dil); its kernel slot is (j - raw) / dil.
struct AxisWin {
  int32_t raw;  // position of kernel slot 0 (may be negative when causal)
  int32_t lo;   // first valid key position
  int32_t hi;   // one past the last valid key position
};

// Window of the query at position p on an axis of length L
// (reference pure.py:52-73: causal start p-(K-1)*d with keys <= p;
// non-causal clamped start with keys < window_end; keys < 0 invalid).
NA_HD AxisWin axis_window(int32_t p, int32_t L, int32_t K, int32_t dil,
                          int32_t causal) {
  AxisWin w;
  if (causal) {
    w.raw = p - (K - 1) * dil;
    w.hi = p + 1;
  } else {
    w.raw = window_start(p, L, K, K / 2, dil);
    w.hi = window_end(w.raw, L, K, dil);
  }
  if (w.hi > L) w.hi = L;
  if (w.raw >= 0) {
    w.lo = w.raw;
  } else {
    const int32_t skip = (-w.raw + dil - 1) / dil;  // slots below zero
    w.lo = w.raw + skip * dil;
  }
  return w;
}

}  // namespace na
