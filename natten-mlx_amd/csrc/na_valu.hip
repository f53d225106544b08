// na_valu.hip — vector-ALU neighborhood-attention kernels.
//
// One aligned group of G lanes (a power of two) owns one (position, head)
// row; each lane holds NT chunks of VEC consecutive head-dim elements, so a
// D-row is read with 16-byte accesses and dot products finish with a
// log2(G)-step xor shuffle.  These kernels cover every dtype, head_dim,
// rank, stride, dilation, causal mask, GQA, varlen and additional-token
// configuration; the MFMA kernels take over the bf16/fp16 cases they tile.
// All arithmetic is fp32; outputs are rounded once to the storage type.
#include "na_common.h"
#include "na_launch.h"
#include "na_row.h"

namespace na {
namespace {

// Decode idx = (((b * E0 + x0) * E1 + x1) * E2 + x2) * Hn + h.
struct Pos {
  int32_t b, x[3], h;
};
__device__ __forceinline__ Pos decode(int64_t idx, int32_t e0, int32_t e1,
                                      int32_t e2, int32_t Hn) {
  Pos p;
  p.h = (int32_t)(idx % Hn);
  idx /= Hn;
  p.x[2] = (int32_t)(idx % e2);
  idx /= e2;
  p.x[1] = (int32_t)(idx % e1);
  idx /= e1;
  p.x[0] = (int32_t)(idx % e0);
  p.b = (int32_t)(idx / e0);
  return p;
}

__device__ __forceinline__ int32_t gcd_i(int32_t a, int32_t b) {
  while (b) {
    const int32_t t = a % b;
    a = b;
    b = t;
  }
  return a;
}

// Output indices o (stepping o_step from o_begin, below o_end) whose window
// may contain key position j on axis a; members are confirmed with
// prob_window.  Every window lies in [p - K*d, p + K*d) for p = o*s.
struct InvRange {
  int32_t begin, end, step;
};
__device__ __forceinline__ InvRange inv_candidates(const Prob &P, int a,
                                                   int32_t j, int32_t O) {
  InvRange r;
  if (P.dense) {
    r.begin = 0;
    r.end = O;
    r.step = 1;
    return r;
  }
  const Axis &x = P.ax[a];
  const int32_t plo = x.causal ? j : j - x.K * x.d + 1;
  const int32_t phi = x.causal ? j + (x.K - 1) * x.d : j + x.K * x.d;
  const int32_t olo = plo <= 0 ? 0 : (plo + x.s - 1) / x.s;
  int32_t ohi = phi / x.s;
  if (ohi > O - 1) ohi = O - 1;
  const int32_t c = x.d / gcd_i(x.s, x.d);
  r.begin = 0;
  r.end = 0;
  r.step = c;
  for (int32_t o = olo; o < olo + c && o <= ohi; ++o) {
    if ((o * x.s - j) % x.d == 0) {
      r.begin = o;
      r.end = ohi + 1;
      break;
    }
  }
  return r;
}

__device__ __forceinline__ bool in_window(const AxisWin &w, int32_t j) {
  return j >= w.lo && j < w.hi;
}

// ---------------------------------------------------------------------------
// Fused forward: online softmax over the window (+ additional tokens).
template <typename T, int VEC, int NT>
__global__ void __launch_bounds__(256)
    k_fwd(Prob P, const T *__restrict__ q, const T *__restrict__ k,
          const T *__restrict__ v, const T *__restrict__ ek,
          const T *__restrict__ ev, T *__restrict__ out,
          float *__restrict__ lse, int G, int lgG, int64_t n_groups) {
  const Group g = make_group(lgG, n_groups);
  const Pos p = decode(g.id, P.ax[0].O, P.ax[1].O, P.ax[2].O, P.H);
  int32_t L[3], O[3];
  sample_extents(P, p.b, L, O);
  const bool inside = p.x[0] < O[0] && p.x[1] < O[1] && p.x[2] < O[2];
  const int hk = p.h / P.rep;
  const int D = P.D;
  const float sl2 = P.scale * kLog2e;

  Row<T, VEC, NT> qr, acc;
  acc.zero();
  float m = -INFINITY, l = 0.f;
  if (inside) {
    const int64_t qt = tok_in(P, p.b, p.x[0] * P.ax[0].s, p.x[1] * P.ax[1].s,
                              p.x[2] * P.ax[2].s);
    qr.load(q + (qt * P.H + p.h) * D, g.lane, G, D);
    const AxisWin w0 = prob_window(P, 0, p.x[0], L[0]);
    const AxisWin w1 = prob_window(P, 1, p.x[1], L[1]);
    const AxisWin w2 = prob_window(P, 2, p.x[2], L[2]);
    const int32_t d0 = prob_step(P, 0), d1 = prob_step(P, 1),
                  d2 = prob_step(P, 2);
    // The window's keys in slot order (row-major over the axes) through two
    // register sets that take turns: a key's K and V rows are loaded while
    // the previous key is processed, so the loads overlap its arithmetic
    // instead of each waiting alone.  Loads past the last key reload it.
    auto count = [](const AxisWin &w, int32_t st) {
      return w.hi > w.lo ? (w.hi - w.lo + st - 1) / st : 0;
    };
    const int32_t nk = count(w0, d0) * count(w1, d1) * count(w2, d2);
    int32_t c0 = w0.lo, c1 = w1.lo, c2 = w2.lo;  // the next key to load
    int32_t left = nk;                            // keys not yet loaded
    // a key row (the query's own token's row where the window is empty)
    int64_t last = (qt * P.Hkv + hk) * D;
    auto next_row = [&]() -> int64_t {
      if (left > 0) {
        last = (tok_in(P, p.b, c0, c1, c2) * P.Hkv + hk) * D;
        --left;
        c2 += d2;
        if (c2 >= w2.hi) {
          c2 = w2.lo;
          c1 += d1;
          if (c1 >= w1.hi) {
            c1 = w1.lo;
            c0 += d0;
          }
        }
      }
      return last;
    };
    auto step = [&](const Row<T, VEC, NT> &kr, const Row<T, VEC, NT> &vr) {
      const float s = group_sum(qr.dot(kr), G) * sl2;
      const float mn = fmaxf(m, s);
      const float alpha = exp2f(m - mn);
      const float pr = exp2f(s - mn);
      l = fmaf(l, alpha, pr);
      acc.scale_add(alpha, pr, vr);
      m = mn;
    };
    Row<T, VEC, NT> ka, va, kb, vb;
    int64_t r = next_row();
    ka.load_nb(k + r, g.lane, G, D);
    va.load_nb(v + r, g.lane, G, D);
    for (int32_t i = 0; i < nk; i += 2) {
      r = next_row();
      kb.load_nb(k + r, g.lane, G, D);
      vb.load_nb(v + r, g.lane, G, D);
      step(ka, va);
      r = next_row();
      ka.load_nb(k + r, g.lane, G, D);
      va.load_nb(v + r, g.lane, G, D);
      if (i + 1 < nk) step(kb, vb);
    }
    for (int32_t n = 0; n < P.n_extra; ++n) {
      const int64_t row = (((int64_t)p.b * P.n_extra + n) * P.Hkv + hk) * D;
      const float s = group_sum(qr.dot_mem(ek + row, g.lane, G, D), G) * sl2;
      const float mn = fmaxf(m, s);
      const float alpha = exp2f(m - mn);
      const float pr = exp2f(s - mn);
      l = fmaf(l, alpha, pr);
      acc.scale_add_mem(alpha, pr, ev + row, g.lane, G, D);
      m = mn;
    }
    acc.mul(1.f / l);
  }
  if (g.live) {
    const int64_t ot = tok_out(P, p.b, p.x[0], p.x[1], p.x[2]);
    acc.store(out + (ot * P.H + p.h) * D, g.lane, G, D);
    if (lse != nullptr && g.lane == 0)
      lse[ot * P.H + p.h] = inside ? (m + __log2f(l)) * kLn2 : 0.f;
  }
}

// delta[q,h] = <dO, O> - dlse  (the softmax-backward row term).
template <typename T, int VEC, int NT>
__global__ void __launch_bounds__(256)
    k_delta(Prob P, const T *__restrict__ out, const T *__restrict__ dout,
            const float *__restrict__ dlse, float *__restrict__ delta, int G,
            int lgG, int64_t n_groups) {
  const Group g = make_group(lgG, n_groups);
  const int64_t row = g.id * P.D;
  Row<T, VEC, NT> o;
  o.load(out + row, g.lane, G, P.D);
  const float dd = group_sum(o.dot_mem(dout + row, g.lane, G, P.D), G);
  if (g.live && g.lane == 0)
    delta[g.id] = dd - (dlse != nullptr ? dlse[g.id] : 0.f);
}

// dQ for every input position (zero where no query sits).
template <typename T, int VEC, int NT>
__global__ void __launch_bounds__(256)
    k_dq(Prob P, const T *__restrict__ q, const T *__restrict__ k,
         const T *__restrict__ v, const T *__restrict__ ek,
         const T *__restrict__ ev, const float *__restrict__ lse,
         const float *__restrict__ delta, const T *__restrict__ dout,
         T *__restrict__ dq, int G, int lgG, int64_t n_groups) {
  const Group g = make_group(lgG, n_groups);
  const Pos p = decode(g.id, P.ax[0].L, P.ax[1].L, P.ax[2].L, P.H);
  int32_t L[3], O[3];
  sample_extents(P, p.b, L, O);
  int32_t o[3];
  bool is_q = true;
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    is_q = is_q && (p.x[a] % P.ax[a].s == 0) && p.x[a] < L[a];
    o[a] = p.x[a] / P.ax[a].s;
  }
  const int hk = p.h / P.rep;
  const int D = P.D;
  const float sl2 = P.scale * kLog2e;
  Row<T, VEC, NT> qr, dor, acc;
  acc.zero();
  if (is_q) {
    const int64_t qt = tok_in(P, p.b, p.x[0], p.x[1], p.x[2]);
    const int64_t ot = tok_out(P, p.b, o[0], o[1], o[2]);
    qr.load(q + (qt * P.H + p.h) * D, g.lane, G, D);
    dor.load(dout + (ot * P.H + p.h) * D, g.lane, G, D);
    const float lse2 = lse[ot * P.H + p.h] * kLog2e;
    const float dl = delta[ot * P.H + p.h];
    const AxisWin w0 = prob_window(P, 0, o[0], L[0]);
    const AxisWin w1 = prob_window(P, 1, o[1], L[1]);
    const AxisWin w2 = prob_window(P, 2, o[2], L[2]);
    const int32_t d0 = prob_step(P, 0), d1 = prob_step(P, 1),
                  d2 = prob_step(P, 2);
    for (int32_t k0 = w0.lo; k0 < w0.hi; k0 += d0)
      for (int32_t k1 = w1.lo; k1 < w1.hi; k1 += d1)
        for (int32_t k2 = w2.lo; k2 < w2.hi; k2 += d2) {
          const int64_t row = (tok_in(P, p.b, k0, k1, k2) * P.Hkv + hk) * D;
          const float s = group_sum(qr.dot_mem(k + row, g.lane, G, D), G);
          const float dp = group_sum(dor.dot_mem(v + row, g.lane, G, D), G);
          const float pr = exp2f(fmaf(s, sl2, -lse2));
          acc.scale_add_mem(1.f, pr * (dp - dl), k + row, g.lane, G, D);
        }
    for (int32_t n = 0; n < P.n_extra; ++n) {
      const int64_t row = (((int64_t)p.b * P.n_extra + n) * P.Hkv + hk) * D;
      const float s = group_sum(qr.dot_mem(ek + row, g.lane, G, D), G);
      const float dp = group_sum(dor.dot_mem(ev + row, g.lane, G, D), G);
      const float pr = exp2f(fmaf(s, sl2, -lse2));
      acc.scale_add_mem(1.f, pr * (dp - dl), ek + row, g.lane, G, D);
    }
    acc.mul(P.scale);
  }
  if (g.live) acc.store(dq + g.id * D, g.lane, G, D);
}

// dK, dV for every key position by gathering over its inverse neighborhood.
template <typename T, int VEC, int NT>
__global__ void __launch_bounds__(256)
    k_dkdv(Prob P, const T *__restrict__ q, const T *__restrict__ k,
           const T *__restrict__ v, const float *__restrict__ lse,
           const float *__restrict__ delta, const T *__restrict__ dout,
           T *__restrict__ dk, T *__restrict__ dv, int G, int lgG,
           int64_t n_groups) {
  const Group g = make_group(lgG, n_groups);
  const Pos p = decode(g.id, P.ax[0].L, P.ax[1].L, P.ax[2].L, P.Hkv);
  int32_t L[3], O[3];
  sample_extents(P, p.b, L, O);
  const bool inside = p.x[0] < L[0] && p.x[1] < L[1] && p.x[2] < L[2];
  const int D = P.D;
  const float sl2 = P.scale * kLog2e;
  Row<T, VEC, NT> kr, vr, dka, dva;
  dka.zero();
  dva.zero();
  if (inside) {
    kr.load(k + g.id * D, g.lane, G, D);
    vr.load(v + g.id * D, g.lane, G, D);
    const InvRange r0 = inv_candidates(P, 0, p.x[0], O[0]);
    const InvRange r1 = inv_candidates(P, 1, p.x[1], O[1]);
    const InvRange r2 = inv_candidates(P, 2, p.x[2], O[2]);
    for (int32_t o0 = r0.begin; o0 < r0.end; o0 += r0.step) {
      if (!in_window(prob_window(P, 0, o0, L[0]), p.x[0])) continue;
      for (int32_t o1 = r1.begin; o1 < r1.end; o1 += r1.step) {
        if (!in_window(prob_window(P, 1, o1, L[1]), p.x[1])) continue;
        for (int32_t o2 = r2.begin; o2 < r2.end; o2 += r2.step) {
          if (!in_window(prob_window(P, 2, o2, L[2]), p.x[2])) continue;
          const int64_t qt = tok_in(P, p.b, o0 * P.ax[0].s, o1 * P.ax[1].s,
                                    o2 * P.ax[2].s);
          const int64_t ot = tok_out(P, p.b, o0, o1, o2);
          for (int h = p.h * P.rep; h < (p.h + 1) * P.rep; ++h) {
            const T *qrow = q + (qt * P.H + h) * D;
            const T *drow = dout + (ot * P.H + h) * D;
            const float s = group_sum(kr.dot_mem(qrow, g.lane, G, D), G);
            const float dp = group_sum(vr.dot_mem(drow, g.lane, G, D), G);
            const float pr =
                exp2f(fmaf(s, sl2, -lse[ot * P.H + h] * kLog2e));
            const float ds = pr * (dp - delta[ot * P.H + h]);
            dva.scale_add_mem(1.f, pr, drow, g.lane, G, D);
            dka.scale_add_mem(1.f, ds, qrow, g.lane, G, D);
          }
        }
      }
    }
    dka.mul(P.scale);
  }
  if (g.live) {
    dka.store(dk + g.id * D, g.lane, G, D);
    dva.store(dv + g.id * D, g.lane, G, D);
  }
}


// ---------------------------------------------------------------------------
// Split operators.  Slot n of the last logits axis is row-major over
// (k0, k1, k2); slot positions are raw + k*d and valid iff lo <= pos < hi.

template <typename T, int VEC, int NT>
__global__ void __launch_bounds__(256)
    k_qk(Prob P, const T *__restrict__ q, const T *__restrict__ k,
         T *__restrict__ logits, int G, int lgG, int64_t n_groups) {
  const Group g = make_group(lgG, n_groups);
  const Pos p = decode(g.id, P.ax[0].O, P.ax[1].O, P.ax[2].O, P.H);
  const int hk = p.h / P.rep;
  const int D = P.D;
  const int64_t qt = tok_in(P, p.b, p.x[0] * P.ax[0].s, p.x[1] * P.ax[1].s,
                            p.x[2] * P.ax[2].s);
  Row<T, VEC, NT> qr;
  qr.load(q + (qt * P.H + p.h) * D, g.lane, G, D);
  AxisWin w[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) w[a] = prob_window(P, a, p.x[a], P.ax[a].L);
  T *dst = logits + g.id * P.kprod;
  int n = 0;
  for (int k0 = 0; k0 < P.ax[0].K; ++k0) {
    const int32_t j0 = w[0].raw + k0 * P.ax[0].d;
    for (int k1 = 0; k1 < P.ax[1].K; ++k1) {
      const int32_t j1 = w[1].raw + k1 * P.ax[1].d;
      for (int k2 = 0; k2 < P.ax[2].K; ++k2, ++n) {
        const int32_t j2 = w[2].raw + k2 * P.ax[2].d;
        const bool ok = in_window(w[0], j0) && in_window(w[1], j1) &&
                        in_window(w[2], j2);
        float s = -INFINITY;
        if (ok) {
          const int64_t row = (tok_in(P, p.b, j0, j1, j2) * P.Hkv + hk) * D;
          s = group_sum(qr.dot_mem(k + row, g.lane, G, D), G) * P.scale;
        }
        if (g.live && g.lane == 0) dst[n] = from_f32<T>(s);
      }
    }
  }
}

template <typename T, int VEC, int NT>
__global__ void __launch_bounds__(256)
    k_av(Prob P, const T *__restrict__ attn, const T *__restrict__ v,
         T *__restrict__ out, int G, int lgG, int64_t n_groups) {
  const Group g = make_group(lgG, n_groups);
  const Pos p = decode(g.id, P.ax[0].O, P.ax[1].O, P.ax[2].O, P.H);
  const int hk = p.h / P.rep;
  const int D = P.D;
  AxisWin w[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) w[a] = prob_window(P, a, p.x[a], P.ax[a].L);
  const T *arow = attn + g.id * P.kprod;
  Row<T, VEC, NT> acc;
  acc.zero();
  int n = 0;
  for (int k0 = 0; k0 < P.ax[0].K; ++k0) {
    const int32_t j0 = w[0].raw + k0 * P.ax[0].d;
    for (int k1 = 0; k1 < P.ax[1].K; ++k1) {
      const int32_t j1 = w[1].raw + k1 * P.ax[1].d;
      for (int k2 = 0; k2 < P.ax[2].K; ++k2, ++n) {
        const int32_t j2 = w[2].raw + k2 * P.ax[2].d;
        if (in_window(w[0], j0) && in_window(w[1], j1) &&
            in_window(w[2], j2)) {
          const int64_t row = (tok_in(P, p.b, j0, j1, j2) * P.Hkv + hk) * D;
          acc.scale_add_mem(1.f, to_f32(arow[n]), v + row, g.lane, G, D);
        }
      }
    }
  }
  if (g.live) acc.store(out + g.id * D, g.lane, G, D);
}

// dQ of the split QK op for every input position.
template <typename T, int VEC, int NT>
__global__ void __launch_bounds__(256)
    k_qk_dq(Prob P, const T *__restrict__ k, const T *__restrict__ dlogits,
            T *__restrict__ dq, int G, int lgG, int64_t n_groups) {
  const Group g = make_group(lgG, n_groups);
  const Pos p = decode(g.id, P.ax[0].L, P.ax[1].L, P.ax[2].L, P.H);
  const int hk = p.h / P.rep;
  const int D = P.D;
  bool is_q = true;
  int32_t o[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    is_q = is_q && (p.x[a] % P.ax[a].s == 0);
    o[a] = p.x[a] / P.ax[a].s;
  }
  Row<T, VEC, NT> acc;
  acc.zero();
  if (is_q) {
    AxisWin w[3];
#pragma unroll
    for (int a = 0; a < 3; ++a) w[a] = prob_window(P, a, o[a], P.ax[a].L);
    const T *grow =
        dlogits + (tok_out(P, p.b, o[0], o[1], o[2]) * P.H + p.h) * P.kprod;
    int n = 0;
    for (int k0 = 0; k0 < P.ax[0].K; ++k0) {
      const int32_t j0 = w[0].raw + k0 * P.ax[0].d;
      for (int k1 = 0; k1 < P.ax[1].K; ++k1) {
        const int32_t j1 = w[1].raw + k1 * P.ax[1].d;
        for (int k2 = 0; k2 < P.ax[2].K; ++k2, ++n) {
          const int32_t j2 = w[2].raw + k2 * P.ax[2].d;
          if (in_window(w[0], j0) && in_window(w[1], j1) &&
              in_window(w[2], j2)) {
            const int64_t row = (tok_in(P, p.b, j0, j1, j2) * P.Hkv + hk) * D;
            acc.scale_add_mem(1.f, to_f32(grow[n]), k + row, g.lane, G, D);
          }
        }
      }
    }
    acc.mul(P.scale);
  }
  if (g.live) acc.store(dq + g.id * D, g.lane, G, D);
}

// Inverse-neighborhood gather shared by the split backward ops:
//   out[key] = mult * sum over (query o, head h, slot n) with nbr(o,n)=key
//              of g[o, h, n] * X[o, h]
// X is indexed at the query's input token (dK of QK: X = q) or at its
// output token (dV of AV: X = dout).
template <typename T, int VEC, int NT, bool X_AT_INPUT>
__global__ void __launch_bounds__(256)
    k_inverse(Prob P, const T *__restrict__ gsl, const T *__restrict__ X,
              float mult, T *__restrict__ dst, int G, int lgG,
              int64_t n_groups) {
  const Group g = make_group(lgG, n_groups);
  const Pos p = decode(g.id, P.ax[0].L, P.ax[1].L, P.ax[2].L, P.Hkv);
  const int D = P.D;
  Row<T, VEC, NT> acc;
  acc.zero();
  int32_t O[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) O[a] = P.ax[a].O;
  const InvRange r0 = inv_candidates(P, 0, p.x[0], O[0]);
  const InvRange r1 = inv_candidates(P, 1, p.x[1], O[1]);
  const InvRange r2 = inv_candidates(P, 2, p.x[2], O[2]);
  for (int32_t o0 = r0.begin; o0 < r0.end; o0 += r0.step) {
    const AxisWin w0 = prob_window(P, 0, o0, P.ax[0].L);
    if (!in_window(w0, p.x[0])) continue;
    const int n0 = (p.x[0] - w0.raw) / P.ax[0].d;
    for (int32_t o1 = r1.begin; o1 < r1.end; o1 += r1.step) {
      const AxisWin w1 = prob_window(P, 1, o1, P.ax[1].L);
      if (!in_window(w1, p.x[1])) continue;
      const int n1 = (p.x[1] - w1.raw) / P.ax[1].d;
      for (int32_t o2 = r2.begin; o2 < r2.end; o2 += r2.step) {
        const AxisWin w2 = prob_window(P, 2, o2, P.ax[2].L);
        if (!in_window(w2, p.x[2])) continue;
        const int n2 = (p.x[2] - w2.raw) / P.ax[2].d;
        const int n = (n0 * P.ax[1].K + n1) * P.ax[2].K + n2;
        const int64_t ot = tok_out(P, p.b, o0, o1, o2);
        const int64_t xt =
            X_AT_INPUT ? tok_in(P, p.b, o0 * P.ax[0].s, o1 * P.ax[1].s,
                                o2 * P.ax[2].s)
                       : ot;
        for (int h = p.h * P.rep; h < (p.h + 1) * P.rep; ++h) {
          const float gv = to_f32(gsl[(ot * P.H + h) * P.kprod + n]);
          acc.scale_add_mem(1.f, gv, X + (xt * P.H + h) * D, g.lane, G, D);
        }
      }
    }
  }
  acc.mul(mult);
  if (g.live) acc.store(dst + g.id * D, g.lane, G, D);
}

// dAttn of the split AV op: <dout, v_nbr> on valid slots, 0 elsewhere.
template <typename T, int VEC, int NT>
__global__ void __launch_bounds__(256)
    k_dattn(Prob P, const T *__restrict__ v, const T *__restrict__ dout,
            T *__restrict__ dattn, int G, int lgG, int64_t n_groups) {
  const Group g = make_group(lgG, n_groups);
  const Pos p = decode(g.id, P.ax[0].O, P.ax[1].O, P.ax[2].O, P.H);
  const int hk = p.h / P.rep;
  const int D = P.D;
  Row<T, VEC, NT> dor;
  dor.load(dout + g.id * D, g.lane, G, D);
  AxisWin w[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) w[a] = prob_window(P, a, p.x[a], P.ax[a].L);
  T *dst = dattn + g.id * P.kprod;
  int n = 0;
  for (int k0 = 0; k0 < P.ax[0].K; ++k0) {
    const int32_t j0 = w[0].raw + k0 * P.ax[0].d;
    for (int k1 = 0; k1 < P.ax[1].K; ++k1) {
      const int32_t j1 = w[1].raw + k1 * P.ax[1].d;
      for (int k2 = 0; k2 < P.ax[2].K; ++k2, ++n) {
        const int32_t j2 = w[2].raw + k2 * P.ax[2].d;
        float s = 0.f;
        if (in_window(w[0], j0) && in_window(w[1], j1) &&
            in_window(w[2], j2)) {
          const int64_t row = (tok_in(P, p.b, j0, j1, j2) * P.Hkv + hk) * D;
          s = group_sum(dor.dot_mem(v + row, g.lane, G, D), G);
        }
        if (g.live && g.lane == 0) dst[n] = from_f32<T>(s);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Device neighbor table (pure.py:24-152 layout) for bit-exact checks.
__global__ void k_table(Prob P, int32_t *__restrict__ index,
                        uint8_t *__restrict__ valid, int64_t n) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= n) return;
  const int slot = (int)(id % P.kprod);
  int64_t r = id / P.kprod;
  int32_t o[3];
  o[2] = (int32_t)(r % P.ax[2].O);
  r /= P.ax[2].O;
  o[1] = (int32_t)(r % P.ax[1].O);
  o[0] = (int32_t)(r / P.ax[1].O);
  int32_t kk[3];
  kk[2] = slot % P.ax[2].K;
  kk[1] = (slot / P.ax[2].K) % P.ax[1].K;
  kk[0] = slot / (P.ax[2].K * P.ax[1].K);
  bool ok = true;
  int64_t lin = 0;
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    const AxisWin w = axis_window(o[a] * P.ax[a].s, P.ax[a].L, P.ax[a].K,
                                  P.ax[a].d, P.ax[a].causal);
    const int32_t j = w.raw + kk[a] * P.ax[a].d;
    ok = ok && in_window(w, j);
    const int32_t jc = j < 0 ? 0 : (j > P.ax[a].L - 1 ? P.ax[a].L - 1 : j);
    lin = lin * P.ax[a].L + jc;
  }
  index[id] = (int32_t)lin;
  valid[id] = ok ? 1 : 0;
}

// ---------------------------------------------------------------------------
// Launch helpers (launch shapes: na_row.h).

template <typename T>
void fwd_t(const Prob &P, const void *q, const void *k, const void *v,
           const void *ek, const void *ev, void *out, float *lse,
           hipStream_t st) {
  const Shape s = pick_shape<T>(P.D);
  const int64_t n = (int64_t)P.B * P.ax[0].O * P.ax[1].O * P.ax[2].O * P.H;
#define L_(TT, V, N)                                                        \
  hipLaunchKernelGGL((k_fwd<TT, V, N>), grid_for(n, s.lgG), dim3(256), 0,  \
                     st, P, (const TT *)q, (const TT *)k, (const TT *)v,    \
                     (const TT *)ek, (const TT *)ev, (TT *)out, lse, s.G,   \
                     s.lgG, n)
  NA_VALU_DISPATCH(T, s, L_);
#undef L_
}

template <typename T>
void bwd_t(const Prob &P, const void *q, const void *k, const void *v,
           const void *ek, const void *ev, const void *out, const float *lse,
           const void *dout, const float *dlse, void *dq, void *dk, void *dv,
           float *delta, hipStream_t st) {
  const Shape s = pick_shape<T>(P.D);
  const int64_t n_out = (int64_t)P.B * P.ax[0].O * P.ax[1].O * P.ax[2].O * P.H;
  const int64_t n_in_q = (int64_t)P.B * P.ax[0].L * P.ax[1].L * P.ax[2].L * P.H;
  const int64_t n_in_kv =
      (int64_t)P.B * P.ax[0].L * P.ax[1].L * P.ax[2].L * P.Hkv;
#define L_(TT, V, N)                                                          \
  do {                                                                        \
    hipLaunchKernelGGL((k_delta<TT, V, N>), grid_for(n_out, s.lgG),           \
                       dim3(256), 0, st, P, (const TT *)out,                  \
                       (const TT *)dout, dlse, delta, s.G, s.lgG, n_out);     \
    hipLaunchKernelGGL((k_dq<TT, V, N>), grid_for(n_in_q, s.lgG), dim3(256),  \
                       0, st, P, (const TT *)q, (const TT *)k, (const TT *)v, \
                       (const TT *)ek, (const TT *)ev, lse, delta,            \
                       (const TT *)dout, (TT *)dq, s.G, s.lgG, n_in_q);       \
    hipLaunchKernelGGL((k_dkdv<TT, V, N>), grid_for(n_in_kv, s.lgG),          \
                       dim3(256), 0, st, P, (const TT *)q, (const TT *)k,     \
                       (const TT *)v, lse, delta, (const TT *)dout,           \
                       (TT *)dk, (TT *)dv, s.G, s.lgG, n_in_kv);              \
  } while (0)
  NA_VALU_DISPATCH(T, s, L_);
#undef L_
}

template <typename T>
void delta_t(const Prob &P, const void *out, const void *dout, const float *dlse,
             float *delta, hipStream_t st) {
  const Shape s = pick_shape<T>(P.D);
  const int64_t n = (int64_t)P.B * P.ax[0].O * P.ax[1].O * P.ax[2].O * P.H;
#define L_(TT, V, N)                                                         \
  hipLaunchKernelGGL((k_delta<TT, V, N>), grid_for(n, s.lgG), dim3(256), 0, \
                     st, P, (const TT *)out, (const TT *)dout, dlse, delta,  \
                     s.G, s.lgG, n)
  NA_VALU_DISPATCH(T, s, L_);
#undef L_
}

template <typename T>
void qk_t(const Prob &P, const void *q, const void *k, void *logits,
          hipStream_t st) {
  const Shape s = pick_shape<T>(P.D);
  const int64_t n = (int64_t)P.B * P.ax[0].O * P.ax[1].O * P.ax[2].O * P.H;
#define L_(TT, V, N)                                                      \
  hipLaunchKernelGGL((k_qk<TT, V, N>), grid_for(n, s.lgG), dim3(256), 0, \
                     st, P, (const TT *)q, (const TT *)k, (TT *)logits,   \
                     s.G, s.lgG, n)
  NA_VALU_DISPATCH(T, s, L_);
#undef L_
}

template <typename T>
void av_t(const Prob &P, const void *attn, const void *v, void *out,
          hipStream_t st) {
  const Shape s = pick_shape<T>(P.D);
  const int64_t n = (int64_t)P.B * P.ax[0].O * P.ax[1].O * P.ax[2].O * P.H;
#define L_(TT, V, N)                                                      \
  hipLaunchKernelGGL((k_av<TT, V, N>), grid_for(n, s.lgG), dim3(256), 0, \
                     st, P, (const TT *)attn, (const TT *)v, (TT *)out,   \
                     s.G, s.lgG, n)
  NA_VALU_DISPATCH(T, s, L_);
#undef L_
}

template <typename T>
void qk_bwd_t(const Prob &P, const void *q, const void *k, const void *dl,
              void *dq, void *dk, hipStream_t st) {
  const Shape s = pick_shape<T>(P.D);
  const int64_t n_q = (int64_t)P.B * P.ax[0].L * P.ax[1].L * P.ax[2].L * P.H;
  const int64_t n_kv =
      (int64_t)P.B * P.ax[0].L * P.ax[1].L * P.ax[2].L * P.Hkv;
#define L_(TT, V, N)                                                          \
  do {                                                                        \
    hipLaunchKernelGGL((k_qk_dq<TT, V, N>), grid_for(n_q, s.lgG), dim3(256),  \
                       0, st, P, (const TT *)k, (const TT *)dl, (TT *)dq,     \
                       s.G, s.lgG, n_q);                                      \
    hipLaunchKernelGGL((k_inverse<TT, V, N, true>), grid_for(n_kv, s.lgG),    \
                       dim3(256), 0, st, P, (const TT *)dl, (const TT *)q,    \
                       P.scale, (TT *)dk, s.G, s.lgG, n_kv);                  \
  } while (0)
  NA_VALU_DISPATCH(T, s, L_);
#undef L_
}

template <typename T>
void av_bwd_t(const Prob &P, const void *attn, const void *v, const void *dout,
              void *dattn, void *dv, hipStream_t st) {
  const Shape s = pick_shape<T>(P.D);
  const int64_t n_o = (int64_t)P.B * P.ax[0].O * P.ax[1].O * P.ax[2].O * P.H;
  const int64_t n_kv =
      (int64_t)P.B * P.ax[0].L * P.ax[1].L * P.ax[2].L * P.Hkv;
#define L_(TT, V, N)                                                          \
  do {                                                                        \
    hipLaunchKernelGGL((k_dattn<TT, V, N>), grid_for(n_o, s.lgG), dim3(256),  \
                       0, st, P, (const TT *)v, (const TT *)dout,             \
                       (TT *)dattn, s.G, s.lgG, n_o);                         \
    hipLaunchKernelGGL((k_inverse<TT, V, N, false>), grid_for(n_kv, s.lgG),   \
                       dim3(256), 0, st, P, (const TT *)attn,                 \
                       (const TT *)dout, 1.f, (TT *)dv, s.G, s.lgG, n_kv);    \
  } while (0)
  NA_VALU_DISPATCH(T, s, L_);
#undef L_
}

}  // namespace

void valu_fwd(const Prob &P, int dtype, const void *q, const void *k,
              const void *v, const void *ek, const void *ev, void *out,
              float *lse, hipStream_t st) {
  NA_BY_DTYPE(dtype, fwd_t, P, q, k, v, ek, ev, out, lse, st);
}

void valu_bwd(const Prob &P, int dtype, const void *q, const void *k,
              const void *v, const void *ek, const void *ev, const void *out,
              const float *lse, const void *dout, const float *dlse, void *dq,
              void *dk, void *dv, float *delta, hipStream_t st) {
  NA_BY_DTYPE(dtype, bwd_t, P, q, k, v, ek, ev, out, lse, dout, dlse, dq, dk,
              dv, delta, st);
}

void valu_delta(const Prob &P, int dtype, const void *out, const void *dout,
                const float *dlse, float *delta, hipStream_t st) {
  NA_BY_DTYPE(dtype, delta_t, P, out, dout, dlse, delta, st);
}

void valu_qk(const Prob &P, int dtype, const void *q, const void *k,
             void *logits, hipStream_t st) {
  NA_BY_DTYPE(dtype, qk_t, P, q, k, logits, st);
}

void valu_av(const Prob &P, int dtype, const void *attn, const void *v,
             void *out, hipStream_t st) {
  NA_BY_DTYPE(dtype, av_t, P, attn, v, out, st);
}

void valu_qk_bwd(const Prob &P, int dtype, const void *q, const void *k,
                 const void *dl, void *dq, void *dk, hipStream_t st) {
  NA_BY_DTYPE(dtype, qk_bwd_t, P, q, k, dl, dq, dk, st);
}

void valu_av_bwd(const Prob &P, int dtype, const void *attn, const void *v,
                 const void *dout, void *dattn, void *dv, hipStream_t st) {
  NA_BY_DTYPE(dtype, av_bwd_t, P, attn, v, dout, dattn, dv, st);
}


void table(const Prob &P, int32_t *index, uint8_t *valid, hipStream_t st) {
  const int64_t n =
      (int64_t)P.ax[0].O * P.ax[1].O * P.ax[2].O * (int64_t)P.kprod;
  if (n == 0) return;
  hipLaunchKernelGGL(k_table, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     st, P, index, valid, n);
}

}  // namespace na
