// na_mfma.hip — matrix-core (gfx950 MFMA) kernels for the fused op.
//
// Tiling.  With dilation d an axis splits into d independent phases
// (positions r, r+d, r+2d, ...), each an undilated neighborhood problem on
// its "sub-grid".  A wave owns a tile of 32 queries: a T0 x T1 x T2 box
// (powers of two) of one phase.  The union of their windows is again a box
// on the same sub-grid, enumerated row-major with the innermost extent
// padded to a power of two P2 >= 8, so the coordinates of a chunk of 32
// keys follow from shifts and wave-uniform divisions.
//
// Forward, per chunk of 32 keys (mfma_f32_32x32x16, fp32 accumulate):
//   S^T[key][q] = K_chunk . Q^T          (A = K rows, B = Q rows: global)
//   online softmax per query column: a lane owns 16 scores of one query,
//   the other 16 sit in lane ^ 32, so one cross-lane max per chunk
//   O^T[d][q] += V^T[d][key] . P^T        (A = V^T from LDS, B = P regs)
// The 16 scores a lane holds (keys 8i + 4h + j) feed the next MFMA's B
// operand directly when its k index is permuted the same way on the A side.
//
// Backward is one launch with two roles, deterministic and atomic-free:
//   dQ tiles   (as forward)  dS^T = P^T (dP^T - delta),  dQ^T += K^T . dS^T
//   dK/dV tiles (32 keys)    over the queries whose windows contain them
//                            (inverse neighborhood, a box per axis):
//                            dV^T += dO^T . P,  dK^T += Q^T . dS
// delta = rowsum(dO * O) - dlse: at head_dim 32 each role recomputes it from
// O and dO (cheaper than one more launch on these short problems); from
// head_dim 64 a pre-pass writes one fp32 per (query, head) and neither role
// reads O, which keeps the prefetching loops within two waves per SIMD.
#include "na_mfma.h"

namespace na {
namespace {

// ---------------------------------------------------------------------------
// Layout self-check: C = A . B for fixed small-integer A (32x16), B (16x32),
// using the operand and result layouts every kernel here assumes.
template <typename T>
__global__ void __launch_bounds__(64) k_selftest(float *out) {
  typedef typename Mf<T>::v8 v8;
  const int lane = threadIdx.x, n = lane & 31, h = lane >> 5;
  v8 a, bv;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = 8 * h + e;
    a[e] = (typename Mf<T>::e)(float)(((n + 2 * k) % 7) - 3);   // A[m=n][k]
    bv[e] = (typename Mf<T>::e)(float)(((3 * k + n) % 5) - 2);  // B[k][n]
  }
  const f32x16 c = Mf<T>::mma(a, bv, zero16());
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = 8 * (r >> 2) + 4 * h + (r & 3);
    out[m * 32 + n] = c[r];
  }
}

// ---------------------------------------------------------------------------
// A workgroup of W waves owns one tile; wave w walks chunks w, w + W, ...
// with its own LDS transpose buffer, and the partial results are combined
// in LDS in wave order at the end (deterministic).  Inside the chunk loops a
// wave only synchronises with itself.
// Backward chunk loops without next-chunk prefetch at head_dim 32: there the
// registers the prefetch needs would cost the kernel a wave per SIMD
// (123 VGPRs: four waves, all of config 2's 3136 waves resident at once).
constexpr bool kLeanBwd(int D) { return D == 32; }
// From head_dim 64 the backward reads delta from a pre-pass instead of
// recomputing it from O.
constexpr bool kPreDelta(int D) { return !kLeanBwd(D); }

// LDS row stride (elements) of a dK/dV tile's K / V rows: 16 bytes of skew.
constexpr int kKvRow(int D) { return D + 8; }
// Per-wave LDS of the backward: two transposed chunks, lse / delta of a
// chunk, and (lean variant) the dK/dV tile's K and V rows.
constexpr int bwd_wave_lds(int D, int esize) {
  return 2 * D * kRow * esize + 256 + (kLeanBwd(D) ? 2 * 32 * kKvRow(D) * esize : 0);
}

// Chunks of K/V rows a wave loads together (registers: 16*D/8 per chunk).
constexpr int group_chunks(int D) { return D == 32 ? 6 : D == 64 ? 3 : 2; }
// LDS row stride (elements) of a group's V^T: 32 per chunk plus 4 of skew.
constexpr int group_row(int NB) { return 32 * NB + 4; }

// Online-softmax state of one query column (the lane pair n, n + 32).
template <int NC>
struct Softmax {
  f32x16 o[NC];
  float m, l;
};

// One 32-key chunk of the forward: S^T = K.Q^T, masked online softmax,
// O^T += V^T.P^T (V^T staged through this wave's LDS buffer).
template <typename T, int D>
__device__ __forceinline__ void fwd_compute(Softmax<D / 32> &st,
                                            const typename Mf<T>::v8 *qf,
                                            const typename Mf<T>::v8 *kf,
                                            const typename Mf<T>::v8 *vf,
                                            const bool ok[16], float sl2,
                                            typename Mf<T>::e *vt, int n,
                                            int h) {
  typedef Mf<T> M;
  typedef typename M::v8 v8;
  constexpr int NK = D / 16, NC = D / 32;
  f32x16 s = zero16();
#pragma unroll
  for (int t = 0; t < NK; ++t) s = M::mma(kf[t], qf[t], s);
  // raw scores, -inf outside the window; the max commutes with the
  // positive scale, which is folded into the exponent's fma
  float sv[16];
  float mx = -INFINITY;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    sv[e] = ok[e] ? s[e] : -INFINITY;
    mx = fmaxf(mx, sv[e]);
  }
  mx = fmaxf(mx, __shfl_xor(mx, 32)) * sl2;
  // The reference point st.m may trail the running max by up to 8 (a
  // factor 2^8 in P): exact after the final division by l, and it spares
  // the O rescale on chunks that do not raise any query's max by more.
  if (__builtin_amdgcn_ballot_w64(mx > st.m + 8.f) != 0) {
    const float mn = fmaxf(st.m, mx);
    const float alpha = __builtin_amdgcn_exp2f(st.m - (mn == -INFINITY ? 0.f : mn));
    st.l *= alpha;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
#pragma unroll
      for (int e = 0; e < 16; ++e) st.o[cc][e] *= alpha;
    st.m = mn;
  }
  const float mu = st.m == -INFINITY ? 0.f : st.m;
  float ps = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    sv[e] = __builtin_amdgcn_exp2f(fmaf(sv[e], sl2, -mu));
    ps += sv[e];
  }
  st.l += ps;
  wave_lds_sync();
#pragma unroll
  for (int t = 0; t < NK; ++t)
#pragma unroll
    for (int e = 0; e < 8; ++e) vt[(16 * t + 8 * h + e) * kRow + n] = vf[t][e];
  wave_lds_sync();
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const v8 bp = pack8<T>(sv + 8 * kb);
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
      st.o[cc] = M::mma(lds_a<T>(vt + (32 * cc + n) * kRow + 16 * kb, h), bp,
                        st.o[cc]);
  }
}

// A group of up to NB box chunks of the forward, in two phases: the score
// tiles of every chunk (back-to-back MFMAs) and one max over them, then the
// exponentials and O^T += V^T . P^T with the group's V^T staged in LDS
// behind a single wave sync.  The reference point st.m trails the running
// max by at most 8 (see fwd_compute).
template <typename T, int D, int NB>
__device__ __forceinline__ void fwd_group(Softmax<D / 32> &st,
                                          const typename Mf<T>::v8 *qf,
                                          const typename Mf<T>::v8 (*kg)[D / 16],
                                          const typename Mf<T>::v8 (*vg)[D / 16],
                                          const ChunkRows *cr, const QTile &Q,
                                          int w, int W, int i0, int n_own,
                                          float sl2, typename Mf<T>::e *vt,
                                          int n, int h) {
  typedef Mf<T> M;
  typedef typename M::v8 v8;
  constexpr int NK = D / 16, NC = D / 32, RG = group_row(NB);
  float sv[NB][16];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    if (i0 + j >= n_own) break;
    f32x16 s = zero16();
#pragma unroll
    for (int t = 0; t < NK; ++t) s = M::mma(kg[j][t], qf[t], s);
    bool ok[16];
    chunk_mask(Q.bx, cr[j], 32 * (w + W * (i0 + j)), h, Q.wlo, Q.ww, ok);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      sv[j][e] = ok[e] ? s[e] : -INFINITY;
      mx = fmaxf(mx, sv[j][e]);
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 32)) * sl2;
  if (__builtin_amdgcn_ballot_w64(mx > st.m + 8.f) != 0) {
    const float mn = fmaxf(st.m, mx);
    const float alpha = __builtin_amdgcn_exp2f(st.m - (mn == -INFINITY ? 0.f : mn));
    st.l *= alpha;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
#pragma unroll
      for (int e = 0; e < 16; ++e) st.o[cc][e] *= alpha;
    st.m = mn;
  }
  const float mu = st.m == -INFINITY ? 0.f : st.m;
  wave_lds_sync();
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    if (i0 + j >= n_own) break;
#pragma unroll
    for (int t = 0; t < NK; ++t)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        vt[(16 * t + 8 * h + e) * RG + 32 * j + n] = vg[j][t][e];
  }
  wave_lds_sync();
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    if (i0 + j >= n_own) break;
    float ps = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      sv[j][e] = __builtin_amdgcn_exp2f(fmaf(sv[j][e], sl2, -mu));
      ps += sv[j][e];
    }
    st.l += ps;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const v8 bp = pack8<T>(sv[j] + 8 * kb);
#pragma unroll
      for (int cc = 0; cc < NC; ++cc)
        st.o[cc] = M::mma(lds_a<T>(vt + (32 * cc + n) * RG + 32 * j + 16 * kb, h),
                          bp, st.o[cc]);
    }
  }
}

// Forward.  GROUPED: the tile's box fits one group of chunks (see
// fwd_group); otherwise chunks are software-pipelined one ahead.
template <typename T, int D, bool GROUPED>
__global__ void __launch_bounds__(256)
    k_mfwd(Prob P, Tiling Tl, const T *__restrict__ q, const T *__restrict__ k,
           const T *__restrict__ v, const T *__restrict__ ek,
           const T *__restrict__ ev, T *__restrict__ out,
           float *__restrict__ lse) {
  typedef Mf<T> M;
  typedef typename M::v8 v8;
  typedef typename M::e E;
  constexpr int NK = D / 16;  // k-steps over head_dim
  constexpr int NC = D / 32;  // 32-row output tiles over head_dim
  extern __shared__ __align__(16) char smem[];

  const int tile = xcd_tile(blockIdx.x, Tl.n_launch);
  if (tile >= Tl.n_q) return;
  const int W = blockDim.x >> 6, w = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63, n = lane & 31, h = lane >> 5;
  E *vt = reinterpret_cast<E *>(smem) + w * D * group_row(group_chunks(D));
  const QTile Q = query_tile(P, Tl, decode_tile(P, Tl, tile, Tl.fH), n);
  const int hk = Q.tc.head / P.rep;
  const float sl2 = P.scale * kLog2e;
  const int64_t qrow = (Q.qtok * P.H + Q.tc.head) * D;

  v8 qf[NK];
#pragma unroll
  for (int t = 0; t < NK; ++t)
    qf[t] = Q.q_valid ? ld8(q + qrow + 16 * t + 8 * h) : zero8<T>();

  Softmax<NC> st;
#pragma unroll
  for (int c = 0; c < NC; ++c) st.o[c] = zero16();
  st.m = -INFINITY;
  st.l = 0.f;

  const BoxAddr ka = box_addr(P, Q.tc, Q.bx, hk, P.Hkv);
  RowCursor rc{0, 0, 0};
  if constexpr (GROUPED) {
    // the whole box in one group of NB chunks (c = w, w + W, ...): every
    // K/V load is issued before the first chunk computes, then the
    // two-phase group softmax
    constexpr int NB = group_chunks(D);
    const int n_own = uni(Q.nbox > w ? (Q.nbox - w + W - 1) / W : 0);
    for (int i0 = 0; i0 < n_own; i0 += NB) {
      ChunkRows cr[NB];
      v8 kg[NB][NK], vg[NB][NK];
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        if (i0 + j >= n_own) break;
        const int c = w + W * (i0 + j);
        cr[j] = chunk_rows(rc, Q.bx, 32 * c);
        int e[3];
        box_point(Q.bx, cr[j], 32 * c, n, e);
        const int off = box_off(ka, e);
        load_kv<T, D>(k + ka.base + off, v + ka.base + off, kg[j], vg[j], h);
      }
      fwd_group<T, D, NB>(st, qf, kg, vg, cr, Q, w, W, i0, n_own, sl2, vt, n, h);
    }
  } else {
    // software-pipelined chunks: the next chunk's K/V loads are in flight
    // while the current chunk computes
    int c = w;
    ChunkRows cr{0, 0, 0};
    v8 kf[NK], vf[NK];
    if (c < Q.nbox) {
      cr = chunk_rows(rc, Q.bx, 32 * c);
      int e[3];
      box_point(Q.bx, cr, 32 * c, n, e);
      const int off = box_off(ka, e);
      load_kv<T, D>(k + ka.base + off, v + ka.base + off, kf, vf, h);
    }
    while (c < Q.nbox) {
      const int cn = c + W;
      ChunkRows crn = cr;
      v8 kn[NK], vn[NK];
      if (cn < Q.nbox) {
        crn = chunk_rows(rc, Q.bx, 32 * cn);
        int e[3];
        box_point(Q.bx, crn, 32 * cn, n, e);
        const int off = box_off(ka, e);
        load_kv<T, D>(k + ka.base + off, v + ka.base + off, kn, vn, h);
      }
      bool ok[16];
      chunk_mask(Q.bx, cr, 32 * c, h, Q.wlo, Q.ww, ok);
      fwd_compute<T, D>(st, qf, kf, vf, ok, sl2, vt, n, h);
      c = cn;
      cr = crn;
#pragma unroll
      for (int t = 0; t < NK; ++t) {
        kf[t] = kn[t];
        vf[t] = vn[t];
      }
    }
  }
  v8 kf[NK], vf[NK];
  for (int cx = first_owned(Q.nbox, w, W); cx < Q.nbox + Q.nextra; cx += W) {
    const int first = 32 * (cx - Q.nbox);
    const int ne = min(first + n, P.n_extra - 1);
    const int64_t row = (((int64_t)Q.tc.b * P.n_extra + ne) * P.Hkv + hk) * D;
    bool ok[16];
    extra_mask(Q.q_valid, first, P.n_extra, h, ok);
    load_kv<T, D>(ek + row, ev + row, kf, vf, h);
    fwd_compute<T, D>(st, qf, kf, vf, ok, sl2, vt, n, h);
  }

  float lt = st.l + __shfl_xor(st.l, 32);
  float m = st.m;
  if (W > 1) {
    // waves 1..W-1 hand (m, l, O^T) to wave 0, which merges them in order
    float *cb = reinterpret_cast<float *>(smem);
    __syncthreads();  // the combine area overlaps the transpose buffers
    if (w > 0) {
      float *mine = cb + (w - 1) * (D * 32 + 64);
#pragma unroll
      for (int cc = 0; cc < NC; ++cc)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          mine[(32 * cc + 8 * (e >> 2) + 4 * h + (e & 3)) * 32 + n] = st.o[cc][e];
      if (h == 0) {
        mine[D * 32 + n] = m;
        mine[D * 32 + 32 + n] = lt;
      }
    }
    __syncthreads();
    if (w > 0) return;
    for (int w2 = 1; w2 < W; ++w2) {
      const float *src = cb + (w2 - 1) * (D * 32 + 64);
      const float m2 = src[D * 32 + n];
      const float l2 = src[D * 32 + 32 + n];
      const float mn = fmaxf(m, m2);
      const float mu = mn == -INFINITY ? 0.f : mn;
      const float a0 = __builtin_amdgcn_exp2f(m - mu);
      const float a2 = __builtin_amdgcn_exp2f(m2 - mu);
#pragma unroll
      for (int cc = 0; cc < NC; ++cc)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          st.o[cc][e] = st.o[cc][e] * a0 +
                        src[(32 * cc + 8 * (e >> 2) + 4 * h + (e & 3)) * 32 + n] * a2;
      lt = lt * a0 + l2 * a2;
      m = mn;
    }
  }
  const float inv = (Q.q_valid && lt > 0.f) ? 1.f / lt : 0.f;
  if (Q.q_tensor) {
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        typename M::v4 wv;
#pragma unroll
        for (int j = 0; j < 4; ++j) wv[j] = (E)(st.o[cc][4 * i + j] * inv);
        *reinterpret_cast<typename M::v4 *>(out + qrow + 32 * cc + 8 * i + 4 * h) = wv;
      }
    if (lse != nullptr && h == 0)
      lse[qrow / D] = Q.q_valid ? (m + __log2f(lt)) * kLn2 : 0.f;
  }
}

// Sum partial f32x16 accumulators of waves 1..W-1 into wave 0 (in wave
// order).  Returns false for the waves that are done.
template <int NC, int NA>
__device__ __forceinline__ bool combine_sum(char *smem, int W, int w, int n,
                                            int h, f32x16 (*acc)[NC]) {
  if (W == 1) return true;
  float *cb = reinterpret_cast<float *>(smem);
  constexpr int PER = NA * NC * 16 * 64;  // floats per wave
  __syncthreads();
  if (w > 0) {
    float *mine = cb + (w - 1) * PER;
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int cc = 0; cc < NC; ++cc)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          mine[((a * NC + cc) * 16 + e) * 64 + h * 32 + n] = acc[a][cc][e];
  }
  __syncthreads();
  if (w > 0) return false;
  for (int w2 = 1; w2 < W; ++w2) {
    const float *src = cb + (w2 - 1) * PER;
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int cc = 0; cc < NC; ++cc)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          acc[a][cc][e] += src[((a * NC + cc) * 16 + e) * 64 + h * 32 + n];
  }
  return true;
}

// One 32-key chunk of the dQ role: S^T = K.Q^T, dP^T = V.dO^T,
// dS^T = P^T (dP^T - delta), dQ^T += K^T.dS^T (K^T via LDS).
template <typename T, int D>
__device__ __forceinline__ void dq_compute(f32x16 *acc,
                                           const typename Mf<T>::v8 *qf,
                                           const typename Mf<T>::v8 *df,
                                           const typename Mf<T>::v8 *kf,
                                           const typename Mf<T>::v8 *vf,
                                           const bool ok[16], float sl2,
                                           float lse2, float dl,
                                           typename Mf<T>::e *ta, int n,
                                           int h) {
  typedef Mf<T> M;
  typedef typename M::v8 v8;
  constexpr int NK = D / 16, NC = D / 32;
  f32x16 s = zero16(), dp = zero16();
#pragma unroll
  for (int t = 0; t < NK; ++t) {
    s = M::mma(kf[t], qf[t], s);
    dp = M::mma(vf[t], df[t], dp);
  }
  float ds[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const float p = ok[e] ? __builtin_amdgcn_exp2f(fmaf(s[e], sl2, -lse2)) : 0.f;
    ds[e] = p * (dp[e] - dl);
  }
  wave_lds_sync();
#pragma unroll
  for (int t = 0; t < NK; ++t)
#pragma unroll
    for (int e = 0; e < 8; ++e) ta[(16 * t + 8 * h + e) * kRow + n] = kf[t][e];
  wave_lds_sync();
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const v8 bs = pack8<T>(ds + 8 * kb);
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
      acc[cc] = M::mma(lds_a<T>(ta + (32 * cc + n) * kRow + 16 * kb, h), bs,
                       acc[cc]);
  }
}

// ---------------------------------------------------------------------------
// Backward: blocks [0, n_q) are dQ tiles, [n_q, n_q + n_k) dK/dV tiles.
template <typename T, int D>
__global__ void __launch_bounds__(256)
    k_mbwd(Prob P, Tiling Tl, const T *__restrict__ q, const T *__restrict__ k,
           const T *__restrict__ v, const T *__restrict__ ek,
           const T *__restrict__ ev, const T *__restrict__ out,
           const float *__restrict__ lse, const T *__restrict__ dout,
           const float *__restrict__ dlse, const float *__restrict__ delta,
           T *__restrict__ dq,
           T *__restrict__ dk, T *__restrict__ dv) {
  typedef Mf<T> M;
  typedef typename M::v8 v8;
  typedef typename M::e E;
  constexpr int NK = D / 16;
  constexpr int NC = D / 32;
  extern __shared__ __align__(16) char smem[];

  const int tile = xcd_tile(blockIdx.x, Tl.n_launch);
  if (tile >= Tl.n_q + Tl.n_k) return;
  const int W = blockDim.x >> 6, w = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63, n = lane & 31, h = lane >> 5;
  // Tiles come in groups of rep + 1 over one spatial tile of one KV head:
  // rep dQ tiles (one per query head of the group), then the dK/dV tile,
  // so both roles spread evenly over the XCDs and share the group's data.
  const uint32_t grp = fdiv((uint32_t)tile, Tl.fRep1);
  const int role = tile - (int)grp * (P.rep + 1);
  TileCtx tcg = decode_tile(P, Tl, (int)grp, Tl.fHk);
  // per-wave scratch: two transposed chunks + per-query lse / delta
  char *mys = smem + w * bwd_wave_lds(D, (int)sizeof(E));
  E *ta = reinterpret_cast<E *>(mys);                 // K^T (dQ) or Q^T (dK/dV)
  E *tb = ta + D * kRow;                              // dO^T (dK/dV)
  float *s_lse = reinterpret_cast<float *>(tb + D * kRow);
  float *s_del = s_lse + 32;
  E *kvs = reinterpret_cast<E *>(s_del + 32);         // K, V rows of a dK/dV tile
  const float sl2 = P.scale * kLog2e;

  if (role < P.rep) {
    // ------------------------------- dQ role -------------------------------
    const int hk = tcg.head;
    tcg.head = hk * P.rep + role;
    const QTile Q = query_tile(P, Tl, tcg, n);
    const int64_t qrow = (Q.qtok * P.H + Q.tc.head) * D;
    v8 qf[NK], df[NK];
    float dl = 0.f;
#pragma unroll
    for (int t = 0; t < NK; ++t) {
      qf[t] = Q.q_valid ? ld8(q + qrow + 16 * t + 8 * h) : zero8<T>();
      df[t] = Q.q_valid ? ld8(dout + qrow + 16 * t + 8 * h) : zero8<T>();
      if constexpr (!kPreDelta(D)) {
        const v8 of = Q.q_valid ? ld8(out + qrow + 16 * t + 8 * h) : zero8<T>();
#pragma unroll
        for (int e = 0; e < 8; ++e) dl = fmaf((float)df[t][e], (float)of[e], dl);
      }
    }
    const int64_t lrow = Q.qtok * P.H + Q.tc.head;
    if constexpr (kPreDelta(D)) {
      dl = Q.q_valid ? delta[lrow] : 0.f;
    } else {
      dl += __shfl_xor(dl, 32);
      if (Q.q_valid && dlse != nullptr) dl -= dlse[lrow];
    }
    const float lse2 = Q.q_valid ? lse[lrow] * kLog2e : 0.f;

    f32x16 acc[1][NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[0][c] = zero16();

    v8 kf[NK], vf[NK];
    if constexpr (kLeanBwd(D)) {
      // box chunks, loaded when used (see the dK/dV role on occupancy)
      const BoxAddr ka = box_addr(P, Q.tc, Q.bx, hk, P.Hkv);
      RowCursor rc{0, 0, 0};
      for (int c = w; c < Q.nbox; c += W) {
        const ChunkRows cr = chunk_rows(rc, Q.bx, 32 * c);
        int e[3];
        box_point(Q.bx, cr, 32 * c, n, e);
        const int off = box_off(ka, e);
        load_kv<T, D>(k + ka.base + off, v + ka.base + off, kf, vf, h);
        bool ok[16];
        chunk_mask(Q.bx, cr, 32 * c, h, Q.wlo, Q.ww, ok);
        dq_compute<T, D>(acc[0], qf, df, kf, vf, ok, sl2, lse2, dl, ta, n, h);
      }
    } else {
      // software-pipelined chunks: the next chunk's K/V loads are in flight
      // while the current chunk computes
      const BoxAddr ka = box_addr(P, Q.tc, Q.bx, hk, P.Hkv);
      RowCursor rc{0, 0, 0};
      int c = w;
      ChunkRows cr{0, 0, 0};
      if (c < Q.nbox) {
        cr = chunk_rows(rc, Q.bx, 32 * c);
        int e[3];
        box_point(Q.bx, cr, 32 * c, n, e);
        const int off = box_off(ka, e);
        load_kv<T, D>(k + ka.base + off, v + ka.base + off, kf, vf, h);
      }
      while (c < Q.nbox) {
        const int cn = c + W;
        ChunkRows crn = cr;
        v8 kn[NK], vn[NK];
        if (cn < Q.nbox) {
          crn = chunk_rows(rc, Q.bx, 32 * cn);
          int e[3];
          box_point(Q.bx, crn, 32 * cn, n, e);
          const int off = box_off(ka, e);
          load_kv<T, D>(k + ka.base + off, v + ka.base + off, kn, vn, h);
        }
        bool ok[16];
        chunk_mask(Q.bx, cr, 32 * c, h, Q.wlo, Q.ww, ok);
        dq_compute<T, D>(acc[0], qf, df, kf, vf, ok, sl2, lse2, dl, ta, n, h);
        c = cn;
        cr = crn;
#pragma unroll
        for (int t = 0; t < NK; ++t) {
          kf[t] = kn[t];
          vf[t] = vn[t];
        }
      }
    }
    for (int cx = first_owned(Q.nbox, w, W); cx < Q.nbox + Q.nextra; cx += W) {
      const int first = 32 * (cx - Q.nbox);
      const int ne = min(first + n, P.n_extra - 1);
      const int64_t row = (((int64_t)Q.tc.b * P.n_extra + ne) * P.Hkv + hk) * D;
      bool ok[16];
      extra_mask(Q.q_valid, first, P.n_extra, h, ok);
      load_kv<T, D>(ek + row, ev + row, kf, vf, h);
      dq_compute<T, D>(acc[0], qf, df, kf, vf, ok, sl2, lse2, dl, ta, n, h);
    }
    if (!combine_sum<NC, 1>(smem, W, w, n, h, acc)) return;
    if (Q.q_tensor) {
#pragma unroll
      for (int cc = 0; cc < NC; ++cc)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          typename M::v4 wv;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            wv[j] = (E)(Q.q_valid ? acc[0][cc][4 * i + j] * P.scale : 0.f);
          *reinterpret_cast<typename M::v4 *>(dq + qrow + 32 * cc + 8 * i + 4 * h) = wv;
        }
    }
    return;
  }

  // ------------------------------ dK/dV role -------------------------------
  const TileCtx tc = tcg;
  const int hk = tc.head;
  int u[3];
  tile_slot(Tl, n, u);
  const bool k_tensor = (u[0] < tc.nt[0]) & (u[1] < tc.nt[1]) & (u[2] < tc.nt[2]);
  const bool k_valid = (u[0] < tc.nv[0]) & (u[1] < tc.nv[1]) & (u[2] < tc.nv[2]);
  const bool any = (tc.nv[0] > 0) & (tc.nv[1] > 0) & (tc.nv[2] > 0);
  int pos[3], Lr[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    pos[a] = tc.r[a] + P.ax[a].d * (tc.i0[a] + u[a]);
    Lr[a] = P.ax[a].d == 1 ? tc.L[a]
            : tc.L[a] > tc.r[a]
                ? (int)fdiv((uint32_t)(tc.L[a] - 1 - tc.r[a]), Tl.fd[a]) + 1
                : 0;
  }
  const int64_t krow =
      (tok_in(P, tc.b, pos[0], pos[1], pos[2]) * P.Hkv + hk) * D;

  // query box = union of the tile keys' inverse neighborhoods
  Box bx;
  int wlo[3], ww[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    int lo0 = 0, hi0 = 0, lo1 = 0, hi1 = 0;
    if (any) {
      sub_inverse(P, Tl, a, tc.L[a], tc.r[a], Lr[a], tc.i0[a], lo0, hi0);
      sub_inverse(P, Tl, a, tc.L[a], tc.r[a], Lr[a], tc.i0[a] + tc.nv[a] - 1,
                  lo1, hi1);
    }
    bx.lo[a] = uni(lo0);
    bx.E[a] = uni(any ? max(hi1 - lo0 + 1, 1) : 1);
    int lo = 0, hi = -1;
    if (k_valid)
      sub_inverse(P, Tl, a, tc.L[a], tc.r[a], Lr[a], tc.i0[a] + u[a], lo, hi);
    wlo[a] = lo - bx.lo[a];
    ww[a] = k_valid ? max(hi - lo + 1, 0) : 0;
  }
  box_init(bx);
  bx.lgP = uni(bx.lgP);
  const int nchunk = uni(any ? (bx.slots + 31) >> 5 : 0);

  // the tile's K and V rows (B operands of every chunk): in LDS for the
  // lean variant, whose register peak sets the kernel's occupancy, else in
  // registers
  v8 kf[NK], vf[NK];
  if constexpr (kLeanBwd(D)) {
    E *kr = kvs + n * kKvRow(D);
    E *vr = kvs + (32 + n) * kKvRow(D);
#pragma unroll
    for (int t = 0; t < NK; ++t) {
      *reinterpret_cast<v8 *>(kr + 16 * t + 8 * h) =
          k_valid ? ld8(k + krow + 16 * t + 8 * h) : zero8<T>();
      *reinterpret_cast<v8 *>(vr + 16 * t + 8 * h) =
          k_valid ? ld8(v + krow + 16 * t + 8 * h) : zero8<T>();
    }
  } else {
#pragma unroll
    for (int t = 0; t < NK; ++t) {
      kf[t] = k_valid ? ld8(k + krow + 16 * t + 8 * h) : zero8<T>();
      vf[t] = k_valid ? ld8(v + krow + 16 * t + 8 * h) : zero8<T>();
    }
  }
  const E *kfl = kvs + n * kKvRow(D) + 8 * h;
  const E *vfl = kvs + (32 + n) * kKvRow(D) + 8 * h;
  f32x16 acc[2][NC];  // [0] = dK^T, [1] = dV^T
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    acc[0][c] = zero16();
    acc[1][c] = zero16();
  }

  for (int hq = hk * P.rep; hq < (hk + 1) * P.rep; ++hq) {
    const BoxAddr qa_addr = box_addr(P, tc, bx, hq, P.H);
    const int64_t lbase = qa_addr.base / D;  // lse/dlse/delta offset of the box origin
    if constexpr (kLeanBwd(D)) {
      // query chunks; padding slots load a real (clamped) query and the mask
      // removes them.  No next-chunk prefetch here: this role's register peak
      // sets the whole kernel's occupancy, and at four waves per SIMD the
      // other resident waves hide the chunk loads instead.
      RowCursor rc{0, 0, 0};
      for (int c = w; c < nchunk; c += W) {
        const ChunkRows cr = chunk_rows(rc, bx, 32 * c);
        v8 qa[NK], da[NK];
        float dl = 0.f, lsev, dlsev;
        {
          int e[3];
          box_point(bx, cr, 32 * c, n, e);
          const int off = box_off(qa_addr, e);
          const int64_t qrow = qa_addr.base + off;
          const int64_t lrow = lbase + off / D;
          v8 oa[NK];
#pragma unroll
          for (int t = 0; t < NK; ++t) {
            qa[t] = ld8(q + qrow + 16 * t + 8 * h);
            da[t] = ld8(dout + qrow + 16 * t + 8 * h);
            oa[t] = ld8(out + qrow + 16 * t + 8 * h);
          }
          lsev = lse[lrow];
          dlsev = dlse != nullptr ? dlse[lrow] : 0.f;
#pragma unroll
          for (int t = 0; t < NK; ++t)
#pragma unroll
            for (int i = 0; i < 8; ++i) dl = fmaf((float)da[t][i], (float)oa[t][i], dl);
        }
        dl += __shfl_xor(dl, 32);
        dl -= dlsev;
        const float l2 = lsev * kLog2e;

        wave_lds_sync();
#pragma unroll
        for (int t = 0; t < NK; ++t)
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            ta[(16 * t + 8 * h + i) * kRow + n] = qa[t][i];
            tb[(16 * t + 8 * h + i) * kRow + n] = da[t][i];
          }
        if (h == 0) {
          s_lse[n] = l2;
          s_del[n] = dl;
        }
        wave_lds_sync();

        f32x16 s = zero16(), dp = zero16();
#pragma unroll
        for (int t = 0; t < NK; ++t) {
          s = M::mma(qa[t], *reinterpret_cast<const v8 *>(kfl + 16 * t), s);
          dp = M::mma(da[t], *reinterpret_cast<const v8 *>(vfl + 16 * t), dp);
        }
        bool ok[16];
        chunk_mask(bx, cr, 32 * c, h, wlo, ww, ok);
        float p[16], ds[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 l4 = *reinterpret_cast<const float4 *>(s_lse + 8 * i + 4 * h);
          const float4 d4 = *reinterpret_cast<const float4 *>(s_del + 8 * i + 4 * h);
          const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
          const float dv4[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int e2 = 4 * i + j;
            p[e2] = ok[e2] ? __builtin_amdgcn_exp2f(fmaf(s[e2], sl2, -lv[j])) : 0.f;
            ds[e2] = p[e2] * (dp[e2] - dv4[j]);
          }
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const v8 bp = pack8<T>(p + 8 * kb);
          const v8 bs = pack8<T>(ds + 8 * kb);
#pragma unroll
          for (int cc = 0; cc < NC; ++cc) {
            acc[1][cc] = M::mma(lds_a<T>(tb + (32 * cc + n) * kRow + 16 * kb, h),
                                bp, acc[1][cc]);
            acc[0][cc] = M::mma(lds_a<T>(ta + (32 * cc + n) * kRow + 16 * kb, h),
                                bs, acc[0][cc]);
          }
        }
      }
    } else {
      // query chunks, software-pipelined like the forward; padding slots
      // load a real (clamped) query and the mask removes them
      RowCursor rc{0, 0, 0};
      int c = w;
      ChunkRows cr{0, 0, 0};
      v8 qa[NK], da[NK];
      float lsev = 0.f, delv = 0.f;
      if (c < nchunk) {
        cr = chunk_rows(rc, bx, 32 * c);
        int e[3];
        box_point(bx, cr, 32 * c, n, e);
        const int off = box_off(qa_addr, e);
        const int64_t qrow = qa_addr.base + off;
        const int64_t lrow = lbase + off / D;
#pragma unroll
        for (int t = 0; t < NK; ++t) {
          qa[t] = ld8(q + qrow + 16 * t + 8 * h);
          da[t] = ld8(dout + qrow + 16 * t + 8 * h);
        }
        lsev = lse[lrow];
        delv = delta[lrow];
      }
      while (c < nchunk) {
        const int cn = c + W;
        ChunkRows crn = cr;
        v8 qn[NK], dn[NK];
        float lsen = 0.f, deln = 0.f;
        if (cn < nchunk) {
          crn = chunk_rows(rc, bx, 32 * cn);
          int e[3];
          box_point(bx, crn, 32 * cn, n, e);
          const int off = box_off(qa_addr, e);
          const int64_t qrow = qa_addr.base + off;
          const int64_t lrow = lbase + off / D;
#pragma unroll
          for (int t = 0; t < NK; ++t) {
            qn[t] = ld8(q + qrow + 16 * t + 8 * h);
            dn[t] = ld8(dout + qrow + 16 * t + 8 * h);
          }
          lsen = lse[lrow];
          deln = delta[lrow];
        }
        const float dl = delv;
        const float l2 = lsev * kLog2e;

        wave_lds_sync();
#pragma unroll
        for (int t = 0; t < NK; ++t)
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            ta[(16 * t + 8 * h + i) * kRow + n] = qa[t][i];
            tb[(16 * t + 8 * h + i) * kRow + n] = da[t][i];
          }
        if (h == 0) {
          s_lse[n] = l2;
          s_del[n] = dl;
        }
        wave_lds_sync();

        f32x16 s = zero16(), dp = zero16();
#pragma unroll
        for (int t = 0; t < NK; ++t) {
          s = M::mma(qa[t], kf[t], s);
          dp = M::mma(da[t], vf[t], dp);
        }
        bool ok[16];
        chunk_mask(bx, cr, 32 * c, h, wlo, ww, ok);
        float p[16], ds[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 l4 = *reinterpret_cast<const float4 *>(s_lse + 8 * i + 4 * h);
          const float4 d4 = *reinterpret_cast<const float4 *>(s_del + 8 * i + 4 * h);
          const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
          const float dv4[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int e2 = 4 * i + j;
            p[e2] = ok[e2] ? __builtin_amdgcn_exp2f(fmaf(s[e2], sl2, -lv[j])) : 0.f;
            ds[e2] = p[e2] * (dp[e2] - dv4[j]);
          }
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const v8 bp = pack8<T>(p + 8 * kb);
          const v8 bs = pack8<T>(ds + 8 * kb);
#pragma unroll
          for (int cc = 0; cc < NC; ++cc) {
            acc[1][cc] = M::mma(lds_a<T>(tb + (32 * cc + n) * kRow + 16 * kb, h),
                                bp, acc[1][cc]);
            acc[0][cc] = M::mma(lds_a<T>(ta + (32 * cc + n) * kRow + 16 * kb, h),
                                bs, acc[0][cc]);
          }
        }
        c = cn;
        cr = crn;
        lsev = lsen;
        delv = deln;
#pragma unroll
        for (int t = 0; t < NK; ++t) {
          qa[t] = qn[t];
          da[t] = dn[t];
        }
      }
    }
  }
  if (!combine_sum<NC, 2>(smem, W, w, n, h, acc)) return;
  if (k_tensor) {
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        typename M::v4 wk, wv;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          wk[j] = (E)(k_valid ? acc[0][cc][4 * i + j] * P.scale : 0.f);
          wv[j] = (E)(k_valid ? acc[1][cc][4 * i + j] : 0.f);
        }
        *reinterpret_cast<typename M::v4 *>(dk + krow + 32 * cc + 8 * i + 4 * h) = wk;
        *reinterpret_cast<typename M::v4 *>(dv + krow + 32 * cc + 8 * i + 4 * h) = wv;
      }
  }
}

// ---------------------------------------------------------------------------
// Host side: LDS sizes, eligibility, launch.

// Waves up to which the whole forward launch is resident at once (two per
// SIMD on 256 CUs x 4 SIMDs at the grouped kernel's register use).
constexpr int64_t kGroupedMaxWaves = 2048;

size_t fwd_lds(int D, int W, int esize) {
  const size_t tr = (size_t)W * D * group_row(group_chunks(D)) * esize;
  const size_t cb = (size_t)(W - 1) * (D * 32 + 64) * sizeof(float);
  return tr > cb ? tr : cb;
}

size_t bwd_lds(int D, int W, int esize) {
  const size_t tr = (size_t)W * bwd_wave_lds(D, esize);
  const size_t cb = (size_t)(W - 1) * 2 * (D / 32) * 16 * 64 * sizeof(float);
  return tr > cb ? tr : cb;
}

}  // namespace

bool mfma_eligible(const Prob &P, int dtype) {
  if (dtype != NA_BF16 && dtype != NA_F16) return false;
  if (P.D != 32 && P.D != 64 && P.D != 128) return false;
  // the forward folds the scale into the exponent after taking the max of
  // raw scores, which needs a positive finite scale
  if (!(P.scale > 0.f) || !std::isfinite(P.scale)) return false;
  for (int a = 0; a < 3; ++a) {
    const Axis &x = P.ax[a];
    if (x.s != 1) return false;
    if (!P.dense && !x.causal && (x.K % 2) == 0) return false;
  }
  return true;
}

#define NA_MFMA_D(D_, BODY)      \
  do {                           \
    if ((D_) == 32) {            \
      BODY(32);                  \
    } else if ((D_) == 64) {     \
      BODY(64);                  \
    } else {                     \
      BODY(128);                 \
    }                            \
  } while (0)

void mfma_fwd(const Prob &P, int dtype, const void *q, const void *k,
              const void *v, const void *ek, const void *ev, void *out,
              float *lse, hipStream_t st) {
  double chunks = 1.0;
  Tiling Tl = choose_tiling(P, P.H, P.Hkv, &chunks);
  Tl.n_launch = (Tl.n_q + 7) & ~7;
  if (Tl.n_q == 0) return;
  const int W = waves_for(chunks, 4, "NATTEN_AMD_FWD_WAVES");
  const size_t lds = fwd_lds(P.D, W, 2);
  // The grouped kernel trades occupancy (more VGPRs) for one memory wait
  // per tile: a gain only while the launch is a single round of waves.
  // Box chunks per tile (the cost model's count includes additional tokens):
  const double box_chunks = chunks - std::ceil(P.n_extra / 32.0);
#define FWD_(DD)                                                               \
  do {                                                                         \
    const bool grouped = std::ceil(box_chunks / W) <= group_chunks(DD) &&      \
                         (int64_t)Tl.n_q * W <= kGroupedMaxWaves;              \
    if (dtype == NA_BF16) {                                                    \
      if (grouped) FWD_LAUNCH(bf16_t, DD, true); else FWD_LAUNCH(bf16_t, DD, false); \
    } else {                                                                   \
      if (grouped) FWD_LAUNCH(f16_t, DD, true); else FWD_LAUNCH(f16_t, DD, false); \
    }                                                                          \
  } while (0)
#define FWD_LAUNCH(TT, DD, GG)                                                 \
  hipLaunchKernelGGL((k_mfwd<TT, DD, GG>), dim3(Tl.n_launch), dim3(64 * W),   \
                     lds, st, P, Tl, (const TT *)q, (const TT *)k,             \
                     (const TT *)v, (const TT *)ek, (const TT *)ev, (TT *)out, \
                     lse)
  NA_MFMA_D(P.D, FWD_);
#undef FWD_LAUNCH
#undef FWD_
}

bool mfma_bwd_reads_delta(const Prob &P) { return kPreDelta(P.D); }

void mfma_bwd(const Prob &P, int dtype, const void *q, const void *k,
              const void *v, const void *ek, const void *ev, const void *out,
              const float *lse, const void *dout, const float *dlse,
              const float *delta, void *dq, void *dk, void *dv,
              hipStream_t st) {
  double chunks = 1.0;
  Tiling Tl = choose_tiling(P, P.H, P.Hkv, &chunks);
  Tl.n_launch = (Tl.n_q + Tl.n_k + 7) & ~7;
  if (Tl.n_q + Tl.n_k == 0) return;
  const int W = waves_for(chunks * P.rep, P.D >= 128 ? 2 : 4, "NATTEN_AMD_BWD_WAVES");
  const size_t lds = bwd_lds(P.D, W, 2);
#define BWD_(DD)                                                               \
  if (dtype == NA_BF16)                                                        \
    hipLaunchKernelGGL((k_mbwd<bf16_t, DD>), dim3(Tl.n_launch), dim3(64 * W),   \
                       lds, st, P, Tl, (const bf16_t *)q, (const bf16_t *)k,   \
                       (const bf16_t *)v, (const bf16_t *)ek,                  \
                       (const bf16_t *)ev, (const bf16_t *)out, lse,           \
                       (const bf16_t *)dout, dlse, delta, (bf16_t *)dq,        \
                       (bf16_t *)dk,                                           \
                       (bf16_t *)dv);                                          \
  else                                                                         \
    hipLaunchKernelGGL((k_mbwd<f16_t, DD>), dim3(Tl.n_launch), dim3(64 * W),    \
                       lds, st, P, Tl, (const f16_t *)q, (const f16_t *)k,     \
                       (const f16_t *)v, (const f16_t *)ek,                    \
                       (const f16_t *)ev, (const f16_t *)out, lse,             \
                       (const f16_t *)dout, dlse, delta, (f16_t *)dq,          \
                       (f16_t *)dk,                                            \
                       (f16_t *)dv)
  NA_MFMA_D(P.D, BWD_);
#undef BWD_
}

void mfma_selftest(int dtype, float *out, hipStream_t st) {
  if (dtype == NA_BF16)
    hipLaunchKernelGGL(k_selftest<bf16_t>, dim3(1), dim3(64), 0, st, out);
  else
    hipLaunchKernelGGL(k_selftest<f16_t>, dim3(1), dim3(64), 0, st, out);
}

}  // namespace na
