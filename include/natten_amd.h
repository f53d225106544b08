/*
 * natten_amd.h — C ABI of the MI355X (gfx950) neighborhood-attention library
 * (libnatten_amd.so).
 *
 * The library replaces the accelerated tiers behind natten-mlx's backend
 * registry (reference: src/natten_mlx/_core/ops.py:14-135, the nanobind
 * module src/natten_mlx/_core/_nanobind_ext.cpp:22-278 and the Metal
 * kernels under src/natten_mlx/_core/nanobind/ and _core/_metal_sources.py).
 * Every entry point works on caller-owned device buffers in the reference's
 * spatial-first layout and never allocates or frees device memory:
 *
 *   query / out / dq          [B, X0, X1, X2, H,    D]   (rank < 3: leading X = 1)
 *   key / value / dk / dv     [B, X0, X1, X2, H_kv, D]
 *   extra key / value         [B, N_extra, H_kv, D]
 *   logits / attn             [B, O0, O1, O2, H, K0*K1*K2]   O_a = ceil(X_a / stride_a)
 *   lse / dlse                [B, O0, O1, O2, H]  float32
 *
 * All tensors are dense and contiguous.  Query head h reads key/value head
 * h / (H / H_kv) (GQA/MQA without materialising the repeat, reference
 * functional.py:29-68).  Launches are asynchronous on the caller's HIP stream
 * (a hipStream_t passed as void*, NULL = default stream); nothing
 * synchronises the device.  Return value: NA_OK or an NA_ERR_* code, with a
 * thread-local message in na_last_error().  No C++ exception crosses the ABI.
 */
#ifndef NATTEN_AMD_H
#define NATTEN_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NA_ABI_VERSION 2

enum na_dtype { NA_F32 = 0, NA_F16 = 1, NA_BF16 = 2 };

enum na_status {
  NA_OK = 0,
  NA_ERR_INVALID = 1,     /* malformed parameters or shapes */
  NA_ERR_UNSUPPORTED = 2, /* valid request this build does not implement */
  NA_ERR_LAUNCH = 3,      /* HIP launch / runtime failure */
  NA_ERR_WORKSPACE = 4    /* workspace missing or too small */
};

/* na_params.flags */
enum na_flags {
  /* Every query attends to every key of its sample (the FMHA fast path of
   * functional.py:141-187, taken when the kernel covers the extent). */
  NA_FLAG_DENSE = 1,
  /* Run the generic vector-ALU kernels even where the matrix-core kernels
   * apply (for A/B comparison of the two implementations). */
  NA_FLAG_GENERIC = 2,
  /* Run the 32-query matrix-core kernels where the lean workgroup kernels
   * would apply (A/B comparison; see na_kernel_path). */
  NA_FLAG_NO_LEAN = 4,
  /* With sample_extent: the caller has checked that every sample extent
   * satisfies dilation * kernel_size <= extent on each non-causal axis.
   * Lets na_fwd and na_bwd run such problems on the lean kernels; a sample
   * that breaks the promise gets wrong values in its rows (every memory
   * access stays inside the tensors). */
  NA_FLAG_VARLEN_CLAMPED = 8
};

/*
 * Problem description shared by every entry point.  Per-axis arrays are
 * given for rank axes in order (X0 = depth, X1 = height, X2 = width for
 * rank 3; X0 = length for rank 1) and are normalised internally to three
 * axes by prepending unit axes.  Mirrors the normalised tuples the
 * reference backends receive (ops.py:49-135).
 */
typedef struct na_params {
  int32_t rank;        /* 1, 2 or 3 */
  int32_t batch;       /* B */
  int32_t heads;       /* H (query heads) */
  int32_t kv_heads;    /* H_kv, divides H */
  int32_t head_dim;    /* D */
  int32_t dtype;       /* enum na_dtype of q/k/v/out (and logits/attn) */
  int32_t extent[3];   /* spatial size per axis (the padded maximum for varlen) */
  int32_t kernel[3];   /* neighborhood size per axis */
  int32_t dilation[3];
  int32_t stride[3];
  int32_t causal[3];   /* 0 / 1 per axis */
  float scale;         /* logit scale (the caller resolves None -> D^-0.5) */
  int32_t n_extra;     /* number of additional (global) key/value tokens */
  int32_t flags;       /* enum na_flags */
  /* Optional device pointer to int32 [batch, rank] per-sample extents
   * (varlen, functional.py:697-828); NULL = every sample uses extent[]. */
  const int32_t *sample_extent;
} na_params;

int na_abi_version(void);
const char *na_last_error(void);

/* ---- window math: host twins of the device helpers (bit-exact) --------- */
/* utils/window.py:8-34 */
int32_t na_window_start(int32_t index, int32_t length, int32_t kernel_size,
                        int32_t neighborhood_size, int32_t dilation);
/* utils/window.py:37-39 */
int32_t na_window_end(int32_t start, int32_t length, int32_t kernel_size,
                      int32_t dilation);
/* utils/window.py:42-62 (also extras/allin1/reference_impl.py:32-45) */
int32_t na_pb_start(int32_t index, int32_t length, int32_t kernel_size,
                    int32_t neighborhood_size, int32_t dilation);
/* dilation-partition form, extras/allin1/reference_impl.py:13-25 */
int32_t na_window_start_partition(int32_t index, int32_t length,
                                  int32_t kernel_size,
                                  int32_t neighborhood_size, int32_t dilation);

/*
 * Device-computed neighbor table for checking the device helpers: writes
 * the clipped linear key index (int32) and validity (uint8) of every
 * (output position, kernel slot) pair, [O0, O1, O2, K0*K1*K2] each, exactly
 * as pure.py:24-152 builds them.  Uses extent[], not sample_extent.
 */
int na_neighbor_table(const na_params *p, int32_t *index, uint8_t *valid,
                      void *stream);

/*
 * Diagnostic with no counterpart in the reference: multiplies two fixed
 * small-integer matrices (A 32x16, B 16x32) with one matrix-core
 * instruction in `dtype` (NA_BF16 / NA_F16) using the operand and result
 * lane layouts the kernels assume, and writes C = A.B as float32 [32][32]
 * row-major into `out` (device).  A[m][k] = (m + 2k) % 7 - 3,
 * B[k][n] = (3k + n) % 5 - 2.
 */
int na_mfma_selftest(int32_t dtype, float *out, void *stream);

/*
 * Diagnostic with no counterpart in the reference: the kernel family that
 * na_fwd (backward = 0), na_bwd (backward = 1) or the split ops na_qk_fwd /
 * na_av_fwd / na_qk_bwd / na_av_bwd (backward = 2) run for these
 * parameters, one of na_kernel_path_t, or the negated na_status of invalid
 * parameters.  Launches nothing and reads no device memory.
 */
enum na_kernel_path_t {
  NA_PATH_GENERIC = 0, /* vector-ALU kernels: every dtype / head_dim / stride */
  NA_PATH_MFMA = 1,    /* 32-query matrix-core kernels */
  NA_PATH_LEAN = 2,    /* workgroup-staged 16x16x32 matrix-core kernels */
  NA_PATH_DENSE = 3    /* dense (FMHA) kernels: key or query tiles streamed
                          through LDS */
};
int na_kernel_path(const na_params *p, int32_t backward);

/*
 * Diagnostic with no counterpart in the reference: how na_fwd (backward =
 * 0) or na_bwd (backward = 1) launches for these parameters.  Fields past
 * `path` describe the lean kernels and are 0 on the other paths.  Launches
 * nothing and reads no device memory; returns NA_OK or an NA_ERR_* code.
 */
typedef struct na_plan {
  int32_t path;            /* na_kernel_path_t */
  int32_t tile[3];         /* queries per wave along the three axes */
  int32_t waves;           /* waves per workgroup */
  int32_t box[3];          /* largest staged key box (backward: also the
                              query box of a key tile) */
  int32_t slabs;           /* pieces along axis 0 the box is staged in */
  int32_t grouped_heads;   /* forward: query heads a workgroup runs over one
                              staged box of their key/value head (0: one
                              head per workgroup) */
  int32_t workgroups;      /* workgroups launched */
  int32_t lds_bytes;       /* LDS per workgroup */
  int32_t extra_reduction; /* backward with additional tokens: their
                              gradients on 1 = vector ALU, 2 = matrix cores
                              (0 on the dense path: they are keys of its
                              key-side kernel) */
} na_plan;
int na_kernel_plan(const na_params *p, int32_t backward, na_plan *plan);

/* ---- fused neighborhood attention --------------------------------------- */
/*
 * out = softmax(scale * q k_nbr^T masked) v_nbr over each query's window
 * (plus the n_extra additional tokens, joined into the same softmax, which
 * equals the reference's merge_attentions composition, functional.py:277-292).
 * lse (float32, natural log) may be NULL.  Replaces na{1,2,3}d_forward
 * (ops.py:49-58; pure.py:155-255; fast_metal.py:2524-2763) and the
 * varlen forward (autograd/na1d.py:76-80; pure.py:497-688).  Queries beyond
 * a sample's extent get out = 0 and lse = 0.
 */
int na_fwd(const na_params *p, const void *q, const void *k, const void *v,
           const void *extra_k, const void *extra_v, void *out, float *lse,
           void *stream);

/* Bytes of device workspace na_bwd needs for these parameters. */
size_t na_bwd_workspace_bytes(const na_params *p);

/*
 * Gradients of the fused op given out, lse (from na_fwd) and dout; dlse
 * (gradient w.r.t. the returned lse, float32) may be NULL.  Writes dq, dk,
 * dv in full (zero where nothing contributes: non-strided query positions,
 * varlen padding) and, when n_extra > 0 and the pointers are non-NULL, the
 * additional-token gradients.  Deterministic: no atomics.  Replaces
 * na{1,2,3}d_backward (ops.py:100-110) and the fused SIMD backward that the
 * VJP calls directly (autograd/na2d.py:34-53; fast_metal.py:2390-2521).
 */
int na_bwd(const na_params *p, const void *q, const void *k, const void *v,
           const void *extra_k, const void *extra_v, const void *out,
           const float *lse, const void *dout, const float *dlse, void *dq,
           void *dk, void *dv, void *d_extra_k, void *d_extra_v,
           void *workspace, size_t workspace_bytes, void *stream);

/*
 * na_bwd without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  The workspace
 * is a fixed device array inside the library, one per GPU, of
 * na_bwd_noalloc_max_workspace() bytes (32 MiB); problems whose
 * na_bwd_workspace_bytes exceeds it are rejected with NA_ERR_UNSUPPORTED.
 * Allocates nothing (no hipMalloc / hipFree).  Every call on a GPU shares
 * that GPU's array: calls that overlap on one GPU (on different streams or
 * threads) race and must be serialised by the caller.
 */
size_t na_bwd_noalloc_max_workspace(void);
int na_bwd_noalloc(const na_params *p, const void *q, const void *k,
                   const void *v, const void *extra_k, const void *extra_v,
                   const void *out, const float *lse, const void *dout,
                   const float *dlse, void *dq, void *dk, void *dv,
                   void *d_extra_k, void *d_extra_v, void *stream);

/* ---- split operators ----------------------------------------------------- */
/* logits = scale * <q, k_nbr>, -inf for invalid slots; ops.py:61-80,
 * pure.py:258-283,320-359,404-449.  logits in p->dtype. */
int na_qk_fwd(const na_params *p, const void *q, const void *k, void *logits,
              void *stream);
/* out = sum over valid slots attn * v_nbr; pure.py:286-317,362-401,452-494. */
int na_av_fwd(const na_params *p, const void *attn, const void *v, void *out,
              void *stream);
/* (dq, dk) of na_qk_fwd; ops.py:112-131, pure.py:739-808. */
int na_qk_bwd(const na_params *p, const void *q, const void *k,
              const void *dlogits, void *dq, void *dk, void *stream);
/* (dattn, dv) of na_av_fwd; ops.py:116-135, pure.py:750-808. */
int na_av_bwd(const na_params *p, const void *attn, const void *v,
              const void *dout, void *dattn, void *dv, void *stream);

/* ---- DiNAT all-in-one operators (extras/allin1) -------------------------- */
/*
 * Square window of side `kernel` with one dilation on every axis, rank 1
 * ([B, L, H, X]) or rank 2 ([B, Hh, Hw, H, X]); heads_first = 1 selects the
 * [B, H, L, X] / [B, H, Hh, Hw, X] layout of the lower-level
 * natten{1,2}d* functions.  Windows use the dilation-partition start; slot
 * (k0, k1) is n = k0*K + k1; the bias row of slot k on an axis is
 * clip(pb_start + k, 0, 2K-2).  rpb: float32 [H, 2K-1] (rank 1) or
 * [H, 2K-1, 2K-1] (rank 2).
 */
typedef struct na_rpb_params {
  int32_t rank;        /* 1 or 2 */
  int32_t batch;
  int32_t heads;
  int32_t head_dim;
  int32_t extent[2];   /* L, or (Hh, Hw) */
  int32_t kernel[2];   /* window side per axis (axis 1 unused for rank 1) */
  int32_t dilation[2]; /* dilation per axis (axis 1 unused for rank 1) */
  int32_t heads_first; /* 0: spatial-first rows, 1: heads-first rows */
  int32_t dtype;       /* q / key / value and their gradients */
  float scale;         /* query scale, applied in `dtype` before the dot */
  int32_t has_scale;   /* 0: no scaling (scale=None) */
} na_rpb_params;

/*
 * logits[.., n] = <round(q * scale), key_nbr(n)> + rpb[h, bias rows of n],
 * -inf for invalid slots; logits float32 with K^rank slots per row.
 * rpb may be NULL (zero bias).  Replaces extras/allin1/__init__.py:40-79
 * (na1d_qk_rpb), :112-150 (na2d_qk_rpb); functional_metal.py:1125-1161,
 * 1921-1976.
 */
int na_rpb_qk_fwd(const na_rpb_params *p, const void *q, const void *key,
                  const float *rpb, float *logits, void *stream);
/*
 * out = sum over valid slots attn * value_nbr; attn float32; out in
 * out_dtype (NA_F32 as the reference's Metal kernels, or p->dtype as its
 * MLX fallback).  Replaces extras/allin1/__init__.py:82-109 (na1d_av_fused),
 * :153-180 (na2d_av_fused); functional_metal.py:1164-1199, 1979-2033.
 */
int na_rpb_av_fwd(const na_rpb_params *p, const float *attn, const void *value,
                  void *out, int32_t out_dtype, void *stream);
/* Workspace na_rpb_qk_bwd needs when drpb is requested. */
size_t na_rpb_bwd_workspace_bytes(const na_rpb_params *p);
/*
 * Gradients of na_rpb_qk_fwd: dq = scale * sum dlogits * key_nbr,
 * dk[j] = sum over queries holding j of dlogits * round(q * scale),
 * drpb[h, r] = sum of dlogits over the slots whose bias row is r (float32,
 * deterministic).  Any of dq / dk / drpb may be NULL (not computed).
 * Replaces functional_metal.py:1206-1338 (natten1dqkrpb_backward),
 * 1418-1590 (natten2dqkrpb_backward), 2172-2192, 2216-2244.
 */
int na_rpb_qk_bwd(const na_rpb_params *p, const void *q, const void *key,
                  const float *dlogits, void *dq, void *dk, float *drpb,
                  void *workspace, size_t workspace_bytes, void *stream);
/*
 * Gradients of na_rpb_av_fwd: dattn = <dout, value_nbr> (0 for invalid
 * slots, float32), dvalue[j] = sum over queries holding j of attn * dout.
 * dout has out_dtype.  Either output may be NULL.  Replaces
 * functional_metal.py:1340-1415 (natten1dav_backward), 1592-1918
 * (natten2dav_backward), 2195-2213, 2247-2274.
 */
int na_rpb_av_bwd(const na_rpb_params *p, const float *attn, const void *value,
                  const void *dout, int32_t out_dtype, float *dattn,
                  void *dvalue, void *stream);

/*
 * Host-only diagnostic: the kernel family each allin1 pass of these
 * parameters runs on, as the launchers choose it (no device work).  Rank-1
 * float32 problems take the staged kernels (a block's windows in LDS) or,
 * for large dilations, the phase-major ones; everything else the generic
 * kernels.  qk assumes a bias table, dq a requested drpb (fused_bias: the dq
 * pass also forms the bias gradient's partials).  The kernels' choice has
 * no counterpart in the reference (its Metal kernels are chosen by K and
 * head_dim, functional_metal.py:1921-2033).
 */
enum na_rpb_kernel_t {
  NA_RPB_GENERIC = 0, /* k_rpb_dot / k_rpb_gather / k_rpb_inverse */
  NA_RPB_STAGED = 1,  /* k_r1_dot / k_r1_gather / k_r1_inverse */
  NA_RPB_PHASE = 2    /* k_r1p_dot / k_r1p_gather */
};
typedef struct na_rpb_plan {
  int32_t qk;         /* na_rpb_qk_fwd */
  int32_t av;         /* na_rpb_av_fwd */
  int32_t dq;         /* na_rpb_qk_bwd, dq pass */
  int32_t dk;         /* na_rpb_qk_bwd, dk pass */
  int32_t dattn;      /* na_rpb_av_bwd, dattn pass */
  int32_t dv;         /* na_rpb_av_bwd, dv pass */
  int32_t fused_bias; /* 1: the dq pass forms the drpb partials */
  int32_t block;      /* rows per block of the forward kernels */
} na_rpb_plan;
int na_rpb_kernel_plan(const na_rpb_params *p, na_rpb_plan *plan);

/* ---- merge of attention outputs --------------------------------------- */

#define NA_MERGE_MAX_PARTS 8

typedef struct na_merge_params {
  int32_t n_parts;  /* 2 .. NA_MERGE_MAX_PARTS */
  int32_t head_dim; /* D, the last axis of every output */
  int64_t rows;     /* product of the leading axes ([B, *spatial, H]) */
  int32_t dtype;    /* storage type of the outputs, the merged output and
                       their gradients */
} na_merge_params;

/*
 * Merges outputs that share their queries as if their key/value sets had
 * been concatenated: L = logsumexp_i lse_i, out = sum_i exp(lse_i - L) out_i
 * (the closed form of the reference's sigmoid merge), one pass.  outs / lses
 * are host arrays of n_parts device pointers ([rows, D] in dtype, [rows]
 * float32); lse receives L (float32).  Replaces merge.py:20-68
 * (merge_attentions).
 */
int na_merge_fwd(const na_merge_params *p, const void *const *outs,
                 const float *const *lses, void *out, float *lse,
                 void *stream);
/*
 * Gradients of na_merge_fwd: d_outs[i] = w_i * dout and
 * d_lses[i] = w_i * (<dout, out_i> - sum_j w_j <dout, out_j> + dlse) with
 * w_i = exp(lse_i - L).  dlse may be NULL (zero); d_outs / d_lses may be
 * NULL, as may any of their entries (not computed).  The MLX autodiff of
 * merge.py:56-68 is what this replaces.
 */
int na_merge_bwd(const na_merge_params *p, const void *const *outs,
                 const float *const *lses, const void *dout, const float *dlse,
                 void *const *d_outs, float *const *d_lses, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* NATTEN_AMD_H */
