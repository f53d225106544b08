// na_launch.h — internal launchers behind the C ABI (not exported).
#pragma once

#include <hip/hip_runtime.h>

#include "na_common.h"

namespace na {

// Generic vector-ALU kernels (na_valu.hip): every dtype / head_dim.
void valu_fwd(const Prob &P, int dtype, const void *q, const void *k,
              const void *v, const void *ek, const void *ev, void *out,
              float *lse, hipStream_t st);
void valu_bwd(const Prob &P, int dtype, const void *q, const void *k,
              const void *v, const void *ek, const void *ev, const void *out,
              const float *lse, const void *dout, const float *dlse, void *dq,
              void *dk, void *dv, float *delta, hipStream_t st);
void valu_qk(const Prob &P, int dtype, const void *q, const void *k,
             void *logits, hipStream_t st);
void valu_av(const Prob &P, int dtype, const void *attn, const void *v,
             void *out, hipStream_t st);
void valu_qk_bwd(const Prob &P, int dtype, const void *q, const void *k,
                 const void *dl, void *dq, void *dk, hipStream_t st);
void valu_av_bwd(const Prob &P, int dtype, const void *attn, const void *v,
                 const void *dout, void *dattn, void *dv, hipStream_t st);
void table(const Prob &P, int32_t *index, uint8_t *valid, hipStream_t st);

// DiNAT all-in-one operators (na_rpb.hip): square window K (odd or even),
// uniform dilation, rank 1 or 2, spatial-first or heads-first rows.
struct RpbProb {
  int32_t rank, B, H, D;
  int32_t L0, L1;       // L1 = 1 for rank 1
  int32_t K0, K1;       // window side per axis (K1 = 1 for rank 1)
  int32_t d0, d1;       // dilation per axis (d1 = 1 for rank 1)
  int32_t KK;           // slots per query, K0 * K1
  int32_t R0, R1;       // bias rows per axis, 2K-1 (R1 = 1 for rank 1)
  int32_t heads_first;  // 0: rows ordered [B, L0, L1, H]; 1: [B, H, L0, L1]
  int32_t has_scale;    // q is scaled (and rounded to its dtype) first
  float scale;
  int32_t n_rows;       // B * H * L0 * L1 (< 2^31)
  FastDiv fH, fL0, fL1, fd0, fd1;  // row decode and window arithmetic
};
void rpb_qk_fwd(const RpbProb &A, int dtype, const void *q, const void *key,
                const float *rpb, float *logits, hipStream_t st);
void rpb_av_fwd(const RpbProb &A, int dtype, int out_dtype, const float *attn,
                const void *value, void *out, hipStream_t st);
size_t rpb_bias_workspace_bytes(const RpbProb &A);
void rpb_qk_bwd(const RpbProb &A, int dtype, const void *q, const void *key,
                const float *dlogits, void *dq, void *dk, float *drpb,
                void *workspace, hipStream_t st);
void rpb_av_bwd(const RpbProb &A, int dtype, int out_dtype, const float *attn,
                const void *value, const void *dout, float *dattn, void *dvalue,
                hipStream_t st);
// Kernel family per allin1 pass (0 generic, 1 staged rank-1, 2 phase-major
// rank-1) as the launchers choose it; host only.
struct RpbPlanInfo {
  int32_t qk, av, dq, dk, dattn, dv, fused_bias, block;
};
void rpb_plan(const RpbProb &A, int dtype, RpbPlanInfo *o);

// Matrix-core kernels (na_mfma.hip): bf16/fp16, head_dim 32/64/128,
// stride 1, odd kernel size on every non-causal axis.
// Dense (FMHA) forward: bf16 / fp16, head_dim 32 / 64 / 128, no per-sample
// extents (na_dense.hip).
bool dense_fwd_eligible(const Prob &P, int dtype);
void dense_fwd(const Prob &P, int dtype, const void *q, const void *k,
               const void *v, const void *ek, const void *ev, void *out,
               float *lse, hipStream_t st);
// Dense backward (same problems): k_ddkv (dk, dv and, when dek / dev are
// non-null, the additional tokens' gradients) and k_ddq (dq); delta rows
// (rowsum(dO * O) - dLSE) from the delta pass.
void dense_bwd(const Prob &P, int dtype, const void *q, const void *k,
               const void *v, const void *ek, const void *ev, const void *dout,
               const float *lse, const float *delta, void *dq, void *dk, void *dv,
               void *dek, void *dev, hipStream_t st);

bool mfma_eligible(const Prob &P, int dtype);
void mfma_fwd(const Prob &P, int dtype, const void *q, const void *k,
              const void *v, const void *ek, const void *ev, void *out,
              float *lse, hipStream_t st);
// delta: rowsum(dO * O) - dlse per (query, head), from valu_delta; read only
// where mfma_bwd_reads_delta(P), else recomputed from out and dlse.
bool mfma_bwd_reads_delta(const Prob &P);
void mfma_bwd(const Prob &P, int dtype, const void *q, const void *k,
              const void *v, const void *ek, const void *ev, const void *out,
              const float *lse, const void *dout, const float *dlse,
              const float *delta, void *dq, void *dk, void *dv,
              hipStream_t st);
void mfma_selftest(int dtype, float *out, hipStream_t st);

// Lean matrix-core fused forward (na_lean.hip): the MFMA-eligible problems
// that are not dense, with d*K <= L on every non-causal axis (and d*K <= L_b
// for every sample when per-sample extents are given, Prob::varlen_clamped).
bool lean_eligible(const Prob &P, int dtype);
void lean_fwd(const Prob &P, int dtype, const void *q, const void *k,
              const void *v, const void *ek, const void *ev, void *out,
              float *lse, hipStream_t st);
// Launch plan of the lean fused kernels (a diagnostic): wave tile T, waves
// per workgroup W, staged box Em, number of axis-0 slabs the box is staged
// in, grouped query heads (forward), workgroups launched and LDS bytes.
// False when the problem does not run on them.
struct LeanPlanInfo {
  int T[3], W, Em[3], slabs, hl, workgroups, lds;
};
bool lean_plan(const Prob &P, int dtype, bool backward, LeanPlanInfo *o);
// Lean fused backward: one launch, no workspace (delta is computed in the
// kernel); dlse may be null.  Per-sample extents and additional tokens as
// in lean_fwd (ek / ev: their contribution to dq; their own gradients come
// from dextra).  delta_out (nullable; with additional tokens only): the
// kernel also writes each query row's delta there, for dextra.
bool lean_bwd_eligible(const Prob &P, int dtype);
void lean_bwd(const Prob &P, int dtype, const void *q, const void *k,
              const void *v, const void *ek, const void *ev,
              const void *out, const float *lse,
              const void *dout, const float *dlse, void *dq, void *dk,
              void *dv, float *delta_out, hipStream_t st);

// Lean split ops (na_lsplit.hip): the lean problem class without varlen,
// additional tokens or dense mode, where the compact rows fit LDS.
// lsplit_qk: out[q, slot] = scale * <x_q, y_key(slot)> (fill outside the
// window); lsplit_av: out_q = scale * sum_slot a[q, slot] * y_key(slot);
// lsplit_inv: z_key = scale * sum over queries q holding the key (all query
// heads of its group) of a[q, slot(q, key)] * x_q.
bool lsplit_eligible(const Prob &P, int dtype);
// Vector-ALU gather alternative to lsplit_qk (na_vsplit.hip; rank 2,
// non-causal, same odd K <= 7 on both axes): false where it does not apply.
bool vsplit_on();
bool vsplit_qk(const Prob &P, int dtype, const void *x, const void *y, void *out,
               float scale, hipStream_t st);
void lsplit_qk(const Prob &P, int dtype, const void *x, const void *y,
               void *out, float scale, float fill, hipStream_t st);
void lsplit_av(const Prob &P, int dtype, const void *a, const void *y,
               void *out, float scale, hipStream_t st);
void lsplit_inv(const Prob &P, int dtype, const void *a, const void *x,
                void *z, float scale, hipStream_t st);
// The split backward calls: dq (lsplit_av over dlogits and the keys) and
// dk (lsplit_inv over dlogits and the queries); dattn (lsplit_qk over dout
// and the values) and dv (lsplit_inv over attn and dout) — each pair in one
// launch where that applies.
void lsplit_qk_bwd(const Prob &P, int dtype, const void *q, const void *k,
                   const void *dlogits, void *dq, void *dk, hipStream_t st);
void lsplit_av_bwd(const Prob &P, int dtype, const void *attn, const void *v,
                   const void *dout, void *dattn, void *dv, hipStream_t st);

// Matrix-core split ops (na_msplit.hip): the MFMA-eligible problems with
// d*K <= L on every non-causal axis and at most 512 kernel slots.
bool msplit_eligible(const Prob &P, int dtype);
// out[q, slot] = scale * <x_q, y_key(slot)>, `fill` outside the window.
void msplit_qk(const Prob &P, int dtype, const void *x, const void *y,
               void *out, float scale, float fill, hipStream_t st);
// out_q = scale * sum_slot a[q, slot] * y_key(slot).
void msplit_av(const Prob &P, int dtype, const void *a, const void *y,
               void *out, float scale, hipStream_t st);
// out_key = scale * sum over (q, slot) holding the key of a[q, slot] * x_q.
void msplit_inv(const Prob &P, int dtype, const void *a, const void *x,
                void *out, float scale, hipStream_t st);

// Merge of attention outputs sharing their queries (na_merge.hip): up to
// kMergeMaxParts parts of rows x D elements in `dtype`, LSEs float32.
constexpr int kMergeMaxParts = 8;
void merge_fwd(int dtype, int n, int64_t rows, int D, const void *const *outs,
               const float *const *lses, void *out, float *lse,
               hipStream_t st);
void merge_bwd(int dtype, int n, int64_t rows, int D, const void *const *outs,
               const float *const *lses, const void *dout, const float *dlse,
               void *const *d_outs, float *const *d_lses, hipStream_t st);

// Generic pieces reused around the MFMA backward.
void valu_delta(const Prob &P, int dtype, const void *out, const void *dout,
                const float *dlse, float *delta, hipStream_t st);

// Gradients of the additional tokens (na_dextra.hip): a two-pass segment
// reduction over every query of the sample, reading delta (rowsum(dO * O) -
// dlse per (query, head)); `part` is a float workspace of
// dextra_workspace_bytes(P); `matrix` allows the matrix-core variant
// (bf16 / fp16, head_dim 32 / 64 / 128).
size_t dextra_workspace_bytes(const Prob &P);
// Whether dextra runs the matrix-core reduction (else the vector-ALU one).
bool dextra_uses_matrix(const Prob &P, int dtype, bool matrix);
void dextra(const Prob &P, int dtype, const void *q, const void *ek,
            const void *ev, const float *lse, const float *delta,
            const void *dout, void *dek, void *dev, float *part, bool matrix,
            hipStream_t st);

}  // namespace na
