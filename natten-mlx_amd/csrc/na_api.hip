// na_api.hip — the exported C ABI (include/natten_amd.h): parameter
// validation, problem normalisation and kernel selection.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <string>

#include "na_common.h"
#include "na_launch.h"

namespace {

thread_local std::string g_error;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int launch_status(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(NA_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  g_error.clear();
  return NA_OK;
}

constexpr int kMaxHeadDim = 1024;

// Normalise the public parameters to the three-axis device problem.
int make_prob(const na_params *p, na::Prob *P, bool allow_varlen) {
  if (p == nullptr) return fail(NA_ERR_INVALID, "params is NULL");
  if (p->rank < 1 || p->rank > 3)
    return fail(NA_ERR_INVALID, "rank must be 1, 2 or 3, got %d", p->rank);
  if (p->batch < 0 || p->heads < 1 || p->kv_heads < 1 || p->head_dim < 1)
    return fail(NA_ERR_INVALID,
                "batch/heads/kv_heads/head_dim must be positive "
                "(got %d/%d/%d/%d)",
                p->batch, p->heads, p->kv_heads, p->head_dim);
  if (p->heads % p->kv_heads != 0)
    return fail(NA_ERR_INVALID,
                "heads (%d) must be divisible by kv_heads (%d)", p->heads,
                p->kv_heads);
  if (p->dtype != NA_F32 && p->dtype != NA_F16 && p->dtype != NA_BF16)
    return fail(NA_ERR_INVALID, "unknown dtype %d", p->dtype);
  if (p->n_extra < 0)
    return fail(NA_ERR_INVALID, "n_extra must be >= 0, got %d", p->n_extra);
  if (!allow_varlen && p->sample_extent != nullptr)
    return fail(NA_ERR_UNSUPPORTED,
                "per-sample extents are only supported by na_fwd/na_bwd");
  if ((p->head_dim % 8 != 0 && p->head_dim > 128) ||
      p->head_dim > kMaxHeadDim)
    return fail(NA_ERR_UNSUPPORTED, "head_dim %d is not supported",
                p->head_dim);
  const bool dense = (p->flags & NA_FLAG_DENSE) != 0;
  P->rank = p->rank;
  P->B = p->batch;
  P->H = p->heads;
  P->Hkv = p->kv_heads;
  P->rep = p->heads / p->kv_heads;
  P->D = p->head_dim;
  P->scale = p->scale;
  P->n_extra = p->n_extra;
  P->dense = dense ? 1 : 0;
  P->sample_extent = p->sample_extent;
  P->varlen_clamped = (p->flags & NA_FLAG_VARLEN_CLAMPED) != 0 ? 1 : 0;
  P->kprod = 1;
  const int lead = 3 - p->rank;
  for (int a = 0; a < 3; ++a) {
    na::Axis &x = P->ax[a];
    if (a < lead) {
      x.L = 1;
      x.K = 1;
      x.d = 1;
      x.s = 1;
      x.causal = 0;
    } else {
      const int i = a - lead;
      x.L = p->extent[i];
      x.K = p->kernel[i];
      x.d = p->dilation[i];
      x.s = p->stride[i];
      x.causal = p->causal[i] ? 1 : 0;
      if (x.L < 1)
        return fail(NA_ERR_INVALID, "extent[%d] must be positive, got %d", i,
                    x.L);
      if (x.K < 1 || x.d < 1 || x.s < 1)
        return fail(NA_ERR_INVALID,
                    "kernel/dilation/stride[%d] must be positive "
                    "(got %d/%d/%d)",
                    i, x.K, x.d, x.s);
      if (!dense && x.K > x.L)
        return fail(NA_ERR_INVALID, "kernel_size[%d]=%d exceeds extent %d", i,
                    x.K, x.L);
      if (dense && (x.s != 1 || x.causal))
        return fail(NA_ERR_INVALID,
                    "dense attention requires stride 1 and no causal mask");
      if (dense) {  // every key of the sample: no window, no dilation phases
        x.K = x.L;
        x.d = 1;
      }
    }
    x.O = (x.L + x.s - 1) / x.s;
    P->kprod *= x.K;
  }
  return NA_OK;
}

hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

bool use_mfma(const na_params *p, const na::Prob &P) {
  return (p->flags & NA_FLAG_GENERIC) == 0 && na::mfma_eligible(P, p->dtype);
}

bool use_dense(const na_params *p, const na::Prob &P) {
  return (p->flags & NA_FLAG_GENERIC) == 0 && na::dense_fwd_eligible(P, p->dtype);
}

bool use_lean(const na_params *p, const na::Prob &P) {
  return (p->flags & (NA_FLAG_GENERIC | NA_FLAG_NO_LEAN)) == 0 &&
         na::lean_eligible(P, p->dtype);
}

bool use_lean_bwd(const na_params *p, const na::Prob &P) {
  return (p->flags & (NA_FLAG_GENERIC | NA_FLAG_NO_LEAN)) == 0 &&
         na::lean_bwd_eligible(P, p->dtype);
}

bool use_lsplit(const na_params *p, const na::Prob &P) {
  return (p->flags & (NA_FLAG_GENERIC | NA_FLAG_NO_LEAN)) == 0 &&
         na::lsplit_eligible(P, p->dtype);
}

bool use_msplit(const na_params *p, const na::Prob &P) {
  return (p->flags & NA_FLAG_GENERIC) == 0 && na::msplit_eligible(P, p->dtype);
}

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

size_t delta_bytes(const na::Prob &P) {
  return align256(sizeof(float) * (size_t)P.B * P.ax[0].O * P.ax[1].O *
                  P.ax[2].O * P.H);
}

// The backward's kernels and the workspace they read: delta rows
// (rowsum(dO * O) - dlse per query and head) where a kernel reads them, then
// the additional tokens' gradient partials.  Sized as if the extra-token
// gradients are requested (the workspace query sees no pointers).
enum BwdPath { kBwdLean, kBwdDense, kBwdMfma, kBwdGeneric };
struct BwdPlan {
  BwdPath path;
  bool matrix;       // the extra-token reduction may use matrix cores
  bool need_delta;   // delta rows live in the workspace (written by a delta
                     // pass, or by the lean backward for the reduction)
  size_t delta, total;  // bytes: delta rows, whole workspace
};

BwdPlan bwd_plan(const na_params *p, const na::Prob &P) {
  BwdPlan b{};
  b.matrix = (p->flags & NA_FLAG_GENERIC) == 0;
  const bool extra = P.n_extra > 0;
  if (use_lean_bwd(p, P)) {
    b.path = kBwdLean;
    b.need_delta = extra;
  } else if (use_dense(p, P)) {
    // the additional tokens are keys of the dense kernels: no reduction pass
    b.path = kBwdDense;
    b.need_delta = true;
    b.delta = delta_bytes(P);
    b.total = b.delta;
    return b;
  } else if (use_mfma(p, P)) {
    b.path = kBwdMfma;
    b.need_delta = extra || na::mfma_bwd_reads_delta(P);
  } else {
    b.path = kBwdGeneric;
    b.need_delta = true;
  }
  b.delta = b.need_delta ? delta_bytes(P) : 0;
  b.total = b.delta + (extra ? align256(na::dextra_workspace_bytes(P)) : 0);
  return b;
}

// Validate the all-in-one parameters and build the device problem.
int make_rpb(const na_rpb_params *p, na::RpbProb *A) {
  if (p == nullptr) return fail(NA_ERR_INVALID, "params is NULL");
  if (p->rank != 1 && p->rank != 2)
    return fail(NA_ERR_INVALID, "allin1 rank must be 1 or 2, got %d", p->rank);
  if (p->batch < 0 || p->heads < 1 || p->head_dim < 1)
    return fail(NA_ERR_INVALID,
                "batch/heads/head_dim must be positive (got %d/%d/%d)",
                p->batch, p->heads, p->head_dim);
  if (p->dtype != NA_F32 && p->dtype != NA_F16 && p->dtype != NA_BF16)
    return fail(NA_ERR_INVALID, "unknown dtype %d", p->dtype);
  if ((p->head_dim % 8 != 0 && p->head_dim > 128) ||
      p->head_dim > kMaxHeadDim)
    return fail(NA_ERR_UNSUPPORTED, "head_dim %d is not supported",
                p->head_dim);
  const int32_t K1 = p->rank == 2 ? p->kernel[1] : 1;
  const int32_t d1 = p->rank == 2 ? p->dilation[1] : 1;
  if (p->kernel[0] < 1 || p->dilation[0] < 1 || K1 < 1 || d1 < 1)
    return fail(NA_ERR_INVALID, "kernel and dilation must be positive");
  const int32_t L1 = p->rank == 2 ? p->extent[1] : 1;
  if (p->extent[0] < 1 || L1 < 1)
    return fail(NA_ERR_INVALID, "extents must be positive");
  if ((int64_t)p->kernel[0] * p->dilation[0] > (1 << 20) ||
      (int64_t)K1 * d1 > (1 << 20))
    return fail(NA_ERR_UNSUPPORTED, "kernel * dilation too large");
  const int64_t kk = (int64_t)p->kernel[0] * K1;
  const int64_t rows = (int64_t)p->batch * p->heads * p->extent[0] * L1;
  if (rows >= ((int64_t)1 << 31) || kk >= ((int64_t)1 << 20))
    return fail(NA_ERR_UNSUPPORTED, "allin1 problem too large");
  A->rank = p->rank;
  A->B = p->batch;
  A->H = p->heads;
  A->D = p->head_dim;
  A->K0 = p->kernel[0];
  A->K1 = K1;
  A->d0 = p->dilation[0];
  A->d1 = d1;
  A->L0 = p->extent[0];
  A->L1 = L1;
  A->KK = (int32_t)kk;
  A->R0 = 2 * A->K0 - 1;
  A->R1 = p->rank == 2 ? 2 * K1 - 1 : 1;
  A->heads_first = p->heads_first ? 1 : 0;
  A->has_scale = p->has_scale ? 1 : 0;
  A->scale = p->scale;
  A->n_rows = (int32_t)rows;
  A->fH = na::make_fastdiv((uint32_t)A->H);
  A->fL0 = na::make_fastdiv((uint32_t)A->L0);
  A->fL1 = na::make_fastdiv((uint32_t)A->L1);
  A->fd0 = na::make_fastdiv((uint32_t)A->d0);
  A->fd1 = na::make_fastdiv((uint32_t)A->d1);
  return NA_OK;
}

int check_out_dtype(const na_rpb_params *p, int32_t out_dtype) {
  if (out_dtype != NA_F32 && out_dtype != p->dtype)
    return fail(NA_ERR_INVALID,
                "out_dtype must be NA_F32 or the input dtype (got %d)",
                out_dtype);
  return NA_OK;
}

int check_merge(const na_merge_params *p, const void *const *outs,
                const float *const *lses) {
  static_assert(NA_MERGE_MAX_PARTS == na::kMergeMaxParts,
                "merge part limit of the header and the kernels");
  if (p == nullptr) return fail(NA_ERR_INVALID, "params is NULL");
  if (p->n_parts < 2 || p->n_parts > NA_MERGE_MAX_PARTS)
    return fail(NA_ERR_INVALID, "n_parts must be in [2, %d], got %d",
                NA_MERGE_MAX_PARTS, p->n_parts);
  if (p->dtype != NA_F32 && p->dtype != NA_F16 && p->dtype != NA_BF16)
    return fail(NA_ERR_INVALID, "unknown dtype %d", p->dtype);
  if (p->rows < 0 || p->head_dim < 1)
    return fail(NA_ERR_INVALID, "rows must be >= 0 and head_dim positive");
  if ((p->head_dim % 8 != 0 && p->head_dim > 128) ||
      p->head_dim > kMaxHeadDim)
    return fail(NA_ERR_UNSUPPORTED, "head_dim %d is not supported",
                p->head_dim);
  if (p->rows * p->head_dim > ((int64_t)1 << 38))
    return fail(NA_ERR_UNSUPPORTED, "merge problem too large");
  if (outs == nullptr || lses == nullptr)
    return fail(NA_ERR_INVALID, "outs/lses must be non-NULL");
  for (int i = 0; i < p->n_parts; ++i)
    if (outs[i] == nullptr || lses[i] == nullptr)
      return fail(NA_ERR_INVALID, "outs[%d]/lses[%d] is NULL", i, i);
  return NA_OK;
}

// ---- fixed scratch for na_bwd_noalloc -----------------------------------
// The backward's workspace (delta rows and the additional tokens' gradient
// partials) for callers that cannot allocate: a file-scope device array,
// one copy per GPU the library runs on, held until the process ends.  Host
// code never passes `scratch` itself (its host-side name is not a device
// address): the device address comes from hipGetSymbolAddress, once per
// device, with that device current, and is kept per device.
constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// The scratch of the device the kernels run on: that of `stream` (a null
// stream runs on the current device).  The address is looked up with that
// device current (each device holds its own copy of the array at its own
// address); the caller's current device is restored afterwards.
int scratch_of_stream_device(hipStream_t stream, void **out) {
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess)
    return fail(NA_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  int dev = cur;
  if (stream != nullptr) {
    hipDevice_t sd = -1;
    e = hipStreamGetDevice(stream, &sd);
    if (e != hipSuccess)
      return fail(NA_ERR_INVALID, "hipStreamGetDevice: %s", hipGetErrorString(e));
    dev = (int)sd;
  }
  if (dev < 0 || dev >= kMaxDevices)
    return fail(NA_ERR_UNSUPPORTED, "device %d is beyond the %d devices na_bwd_noalloc serves",
                dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess)
      return fail(NA_ERR_LAUNCH, "hipSetDevice(%d): %s", dev, hipGetErrorString(e));
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    const hipError_t er = dev != cur ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess || ptr == nullptr)
      return fail(NA_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
    if (er != hipSuccess)
      return fail(NA_ERR_LAUNCH, "hipSetDevice(%d): %s", cur, hipGetErrorString(er));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return NA_OK;
}

}  // namespace

extern "C" {

int na_abi_version(void) { return NA_ABI_VERSION; }

const char *na_last_error(void) { return g_error.c_str(); }

int32_t na_window_start(int32_t index, int32_t length, int32_t kernel_size,
                        int32_t neighborhood_size, int32_t dilation) {
  return na::window_start(index, length, kernel_size, neighborhood_size,
                          dilation);
}

int32_t na_window_end(int32_t start, int32_t length, int32_t kernel_size,
                      int32_t dilation) {
  return na::window_end(start, length, kernel_size, dilation);
}

int32_t na_pb_start(int32_t index, int32_t length, int32_t kernel_size,
                    int32_t neighborhood_size, int32_t dilation) {
  return na::pb_start(index, length, kernel_size, neighborhood_size, dilation);
}

int32_t na_window_start_partition(int32_t index, int32_t length,
                                  int32_t kernel_size,
                                  int32_t neighborhood_size,
                                  int32_t dilation) {
  return na::window_start_partition(index, length, kernel_size,
                                    neighborhood_size, dilation);
}

int na_mfma_selftest(int32_t dtype, float *out, void *stream) {
  if (dtype != NA_BF16 && dtype != NA_F16)
    return fail(NA_ERR_INVALID, "selftest dtype must be bf16 or fp16");
  if (out == nullptr) return fail(NA_ERR_INVALID, "out must be non-NULL");
  na::mfma_selftest(dtype, out, as_stream(stream));
  return launch_status("na_mfma_selftest");
}

int na_kernel_path(const na_params *p, int32_t backward) {
  na::Prob P;
  const int rc = make_prob(p, &P, backward != 2);
  if (rc != NA_OK) return -rc;
  if (backward == 2) {
    if (use_lsplit(p, P)) return NA_PATH_LEAN;
    if (use_msplit(p, P)) return NA_PATH_MFMA;
    return NA_PATH_GENERIC;
  }
  if (backward ? use_lean_bwd(p, P) : use_lean(p, P)) return NA_PATH_LEAN;
  if (use_dense(p, P)) return NA_PATH_DENSE;
  if (use_mfma(p, P)) return NA_PATH_MFMA;
  return NA_PATH_GENERIC;
}

int na_kernel_plan(const na_params *p, int32_t backward, na_plan *plan) {
  if (plan == nullptr) return fail(NA_ERR_INVALID, "plan is NULL");
  if (backward != 0 && backward != 1)
    return fail(NA_ERR_INVALID, "backward must be 0 or 1, got %d", backward);
  na::Prob P;
  const int rc = make_prob(p, &P, true);
  if (rc != NA_OK) return rc;
  *plan = na_plan{};
  const bool lean = backward ? use_lean_bwd(p, P) : use_lean(p, P);
  plan->path = lean                         ? NA_PATH_LEAN
               : use_dense(p, P)              ? NA_PATH_DENSE
               : use_mfma(p, P)               ? NA_PATH_MFMA
                                              : NA_PATH_GENERIC;
  if (lean) {
    na::LeanPlanInfo L{};
    if (na::lean_plan(P, p->dtype, backward != 0, &L)) {
      for (int a = 0; a < 3; ++a) {
        plan->tile[a] = L.T[a];
        plan->box[a] = L.Em[a];
      }
      plan->waves = L.W;
      plan->slabs = L.slabs;
      plan->grouped_heads = L.hl;
      plan->workgroups = L.workgroups;
      plan->lds_bytes = L.lds;
    }
  }
  if (backward && P.n_extra > 0 && plan->path != NA_PATH_DENSE)
    plan->extra_reduction =
        na::dextra_uses_matrix(P, p->dtype, (p->flags & NA_FLAG_GENERIC) == 0) ? 2 : 1;
  g_error.clear();
  return NA_OK;
}

int na_neighbor_table(const na_params *p, int32_t *index, uint8_t *valid,
                      void *stream) {
  na::Prob P;
  const int rc = make_prob(p, &P, false);
  if (rc != NA_OK) return rc;
  if (P.dense) return fail(NA_ERR_INVALID, "neighbor table of a dense problem");
  if (index == nullptr || valid == nullptr)
    return fail(NA_ERR_INVALID, "index/valid must be non-NULL");
  na::table(P, index, valid, as_stream(stream));
  return launch_status("na_neighbor_table");
}

int na_fwd(const na_params *p, const void *q, const void *k, const void *v,
           const void *extra_k, const void *extra_v, void *out, float *lse,
           void *stream) {
  na::Prob P;
  const int rc = make_prob(p, &P, true);
  if (rc != NA_OK) return rc;
  if (P.B == 0) return NA_OK;
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr)
    return fail(NA_ERR_INVALID, "q/k/v/out must be non-NULL");
  if (P.n_extra > 0 && (extra_k == nullptr || extra_v == nullptr))
    return fail(NA_ERR_INVALID, "n_extra > 0 needs extra_k and extra_v");
  if (use_lean(p, P))
    na::lean_fwd(P, p->dtype, q, k, v, extra_k, extra_v, out, lse,
                 as_stream(stream));
  else if (use_dense(p, P))
    na::dense_fwd(P, p->dtype, q, k, v, extra_k, extra_v, out, lse,
                  as_stream(stream));
  else if (use_mfma(p, P))
    na::mfma_fwd(P, p->dtype, q, k, v, extra_k, extra_v, out, lse,
                 as_stream(stream));
  else
    na::valu_fwd(P, p->dtype, q, k, v, extra_k, extra_v, out, lse,
                 as_stream(stream));
  return launch_status("na_fwd");
}

size_t na_bwd_workspace_bytes(const na_params *p) {
  na::Prob P;
  if (make_prob(p, &P, true) != NA_OK) return 0;
  return bwd_plan(p, P).total;
}

int na_bwd(const na_params *p, const void *q, const void *k, const void *v,
           const void *extra_k, const void *extra_v, const void *out,
           const float *lse, const void *dout, const float *dlse, void *dq,
           void *dk, void *dv, void *d_extra_k, void *d_extra_v,
           void *workspace, size_t workspace_bytes, void *stream) {
  na::Prob P;
  const int rc = make_prob(p, &P, true);
  if (rc != NA_OK) return rc;
  if (P.B == 0) return NA_OK;
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr ||
      lse == nullptr || dout == nullptr || dq == nullptr || dk == nullptr ||
      dv == nullptr)
    return fail(NA_ERR_INVALID,
                "q/k/v/out/lse/dout/dq/dk/dv must be non-NULL");
  if (P.n_extra > 0 && (extra_k == nullptr || extra_v == nullptr))
    return fail(NA_ERR_INVALID, "n_extra > 0 needs extra_k and extra_v");
  const BwdPlan plan = bwd_plan(p, P);
  if (plan.total > 0 && (workspace == nullptr || workspace_bytes < plan.total))
    return fail(NA_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", plan.total,
                workspace == nullptr ? (size_t)0 : workspace_bytes);
  float *delta = static_cast<float *>(workspace);
  float *xpart = plan.total > 0 ? reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                                            plan.delta)
                                : nullptr;
  const hipStream_t st = as_stream(stream);
  const bool dextra =
      P.n_extra > 0 && d_extra_k != nullptr && d_extra_v != nullptr;
  // the lean backward computes delta inside, and writes its rows for the
  // extra-token reduction that follows it
  if (plan.path == kBwdLean) {
    na::lean_bwd(P, p->dtype, q, k, v, extra_k, extra_v, out, lse, dout, dlse,
                 dq, dk, dv, dextra ? delta : nullptr, st);
  } else if (plan.path == kBwdDense) {
    na::valu_delta(P, p->dtype, out, dout, dlse, delta, st);
    na::dense_bwd(P, p->dtype, q, k, v, extra_k, extra_v, dout, lse, delta, dq, dk, dv,
                  dextra ? d_extra_k : nullptr, dextra ? d_extra_v : nullptr, st);
    return launch_status("na_bwd");
  } else if (plan.path == kBwdMfma) {
    if (dextra || na::mfma_bwd_reads_delta(P))
      na::valu_delta(P, p->dtype, out, dout, dlse, delta, st);
    na::mfma_bwd(P, p->dtype, q, k, v, extra_k, extra_v, out, lse, dout, dlse,
                 delta, dq, dk, dv, st);
  } else {
    na::valu_bwd(P, p->dtype, q, k, v, extra_k, extra_v, out, lse, dout, dlse,
                 dq, dk, dv, delta, st);
  }
  if (dextra)
    na::dextra(P, p->dtype, q, extra_k, extra_v, lse, delta, dout, d_extra_k,
               d_extra_v, xpart, plan.matrix, st);
  return launch_status("na_bwd");
}

size_t na_bwd_noalloc_max_workspace(void) { return kScratchBytes; }

int na_bwd_noalloc(const na_params *p, const void *q, const void *k,
                   const void *v, const void *extra_k, const void *extra_v,
                   const void *out, const float *lse, const void *dout,
                   const float *dlse, void *dq, void *dk, void *dv,
                   void *d_extra_k, void *d_extra_v, void *stream) {
  na::Prob P;
  const int rc = make_prob(p, &P, true);
  if (rc != NA_OK) return rc;
  const size_t need = bwd_plan(p, P).total;
  if (need > kScratchBytes)
    return fail(NA_ERR_UNSUPPORTED,
                "na_bwd_noalloc: this problem needs %zu bytes of scratch, above its "
                "fixed maximum of %zu; use na_bwd with a caller workspace",
                need, kScratchBytes);
  void *ws = nullptr;
  const int src = scratch_of_stream_device(as_stream(stream), &ws);
  if (src != NA_OK) return src;
  // every byte the kernels read from the workspace is written earlier in
  // the same call (delta rows; one partial per reduction segment), so the
  // previous call's contents need no clearing
  return na_bwd(p, q, k, v, extra_k, extra_v, out, lse, dout, dlse, dq, dk, dv,
                d_extra_k, d_extra_v, ws, kScratchBytes, stream);
}

int na_qk_fwd(const na_params *p, const void *q, const void *k, void *logits,
              void *stream) {
  na::Prob P;
  const int rc = make_prob(p, &P, false);
  if (rc != NA_OK) return rc;
  if (P.dense) return fail(NA_ERR_INVALID, "split ops take no dense flag");
  if (P.B == 0) return NA_OK;
  if (q == nullptr || k == nullptr || logits == nullptr)
    return fail(NA_ERR_INVALID, "q/k/logits must be non-NULL");
  if (use_lsplit(p, P) && na::vsplit_on() &&
      na::vsplit_qk(P, p->dtype, q, k, logits, P.scale, as_stream(stream)))
    ;
  else if (use_lsplit(p, P))
    na::lsplit_qk(P, p->dtype, q, k, logits, P.scale, -INFINITY,
                  as_stream(stream));
  else if (use_msplit(p, P))
    na::msplit_qk(P, p->dtype, q, k, logits, P.scale, -INFINITY,
                  as_stream(stream));
  else
    na::valu_qk(P, p->dtype, q, k, logits, as_stream(stream));
  return launch_status("na_qk_fwd");
}

int na_av_fwd(const na_params *p, const void *attn, const void *v, void *out,
              void *stream) {
  na::Prob P;
  const int rc = make_prob(p, &P, false);
  if (rc != NA_OK) return rc;
  if (P.dense) return fail(NA_ERR_INVALID, "split ops take no dense flag");
  if (P.B == 0) return NA_OK;
  if (attn == nullptr || v == nullptr || out == nullptr)
    return fail(NA_ERR_INVALID, "attn/v/out must be non-NULL");
  if (use_lsplit(p, P))
    na::lsplit_av(P, p->dtype, attn, v, out, 1.f, as_stream(stream));
  else if (use_msplit(p, P))
    na::msplit_av(P, p->dtype, attn, v, out, 1.f, as_stream(stream));
  else
    na::valu_av(P, p->dtype, attn, v, out, as_stream(stream));
  return launch_status("na_av_fwd");
}

int na_qk_bwd(const na_params *p, const void *q, const void *k,
              const void *dlogits, void *dq, void *dk, void *stream) {
  na::Prob P;
  const int rc = make_prob(p, &P, false);
  if (rc != NA_OK) return rc;
  if (P.dense) return fail(NA_ERR_INVALID, "split ops take no dense flag");
  if (P.B == 0) return NA_OK;
  if (q == nullptr || k == nullptr || dlogits == nullptr || dq == nullptr ||
      dk == nullptr)
    return fail(NA_ERR_INVALID, "q/k/dlogits/dq/dk must be non-NULL");
  if (use_lsplit(p, P)) {
    na::lsplit_qk_bwd(P, p->dtype, q, k, dlogits, dq, dk, as_stream(stream));
  } else if (use_msplit(p, P)) {
    na::msplit_av(P, p->dtype, dlogits, k, dq, P.scale, as_stream(stream));
    na::msplit_inv(P, p->dtype, dlogits, q, dk, P.scale, as_stream(stream));
  } else {
    na::valu_qk_bwd(P, p->dtype, q, k, dlogits, dq, dk, as_stream(stream));
  }
  return launch_status("na_qk_bwd");
}

int na_av_bwd(const na_params *p, const void *attn, const void *v,
              const void *dout, void *dattn, void *dv, void *stream) {
  na::Prob P;
  const int rc = make_prob(p, &P, false);
  if (rc != NA_OK) return rc;
  if (P.dense) return fail(NA_ERR_INVALID, "split ops take no dense flag");
  if (P.B == 0) return NA_OK;
  if (attn == nullptr || v == nullptr || dout == nullptr || dattn == nullptr ||
      dv == nullptr)
    return fail(NA_ERR_INVALID, "attn/v/dout/dattn/dv must be non-NULL");
  if (use_lsplit(p, P)) {
    na::lsplit_av_bwd(P, p->dtype, attn, v, dout, dattn, dv, as_stream(stream));
  } else if (use_msplit(p, P)) {
    na::msplit_qk(P, p->dtype, dout, v, dattn, 1.f, 0.f, as_stream(stream));
    na::msplit_inv(P, p->dtype, attn, dout, dv, 1.f, as_stream(stream));
  } else {
    na::valu_av_bwd(P, p->dtype, attn, v, dout, dattn, dv, as_stream(stream));
  }
  return launch_status("na_av_bwd");
}

int na_rpb_qk_fwd(const na_rpb_params *p, const void *q, const void *key,
                  const float *rpb, float *logits, void *stream) {
  na::RpbProb A;
  const int rc = make_rpb(p, &A);
  if (rc != NA_OK) return rc;
  if (A.n_rows == 0) return NA_OK;
  if (q == nullptr || key == nullptr || logits == nullptr)
    return fail(NA_ERR_INVALID, "q/key/logits must be non-NULL");
  na::rpb_qk_fwd(A, p->dtype, q, key, rpb, logits, as_stream(stream));
  return launch_status("na_rpb_qk_fwd");
}

int na_rpb_av_fwd(const na_rpb_params *p, const float *attn, const void *value,
                  void *out, int32_t out_dtype, void *stream) {
  na::RpbProb A;
  int rc = make_rpb(p, &A);
  if (rc != NA_OK) return rc;
  rc = check_out_dtype(p, out_dtype);
  if (rc != NA_OK) return rc;
  if (A.n_rows == 0) return NA_OK;
  if (attn == nullptr || value == nullptr || out == nullptr)
    return fail(NA_ERR_INVALID, "attn/value/out must be non-NULL");
  na::rpb_av_fwd(A, p->dtype, out_dtype, attn, value, out, as_stream(stream));
  return launch_status("na_rpb_av_fwd");
}

size_t na_rpb_bwd_workspace_bytes(const na_rpb_params *p) {
  na::RpbProb A;
  if (make_rpb(p, &A) != NA_OK) return 0;
  return align256(na::rpb_bias_workspace_bytes(A));
}

int na_rpb_qk_bwd(const na_rpb_params *p, const void *q, const void *key,
                  const float *dlogits, void *dq, void *dk, float *drpb,
                  void *workspace, size_t workspace_bytes, void *stream) {
  na::RpbProb A;
  const int rc = make_rpb(p, &A);
  if (rc != NA_OK) return rc;
  if (drpb != nullptr) {
    const size_t need = align256(na::rpb_bias_workspace_bytes(A));
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
      return fail(NA_ERR_WORKSPACE,
                  "na_rpb_qk_bwd needs a %zu-byte workspace for drpb (got %zu)",
                  need, workspace_bytes);
  }
  if (A.n_rows == 0) {  // empty batch: drpb (if requested) is all zero
    if (drpb != nullptr)
      na::rpb_qk_bwd(A, p->dtype, q, key, dlogits, nullptr, nullptr, drpb,
                     workspace, as_stream(stream));
    return launch_status("na_rpb_qk_bwd");
  }
  if (q == nullptr || key == nullptr || dlogits == nullptr)
    return fail(NA_ERR_INVALID, "q/key/dlogits must be non-NULL");
  na::rpb_qk_bwd(A, p->dtype, q, key, dlogits, dq, dk, drpb, workspace,
                 as_stream(stream));
  return launch_status("na_rpb_qk_bwd");
}

int na_rpb_kernel_plan(const na_rpb_params *p, na_rpb_plan *plan) {
  if (plan == nullptr) return fail(NA_ERR_INVALID, "plan is NULL");
  na::RpbProb A;
  const int rc = make_rpb(p, &A);
  if (rc != NA_OK) return rc;
  na::RpbPlanInfo o{};
  na::rpb_plan(A, p->dtype, &o);
  plan->qk = o.qk;
  plan->av = o.av;
  plan->dq = o.dq;
  plan->dk = o.dk;
  plan->dattn = o.dattn;
  plan->dv = o.dv;
  plan->fused_bias = o.fused_bias;
  plan->block = o.block;
  return NA_OK;
}

int na_rpb_av_bwd(const na_rpb_params *p, const float *attn, const void *value,
                  const void *dout, int32_t out_dtype, float *dattn,
                  void *dvalue, void *stream) {
  na::RpbProb A;
  int rc = make_rpb(p, &A);
  if (rc != NA_OK) return rc;
  rc = check_out_dtype(p, out_dtype);
  if (rc != NA_OK) return rc;
  if (A.n_rows == 0) return NA_OK;
  if (attn == nullptr || value == nullptr || dout == nullptr)
    return fail(NA_ERR_INVALID, "attn/value/dout must be non-NULL");
  na::rpb_av_bwd(A, p->dtype, out_dtype, attn, value, dout, dattn, dvalue,
                 as_stream(stream));
  return launch_status("na_rpb_av_bwd");
}

int na_merge_fwd(const na_merge_params *p, const void *const *outs,
                 const float *const *lses, void *out, float *lse,
                 void *stream) {
  const int rc = check_merge(p, outs, lses);
  if (rc != NA_OK) return rc;
  if (p->rows == 0) return NA_OK;
  if (out == nullptr || lse == nullptr)
    return fail(NA_ERR_INVALID, "out/lse must be non-NULL");
  na::merge_fwd(p->dtype, p->n_parts, p->rows, p->head_dim, outs, lses, out,
                lse, as_stream(stream));
  return launch_status("na_merge_fwd");
}

int na_merge_bwd(const na_merge_params *p, const void *const *outs,
                 const float *const *lses, const void *dout, const float *dlse,
                 void *const *d_outs, float *const *d_lses, void *stream) {
  const int rc = check_merge(p, outs, lses);
  if (rc != NA_OK) return rc;
  if (p->rows == 0) return NA_OK;
  if (dout == nullptr) return fail(NA_ERR_INVALID, "dout must be non-NULL");
  na::merge_bwd(p->dtype, p->n_parts, p->rows, p->head_dim, outs, lses, dout,
                dlse, d_outs, d_lses, as_stream(stream));
  return launch_status("na_merge_bwd");
}

}  // extern "C"
