// The fused op as a torch custom operator with its autograd node in C++
// (natten_amd::na_fused), over the C ABI of libnatten_amd.so.
//
// The reference's autograd layer (autograd/na1d.py:34-53, na2d.py:34-64,
// na3d.py) wraps the fused forward / backward in an mx.custom_function; the
// Python twin here is autograd/fused.py's _FusedNA.  This node does the same
// work without Python in the backward and without ctypes marshalling in
// either direction: an eager training step is host-bound (the config-2
// kernels take ~21 us per step, the host path several times that), so the
// per-call host cost is what a caller who does not capture graphs sees.
//
// Built with the host compiler against torch's headers only (no HIP
// headers): the caller passes torch's current stream handle, and the
// backward launches on the forward's stream (torch runs a node's backward
// on the stream of its forward).

#include <ATen/ATen.h>
#include <torch/csrc/autograd/custom_function.h>
#include <torch/library.h>

#include <cstdint>
#include <vector>

#include "natten_amd.h"

namespace {

using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

void check_rc(int rc, const char *what) {
  TORCH_CHECK(rc == NA_OK, "natten_amd ", what, " failed (", rc, "): ", na_last_error());
}

void check_device(const at::Tensor &t) {
  if (!t.defined()) return;
  TORCH_CHECK(t.is_cuda(),
              "natten_amd's hip backend runs on MI355X (HIP) tensors only; got a tensor on ",
              t.device(), ". There is no CPU implementation.");
}

int32_t dtype_code(at::ScalarType s) {
  switch (s) {
    case at::kFloat:
      return NA_F32;
    case at::kHalf:
      return NA_F16;
    case at::kBFloat16:
      return NA_BF16;
    default:
      TORCH_CHECK(false, "natten_amd supports float32/float16/bfloat16 tensors, got ", s);
  }
  return -1;
}

const void *cptr(const at::Tensor &t) { return t.defined() ? t.data_ptr() : nullptr; }
void *mptr(const at::Tensor &t) { return t.defined() ? t.data_ptr() : nullptr; }

// q [B, X..., H, D], k [B, X..., H_kv, D]; per-axis fields hold the rank's
// axes first and 1 (0 for causal) after them, as na_params documents.
na_params make_params(const at::Tensor &q, const at::Tensor &k, at::IntArrayRef kernel,
                      at::IntArrayRef stride, at::IntArrayRef dilation,
                      at::IntArrayRef causal, double scale, int64_t n_extra, int64_t flags,
                      const at::Tensor &sample_extent) {
  const int64_t rank = q.dim() - 3;
  TORCH_CHECK(rank >= 1 && rank <= 3, "natten_amd: q must be [B, *spatial, heads, dim]");
  TORCH_CHECK((int64_t)kernel.size() == rank && (int64_t)stride.size() == rank &&
                  (int64_t)dilation.size() == rank && (int64_t)causal.size() == rank,
              "natten_amd: per-axis parameters must have one entry per spatial axis");
  na_params p{};
  p.rank = (int32_t)rank;
  p.batch = (int32_t)q.size(0);
  p.heads = (int32_t)q.size(-2);
  p.kv_heads = (int32_t)k.size(-2);
  p.head_dim = (int32_t)q.size(-1);
  p.dtype = dtype_code(q.scalar_type());
  for (int a = 0; a < 3; ++a) {
    p.extent[a] = 1;
    p.kernel[a] = 1;
    p.dilation[a] = 1;
    p.stride[a] = 1;
    p.causal[a] = 0;
  }
  for (int64_t a = 0; a < rank; ++a) {
    p.extent[a] = (int32_t)q.size(1 + a);
    p.kernel[a] = (int32_t)kernel[a];
    p.dilation[a] = (int32_t)dilation[a];
    p.stride[a] = (int32_t)stride[a];
    p.causal[a] = causal[a] != 0 ? 1 : 0;
  }
  p.scale = (float)scale;
  p.n_extra = (int32_t)n_extra;
  p.flags = (int32_t)flags;
  p.sample_extent =
      sample_extent.defined() ? static_cast<const int32_t *>(sample_extent.data_ptr()) : nullptr;
  return p;
}

at::Tensor contig(const at::Tensor &t) { return t.defined() ? t.contiguous() : t; }

struct FusedNA : public torch::autograd::Function<FusedNA> {
  // The optional inputs come as std::optional so that an absent one is not
  // taken for an (undefined) variable input of the node.
  static variable_list forward(AutogradContext *ctx, at::Tensor q, at::Tensor k, at::Tensor v,
                               std::optional<at::Tensor> extra_k_opt,
                               std::optional<at::Tensor> extra_v_opt,
                               std::optional<at::Tensor> sample_extent_opt,
                               std::vector<int64_t> kernel, std::vector<int64_t> stride,
                               std::vector<int64_t> dilation, std::vector<int64_t> causal,
                               double scale, int64_t flags, int64_t stream) {
    at::Tensor extra_k = extra_k_opt.value_or(at::Tensor());
    at::Tensor extra_v = extra_v_opt.value_or(at::Tensor());
    const at::Tensor sample_extent = sample_extent_opt.value_or(at::Tensor());
    for (const at::Tensor *t : std::initializer_list<const at::Tensor *>{
             &q, &k, &v, &extra_k, &extra_v, &sample_extent})
      check_device(*t);
    // the shape rules the functional layer has already applied, restated for
    // direct callers of the operator
    TORCH_CHECK(q.dim() == k.dim() && q.dim() == v.dim() && q.size(0) == k.size(0) &&
                    q.size(0) == v.size(0) && k.sizes() == v.sizes() && q.size(-1) == k.size(-1),
                "natten_amd na_fused: q [B, *spatial, H, D], k / v [B, *spatial, H_kv, D]");
    for (int64_t a = 1; a + 2 < q.dim(); ++a)
      TORCH_CHECK(q.size(a) == k.size(a), "natten_amd na_fused: spatial extents differ");
    TORCH_CHECK(k.size(-2) > 0 && q.size(-2) % k.size(-2) == 0,
                "natten_amd na_fused: heads_q must be divisible by heads_kv");
    TORCH_CHECK(k.scalar_type() == q.scalar_type() && v.scalar_type() == q.scalar_type(),
                "natten_amd na_fused: q, k and v must share a dtype");
    TORCH_CHECK(extra_k.defined() == extra_v.defined(),
                "natten_amd na_fused: extra_k and extra_v come together");
    if (extra_k.defined())
      TORCH_CHECK(extra_k.dim() == 4 && extra_k.sizes() == extra_v.sizes() &&
                      extra_k.size(0) == q.size(0) && extra_k.size(2) == k.size(-2) &&
                      extra_k.size(3) == q.size(-1) && extra_k.scalar_type() == q.scalar_type() &&
                      extra_v.scalar_type() == q.scalar_type(),
                  "natten_amd na_fused: extra_k / extra_v [B, N_extra, H_kv, D] in q's dtype");
    if (sample_extent.defined())
      TORCH_CHECK(sample_extent.scalar_type() == at::kInt && sample_extent.is_contiguous() &&
                      sample_extent.numel() == q.size(0) * (q.dim() - 3),
                  "natten_amd na_fused: sample_extent is a contiguous int32 [B, rank] tensor");
    q = q.contiguous();
    k = contig(k);
    v = contig(v);
    extra_k = contig(extra_k);
    extra_v = contig(extra_v);
    const int64_t n_extra = extra_k.defined() ? extra_k.size(1) : 0;
    const na_params p = make_params(q, k, kernel, stride, dilation, causal, scale, n_extra, flags,
                                    sample_extent);
    std::vector<int64_t> osz(q.sizes().begin(), q.sizes().end());
    for (size_t a = 0; a < kernel.size(); ++a)
      osz[1 + a] = (osz[1 + a] + stride[a] - 1) / stride[a];
    at::Tensor out = at::empty(osz, q.options());
    osz.pop_back();
    at::Tensor lse = at::empty(osz, q.options().dtype(at::kFloat));
    check_rc(na_fwd(&p, q.data_ptr(), k.data_ptr(), v.data_ptr(), cptr(extra_k), cptr(extra_v),
                    out.data_ptr(), static_cast<float *>(lse.data_ptr()),
                    reinterpret_cast<void *>(stream)),
             "na_fwd");
    ctx->save_for_backward({q, k, v, extra_k, extra_v, out, lse, sample_extent});
    ctx->saved_data["kernel"] = kernel;
    ctx->saved_data["stride"] = stride;
    ctx->saved_data["dilation"] = dilation;
    ctx->saved_data["causal"] = causal;
    ctx->saved_data["scale"] = scale;
    ctx->saved_data["flags"] = flags;
    ctx->saved_data["stream"] = stream;
    // lse is differentiable too: its gradient enters the backward as
    // delta - dlse
    ctx->set_materialize_grads(false);
    return {out, lse};
  }

  static variable_list backward(AutogradContext *ctx, variable_list grads) {
    const variable_list s = ctx->get_saved_variables();
    const at::Tensor &q = s[0], &k = s[1], &v = s[2], &extra_k = s[3], &extra_v = s[4],
                     &out = s[5], &lse = s[6], &sample_extent = s[7];
    at::Tensor gout = grads[0], glse = grads.size() > 1 ? grads[1] : at::Tensor();
    if (!gout.defined()) gout = at::zeros_like(out);
    gout = gout.contiguous();
    if (gout.scalar_type() != q.scalar_type()) gout = gout.to(q.scalar_type());
    if (glse.defined()) {
      glse = glse.contiguous();
      if (glse.scalar_type() != at::kFloat) glse = glse.to(at::kFloat);
    }
    const auto kernel = ctx->saved_data["kernel"].toIntVector();
    const auto stride = ctx->saved_data["stride"].toIntVector();
    const auto dilation = ctx->saved_data["dilation"].toIntVector();
    const auto causal = ctx->saved_data["causal"].toIntVector();
    const double scale = ctx->saved_data["scale"].toDouble();
    const int64_t flags = ctx->saved_data["flags"].toInt();
    void *stream = reinterpret_cast<void *>(ctx->saved_data["stream"].toInt());
    const int64_t n_extra = extra_k.defined() ? extra_k.size(1) : 0;
    const na_params p = make_params(q, k, kernel, stride, dilation, causal, scale, n_extra, flags,
                                    sample_extent);
    const size_t ws_bytes = na_bwd_workspace_bytes(&p);
    at::Tensor dq = at::empty_like(q), dk = at::empty_like(k), dv = at::empty_like(v);
    at::Tensor dek = n_extra ? at::empty_like(extra_k) : at::Tensor();
    at::Tensor dev = n_extra ? at::empty_like(extra_v) : at::Tensor();
    at::Tensor ws = ws_bytes ? at::empty({(int64_t)ws_bytes}, q.options().dtype(at::kByte))
                             : at::Tensor();
    const float *dlse = glse.defined() ? static_cast<const float *>(glse.data_ptr()) : nullptr;
    check_rc(na_bwd(&p, q.data_ptr(), k.data_ptr(), v.data_ptr(), cptr(extra_k), cptr(extra_v),
                    out.data_ptr(), static_cast<const float *>(lse.data_ptr()), gout.data_ptr(),
                    dlse, dq.data_ptr(),
                    dk.data_ptr(), dv.data_ptr(), mptr(dek), mptr(dev), mptr(ws), ws_bytes,
                    stream),
             "na_bwd");
    // one entry per forward input: q, k, v, extra_k, extra_v, then the
    // non-differentiable sample extents and parameters
    return {dq, dk, dv, dek, dev, at::Tensor(), at::Tensor(), at::Tensor(),
            at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor()};
  }
};

std::tuple<at::Tensor, at::Tensor> na_fused(const at::Tensor &q, const at::Tensor &k,
                                            const at::Tensor &v,
                                            const std::optional<at::Tensor> &extra_k,
                                            const std::optional<at::Tensor> &extra_v,
                                            const std::optional<at::Tensor> &sample_extent,
                                            at::IntArrayRef kernel, at::IntArrayRef stride,
                                            at::IntArrayRef dilation, at::IntArrayRef causal,
                                            double scale, int64_t flags, int64_t stream) {
  auto r = FusedNA::apply(q, k, v, extra_k, extra_v, sample_extent, kernel.vec(), stride.vec(),
                          dilation.vec(), causal.vec(), scale, flags, stream);
  return {r[0], r[1]};
}

}  // namespace

TORCH_LIBRARY(natten_amd, m) {
  m.def(
      "na_fused(Tensor q, Tensor k, Tensor v, Tensor? extra_k, Tensor? extra_v, "
      "Tensor? sample_extent, int[] kernel, int[] stride, int[] dilation, int[] causal, "
      "float scale, int flags, int stream) -> (Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(natten_amd, CompositeImplicitAutograd, m) { m.impl("na_fused", na_fused); }
