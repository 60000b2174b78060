// Row operators on the vk device: softmax (+backward, _safe_softmax) and layer_norm (+backward).
// Reference: csrc/ops_rows.cpp:36-181, registrations :336-341.  Non-contiguous inputs are made
// contiguous on the device first; dtype conversions (half_to_float, _safe_softmax(dtype)) likewise.
#include <ATen/Operators.h>

#include <optional>
#include <string>
#include <tuple>
#include <vector>

#include "common.h"

namespace {

using namespace vkt;

at::Tensor contig(const at::Tensor& t) { return t.is_contiguous() ? t : t.contiguous(); }

// View a tensor as [outer, R, inner] around `dim` (csrc/ops_rows.cpp:43-57).
bool softmax_dims(const at::Tensor& t, int64_t dim, int64_t& outer, int64_t& R, int64_t& inner) {
  if (t.dim() == 0) {
    outer = R = inner = 1;
    return true;
  }
  dim = at::maybe_wrap_dim(dim, t.dim());
  outer = 1;
  inner = 1;
  for (int64_t d = 0; d < dim; ++d) outer *= t.size(d);
  for (int64_t d = dim + 1; d < t.dim(); ++d) inner *= t.size(d);
  R = t.size(dim);
  return true;
}

std::optional<at::Tensor> try_softmax(const at::Tensor& self, int64_t dim, std::optional<at::ScalarType> out_dtype, bool safe,
                                      const char* aten_name) {
  if (!is_vk(self) || self.numel() == 0) return std::nullopt;
  const at::ScalarType dt = out_dtype.value_or(self.scalar_type());
  const char* k = kind_name(dt);
  if (!k || !kind_name(self.scalar_type())) return std::nullopt;
  int64_t outer, R, inner;
  if (!softmax_dims(self, dim, outer, R, inner)) return std::nullopt;
  at::Tensor x = contig(self.scalar_type() == dt ? self : self.to(dt));
  at::Tensor y = at::empty(x.sizes(), x.options());
  hrt_softmax_args P{};
  P.x = addr_of(x);
  P.y = addr_of(y);
  P.outer = outer;
  P.R = R;
  P.inner = inner;
  P.safe = safe ? 1u : 0u;
  launch(std::string("softmax_fwd_") + k, P);
  count_kernel(aten_name);
  return y;
}

at::Tensor k_softmax(const at::Tensor& self, int64_t dim, bool half_to_float) {
  std::optional<at::ScalarType> dt = half_to_float ? std::optional<at::ScalarType>(at::kFloat) : std::nullopt;
  if (auto r = try_softmax(self, dim, dt, false, "aten::_softmax")) return *r;
  return VKT_FALLBACK(_softmax, self, dim, half_to_float);
}

at::Tensor k_safe_softmax(const at::Tensor& self, int64_t dim, std::optional<at::ScalarType> dtype) {
  if (auto r = try_softmax(self, dim, dtype, true, "aten::_safe_softmax")) return *r;
  return VKT_FALLBACK(_safe_softmax, self, dim, dtype);
}

at::Tensor k_softmax_backward(const at::Tensor& g, const at::Tensor& y, int64_t dim, at::ScalarType input_dtype) {
  const char* k = (is_vk(g) && is_vk(y)) ? kind_name(y.scalar_type()) : nullptr;
  int64_t outer, R, inner;
  if (k && kind_name(g.scalar_type()) && kind_name(input_dtype) && g.sizes() == y.sizes() && y.numel() > 0 &&
      softmax_dims(y, dim, outer, R, inner)) {
    // computed in y's dtype, converted to the forward input's dtype (csrc/ops_rows.cpp:86-100)
    at::Tensor gc = contig(g.scalar_type() == y.scalar_type() ? g : g.to(y.scalar_type()));
    at::Tensor yc = contig(y);
    at::Tensor dx = at::empty(yc.sizes(), yc.options());
    hrt_softmax_args P{};
    P.y = addr_of(yc);
    P.g = addr_of(gc);
    P.dx = addr_of(dx);
    P.outer = outer;
    P.R = R;
    P.inner = inner;
    launch(std::string("softmax_bwd_") + k, P);
    count_kernel("aten::_softmax_backward_data");
    return input_dtype == dx.scalar_type() ? dx : dx.to(input_dtype);
  }
  return VKT_FALLBACK(_softmax_backward_data, g, y, dim, input_dtype);
}

int64_t prod(c10::IntArrayRef s) {
  int64_t n = 1;
  for (auto v : s) n *= v;
  return n;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> k_native_layer_norm(const at::Tensor& input, c10::SymIntArrayRef normalized_shape_sym,
                                                                   const std::optional<at::Tensor>& weight,
                                                                   const std::optional<at::Tensor>& bias, double eps) {
  auto normalized_shape = C10_AS_INTARRAYREF_SLOW(normalized_shape_sym);
  const char* k = is_vk(input) ? kind_name(input.scalar_type()) : nullptr;
  const int64_t D = prod(normalized_shape);
  bool ok = k && D > 0 && input.numel() > 0 && (int64_t)normalized_shape.size() <= input.dim();
  auto param_ok = [&](const std::optional<at::Tensor>& p) {
    return !p.has_value() || !p->defined() || (is_vk(*p) && p->scalar_type() == input.scalar_type() && p->numel() == D);
  };
  ok = ok && param_ok(weight) && param_ok(bias);
  if (ok) {
    at::Tensor x = contig(input);
    const int64_t rows = x.numel() / D;
    at::Tensor y = at::empty(x.sizes(), x.options());
    // statistics keep the input's leading dims with the normalized dims set to 1, fp32 (ops_rows.cpp:131-134)
    std::vector<int64_t> stat_shape(x.sizes().begin(), x.sizes().end() - normalized_shape.size());
    stat_shape.insert(stat_shape.end(), normalized_shape.size(), 1);
    at::Tensor mean = at::empty(stat_shape, x.options().dtype(at::kFloat));
    at::Tensor rstd = at::empty(stat_shape, x.options().dtype(at::kFloat));
    at::Tensor w = (weight.has_value() && weight->defined()) ? contig(*weight) : at::Tensor();
    at::Tensor b = (bias.has_value() && bias->defined()) ? contig(*bias) : at::Tensor();
    hrt_ln_args P{};
    P.x = addr_of(x);
    P.y = addr_of(y);
    P.mean = addr_of(mean);
    P.rstd = addr_of(rstd);
    P.w = w.defined() ? addr_of(w) : 0;
    P.b = b.defined() ? addr_of(b) : 0;
    P.rows = rows;
    P.D = D;
    P.eps = (float)eps;
    launch(std::string("ln_fwd_") + k, P);
    count_kernel("aten::native_layer_norm");
    return {y, mean, rstd};
  }
  return VKT_FALLBACK_SYMINT(native_layer_norm, input, normalized_shape_sym, weight, bias, eps);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> k_native_layer_norm_backward(
    const at::Tensor& grad_out, const at::Tensor& input, c10::SymIntArrayRef normalized_shape_sym, const at::Tensor& mean,
    const at::Tensor& rstd, const std::optional<at::Tensor>& weight, const std::optional<at::Tensor>& bias,
    std::array<bool, 3> output_mask) {
  auto normalized_shape = C10_AS_INTARRAYREF_SLOW(normalized_shape_sym);
  const char* k = (is_vk(grad_out) && is_vk(input)) ? kind_name(input.scalar_type()) : nullptr;
  const int64_t D = prod(normalized_shape);
  const bool has_w = weight.has_value() && weight->defined();
  const bool has_b = bias.has_value() && bias->defined();
  const bool ok = k && D > 0 && input.numel() > 0 && grad_out.scalar_type() == input.scalar_type() &&
                  grad_out.sizes() == input.sizes() && is_vk(mean) && is_vk(rstd) && mean.scalar_type() == at::kFloat &&
                  rstd.scalar_type() == at::kFloat && mean.numel() * D == input.numel() && rstd.numel() * D == input.numel() &&
                  (!has_w || (is_vk(*weight) && weight->scalar_type() == input.scalar_type() && weight->numel() == D)) &&
                  (!has_b || (is_vk(*bias) && bias->scalar_type() == input.scalar_type() && bias->numel() == D));
  if (ok) {
    at::Tensor g = contig(grad_out), x = contig(input), mu = contig(mean), rs = contig(rstd);
    at::Tensor w = has_w ? contig(*weight) : at::Tensor();
    const int64_t rows = x.numel() / D;
    at::Tensor dx, dw, db, ws;
    const bool want_dw = output_mask[1] && has_w;
    const bool want_db = output_mask[2] && has_b;
    hrt_ln_args P{};
    P.x = addr_of(x);
    P.g = addr_of(g);
    P.mean = addr_of(mu);
    P.rstd = addr_of(rs);
    P.w = has_w ? addr_of(w) : 0;
    P.rows = rows;
    P.D = D;
    if (output_mask[0]) {
      dx = at::empty(x.sizes(), x.options());
      P.dx = addr_of(dx);
    }
    if (want_dw || want_db) {
      ws = at::empty({hrt_ln_chunks(rows), 2, D}, x.options().dtype(at::kFloat));
      P.ws = addr_of(ws);
    }
    if (P.dx || P.ws) launch(std::string("ln_bwd_") + k, P);
    if (want_dw || want_db) {
      if (want_dw) dw = at::empty(weight->sizes(), weight->options());
      if (want_db) db = at::empty(bias->sizes(), bias->options());
      P.dw = want_dw ? addr_of(dw) : 0;
      P.db = want_db ? addr_of(db) : 0;
      launch(std::string("ln_wgrad_") + k, P);
    }
    count_kernel("aten::native_layer_norm_backward");
    return {dx, dw, db};
  }
  return VKT_FALLBACK_SYMINT(native_layer_norm_backward, grad_out, input, normalized_shape_sym, mean, rstd, weight, bias,
                             output_mask);
}

}  // namespace

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("_softmax", &k_softmax);
  m.impl("_safe_softmax", &k_safe_softmax);
  m.impl("_softmax_backward_data", &k_softmax_backward);
  m.impl("native_layer_norm", &k_native_layer_norm);
  m.impl("native_layer_norm_backward", &k_native_layer_norm_backward);
}
