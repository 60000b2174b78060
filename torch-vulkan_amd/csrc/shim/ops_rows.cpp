// Row operators on the vk device: softmax (+backward, _safe_softmax), layer_norm (+backward), sum / mean
// and cat.  Reference: csrc/ops_rows.cpp:36-332, registrations :336-346.  Non-contiguous inputs of the
// row kernels are made contiguous on the device first; dtype conversions (half_to_float,
// _safe_softmax(dtype)) likewise; the reduction reads any strided view in place.
#include <ATen/Operators.h>
#include <ATen/WrapDimUtilsMulti.h>
#include <ATen/native/TypeProperties.h>

#include <bitset>
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

// ---- sum / mean (reference: try_reduce and its users, csrc/ops_rows.cpp:183-270) -------------------------
// Any subset of up to 8 dimensions of a strided f32/bf16/f16 view, optional output dtype (a float kind);
// fp32 accumulation, one rounding.  The kernel picks its layout and, for few outputs, splits the reduced
// range into fp32 partial sums in a workspace this adapter allocates.
std::optional<at::Tensor> try_reduce(const at::Tensor& self, at::OptionalIntArrayRef dim_opt, bool keepdim,
                                     std::optional<at::ScalarType> dtype, bool mean, const char* aten_name) {
  if (!is_vk(self) || float_code(self.scalar_type()) < 0) return std::nullopt;
  const at::ScalarType odt = dtype.value_or(self.scalar_type());
  const int64_t nd = self.dim();
  if (float_code(odt) < 0 || nd > HRT_MAX_DIMS) return std::nullopt;
  std::bitset<at::dim_bitset_size> red;
  if (!dim_opt.has_value() || dim_opt->empty()) {
    for (int64_t d = 0; d < nd; ++d) red.set(d);
  } else {
    red = at::dim_list_to_bitset(*dim_opt, nd);  // wraps negative dims, rejects repeats as PyTorch does
  }
  hrt_reduce_args A{};
  std::vector<int64_t> out_sizes;
  int64_t n_red = 1;
  A.ndim = (int32_t)nd;
  for (int64_t d = 0; d < nd; ++d) {
    if (self.stride(d) < 0) return std::nullopt;
    A.sizes[d] = self.size(d);
    A.strides[d] = self.stride(d);
    if (red.test(d)) {
      A.reduce_mask |= 1u << d;
      n_red *= self.size(d);
      if (keepdim) out_sizes.push_back(1);
    } else {
      out_sizes.push_back(self.size(d));
    }
  }
  at::Tensor out = at::empty(out_sizes, self.options().dtype(odt));
  A.x = addr_of(self);
  A.out = addr_of(out);
  A.x_dtype = float_code(self.scalar_type());
  A.out_dtype = float_code(odt);
  A.div = mean ? (float)n_red : 1.0f;
  const int64_t ws_floats = hrt_reduce_workspace(&A);
  TORCH_CHECK(ws_floats >= 0, "vk: reduce_sum rejected its arguments");
  at::Tensor ws;
  if (ws_floats > 0) {
    ws = at::empty({ws_floats}, self.options().dtype(at::kFloat));
    A.ws = addr_of(ws);
  }
  if (out.numel() > 0) launch("reduce_sum", A);
  count_kernel(aten_name);
  return out;
}

at::Tensor k_sum_dim(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim, std::optional<at::ScalarType> dtype) {
  if (auto r = try_reduce(self, dim, keepdim, dtype, false, "aten::sum.dim_IntList")) return *r;
  return VKT_FALLBACK(sum_dim_IntList, self, dim, keepdim, dtype);
}
at::Tensor k_mean_dim(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim, std::optional<at::ScalarType> dtype) {
  if (auto r = try_reduce(self, dim, keepdim, dtype, true, "aten::mean.dim")) return *r;
  return VKT_FALLBACK(mean_dim, self, dim, keepdim, dtype);
}
at::Tensor k_sum(const at::Tensor& self, std::optional<at::ScalarType> dtype) {
  if (auto r = try_reduce(self, std::nullopt, false, dtype, false, "aten::sum")) return *r;
  return VKT_FALLBACK(sum, self, dtype);
}
at::Tensor k_mean(const at::Tensor& self, std::optional<at::ScalarType> dtype) {
  if (auto r = try_reduce(self, std::nullopt, false, dtype, true, "aten::mean")) return *r;
  return VKT_FALLBACK(mean, self, dtype);
}

// ---- cat (reference: k_cat, csrc/ops_rows.cpp:272-332) -----------------------------------------------
// The output is allocated on the device and every part is copied into its slice by the strided
// copy/cast kernel.  Parts of float kinds may differ in dtype (PyTorch's result type); other dtypes must
// all be the same.  1-D empty parts are skipped (PyTorch's legacy rule, as the reference does).
// Same-dtype contiguous parts whose rows (the elements from `dim` on) are whole 16-byte chunks: one
// "cat_rows16" launch per 8 parts instead of one copy per part.
bool cat_one_launch(const at::Tensor& out, const std::vector<at::Tensor>& parts, int64_t dim) {
  const int64_t es = (int64_t)out.element_size();
  int64_t outer = 1, inner = 1;
  for (int64_t d = 0; d < dim; ++d) outer *= out.size(d);
  for (int64_t d = dim + 1; d < out.dim(); ++d) inner *= out.size(d);
  const int64_t orow = out.size(dim) * inner * es;
  if (outer == 0 || orow == 0 || orow % 16 || reinterpret_cast<uintptr_t>(out.data_ptr()) % 16) return false;
  std::vector<const at::Tensor*> use;
  for (const auto& t : parts) {
    if (t.size(dim) == 0) continue;
    if (t.scalar_type() != out.scalar_type() || !t.is_contiguous() || (t.size(dim) * inner * es) % 16 ||
        reinterpret_cast<uintptr_t>(t.data_ptr()) % 16)
      return false;
    use.push_back(&t);
  }
  int64_t col = 0;
  for (size_t g = 0; g < use.size(); g += HRT_CAT_MAX_PARTS) {
    hrt_cat_args A{};
    A.out = (uint64_t)out.data_ptr();
    A.outer = outer;
    A.out_row_bytes = orow;
    for (size_t k = g; k < use.size() && k < g + HRT_CAT_MAX_PARTS; ++k) {
      const int i = A.nparts++;
      A.src[i] = (uint64_t)use[k]->data_ptr();
      A.row_bytes[i] = use[k]->size(dim) * inner * es;
      A.col[i] = col;
      col += A.row_bytes[i];
    }
    launch("cat_rows16", A);
  }
  return true;
}

at::Tensor k_cat(const at::ITensorListRef& tensors, int64_t dim) {
  std::vector<at::Tensor> parts;
  bool ok = true, all_float = true, same = true;
  at::ScalarType dt = at::kFloat;
  bool first = true;
  for (const at::Tensor& t : tensors) {
    ok = ok && is_vk(t);
    all_float = all_float && float_code(t.scalar_type()) >= 0;
    if (first) dt = t.scalar_type();
    same = same && t.scalar_type() == dt;
    first = false;
    if (!(t.dim() == 1 && t.size(0) == 0)) parts.push_back(t);
  }
  ok = ok && !first && (same || all_float) && !parts.empty();
  if (ok) {
    const at::ScalarType odt = same ? dt : at::native::result_type(tensors);
    const int64_t nd = parts[0].dim();
    ok = nd > 0 && (float_code(odt) >= 0) == all_float;
    if (ok) {
      dim = at::maybe_wrap_dim(dim, nd);
      std::vector<int64_t> sizes(parts[0].sizes().begin(), parts[0].sizes().end());
      sizes[dim] = 0;
      for (const auto& t : parts) {
        ok = ok && t.dim() == nd;
        for (int64_t d = 0; ok && d < nd; ++d)
          if (d != dim) ok = t.size(d) == parts[0].size(d);
        if (!ok) break;
        sizes[dim] += t.size(dim);
      }
      if (ok) {
        at::Tensor out = at::empty(sizes, parts[0].options().dtype(odt));
        if (!cat_one_launch(out, parts, dim)) {
          int64_t off = 0;
          for (const auto& t : parts) {
            if (t.size(dim) > 0) out.narrow(dim, off, t.size(dim)).copy_(t);
            off += t.size(dim);
          }
        }
        count_kernel("aten::cat");
        return out;
      }
    }
  }
  return VKT_FALLBACK(cat, tensors, dim);
}

}  // namespace

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("sum.dim_IntList", &k_sum_dim);
  m.impl("mean.dim", &k_mean_dim);
  m.impl("sum", &k_sum);
  m.impl("mean", &k_mean);
  m.impl("cat", &k_cat);
  m.impl("_softmax", &k_softmax);
  m.impl("_safe_softmax", &k_safe_softmax);
  m.impl("_softmax_backward_data", &k_softmax_backward);
  m.impl("native_layer_norm", &k_native_layer_norm);
  m.impl("native_layer_norm_backward", &k_native_layer_norm_backward);
}
