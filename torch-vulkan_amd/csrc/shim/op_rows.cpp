// Row operators on the vk device: softmax (_softmax, _safe_softmax, _softmax_backward_data) and layer_norm
// (native_layer_norm and its backward).  The reference registers the same five (csrc/ops_rows.cpp:336-341)
// with these rules, which fix what PyTorch sees:
//   * float kinds only (f32/bf16/f16); a requested result dtype (half_to_float, _safe_softmax's dtype)
//     converts the input first, and the softmax backward computes in the output's dtype and returns the
//     forward input's dtype;
//   * _safe_softmax gives exact 0 for rows that are entirely -inf;
//   * layer_norm's mean and rstd are fp32 and shaped like the input with the normalized dimensions set to 1;
//     weight and bias, when given, must be vk tensors of the input's dtype with D elements;
//   * everything else runs on the CPU.
// Non-contiguous operands are made contiguous on the device before the row kernels run.
#include <c10/util/accumulate.h>

#include "common.h"

namespace {

using namespace vkt;

// ---- softmax ------------------------------------------------------------------------------------------------
// A contiguous tensor seen as [outer, R, inner] around dimension `dim` (R = its length).
struct RowSpan {
  int64_t outer, R, inner;
};

RowSpan span_around(const at::Tensor& t, int64_t dim) {
  if (t.dim() == 0) return {1, 1, 1};
  const int64_t d = at::maybe_wrap_dim(dim, t.dim());
  const c10::IntArrayRef s = t.sizes();
  const int64_t inner = c10::multiply_integers(s.begin() + d + 1, s.end());
  return {c10::multiply_integers(s.begin(), s.begin() + d), s[d], inner};
}

hrt_softmax_args softmax_args(const RowSpan& r) {
  hrt_softmax_args A{};
  A.outer = r.outer, A.R = r.R, A.inner = r.inner;
  return A;
}

// Forward in dtype `compute` (the input converted to it when it differs).
std::optional<at::Tensor> softmax_vk(const at::Tensor& self, int64_t dim, at::ScalarType compute, bool safe, const char* op) {
  if (!on_vk(self) || self.numel() == 0 || float_code(self.scalar_type()) < 0 || float_code(compute) < 0) return std::nullopt;
  const at::Tensor x = dense(self.scalar_type() == compute ? self : self.to(compute));
  at::Tensor y = at::empty_like(x, at::MemoryFormat::Contiguous);
  hrt_softmax_args A = softmax_args(span_around(x, dim));
  A.x = dptr(x), A.y = dptr(y), A.safe = safe ? 1u : 0u;
  queue(typed("softmax_fwd", compute), A);
  note_gpu(op);
  return y;
}

at::Tensor k_softmax(const at::Tensor& self, int64_t dim, bool half_to_float) {
  const at::ScalarType compute = half_to_float ? at::kFloat : self.scalar_type();
  if (auto y = softmax_vk(self, dim, compute, false, "aten::_softmax")) return *y;
  return VKT_CPU(_softmax, self, dim, half_to_float);
}

at::Tensor k_safe_softmax(const at::Tensor& self, int64_t dim, std::optional<at::ScalarType> dtype) {
  if (auto y = softmax_vk(self, dim, dtype.value_or(self.scalar_type()), true, "aten::_safe_softmax")) return *y;
  return VKT_CPU(_safe_softmax, self, dim, dtype);
}

at::Tensor k_softmax_backward(const at::Tensor& grad, const at::Tensor& out, int64_t dim, at::ScalarType input_dtype) {
  const at::ScalarType compute = out.scalar_type();
  const bool ok = on_vk(grad) && on_vk(out) && out.numel() > 0 && grad.sizes().equals(out.sizes()) &&
                  float_code(compute) >= 0 && float_code(grad.scalar_type()) >= 0 && float_code(input_dtype) >= 0;
  if (!ok) return VKT_CPU(_softmax_backward_data, grad, out, dim, input_dtype);
  const at::Tensor y = dense(out), g = dense(grad.scalar_type() == compute ? grad : grad.to(compute));
  at::Tensor dx = at::empty_like(y, at::MemoryFormat::Contiguous);
  hrt_softmax_args A = softmax_args(span_around(y, dim));
  A.y = dptr(y), A.g = dptr(g), A.dx = dptr(dx);
  queue(typed("softmax_bwd", compute), A);
  note_gpu("aten::_softmax_backward_data");
  return input_dtype == compute ? dx : dx.to(input_dtype);
}

// ---- layer_norm ----------------------------------------------------------------------------------------------
// rows x D: D = the product of the normalized (trailing) dimensions.
struct LnShape {
  int64_t rows, D;
};

std::optional<LnShape> ln_shape(const at::Tensor& x, c10::IntArrayRef normalized) {
  if (!on_vk(x) || float_code(x.scalar_type()) < 0 || x.numel() == 0) return std::nullopt;
  if (static_cast<int64_t>(normalized.size()) > x.dim()) return std::nullopt;
  const int64_t D = c10::multiply_integers(normalized);
  if (D <= 0) return std::nullopt;
  return LnShape{x.numel() / D, D};
}

// An affine parameter the kernels can read: absent, or a vk tensor of x's dtype with D elements.
// Returns false for a parameter that disqualifies the call; `dev` gets the dense tensor (or stays undefined).
bool affine_param(const std::optional<at::Tensor>& p, const at::Tensor& x, int64_t D, at::Tensor* dev) {
  if (!present(p)) return true;
  if (!on_vk(*p) || p->scalar_type() != x.scalar_type() || p->numel() != D) return false;
  *dev = dense(*p);
  return true;
}

// mean / rstd shape: x's sizes with the normalized dimensions set to 1.
std::vector<int64_t> stat_sizes(const at::Tensor& x, size_t normalized_dims) {
  std::vector<int64_t> s = x.sizes().vec();
  std::fill(s.end() - static_cast<std::ptrdiff_t>(normalized_dims), s.end(), 1);
  return s;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> k_layer_norm(const at::Tensor& input, c10::SymIntArrayRef normalized_sym,
                                                           const std::optional<at::Tensor>& weight,
                                                           const std::optional<at::Tensor>& bias, double eps) {
  const c10::IntArrayRef normalized = C10_AS_INTARRAYREF_SLOW(normalized_sym);
  const std::optional<LnShape> sh = ln_shape(input, normalized);
  at::Tensor w, b;
  if (!sh || !affine_param(weight, input, sh->D, &w) || !affine_param(bias, input, sh->D, &b))
    return VKT_CPU_SYMINT(native_layer_norm, input, normalized_sym, weight, bias, eps);
  const at::Tensor x = dense(input);
  at::Tensor y = at::empty_like(x, at::MemoryFormat::Contiguous);
  const std::vector<int64_t> ss = stat_sizes(x, normalized.size());
  at::Tensor mean = at::empty(ss, x.options().dtype(at::kFloat)), rstd = at::empty(ss, x.options().dtype(at::kFloat));
  hrt_ln_args A{};
  A.x = dptr(x), A.y = dptr(y), A.mean = dptr(mean), A.rstd = dptr(rstd);
  A.w = w.defined() ? dptr(w) : 0;
  A.b = b.defined() ? dptr(b) : 0;
  A.rows = sh->rows, A.D = sh->D, A.eps = static_cast<float>(eps);
  queue(typed("ln_fwd", x.scalar_type()), A);
  note_gpu("aten::native_layer_norm");
  return {y, mean, rstd};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> k_layer_norm_backward(
    const at::Tensor& grad_out, const at::Tensor& input, c10::SymIntArrayRef normalized_sym, const at::Tensor& mean,
    const at::Tensor& rstd, const std::optional<at::Tensor>& weight, const std::optional<at::Tensor>& bias,
    std::array<bool, 3> need) {
  const c10::IntArrayRef normalized = C10_AS_INTARRAYREF_SLOW(normalized_sym);
  const std::optional<LnShape> sh = ln_shape(input, normalized);
  at::Tensor w, unused_b;
  auto stat_ok = [&](const at::Tensor& s) { return on_vk(s) && s.scalar_type() == at::kFloat && s.numel() == sh->rows; };
  const bool ok = sh && on_vk(grad_out) && grad_out.scalar_type() == input.scalar_type() &&
                  grad_out.sizes().equals(input.sizes()) && stat_ok(mean) && stat_ok(rstd) &&
                  affine_param(weight, input, sh->D, &w) && affine_param(bias, input, sh->D, &unused_b);
  if (!ok)
    return VKT_CPU_SYMINT(native_layer_norm_backward, grad_out, input, normalized_sym, mean, rstd, weight, bias, need);
  const at::Tensor x = dense(input), g = dense(grad_out), mu = dense(mean), rs = dense(rstd);
  const bool want_dw = need[1] && present(weight), want_db = need[2] && present(bias);
  at::Tensor dx, dw, db, partial;
  hrt_ln_args A{};
  A.x = dptr(x), A.g = dptr(g), A.mean = dptr(mu), A.rstd = dptr(rs);
  A.w = w.defined() ? dptr(w) : 0;
  A.rows = sh->rows, A.D = sh->D;
  if (need[0]) {
    dx = at::empty_like(x, at::MemoryFormat::Contiguous);
    A.dx = dptr(dx);
  }
  if (want_dw || want_db) {  // per-chunk column sums of g * xhat and g, reduced into dw / db by the same call
    partial = at::empty({hrt_ln_chunks(sh->rows, sh->D), 2, sh->D}, x.options().dtype(at::kFloat));
    A.ws = dptr(partial);
    if (want_dw) dw = at::empty_like(*weight, at::MemoryFormat::Contiguous);
    if (want_db) db = at::empty_like(*bias, at::MemoryFormat::Contiguous);
    A.dw = want_dw ? dptr(dw) : 0;
    A.db = want_db ? dptr(db) : 0;
  }
  if (A.dx != 0 || A.ws != 0) queue(typed("ln_bwd", x.scalar_type()), A);
  note_gpu("aten::native_layer_norm_backward");
  return {dx, dw, db};
}

}  // namespace

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("_softmax", &k_softmax);
  m.impl("_safe_softmax", &k_safe_softmax);
  m.impl("_softmax_backward_data", &k_softmax_backward);
  m.impl("native_layer_norm", &k_layer_norm);
  m.impl("native_layer_norm_backward", &k_layer_norm_backward);
}
