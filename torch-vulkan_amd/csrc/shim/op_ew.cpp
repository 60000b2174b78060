// Device strided copy/cast and fill used by the boundary (`.contiguous()`, `.to(dtype)`, `copy_` into
// views, `zeros`).  Reference: ew_copy csrc/ops_ew.cpp:495-506, try_fill :382-392, dim merging
// ew_prepare :76-129.  Dimensions are merged where both sides allow, size-1 dimensions dropped, so most
// copies reach the kernel as 1-3 dimensional index spaces.
#include <ATen/ExpandUtils.h>
#include <ATen/MemoryOverlap.h>
#include <ATen/Operators.h>

#include <cstring>
#include <initializer_list>
#include <optional>
#include <vector>

#include "common.h"

namespace vkt {
namespace {

int raw_code(size_t elem) {
  switch (elem) {
    case 1: return HRT_RAW8;
    case 2: return HRT_RAW16;
    case 4: return HRT_RAW32;
    case 8: return HRT_RAW64;
    default: return -1;
  }
}

// Collapse [sizes] with two stride sets into at most HRT_MAX_DIMS dimensions.  false if it does not fit.
bool merge_dims(c10::IntArrayRef sizes, c10::IntArrayRef s0, c10::IntArrayRef s1, int32_t* ndim, int64_t* osz, int64_t* os0,
                int64_t* os1) {
  std::vector<int64_t> z, a, b;
  for (size_t d = 0; d < sizes.size(); ++d) {
    if (sizes[d] == 1) continue;
    if (s0[d] < 0 || s1[d] < 0) return false;
    if (!z.empty() && a.back() == s0[d] * sizes[d] && b.back() == s1[d] * sizes[d]) {
      z.back() *= sizes[d];
      a.back() = s0[d];
      b.back() = s1[d];
    } else {
      z.push_back(sizes[d]);
      a.push_back(s0[d]);
      b.push_back(s1[d]);
    }
  }
  if ((int)z.size() > HRT_MAX_DIMS) return false;
  *ndim = (int32_t)z.size();
  for (size_t i = 0; i < z.size(); ++i) {
    osz[i] = z[i];
    os0[i] = a[i];
    os1[i] = b[i];
  }
  return true;
}

}  // namespace

bool ew_copy(const at::Tensor& dst, const at::Tensor& src) {
  if (!on_vk(dst) || !on_vk(src) || dst.sizes() != src.sizes()) return false;
  if (dst.numel() == 0) return true;
  hrt_copy_args A{};
  const int dc = float_code(dst.scalar_type()), sc = float_code(src.scalar_type());
  if (dc >= 0 && sc >= 0) {
    A.dst_dtype = dc;
    A.src_dtype = sc;
  } else if (dst.scalar_type() == src.scalar_type() && raw_code(dst.element_size()) >= 0) {
    A.dst_dtype = A.src_dtype = raw_code(dst.element_size());
  } else {
    return false;
  }
  if (!merge_dims(dst.sizes(), dst.strides(), src.strides(), &A.ndim, A.sizes, A.dst_strides, A.src_strides)) return false;
  A.dst = dptr(dst);
  A.src = dptr(src);
  queue("ew_copy", A);
  note_gpu("aten::copy_");
  return true;
}

bool ew_fill(const at::Tensor& dst, const at::Scalar& v) {
  if (!on_vk(dst)) return false;
  if (dst.numel() == 0) return true;
  uint64_t bits = 0;
  switch (dst.scalar_type()) {
    case at::kFloat: {
      float f = v.to<float>();
      std::memcpy(&bits, &f, 4);
      break;
    }
    case at::kDouble: {
      double f = v.to<double>();
      std::memcpy(&bits, &f, 8);
      break;
    }
    case at::kBFloat16: bits = v.to<c10::BFloat16>().x; break;
    case at::kHalf: bits = v.to<c10::Half>().x; break;
    case at::kLong: {
      int64_t i = v.to<int64_t>();
      std::memcpy(&bits, &i, 8);
      break;
    }
    case at::kInt: {
      int32_t i = v.to<int32_t>();
      std::memcpy(&bits, &i, 4);
      break;
    }
    case at::kShort: {
      int16_t i = v.to<int16_t>();
      std::memcpy(&bits, &i, 2);
      break;
    }
    case at::kChar: {
      int8_t i = v.to<int8_t>();
      std::memcpy(&bits, &i, 1);
      break;
    }
    case at::kByte: bits = v.to<uint8_t>(); break;
    case at::kBool: bits = v.to<bool>() ? 1 : 0; break;
    default: return false;
  }
  hrt_fill_args A{};
  A.dtype = raw_code(dst.element_size());
  if (A.dtype < 0) return false;
  int64_t dummy[HRT_MAX_DIMS];
  if (!merge_dims(dst.sizes(), dst.strides(), dst.strides(), &A.ndim, A.sizes, A.strides, dummy)) return false;
  A.dst = dptr(dst);
  A.value_bits = bits;
  queue("ew_fill", A);
  return true;
}

}  // namespace vkt

// ---- elementwise arithmetic (kernel "ew_map") ---------------------------------------------------------
// The registrations of csrc/ops_ew.cpp:510-550 with the same support rules: vk tensors of f32 / bf16 /
// f16 (bool only as the where condition), broadcasting and arbitrary non-negative strides, host-side
// 0-dim tensors and Scalars as scalar operands; anything else takes the CPU fallback.  Two widenings of
// the reference's rules: operands of different float dtypes run on the device with PyTorch's result
// type (an operand whose value PyTorch rounds to a narrower result type is cast on the device first),
// and the in-place forms of the unary ops are registered too.
namespace {

using vkt::dptr;
using vkt::note_gpu;
using vkt::float_code;
using vkt::on_vk;

bool is_float(const at::Tensor& t) { return float_code(t.scalar_type()) >= 0; }

// A CPU 0-dim tensor next to vk tensors acts as a scalar operand (Python numbers arrive this way).
bool host_scalar(const at::Tensor& t) {
  return t.defined() && t.device().is_cpu() && t.dim() == 0 && !at::isComplexType(t.scalar_type());
}

// Element strides of t broadcast to `sizes` (right-aligned, size-1 dims get stride 0).
bool broadcast_strides(const at::Tensor& t, at::IntArrayRef sizes, int64_t* st) {
  const int nd = (int)sizes.size(), td = (int)t.dim();
  if (td > nd) return false;
  for (int i = 0; i < nd; ++i) {
    const int j = i - (nd - td);
    st[i] = 0;
    if (j < 0) continue;
    if (t.size(j) == sizes[i]) {
      if (t.stride(j) < 0) return false;
      st[i] = sizes[i] == 1 ? 0 : t.stride(j);
    } else if (t.size(j) != 1) {
      return false;
    }
  }
  return true;
}

// Queue ew_map: out (written with its own strides) = f(a, b, c) with the inputs broadcast to out's sizes.
// Dimensions of size 1 are dropped and neighbours merged where every operand allows (reference:
// ew_prepare, csrc/ops_ew.cpp:76-129).  false = the kernel cannot take it; nothing has been queued.
bool run_ew(int op, const at::Tensor& out, const at::Tensor* a, const at::Tensor* b, const at::Tensor* c, float s0,
            float s1, const char* aten_name) {
  const at::IntArrayRef sizes = out.sizes();
  const int nd = (int)sizes.size();
  std::vector<int64_t> st[4];
  const at::Tensor* ops[4] = {&out, a, b, c};
  for (int k = 0; k < 4; ++k) {
    st[k].assign(nd, 0);
    if (ops[k] && !broadcast_strides(*ops[k], sizes, st[k].data())) return false;
  }
  hrt_ew_args A{};
  int m = 0;
  for (int d = 0; d < nd; ++d) {
    if (sizes[d] == 1) continue;
    bool merge = m > 0;
    for (int k = 0; k < 4 && merge; ++k) {
      const int64_t* prev = k == 0 ? A.out_strides : k == 1 ? A.a_strides : k == 2 ? A.b_strides : A.c_strides;
      merge = prev[m - 1] == st[k][d] * sizes[d];
    }
    if (!merge && m == HRT_MAX_DIMS) return false;
    const int slot = merge ? m - 1 : m++;
    A.sizes[slot] = merge ? A.sizes[slot] * sizes[d] : sizes[d];
    A.out_strides[slot] = st[0][d];
    A.a_strides[slot] = st[1][d];
    A.b_strides[slot] = st[2][d];
    A.c_strides[slot] = st[3][d];
  }
  A.ndim = m;
  if (out.numel() == 0) return true;
  A.op = op;
  A.out = dptr(out);
  A.out_dtype = float_code(out.scalar_type());
  A.a = a ? dptr(*a) : 0;
  A.a_dtype = a ? float_code(a->scalar_type()) : HRT_F32;
  A.b = b ? dptr(*b) : 0;
  A.b_dtype = b ? float_code(b->scalar_type()) : HRT_F32;
  A.c = c ? dptr(*c) : 0;
  A.c_dtype = c ? (c->scalar_type() == at::kBool ? HRT_RAW8 : float_code(c->scalar_type())) : HRT_F32;
  A.s0 = s0;
  A.s1 = s1;
  vkt::queue("ew_map", A);
  note_gpu(aten_name);
  return true;
}

// The operand as PyTorch's CPU kernels see it: converted to the result type when that rounds it (a
// 0-dim f32 tensor next to a bf16 tensor takes part as a bf16 value); widening is exact and the kernel
// reads the narrower type directly.
at::Tensor as_compute(const at::Tensor& t, at::ScalarType rt) {
  return (t.scalar_type() == rt || rt == at::kFloat) ? t : t.to(rt);
}

void check_inplace(const at::Tensor& self, std::initializer_list<const at::Tensor*> inputs) {
  at::assert_no_internal_overlap(self);
  for (const at::Tensor* t : inputs) at::assert_no_partial_overlap(self, *t);
}

enum class Bin { Add, Sub, Mul, Div };

// Tensor op Scalar (scalar_left: Scalar op Tensor).  s0/s1 are formed in fp32 as PyTorch's CPU kernels
// form alpha * value.
std::optional<at::Tensor> try_scalar(Bin op, const at::Tensor& t, const at::Scalar& v, const at::Scalar& alpha,
                                     bool scalar_left, at::Tensor* self, const char* aten_name) {
  if (!on_vk(t) || !is_float(t) || v.isComplex() || alpha.isComplex()) return std::nullopt;
  const float fv = v.to<float>(), fa = alpha.to<float>();
  int code;
  float s0, s1 = 0.f;
  if (!scalar_left) {
    switch (op) {
      case Bin::Add: code = HRT_EW_ADD_S; s0 = fa * fv; break;
      case Bin::Sub: code = HRT_EW_ADD_S; s0 = -(fa * fv); break;
      case Bin::Mul: code = HRT_EW_MUL_S; s0 = fv; break;
      default: code = HRT_EW_DIV_S; s0 = fv; break;
    }
  } else {
    switch (op) {
      case Bin::Add: code = HRT_EW_AXPB; s0 = fa; s1 = fv; break;   // v + alpha * t
      case Bin::Sub: code = HRT_EW_AXPB; s0 = -fa; s1 = fv; break;  // v - alpha * t
      case Bin::Mul: code = HRT_EW_MUL_S; s0 = fv; break;
      default: code = HRT_EW_RDIV_S; s0 = fv; break;                // v / t
    }
  }
  if (self) {
    if (scalar_left || !self->is_same(t)) return std::nullopt;
    check_inplace(*self, {});
    if (!run_ew(code, *self, &t, nullptr, nullptr, s0, s1, aten_name)) return std::nullopt;
    return *self;
  }
  at::Tensor out = at::empty(t.sizes(), t.options());
  if (!run_ew(code, out, &t, nullptr, nullptr, s0, s1, aten_name)) return std::nullopt;
  return out;
}

// Reference: try_binary, csrc/ops_ew.cpp:146-239.
std::optional<at::Tensor> try_binary(Bin op, const at::Tensor& a, const at::Tensor& b, const at::Scalar& alpha,
                                     at::Tensor* self, const char* aten_name) {
  if (on_vk(a) && on_vk(b)) {
    if (!is_float(a) || !is_float(b) || alpha.isComplex()) return std::nullopt;
    const at::ScalarType rt = at::result_type(a, b);
    if (float_code(rt) < 0) return std::nullopt;
    std::vector<int64_t> sizes;
    try {
      sizes = at::infer_size(a.sizes(), b.sizes());
    } catch (...) {
      return std::nullopt;
    }
    at::Tensor out;
    if (self) {
      if (self->sizes() != at::IntArrayRef(sizes) || !at::canCast(rt, self->scalar_type()) || !is_float(*self))
        return std::nullopt;
      check_inplace(*self, {&a, &b});
      out = *self;
    } else {
      out = at::empty(sizes, a.options().dtype(rt));
    }
    const at::Tensor ca = as_compute(a, rt), cb = as_compute(b, rt);
    const int code = op == Bin::Add ? HRT_EW_ADD : op == Bin::Sub ? HRT_EW_SUB : op == Bin::Mul ? HRT_EW_MUL : HRT_EW_DIV;
    if (!run_ew(code, out, &ca, &cb, nullptr, alpha.to<float>(), 0.f, aten_name)) return std::nullopt;
    return out;
  }
  if (on_vk(a) && host_scalar(b)) {
    if (at::result_type(a, b) != a.scalar_type()) return std::nullopt;
    return try_scalar(op, a, b.item(), alpha, false, self, aten_name);
  }
  if (!self && host_scalar(a) && on_vk(b)) {
    if (at::result_type(a, b) != b.scalar_type()) return std::nullopt;
    return try_scalar(op, b, a.item(), alpha, true, nullptr, aten_name);
  }
  return std::nullopt;
}

#define VKT_EW_BINARY(NAME, OP, ATEN)                                                                  \
  at::Tensor NAME##_Tensor(const at::Tensor& a, const at::Tensor& b, const at::Scalar& alpha) {          \
    if (auto r = try_binary(OP, a, b, alpha, nullptr, ATEN ".Tensor")) return *r;                        \
    return VKT_CPU(NAME##_Tensor, a, b, alpha);                                                     \
  }                                                                                                      \
  at::Tensor& NAME##__Tensor(at::Tensor& self, const at::Tensor& b, const at::Scalar& alpha) {           \
    if (try_binary(OP, self, b, alpha, &self, ATEN "_.Tensor")) return self;                             \
    return VKT_CPU(NAME##__Tensor, self, b, alpha);                                                 \
  }                                                                                                      \
  at::Tensor NAME##_Scalar(const at::Tensor& a, const at::Scalar& b, const at::Scalar& alpha) {          \
    if (auto r = try_scalar(OP, a, b, alpha, false, nullptr, ATEN ".Scalar")) return *r;                 \
    return VKT_CPU(NAME##_Scalar, a, b, alpha);                                                     \
  }                                                                                                      \
  at::Tensor& NAME##__Scalar(at::Tensor& self, const at::Scalar& b, const at::Scalar& alpha) {           \
    if (try_scalar(OP, self, b, alpha, false, &self, ATEN "_.Scalar")) return self;                      \
    return VKT_CPU(NAME##__Scalar, self, b, alpha);                                                 \
  }

#define VKT_EW_BINARY_NOALPHA(NAME, OP, ATEN)                                                          \
  at::Tensor NAME##_Tensor(const at::Tensor& a, const at::Tensor& b) {                                   \
    if (auto r = try_binary(OP, a, b, 1.0, nullptr, ATEN ".Tensor")) return *r;                          \
    return VKT_CPU(NAME##_Tensor, a, b);                                                            \
  }                                                                                                      \
  at::Tensor& NAME##__Tensor(at::Tensor& self, const at::Tensor& b) {                                    \
    if (try_binary(OP, self, b, 1.0, &self, ATEN "_.Tensor")) return self;                               \
    return VKT_CPU(NAME##__Tensor, self, b);                                                        \
  }                                                                                                      \
  at::Tensor NAME##_Scalar(const at::Tensor& a, const at::Scalar& b) {                                   \
    if (auto r = try_scalar(OP, a, b, 1.0, false, nullptr, ATEN ".Scalar")) return *r;                   \
    return VKT_CPU(NAME##_Scalar, a, b);                                                            \
  }                                                                                                      \
  at::Tensor& NAME##__Scalar(at::Tensor& self, const at::Scalar& b) {                                    \
    if (try_scalar(OP, self, b, 1.0, false, &self, ATEN "_.Scalar")) return self;                        \
    return VKT_CPU(NAME##__Scalar, self, b);                                                        \
  }

VKT_EW_BINARY(add, Bin::Add, "aten::add")
VKT_EW_BINARY(sub, Bin::Sub, "aten::sub")
VKT_EW_BINARY_NOALPHA(mul, Bin::Mul, "aten::mul")
VKT_EW_BINARY_NOALPHA(div, Bin::Div, "aten::div")

// ---- unary (reference: try_unary and its users, csrc/ops_ew.cpp:283-334) ------------------------------
std::optional<at::Tensor> try_unary(int code, const at::Tensor& a, float s0, at::Tensor* self, const char* aten_name) {
  if (!on_vk(a) || !is_float(a)) return std::nullopt;
  if (self) {
    check_inplace(*self, {});
    if (!run_ew(code, *self, self, nullptr, nullptr, s0, 0.f, aten_name)) return std::nullopt;
    return *self;
  }
  at::Tensor out = at::empty(a.sizes(), a.options());
  if (!run_ew(code, out, &a, nullptr, nullptr, s0, 0.f, aten_name)) return std::nullopt;
  return out;
}

#define VKT_EW_UNARY(NAME, CODE)                                                                       \
  at::Tensor k_##NAME(const at::Tensor& a) {                                                             \
    if (auto r = try_unary(CODE, a, 0.f, nullptr, "aten::" #NAME)) return *r;                            \
    return VKT_CPU(NAME, a);                                                                        \
  }                                                                                                      \
  at::Tensor& k_##NAME##_(at::Tensor& self) {                                                            \
    if (try_unary(CODE, self, 0.f, &self, "aten::" #NAME "_")) return self;                              \
    return VKT_CPU(NAME##_, self);                                                                  \
  }

VKT_EW_UNARY(neg, HRT_EW_NEG)
VKT_EW_UNARY(rsqrt, HRT_EW_RSQRT)
VKT_EW_UNARY(reciprocal, HRT_EW_RECIP)
VKT_EW_UNARY(exp, HRT_EW_EXP)
VKT_EW_UNARY(sin, HRT_EW_SIN)
VKT_EW_UNARY(cos, HRT_EW_COS)
VKT_EW_UNARY(sqrt, HRT_EW_SQRT)
VKT_EW_UNARY(tanh, HRT_EW_TANH)
VKT_EW_UNARY(sigmoid, HRT_EW_SIGMOID)
VKT_EW_UNARY(relu, HRT_EW_RELU)
VKT_EW_UNARY(silu, HRT_EW_SILU)

bool real_scalar(const at::Scalar& s) { return s.isFloatingPoint() || s.isIntegral(false); }

at::Tensor k_pow_Tensor_Scalar(const at::Tensor& a, const at::Scalar& e) {
  if (real_scalar(e))
    if (auto r = try_unary(HRT_EW_POW_S, a, e.to<float>(), nullptr, "aten::pow.Tensor_Scalar")) return *r;
  return VKT_CPU(pow_Tensor_Scalar, a, e);
}
at::Tensor& k_pow__Scalar(at::Tensor& self, const at::Scalar& e) {
  if (real_scalar(e) && try_unary(HRT_EW_POW_S, self, e.to<float>(), &self, "aten::pow_.Scalar")) return self;
  return VKT_CPU(pow__Scalar, self, e);
}

int gelu_code(c10::string_view approximate, bool backward) {
  if (approximate == "none") return backward ? HRT_EW_GELU_ERF_BWD : HRT_EW_GELU_ERF;
  if (approximate == "tanh") return backward ? HRT_EW_GELU_TANH_BWD : HRT_EW_GELU_TANH;
  return -1;
}

at::Tensor k_gelu(const at::Tensor& a, c10::string_view approximate) {
  const int code = gelu_code(approximate, false);
  if (code >= 0)
    if (auto r = try_unary(code, a, 0.f, nullptr, "aten::gelu")) return *r;
  return VKT_CPU(gelu, a, approximate);
}
at::Tensor& k_gelu_(at::Tensor& self, c10::string_view approximate) {
  const int code = gelu_code(approximate, false);
  if (code >= 0 && try_unary(code, self, 0.f, &self, "aten::gelu_")) return self;
  return VKT_CPU(gelu_, self, approximate);
}

// ---- activation backward (grad, input) (reference: csrc/ops_ew.cpp:336-372) ---------------------------
std::optional<at::Tensor> try_backward(int code, const at::Tensor& g, const at::Tensor& x, const char* aten_name) {
  if (!on_vk(g) || !on_vk(x) || !is_float(g) || g.scalar_type() != x.scalar_type()) return std::nullopt;
  std::vector<int64_t> sizes;
  try {
    sizes = at::infer_size(g.sizes(), x.sizes());
  } catch (...) {
    return std::nullopt;
  }
  at::Tensor out = at::empty(sizes, g.options());
  if (!run_ew(code, out, &g, &x, nullptr, 0.f, 0.f, aten_name)) return std::nullopt;
  return out;
}

at::Tensor k_silu_backward(const at::Tensor& g, const at::Tensor& x) {
  if (auto r = try_backward(HRT_EW_SILU_BWD, g, x, "aten::silu_backward")) return *r;
  return VKT_CPU(silu_backward, g, x);
}
at::Tensor k_gelu_backward(const at::Tensor& g, const at::Tensor& x, c10::string_view approximate) {
  const int code = gelu_code(approximate, true);
  if (code >= 0)
    if (auto r = try_backward(code, g, x, "aten::gelu_backward")) return *r;
  return VKT_CPU(gelu_backward, g, x, approximate);
}

// ---- where (reference: csrc/ops_ew.cpp:374-392) --------------------------------------------------------
at::Tensor k_where_self(const at::Tensor& cond, const at::Tensor& a, const at::Tensor& b) {
  if (on_vk(cond) && on_vk(a) && on_vk(b) && cond.scalar_type() == at::kBool && is_float(a) && is_float(b)) {
    const at::ScalarType rt = at::result_type(a, b);
    std::vector<int64_t> sizes;
    bool ok = float_code(rt) >= 0;
    try {
      if (ok) sizes = at::infer_size(at::infer_size(a.sizes(), b.sizes()), cond.sizes());
    } catch (...) {
      ok = false;
    }
    if (ok) {
      at::Tensor out = at::empty(sizes, a.options().dtype(rt));
      const at::Tensor ca = as_compute(a, rt), cb = as_compute(b, rt);
      if (run_ew(HRT_EW_WHERE, out, &ca, &cb, &cond, 0.f, 0.f, "aten::where.self")) return out;
    }
  }
  return VKT_CPU(where_self, cond, a, b);
}

// ---- optimizer forms: addcmul(_), addcdiv(_), lerp(_).Scalar (reference: csrc/ops_ew.cpp:394-455) -------
std::optional<at::Tensor> try_ternary(int code, const at::Tensor& a, const at::Tensor& b, const at::Tensor* c,
                                      const at::Scalar& s, at::Tensor* self, const char* aten_name) {
  if (!on_vk(a) || !on_vk(b) || (c && !on_vk(*c)) || !is_float(a) || s.isComplex()) return std::nullopt;
  if (b.scalar_type() != a.scalar_type() || (c && c->scalar_type() != a.scalar_type())) return std::nullopt;
  std::vector<int64_t> sizes;
  try {
    sizes = at::infer_size(a.sizes(), b.sizes());
    if (c) sizes = at::infer_size(sizes, c->sizes());
  } catch (...) {
    return std::nullopt;
  }
  at::Tensor out;
  if (self) {
    if (self->sizes() != at::IntArrayRef(sizes)) return std::nullopt;
    if (c) check_inplace(*self, {&b, c});
    else check_inplace(*self, {&b});
    out = *self;
  } else {
    out = at::empty(sizes, a.options());
  }
  if (!run_ew(code, out, &a, &b, c, s.to<float>(), 0.f, aten_name)) return std::nullopt;
  return out;
}

at::Tensor k_addcmul(const at::Tensor& self, const at::Tensor& t1, const at::Tensor& t2, const at::Scalar& value) {
  if (auto r = try_ternary(HRT_EW_ADDCMUL, self, t1, &t2, value, nullptr, "aten::addcmul")) return *r;
  return VKT_CPU(addcmul, self, t1, t2, value);
}
at::Tensor& k_addcmul_(at::Tensor& self, const at::Tensor& t1, const at::Tensor& t2, const at::Scalar& value) {
  if (try_ternary(HRT_EW_ADDCMUL, self, t1, &t2, value, &self, "aten::addcmul_")) return self;
  return VKT_CPU(addcmul_, self, t1, t2, value);
}
at::Tensor k_addcdiv(const at::Tensor& self, const at::Tensor& t1, const at::Tensor& t2, const at::Scalar& value) {
  if (auto r = try_ternary(HRT_EW_ADDCDIV, self, t1, &t2, value, nullptr, "aten::addcdiv")) return *r;
  return VKT_CPU(addcdiv, self, t1, t2, value);
}
at::Tensor& k_addcdiv_(at::Tensor& self, const at::Tensor& t1, const at::Tensor& t2, const at::Scalar& value) {
  if (try_ternary(HRT_EW_ADDCDIV, self, t1, &t2, value, &self, "aten::addcdiv_")) return self;
  return VKT_CPU(addcdiv_, self, t1, t2, value);
}
at::Tensor k_lerp_Scalar(const at::Tensor& self, const at::Tensor& end, const at::Scalar& weight) {
  if (auto r = try_ternary(HRT_EW_LERP_S, self, end, nullptr, weight, nullptr, "aten::lerp.Scalar")) return *r;
  return VKT_CPU(lerp_Scalar, self, end, weight);
}
at::Tensor& k_lerp__Scalar(at::Tensor& self, const at::Tensor& end, const at::Scalar& weight) {
  if (try_ternary(HRT_EW_LERP_S, self, end, nullptr, weight, &self, "aten::lerp_.Scalar")) return self;
  return VKT_CPU(lerp__Scalar, self, end, weight);
}

}  // namespace

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("add.Tensor", &add_Tensor);
  m.impl("add_.Tensor", &add__Tensor);
  m.impl("add.Scalar", &add_Scalar);
  m.impl("add_.Scalar", &add__Scalar);
  m.impl("sub.Tensor", &sub_Tensor);
  m.impl("sub_.Tensor", &sub__Tensor);
  m.impl("sub.Scalar", &sub_Scalar);
  m.impl("sub_.Scalar", &sub__Scalar);
  m.impl("mul.Tensor", &mul_Tensor);
  m.impl("mul_.Tensor", &mul__Tensor);
  m.impl("mul.Scalar", &mul_Scalar);
  m.impl("mul_.Scalar", &mul__Scalar);
  m.impl("div.Tensor", &div_Tensor);
  m.impl("div_.Tensor", &div__Tensor);
  m.impl("div.Scalar", &div_Scalar);
  m.impl("div_.Scalar", &div__Scalar);
  m.impl("neg", &k_neg);
  m.impl("neg_", &k_neg_);
  m.impl("rsqrt", &k_rsqrt);
  m.impl("rsqrt_", &k_rsqrt_);
  m.impl("reciprocal", &k_reciprocal);
  m.impl("reciprocal_", &k_reciprocal_);
  m.impl("exp", &k_exp);
  m.impl("exp_", &k_exp_);
  m.impl("sin", &k_sin);
  m.impl("sin_", &k_sin_);
  m.impl("cos", &k_cos);
  m.impl("cos_", &k_cos_);
  m.impl("sqrt", &k_sqrt);
  m.impl("sqrt_", &k_sqrt_);
  m.impl("tanh", &k_tanh);
  m.impl("tanh_", &k_tanh_);
  m.impl("sigmoid", &k_sigmoid);
  m.impl("sigmoid_", &k_sigmoid_);
  m.impl("relu", &k_relu);
  m.impl("relu_", &k_relu_);
  m.impl("silu", &k_silu);
  m.impl("silu_", &k_silu_);
  m.impl("pow.Tensor_Scalar", &k_pow_Tensor_Scalar);
  m.impl("pow_.Scalar", &k_pow__Scalar);
  m.impl("gelu", &k_gelu);
  m.impl("gelu_", &k_gelu_);
  m.impl("silu_backward", &k_silu_backward);
  m.impl("gelu_backward", &k_gelu_backward);
  m.impl("where.self", &k_where_self);
  m.impl("addcmul", &k_addcmul);
  m.impl("addcmul_", &k_addcmul_);
  m.impl("addcdiv", &k_addcdiv);
  m.impl("addcdiv_", &k_addcdiv_);
  m.impl("lerp.Scalar", &k_lerp_Scalar);
  m.impl("lerp_.Scalar", &k_lerp__Scalar);
}
