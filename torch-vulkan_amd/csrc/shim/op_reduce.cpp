// Reductions and concatenation on the vk device: sum / mean (aten::sum, sum.dim_IntList, mean, mean.dim)
// and cat.  The reference registers the same operators (csrc/ops_rows.cpp:342-346); its reduction runs
// one workgroup per output over at most 4 kept and 2 reduced dimensions, its cat one copy per part.
#include <ATen/WrapDimUtilsMulti.h>
#include <ATen/native/TypeProperties.h>

#include <bitset>

#include "common.h"

namespace {

using namespace vkt;

// ---- sum / mean (reference: try_reduce and its users, csrc/ops_rows.cpp:183-270) -------------------------
// Any subset of up to 8 dimensions of a strided f32/bf16/f16 view, optional output dtype (a float kind);
// fp32 accumulation, one rounding.  The kernel picks its layout and, for few outputs, splits the reduced
// range into fp32 partial sums in a workspace this adapter allocates.
std::optional<at::Tensor> try_reduce(const at::Tensor& self, at::OptionalIntArrayRef dim_opt, bool keepdim,
                                     std::optional<at::ScalarType> dtype, bool mean, const char* aten_name) {
  if (!on_vk(self) || float_code(self.scalar_type()) < 0) return std::nullopt;
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
  A.x = dptr(self);
  A.out = dptr(out);
  A.x_dtype = float_code(self.scalar_type());
  A.out_dtype = float_code(odt);
  A.div = mean ? (float)n_red : 1.0f;
  const int64_t ws_floats = hrt_reduce_workspace(&A);
  TORCH_CHECK(ws_floats >= 0, "vk: reduce_sum rejected its arguments");
  at::Tensor ws;
  if (ws_floats > 0) {
    ws = at::empty({ws_floats}, self.options().dtype(at::kFloat));
    A.ws = dptr(ws);
  }
  if (out.numel() > 0) queue("reduce_sum", A);
  note_gpu(aten_name);
  return out;
}

at::Tensor k_sum_dim(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim, std::optional<at::ScalarType> dtype) {
  if (auto r = try_reduce(self, dim, keepdim, dtype, false, "aten::sum.dim_IntList")) return *r;
  return VKT_CPU(sum_dim_IntList, self, dim, keepdim, dtype);
}
at::Tensor k_mean_dim(const at::Tensor& self, at::OptionalIntArrayRef dim, bool keepdim, std::optional<at::ScalarType> dtype) {
  if (auto r = try_reduce(self, dim, keepdim, dtype, true, "aten::mean.dim")) return *r;
  return VKT_CPU(mean_dim, self, dim, keepdim, dtype);
}
at::Tensor k_sum(const at::Tensor& self, std::optional<at::ScalarType> dtype) {
  if (auto r = try_reduce(self, std::nullopt, false, dtype, false, "aten::sum")) return *r;
  return VKT_CPU(sum, self, dtype);
}
at::Tensor k_mean(const at::Tensor& self, std::optional<at::ScalarType> dtype) {
  if (auto r = try_reduce(self, std::nullopt, false, dtype, true, "aten::mean")) return *r;
  return VKT_CPU(mean, self, dtype);
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
    queue("cat_rows16", A);
  }
  return true;
}

at::Tensor k_cat(const at::ITensorListRef& tensors, int64_t dim) {
  std::vector<at::Tensor> parts;
  bool ok = true, all_float = true, same = true;
  at::ScalarType dt = at::kFloat;
  bool first = true;
  for (const at::Tensor& t : tensors) {
    ok = ok && on_vk(t);
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
        note_gpu("aten::cat");
        return out;
      }
    }
  }
  return VKT_CPU(cat, tensors, dim);
}

}  // namespace

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("sum.dim_IntList", &k_sum_dim);
  m.impl("mean.dim", &k_mean_dim);
  m.impl("sum", &k_sum);
  m.impl("mean", &k_mean);
  m.impl("cat", &k_cat);
}
