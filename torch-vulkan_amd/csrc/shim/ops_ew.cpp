// Device strided copy/cast and fill used by the boundary (`.contiguous()`, `.to(dtype)`, `copy_` into
// views, `zeros`).  Reference: ew_copy csrc/ops_ew.cpp:495-506, try_fill :382-392, dim merging
// ew_prepare :76-129.  Dimensions are merged where both sides allow, size-1 dimensions dropped, so most
// copies reach the kernel as 1-3 dimensional index spaces.
#include <cstring>
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
  if (!is_vk(dst) || !is_vk(src) || dst.sizes() != src.sizes()) return false;
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
  A.dst = addr_of(dst);
  A.src = addr_of(src);
  launch("ew_copy", A);
  count_kernel("aten::copy_");
  return true;
}

bool ew_fill(const at::Tensor& dst, const at::Scalar& v) {
  if (!is_vk(dst)) return false;
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
  A.dst = addr_of(dst);
  A.value_bits = bits;
  launch("ew_fill", A);
  return true;
}

}  // namespace vkt
