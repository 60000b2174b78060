// Weight-only int8: dequant (reference csrc/ops_quant.cpp:34-59, pybind csrc/shim.cpp:420-423) and the
// fused int8 linear y = x @ deq(q, scale)^T + bias (new op, no reference counterpart).
#include "common.h"

namespace vkt {

at::Tensor dequant_int8_vk(const at::Tensor& q, const at::Tensor& scale, at::ScalarType out_dtype) {
  TORCH_CHECK(is_vk(q) && is_vk(scale), "dequant_int8: q and scale must be vk tensors");
  TORCH_CHECK(q.scalar_type() == at::kChar && q.dim() == 2 && q.is_contiguous(), "dequant_int8: q must be a contiguous 2-D int8 tensor");
  TORCH_CHECK(scale.scalar_type() == at::kBFloat16 && scale.dim() == 2 && scale.is_contiguous(),
              "dequant_int8: scale must be a contiguous 2-D bfloat16 tensor");
  const char* k = kind_name(out_dtype);
  TORCH_CHECK(k != nullptr, "dequant_int8: out_dtype must be float32, bfloat16 or float16");
  const int64_t rows = q.size(0), cols = q.size(1), nblocks = (cols + 63) / 64;
  TORCH_CHECK(scale.size(0) == rows && scale.size(1) == nblocks, "dequant_int8: scale must have shape [rows, ceil(cols/64)] = [",
              rows, ", ", nblocks, "], got ", scale.sizes());
  at::Tensor out = at::empty({rows, cols}, q.options().dtype(out_dtype));
  if (rows * cols == 0) return out;
  hrt_dq8_args A{addr_of(q), addr_of(scale), addr_of(out), rows, cols, nblocks};
  launch(std::string("dq8_") + k, A);
  count_kernel("torch_vulkan::dequant_int8");
  return out;
}

at::Tensor dequant_int8_linear_vk(const at::Tensor& x, const at::Tensor& q, const at::Tensor& scale,
                                  const std::optional<at::Tensor>& bias) {
  TORCH_CHECK(is_vk(x) && is_vk(q) && is_vk(scale), "dequant_int8_linear: x, q and scale must be vk tensors");
  TORCH_CHECK(x.scalar_type() == at::kBFloat16 || x.scalar_type() == at::kHalf, "dequant_int8_linear: x must be bfloat16 or float16");
  TORCH_CHECK(q.scalar_type() == at::kChar && q.dim() == 2 && q.is_contiguous(), "dequant_int8_linear: q must be a contiguous 2-D int8 tensor");
  TORCH_CHECK(scale.scalar_type() == at::kBFloat16 && scale.dim() == 2 && scale.is_contiguous(),
              "dequant_int8_linear: scale must be a contiguous 2-D bfloat16 tensor");
  const int64_t N = q.size(0), K = q.size(1), nblocks = (K + 63) / 64;
  TORCH_CHECK(scale.size(0) == N && scale.size(1) == nblocks, "dequant_int8_linear: scale must have shape [N, ceil(K/64)]");
  TORCH_CHECK(x.dim() >= 1 && x.size(-1) == K, "dequant_int8_linear: x's last dimension must equal q.size(1)");
  at::Tensor x2 = x.reshape({-1, K});
  const int64_t M = x2.size(0);
  std::vector<int64_t> out_shape(x.sizes().begin(), x.sizes().end());
  out_shape.back() = N;
  at::Tensor y = at::empty({M, N}, x.options());
  if (M * N == 0) return y.view(out_shape);
  hrt_mm_dq8_args A{};
  A.x = addr_of(x2);
  A.q = addr_of(q);
  A.scale = addr_of(scale);
  A.y = addr_of(y);
  A.M = M;
  A.N = N;
  A.K = K;
  A.nblocks = nblocks;
  A.x_sm = x2.stride(0);
  A.x_sk = x2.stride(1);
  A.alpha = 1.f;
  A.beta = 1.f;
  at::Tensor ws;  // large M: the weights are dequantized once into this workspace (same values)
  if (M >= 2048) {
    ws = at::empty({N, K}, x.options());
    A.ws = addr_of(ws);
  }
  if (bias.has_value() && bias->defined()) {
    TORCH_CHECK(is_vk(*bias) && bias->scalar_type() == x.scalar_type() && bias->numel() == N && bias->is_contiguous(),
                "dequant_int8_linear: bias must be a contiguous vk tensor of N elements in x's dtype");
    A.bias = addr_of(*bias);
    A.has_bias = 1;
  }
  launch(std::string("mm_dq8_") + kind_name(x.scalar_type()), A);
  count_kernel("torch_vulkan::dequant_int8_linear");
  return y.view(out_shape);
}

}  // namespace vkt
