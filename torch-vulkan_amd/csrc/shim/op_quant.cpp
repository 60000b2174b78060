// Weight-only int8 on the vk device: torch_vulkan.dequant_int8 (the reference's pybind op,
// csrc/shim.cpp:420-423 over csrc/ops_quant.cpp:34-59) and the fused int8 linear (no reference
// counterpart).  Weights are int8 [rows, cols] with one bf16 scale per 64-column block of a row
// ([rows, ceil(cols / 64)]); the dequantized value is float(q) * float(scale) rounded once to the output
// dtype, so every correct implementation agrees bit for bit.
#include "common.h"

namespace {

using namespace vkt;

int64_t scale_blocks(int64_t cols) { return (cols + 63) / 64; }

// Checks shared by both ops; `who` names the op in the messages.
void check_weights(const at::Tensor& q, const at::Tensor& scale, const char* who) {
  TORCH_CHECK(on_vk(q) && on_vk(scale), who, ": q and scale must be on the vk device");
  TORCH_CHECK(q.scalar_type() == at::kChar && q.dim() == 2 && q.is_contiguous(), who,
              ": q must be a contiguous int8 matrix, got ", q.scalar_type(), q.sizes());
  const std::array<int64_t, 2> want = {q.size(0), scale_blocks(q.size(1))};
  TORCH_CHECK(scale.scalar_type() == at::kBFloat16 && scale.is_contiguous() && scale.dim() == 2 &&
                  scale.size(0) == want[0] && scale.size(1) == want[1],
              who, ": scale must be a contiguous bfloat16 [", want[0], ", ", want[1], "] (one scale per 64 columns), got ",
              scale.scalar_type(), scale.sizes());
}

}  // namespace

namespace vkt {

at::Tensor dequant_int8_vk(const at::Tensor& q, const at::Tensor& scale, at::ScalarType out_dtype) {
  check_weights(q, scale, "dequant_int8");
  TORCH_CHECK(float_code(out_dtype) >= 0, "dequant_int8: out_dtype must be float32, bfloat16 or float16, got ", out_dtype);
  at::Tensor out = at::empty(q.sizes(), q.options().dtype(out_dtype));
  if (out.numel() == 0) return out;
  const hrt_dq8_args A{dptr(q), dptr(scale), dptr(out), q.size(0), q.size(1), scale.size(1)};
  queue(typed("dq8", out_dtype), A);
  note_gpu("torch_vulkan::dequant_int8");
  return out;
}

// y = x @ deq(q)^T (+ bias) for x [..., K] bf16/f16, q [N, K]: y [..., N] in x's dtype.  For M >= 2048 rows the
// weights are dequantized once into a workspace and the product runs on them (the fused kernel would
// convert each weight once per 256 rows of x); the values are the same either way.
at::Tensor dequant_int8_linear_vk(const at::Tensor& x, const at::Tensor& q, const at::Tensor& scale,
                                  const std::optional<at::Tensor>& bias) {
  check_weights(q, scale, "dequant_int8_linear");
  TORCH_CHECK(on_vk(x) && (x.scalar_type() == at::kBFloat16 || x.scalar_type() == at::kHalf),
              "dequant_int8_linear: x must be a bfloat16 or float16 vk tensor");
  const int64_t N = q.size(0), K = q.size(1);
  TORCH_CHECK(x.dim() >= 1 && x.size(-1) == K, "dequant_int8_linear: x's last dimension must be ", K, ", got ", x.sizes());
  const at::Tensor rows = x.reshape({-1, K});
  const int64_t M = rows.size(0);
  std::vector<int64_t> out_sizes = x.sizes().vec();
  out_sizes.back() = N;
  at::Tensor y = at::empty({M, N}, x.options());
  if (M == 0 || N == 0) return y.view(out_sizes);
  hrt_mm_dq8_args A{};
  A.x = dptr(rows), A.q = dptr(q), A.scale = dptr(scale), A.y = dptr(y);
  A.M = M, A.N = N, A.K = K, A.nblocks = scale.size(1);
  A.x_sm = rows.stride(0), A.x_sk = rows.stride(1);
  A.alpha = 1.f, A.beta = 1.f;
  if (present(bias)) {
    TORCH_CHECK(on_vk(*bias) && bias->scalar_type() == x.scalar_type() && bias->numel() == N && bias->is_contiguous(),
                "dequant_int8_linear: bias must be a contiguous vk tensor of ", N, " elements in x's dtype");
    A.bias = dptr(*bias), A.has_bias = 1;
  }
  at::Tensor deq;
  if (M >= 2048) {
    deq = at::empty({N, K}, x.options());
    A.ws = dptr(deq);
  }
  queue(typed("mm_dq8", x.scalar_type()), A);
  note_gpu("torch_vulkan::dequant_int8_linear");
  return y.view(out_sizes);
}

}  // namespace vkt
