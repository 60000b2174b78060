// torch.autocast(device_type="vk"): the policy the reference registers (csrc/shim.cpp:376-394), which is
// CUDA's: products and attention run in the autocast dtype, layer_norm / softmax / mse_loss in fp32,
// everything else passes through unchanged.
#include <ATen/autocast_mode.h>
#include <torch/library.h>

TORCH_LIBRARY_IMPL(_, AutocastPrivateUse1, m) { m.fallback(torch::CppFunction::makeFallthrough()); }

TORCH_LIBRARY_IMPL(aten, AutocastPrivateUse1, m) {
  // lower precision
  KERNEL_PRIVATEUSEONE(mm, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(bmm, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(addmm, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(baddbmm, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(matmul, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(linear, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(conv1d, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(conv2d, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(conv3d, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(scaled_dot_product_attention, lower_precision_fp)
  // fp32
  KERNEL_PRIVATEUSEONE(layer_norm, fp32)
  KERNEL_PRIVATEUSEONE(softmax, int, fp32)
  KERNEL_PRIVATEUSEONE(mse_loss, fp32)
}
