// Helpers shared by the "vk" PrivateUse1 shim (namespace vkt).  The shim is the upper half of the
// boundary: it receives ATen calls through TORCH_LIBRARY_IMPL(aten, PrivateUse1) registrations, checks
// what the kernels support, fills an hrt_ops.h argument block and queues it through the hrt C ABI.
// Reference interface: csrc/common.h:1-66.
#pragma once

#include <ATen/ATen.h>
#include <ATen/native/CPUFallback.h>
#include <torch/library.h>

#include <cstdint>
#include <optional>
#include <string>

#include "hrt.h"
#include "hrt_ops.h"

namespace vkt {

constexpr c10::DeviceType kDev = c10::DeviceType::PrivateUse1;

std::string last_error();
void hrt_check(int rc, const char* what);
void ensure_init();

// Per-op statistics: CPU fallbacks and GPU kernel launches (csrc/shim.cpp:53-66).
void count_fallback(const std::string& name);
void count_kernel(const std::string& name);

// Boxed CPU fallback for every op without a vk kernel (csrc/shim.cpp:70-131).
void vk_fallback(const c10::OperatorHandle& op, torch::jit::Stack* stack);

inline bool is_vk(const at::Tensor& t) { return t.defined() && t.device().type() == kDev; }
inline uint64_t addr_of(const at::Tensor& t) { return reinterpret_cast<uint64_t>(t.data_ptr()); }

// Kernel name -> id (cached); throws if unknown.
int kernel_id(const std::string& name);
// Queue an operator kernel (it sizes its own grid); throws with the runtime's message on failure.
void launch(const std::string& kernel, const void* args, uint32_t len);
template <typename A>
inline void launch(const std::string& kernel, const A& args) {
  launch(kernel, &args, (uint32_t)sizeof(A));
}

// Float kind code (HRT_F32/BF16/F16) and its kernel-name suffix; -1 / nullptr for other dtypes.
int float_code(at::ScalarType t);
const char* kind_name(at::ScalarType t);

// Device strided copy with dtype conversion (float kinds) or same-type raw copy.  false = unsupported.
bool ew_copy(const at::Tensor& dst, const at::Tensor& src);
// Device fill of a (possibly strided) tensor.  false = unsupported dtype.
bool ew_fill(const at::Tensor& dst, const at::Scalar& value);

// Matrix-core switches (csrc/common.h:35-44).
void set_coop_enabled(bool on);
bool coop_is_enabled();
uint32_t coop_caps();
void set_coop_range(uint64_t lo, uint64_t hi, int kind);
void reset_coop_calls();
uint64_t coop_calls();

// Fused attention policy: 0 = off, 1 = on, 2 = auto (csrc/ops_attn.cpp:53-77).
void set_fused_attention(int mode);

// Weight-only int8 (csrc/ops_quant.cpp:34-59) and the fused int8 linear (new op).
at::Tensor dequant_int8_vk(const at::Tensor& q, const at::Tensor& scale, at::ScalarType out_dtype);
at::Tensor dequant_int8_linear_vk(const at::Tensor& x, const at::Tensor& q, const at::Tensor& scale,
                                  const std::optional<at::Tensor>& bias);

#define VKT_FALLBACK(op, ...) at::native::call_fallback_fn<&vkt::vk_fallback, at::_ops::op>::call(__VA_ARGS__)
#define VKT_FALLBACK_SYMINT(op, ...) \
  at::native::call_fallback_fn_symint<&vkt::vk_fallback, at::_ops::op>::call(__VA_ARGS__)

}  // namespace vkt
