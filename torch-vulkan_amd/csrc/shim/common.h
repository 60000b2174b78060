// Shared pieces of the "vk" PrivateUse1 shim, the upper half of the boundary: PyTorch calls the adapters
// declared in ops.h through the dispatcher registrations in register.cpp; an adapter decides whether the
// hrt kernels take the call, fills an include/hrt_ops.h argument block and queues it through the C ABI
// (include/hrt.h).  Interface counterpart in the reference: csrc/common.h:1-66.
#pragma once

#include <ATen/ATen.h>
#include <ATen/native/CPUFallback.h>
#include <torch/library.h>

#include <cstdint>
#include <optional>
#include <string>
#include <string_view>

#include "hrt.h"
#include "hrt_ops.h"

namespace vkt {

constexpr c10::DeviceType kDev = c10::DeviceType::PrivateUse1;

// ---- the runtime ------------------------------------------------------------------------------------------
// runtime() initialises libhrt on first use (device selection, stream, kernel table) and throws with the
// runtime's message when that fails; every entry point that reaches the C ABI calls it first.
void runtime();
std::string runtime_error_text();
// Throws "vk: <what>: <runtime message>" unless rc == 0.
void expect_ok(int rc, const char* what);

// ---- kernels ------------------------------------------------------------------------------------------------
// Queue operator kernel `name` (it sizes its own grid) with an argument block; throws with the runtime's
// message when the kernel rejects its arguments.  Kernel ids are looked up once per name.
void queue(std::string_view name, const void* args, uint32_t len);
template <typename A>
inline void queue(std::string_view name, const A& args) {
  queue(name, &args, static_cast<uint32_t>(sizeof(A)));
}

// Float element kinds the kernels compute in: HRT_F32 / HRT_BF16 / HRT_F16, or -1; and the matching
// kernel-name suffix ("f32" / "bf16" / "f16"), or nullptr.
int float_code(at::ScalarType t);
const char* dtype_suffix(at::ScalarType t);
// "<op>_<suffix>", the registry's naming (e.g. "softmax_fwd_bf16").
std::string typed(std::string_view op, at::ScalarType t);

inline bool on_vk(const at::Tensor& t) { return t.defined() && t.device().type() == kDev; }
inline uint64_t dptr(const at::Tensor& t) { return reinterpret_cast<uint64_t>(t.data_ptr()); }
inline at::Tensor dense(const at::Tensor& t) { return t.is_contiguous() ? t : t.contiguous(); }
inline bool present(const std::optional<at::Tensor>& t) { return t.has_value() && t->defined(); }

// ---- accounting -------------------------------------------------------------------------------------------
// Per-operator counts of GPU launches and CPU fallbacks (with the fallback's host time), which the tests
// read through torch_vulkan.kernel_counts() / fallback_counts() (names as the reference's counters,
// csrc/shim.cpp:53-66).
void note_gpu(std::string_view op);
void note_cpu(std::string_view op, uint64_t ns);

// ---- the CPU fallback --------------------------------------------------------------------------------
// Boxed fallback for every operator without a vk kernel (csrc/shim.cpp:70-131): runs PyTorch's CPU
// kernel on host copies and returns vk results whenever an input was on vk.
void cpu_fallback_boxed(const c10::OperatorHandle& op, torch::jit::Stack* stack);

#define VKT_CPU(op, ...) at::native::call_fallback_fn<&vkt::cpu_fallback_boxed, at::_ops::op>::call(__VA_ARGS__)
#define VKT_CPU_SYMINT(op, ...) \
  at::native::call_fallback_fn_symint<&vkt::cpu_fallback_boxed, at::_ops::op>::call(__VA_ARGS__)

// ---- device copies used by several adapters -------------------------------------------------------
// Strided copy with float-kind conversion, or same-type raw copy; false = dtype pair not handled.
bool ew_copy(const at::Tensor& dst, const at::Tensor& src);
// Fill of a (possibly strided) tensor; false = dtype not handled.
bool ew_fill(const at::Tensor& dst, const at::Scalar& value);

// ---- switches --------------------------------------------------------------------------------------------
// Matrix-core gate of the GEMM adapter: on/off (VKT_NO_COOP), and the debug bisection window
// (set_coop_range: only matrix-core-eligible calls numbered [lo, hi) of the chosen kind use MFMA).
void set_coop_enabled(bool on);
bool coop_is_enabled();
uint32_t coop_caps();
void set_coop_range(uint64_t lo, uint64_t hi, int kind);
void reset_coop_calls();
uint64_t coop_calls();
// Fused attention policy: 0 off, 1 on, 2 auto (VKT_FUSED_ATTN / VKT_NO_FUSED_ATTN).
void set_fused_attention(int mode);

// Weight-only int8 (pybind `dequant_int8`) and the fused int8 linear (no reference counterpart).
at::Tensor dequant_int8_vk(const at::Tensor& q, const at::Tensor& scale, at::ScalarType out_dtype);
at::Tensor dequant_int8_linear_vk(const at::Tensor& x, const at::Tensor& q, const at::Tensor& scale,
                                  const std::optional<at::Tensor>& bias);

}  // namespace vkt
