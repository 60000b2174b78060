// The "vk" PrivateUse1 device: allocator, device guard, hooks, host<->device copies, tensor factories,
// views, the boxed CPU fallback with its counters, the autocast policy and the Python bindings.
//
// Reference interface: csrc/shim.cpp:1-493.  The device memory behind `data_ptr()` is an hrt block
// (a plain HIP device pointer carved from a hipMalloc slab); every kernel and device copy is queued
// on the runtime's single HIP stream, so the host only waits for downloads and explicit syncs.
#include <ATen/EmptyTensor.h>
#include <ATen/autocast_mode.h>
#include <ATen/detail/PrivateUse1HooksInterface.h>
#include <ATen/native/CPUFallback.h>
#include <ATen/ops/_reshape_alias_native.h>
#include <ATen/ops/as_strided_native.h>
#include <ATen/ops/unfold_native.h>
#include <ATen/ops/view_native.h>
#include <c10/core/Allocator.h>
#include <c10/core/CPUAllocator.h>
#include <c10/core/impl/DeviceGuardImplInterface.h>
#include <c10/util/Exception.h>
#include <torch/extension.h>
#include <torch/library.h>

#include <atomic>
#include <chrono>
#include <cstring>
#include <cstdlib>
#include <iostream>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>

#include "common.h"

namespace vkt {

// ---- runtime calls ---------------------------------------------------------------------------------
std::string last_error() {
  char buf[2048];
  hrt_last_error(buf, sizeof(buf));
  return buf;
}

void hrt_check(int rc, const char* what) { TORCH_CHECK(rc == 0, "hrt ", what, " failed: ", last_error()); }

void ensure_init() {
  static std::once_flag once;
  std::call_once(once, [] { hrt_check(hrt_init(), "init"); });
}

// ---- statistics ------------------------------------------------------------------------------------
std::mutex g_stats_mu;
std::map<std::string, int64_t> g_fallback_counts, g_kernel_counts;
std::map<std::string, uint64_t> g_fallback_ns_by_op;
std::atomic<uint64_t> g_fallback_ns{0};

void count_fallback(const std::string& name) {
  std::lock_guard<std::mutex> l(g_stats_mu);
  g_fallback_counts[name]++;
}

void count_kernel(const std::string& name) {
  std::lock_guard<std::mutex> l(g_stats_mu);
  g_kernel_counts[name]++;
}

// ---- boxed CPU fallback ----------------------------------------------------------------------------
void vk_fallback(const c10::OperatorHandle& op, torch::jit::Stack* stack) {
  const auto t0 = std::chrono::steady_clock::now();
  const std::string name = op.schema().operator_name().name;
  const size_t nargs = op.schema().arguments().size();
  static const bool trace = std::getenv("VKT_TRACE_FALLBACK") != nullptr;
  bool first_seen = false, first_is_cpu = false, any_vk = false, any_cpu_dense = false;
  std::string desc;
  for (const auto& a : torch::jit::last(*stack, nargs)) {
    if (a.isTensor() && a.toTensor().defined()) {
      const at::Tensor& t = a.toTensor();
      if (!first_seen) {
        first_seen = true;
        first_is_cpu = !is_vk(t);
      }
      any_vk = any_vk || is_vk(t);
      any_cpu_dense = any_cpu_dense || (!is_vk(t) && t.dim() > 0);
      if (trace) desc += std::string(is_vk(t) ? " vk" : " cpu") + c10::str(t.sizes()) + c10::str(t.scalar_type());
    } else if (a.isTensorList()) {
      for (const at::Tensor& t : a.toTensorList()) any_vk = any_vk || is_vk(t);
    }
  }
  if (trace) {
    std::cerr << "[vkt fallback] " << op.schema() << "\n[vkt fallback-args]" << desc << std::endl;
    if (any_vk && any_cpu_dense) std::cerr << "[vkt MIXED-DEVICE] " << op.schema().operator_name() << ":" << desc << std::endl;
  }
  count_fallback(name);
  at::native::cpu_fallback(op, stack);
  // cpu_fallback returns results on the device of the first tensor argument; when that is a CPU scalar
  // next to vk tensors (1 - x), move the results to vk so CPU tensors do not leak into the graph.
  if (first_is_cpu && any_vk) {
    const size_t nret = op.schema().returns().size();
    for (size_t i = 0; i < nret; ++i) {
      auto& v = (*stack)[stack->size() - nret + i];
      if (v.isTensor() && v.toTensor().defined() && !is_vk(v.toTensor())) v = v.toTensor().to(c10::Device(kDev, 0));
    }
  }
  const uint64_t ns =
      (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t0).count();
  g_fallback_ns += ns;
  std::lock_guard<std::mutex> l(g_stats_mu);
  g_fallback_ns_by_op[name] += ns;
}

// ---- kernels -----------------------------------------------------------------------------------------
int kernel_id(const std::string& name) {
  static std::mutex mu;
  static std::unordered_map<std::string, int> cache;
  std::lock_guard<std::mutex> l(mu);
  auto it = cache.find(name);
  if (it != cache.end()) return it->second;
  ensure_init();
  int k = hrt_kernel_index(name.c_str());
  TORCH_CHECK(k >= 0, "vk: kernel '", name, "' is not registered in libhrt");
  cache.emplace(name, k);
  return k;
}

void launch(const std::string& kernel, const void* args, uint32_t len) {
  int k = kernel_id(kernel);
  TORCH_CHECK(hrt_dispatch((uint32_t)k, args, len, 0, 0, 0) == 0, "vk: ", kernel, " failed: ", last_error());
}

int float_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return HRT_F32;
    case at::kBFloat16: return HRT_BF16;
    case at::kHalf: return HRT_F16;
    default: return -1;
  }
}

const char* kind_name(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return "f32";
    case at::kBFloat16: return "bf16";
    case at::kHalf: return "f16";
    default: return nullptr;
  }
}

}  // namespace vkt

using namespace vkt;

namespace {

// ---- allocator ---------------------------------------------------------------------------------------
struct VkAllocator final : public c10::Allocator {
  static void deleter(void* p) {
    if (p) hrt_free(reinterpret_cast<uint64_t>(p));
  }
  c10::DataPtr allocate(size_t n) override {
    ensure_init();
    if (n == 0) return {nullptr, nullptr, &deleter, c10::Device(kDev, 0)};
    uint64_t a = hrt_alloc(n);
    TORCH_CHECK(a != 0, "vk: out of device memory allocating ", n, " bytes: ", last_error());
    void* p = reinterpret_cast<void*>(a);
    return {p, p, &deleter, c10::Device(kDev, 0)};
  }
  c10::DeleterFnPtr raw_deleter() const override { return &deleter; }
  void copy_data(void* dest, const void* src, std::size_t count) const override {
    hrt_check(hrt_copy_d2d(reinterpret_cast<uint64_t>(dest), reinterpret_cast<uint64_t>(src), count), "copy_data");
  }
};
VkAllocator g_allocator;

// Pinned host memory (tensor.pin_memory(), torch.empty(..., pin_memory=True) with vk as the
// accelerator): page-locked buffers from the runtime, whose frees wait for in-flight transfers.
struct VkPinnedAllocator final : public c10::Allocator {
  static void deleter(void* p) {
    if (p) hrt_host_free(reinterpret_cast<uint64_t>(p));
  }
  c10::DataPtr allocate(size_t n) override {
    ensure_init();
    if (n == 0) return {nullptr, nullptr, &deleter, c10::Device(c10::DeviceType::CPU)};
    uint64_t a = hrt_host_alloc(n);
    TORCH_CHECK(a != 0, "vk: cannot allocate ", n, " bytes of pinned host memory: ", last_error());
    void* p = reinterpret_cast<void*>(a);
    return {p, p, &deleter, c10::Device(c10::DeviceType::CPU)};
  }
  c10::DeleterFnPtr raw_deleter() const override { return &deleter; }
  void copy_data(void* dest, const void* src, std::size_t count) const override { std::memcpy(dest, src, count); }
};
VkPinnedAllocator g_pinned_allocator;

// ---- device guard: one device, one stream ----------------------------------------------------------------
struct VkGuardImpl final : public c10::impl::DeviceGuardImplInterface {
  c10::DeviceType type() const override { return kDev; }
  c10::Device exchangeDevice(c10::Device) const override { return c10::Device(kDev, 0); }
  c10::Device getDevice() const override { return c10::Device(kDev, 0); }
  void setDevice(c10::Device) const override {}
  void uncheckedSetDevice(c10::Device) const noexcept override {}
  c10::Stream getStream(c10::Device d) const override { return c10::Stream(c10::Stream::DEFAULT, d); }
  c10::Stream exchangeStream(c10::Stream s) const override { return s; }
  bool queryStream(const c10::Stream&) const override { return true; }
  void synchronizeStream(const c10::Stream&) const override {
    ensure_init();
    hrt_synchronize();
  }
  void synchronizeDevice(const c10::DeviceIndex) const override {
    ensure_init();
    hrt_synchronize();
  }
  c10::DeviceIndex deviceCount() const noexcept override { return 1; }
};
C10_REGISTER_GUARD_IMPL(PrivateUse1, VkGuardImpl);

// ---- hooks ---------------------------------------------------------------------------------------------------
struct VkHooks final : public at::PrivateUse1HooksInterface {
  void init() const override { ensure_init(); }
  bool isBuilt() const override { return true; }
  bool isAvailable() const override { return true; }
  bool hasPrimaryContext(c10::DeviceIndex) const override { return true; }
  at::Device getDeviceFromPtr(void*) const override { return c10::Device(kDev, 0); }
  bool isPinnedPtr(const void* p) const override { return hrt_host_is_pinned(p) == 1; }  // 0 before init
  // non_blocking copies from / to these buffers are asynchronous (hrt_upload_async / hrt_download_async).
  at::Allocator* getPinnedMemoryAllocator() const override { return &g_pinned_allocator; }
  void resizePrivateUse1Bytes(const c10::Storage& storage, size_t newsize) const override {
    auto* impl = storage.unsafeGetStorageImpl();
    const size_t old = impl->nbytes();
    if (newsize == old) return;
    c10::DataPtr fresh = g_allocator.allocate(newsize);
    const size_t keep = std::min(old, newsize);
    if (keep > 0)
      hrt_check(hrt_copy_d2d(reinterpret_cast<uint64_t>(fresh.get()), reinterpret_cast<uint64_t>(impl->data()), keep),
                "resize copy");
    impl->set_data_ptr_noswap(std::move(fresh));
    impl->set_nbytes(newsize);
  }
};
VkHooks g_hooks;
struct HooksRegistrar {
  HooksRegistrar() { at::RegisterPrivateUse1HooksInterface(&g_hooks); }
};
HooksRegistrar g_hooks_registrar;

// ---- transfers ---------------------------------------------------------------------------------------------------
// host src -> device dst (dtype conversion, broadcast and strided destinations are handled on the host
// side first: the host tensor is made dense in dst's dtype, uploaded, then scattered on the device).
void copy_cpu_to_vk(const at::Tensor& dst, const at::Tensor& src) {
  if (dst.numel() == 0) return;
  at::Tensor s = src.to(dst.scalar_type()).expand(dst.sizes()).contiguous();
  if (dst.is_contiguous()) {
    hrt_check(hrt_upload(addr_of(dst), s.data_ptr(), dst.nbytes()), "upload");
    return;
  }
  at::Tensor staged = at::empty(dst.sizes(), dst.options().memory_format(at::MemoryFormat::Contiguous));
  hrt_check(hrt_upload(addr_of(staged), s.data_ptr(), staged.nbytes()), "upload");
  TORCH_CHECK(ew_copy(dst, staged), "vk: no device copy for dtype ", dst.scalar_type());
}

// device src -> host dst.
void copy_vk_to_cpu(const at::Tensor& dst, const at::Tensor& src) {
  if (src.numel() == 0) return;
  at::Tensor dense = src;
  if (!src.is_contiguous()) {
    dense = at::empty(src.sizes(), src.options().memory_format(at::MemoryFormat::Contiguous));
    TORCH_CHECK(ew_copy(dense, src), "vk: no device copy for dtype ", src.scalar_type());
  }
  at::Tensor host = at::empty(dense.sizes(), dense.options().device(at::kCPU));
  hrt_check(hrt_download(host.data_ptr(), addr_of(dense), host.nbytes()), "download");
  dst.copy_(host);
}

// A non_blocking copy between a dense pinned host tensor and a dense device tensor of the same dtype and
// shape is queued asynchronously: host -> device on the copy stream (later device work on dst waits for
// it, other work overlaps it), device -> host in stream order (valid after a synchronize).  Everything
// else is the synchronous path.
bool async_ok(const at::Tensor& host, const at::Tensor& dev) {
  return host.scalar_type() == dev.scalar_type() && host.sizes() == dev.sizes() && host.is_contiguous() &&
         dev.is_contiguous() && host.numel() > 0 && hrt_host_is_pinned(host.data_ptr()) == 1;
}

void copy_impl(const at::Tensor& dst, const at::Tensor& src, bool non_blocking = false) {
  if (!is_vk(src) && !is_vk(dst)) {
    dst.copy_(src);
  } else if (!is_vk(src)) {
    if (non_blocking && async_ok(src, dst)) {
      hrt_check(hrt_upload_async(addr_of(dst), src.data_ptr(), dst.nbytes()), "upload_async");
      count_kernel("aten::copy_ (async H2D)");
      return;
    }
    copy_cpu_to_vk(dst, src);
  } else if (!is_vk(dst)) {
    if (non_blocking && async_ok(dst, src)) {
      hrt_check(hrt_download_async(dst.data_ptr(), addr_of(src), src.nbytes()), "download_async");
      count_kernel("aten::copy_ (async D2H)");
      return;
    }
    copy_vk_to_cpu(dst, src);
  } else if (src.scalar_type() == dst.scalar_type() && src.sizes() == dst.sizes() && src.is_contiguous() &&
             dst.is_contiguous()) {
    if (src.numel() > 0 && addr_of(src) != addr_of(dst))
      hrt_check(hrt_copy_d2d(addr_of(dst), addr_of(src), dst.nbytes()), "d2d");
  } else if (ew_copy(dst, src.sizes() == dst.sizes() ? src : src.expand(dst.sizes()))) {
    // converted / strided / broadcast copy on the device
  } else {
    // dtype pairs without a device conversion (integer casts): convert on the host
    at::Tensor tmp = at::empty(src.sizes(), src.options().device(at::kCPU));
    copy_vk_to_cpu(tmp, src);
    copy_cpu_to_vk(dst, tmp);
  }
}

at::Tensor copy_from(const at::Tensor& self, const at::Tensor& dst, bool non_blocking) {
  copy_impl(dst, self, non_blocking);
  return dst;
}

at::Tensor copy_from_and_resize(const at::Tensor& self, const at::Tensor& dst) {
  if (dst.sizes() != self.sizes()) dst.resize_(self.sizes());
  copy_impl(dst, self);
  return dst;
}

// ---- factories, views, resize ------------------------------------------------------------------------------------
at::Tensor empty_memory_format(c10::IntArrayRef size, std::optional<at::ScalarType> dtype, std::optional<at::Layout>,
                               std::optional<at::Device>, std::optional<bool>,
                               std::optional<at::MemoryFormat> memory_format) {
  return at::detail::empty_generic(size, &g_allocator, c10::DispatchKeySet(c10::DispatchKey::PrivateUse1),
                                   c10::dtype_or_default(dtype), memory_format);
}

at::Tensor empty_strided(c10::IntArrayRef size, c10::IntArrayRef stride, std::optional<at::ScalarType> dtype,
                         std::optional<at::Layout>, std::optional<at::Device>, std::optional<bool>) {
  return at::detail::empty_strided_generic(size, stride, &g_allocator, c10::DispatchKeySet(c10::DispatchKey::PrivateUse1),
                                           c10::dtype_or_default(dtype));
}

// Views must share storage, so they cannot go through the CPU fallback.
at::Tensor view_impl(const at::Tensor& self, c10::SymIntArrayRef size) {
  return at::native::view(self, C10_AS_INTARRAYREF_SLOW(size));
}

at::Tensor as_strided_impl(const at::Tensor& self, c10::SymIntArrayRef size, c10::SymIntArrayRef stride,
                           std::optional<c10::SymInt> storage_offset) {
  return at::native::as_strided_tensorimpl(
      self, C10_AS_INTARRAYREF_SLOW(size), C10_AS_INTARRAYREF_SLOW(stride),
      storage_offset.has_value() ? std::optional<int64_t>(storage_offset->guard_int(__FILE__, __LINE__)) : std::nullopt);
}

at::Tensor reshape_alias_impl(const at::Tensor& self, c10::SymIntArrayRef size, c10::SymIntArrayRef stride) {
  return at::native::_reshape_alias(self, C10_AS_INTARRAYREF_SLOW(size), C10_AS_INTARRAYREF_SLOW(stride));
}

at::Tensor unfold_impl(const at::Tensor& self, int64_t dimension, int64_t size, int64_t step) {
  return at::native::unfold(self, dimension, size, step);
}

// at::native::resize_ would memcpy device memory on the host; grow through the hooks instead (shrinking
// keeps the storage, as csrc/shim.cpp:335-352).
const at::Tensor& resize_impl(const at::Tensor& self, c10::SymIntArrayRef size_sym,
                              std::optional<at::MemoryFormat> memory_format) {
  auto size = C10_AS_INTARRAYREF_SLOW(size_sym);
  auto* impl = self.unsafeGetTensorImpl();
  int64_t numel = 1;
  for (auto s : size) numel *= s;
  if (numel > 0) {
    const size_t needed = (impl->storage_offset() + numel) * self.element_size();
    if (needed > self.storage().nbytes()) g_hooks.resizePrivateUse1Bytes(self.storage(), needed);
  }
  impl->set_sizes_contiguous(size);
  if (memory_format.has_value() && *memory_format != at::MemoryFormat::Contiguous &&
      *memory_format != at::MemoryFormat::Preserve)
    impl->empty_tensor_restride(*memory_format);
  return self;
}

// fill_ and zero_ on the device (at::zeros, masked padding, optimizer state init).
at::Tensor& fill_scalar_impl(at::Tensor& self, const at::Scalar& value) {
  if (is_vk(self) && ew_fill(self, value)) {
    count_kernel("aten::fill_");
    return self;
  }
  return VKT_FALLBACK(fill__Scalar, self, value);
}

at::Tensor& zero_impl(at::Tensor& self) {
  if (is_vk(self) && ew_fill(self, at::Scalar(0))) {
    count_kernel("aten::zero_");
    return self;
  }
  return VKT_FALLBACK(zero_, self);
}

}  // namespace

TORCH_LIBRARY_IMPL(_, PrivateUse1, m) { m.fallback(torch::CppFunction::makeFromBoxedFunction<&vk_fallback>()); }

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("empty.memory_format", &empty_memory_format);
  m.impl("empty_strided", &empty_strided);
  m.impl("_copy_from", &copy_from);
  m.impl("_copy_from_and_resize", &copy_from_and_resize);
  m.impl("view", &view_impl);
  m.impl("as_strided", &as_strided_impl);
  m.impl("_reshape_alias", &reshape_alias_impl);
  m.impl("unfold", &unfold_impl);
  m.impl("resize_", &resize_impl);
  m.impl("fill_.Scalar", &fill_scalar_impl);
  m.impl("zero_", &zero_impl);
}

// ---- autocast(device_type="vk"): matmuls in lower precision, softmax / norms / losses in fp32 ----------------------
TORCH_LIBRARY_IMPL(_, AutocastPrivateUse1, m) { m.fallback(torch::CppFunction::makeFallthrough()); }

TORCH_LIBRARY_IMPL(aten, AutocastPrivateUse1, m) {
  KERNEL_PRIVATEUSEONE(linear, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(mm, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(bmm, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(addmm, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(baddbmm, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(matmul, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(conv1d, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(conv2d, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(conv3d, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(scaled_dot_product_attention, lower_precision_fp)
  KERNEL_PRIVATEUSEONE(layer_norm, fp32)
  KERNEL_PRIVATEUSEONE(softmax, int, fp32)
  KERNEL_PRIVATEUSEONE(mse_loss, fp32)
}

// ---- Python bindings (csrc/shim.cpp:418-493) ------------------------------------------------------------------------
namespace {
float event_elapsed(uint32_t a, uint32_t b) {
  float ms = hrt_event_elapsed_ms(a, b);
  TORCH_CHECK(ms >= 0.f, "hrt event timing failed: ", last_error());
  return ms;
}
}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("init", [] { ensure_init(); });
  m.def("empty_pinned", [](std::vector<int64_t> sizes, at::ScalarType dtype) {
    ensure_init();
    // torch answers is_pinned() only for accelerators it has initialised itself
    at::globalContext().lazyInitDevice(kDev);
    return at::Tensor(at::detail::empty_generic(sizes, &g_pinned_allocator, c10::DispatchKeySet(c10::DispatchKey::CPU),
                                                dtype, std::nullopt));
  });
  m.def("is_pinned", [](const at::Tensor& t) {
    return t.device().is_cpu() && t.numel() > 0 && hrt_host_is_pinned(t.data_ptr()) == 1;
  });
  m.def("stream_stats", [] {
    ensure_init();
    return std::vector<uint64_t>{hrt_stat(2), hrt_stat(3), hrt_stat(5), hrt_stat(6)};
  });
  m.def("dequant_int8", [](const at::Tensor& q, const at::Tensor& scale, at::ScalarType out_dtype) {
    ensure_init();
    return dequant_int8_vk(q, scale, out_dtype);
  });
  m.def("dequant_int8_linear",
        [](const at::Tensor& x, const at::Tensor& q, const at::Tensor& scale, const std::optional<at::Tensor>& bias) {
          ensure_init();
          return dequant_int8_linear_vk(x, q, scale, bias);
        });
  m.def("device_name", [] {
    ensure_init();
    char buf[256];
    hrt_device_name(buf, sizeof(buf));
    return std::string(buf);
  });
  m.def("max_alloc", [] {
    ensure_init();
    return hrt_max_alloc();
  });
  m.def("live_bytes", [] {
    ensure_init();
    return hrt_live_bytes();
  });
  m.def("memory_info", [] {
    ensure_init();
    uint64_t v[3] = {0, 0, 0};
    hrt_check(hrt_memory_info(v), "memory_info");
    return std::make_tuple(v[0], v[1], v[2]);
  });
  m.def("peak_live_bytes", [] {
    ensure_init();
    return hrt_peak_live_bytes();
  });
  m.def("reset_peak_live_bytes", [] {
    ensure_init();
    hrt_reset_peak_live_bytes();
  });
  m.def("set_memory_limit", [](uint64_t bytes) {
    ensure_init();
    hrt_set_memory_limit(bytes);
  });
  m.def("synchronize", [] {
    ensure_init();
    hrt_check(hrt_synchronize(), "synchronize");
  });
  m.def("empty_cache", [] {
    ensure_init();
    return hrt_empty_cache();
  });
  m.def("reserved_bytes", [] {
    ensure_init();
    return hrt_reserved_bytes();
  });
  m.def("live_blocks", [] {
    ensure_init();
    return hrt_live_blocks();
  });
  m.def("slab_count", [] {
    ensure_init();
    return hrt_slab_count();
  });
  m.def("validation_errors", [] { return hrt_validation_errors(); });
  m.def("fallback_counts", [] {
    std::lock_guard<std::mutex> l(g_stats_mu);
    return g_fallback_counts;
  });
  m.def("kernel_counts", [] {
    std::lock_guard<std::mutex> l(g_stats_mu);
    return g_kernel_counts;
  });
  m.def("stats", [] {
    ensure_init();
    std::map<std::string, double> r;
    r["dispatch_s"] = hrt_stat(0) * 1e-9;
    r["dispatch_n"] = (double)hrt_stat(1);
    r["transfer_s"] = hrt_stat(2) * 1e-9;
    r["transfer_n"] = (double)hrt_stat(3);
    r["pipeline_create_s"] = hrt_stat(4) * 1e-9;
    r["upload_MB"] = hrt_stat(5) / 1048576.0;
    r["download_MB"] = hrt_stat(6) / 1048576.0;
    r["gpu_wait_s"] = hrt_stat(7) * 1e-9;
    r["fallback_s"] = g_fallback_ns.load() * 1e-9;
    return r;
  });
  m.def("fallback_time_by_op", [] {
    std::lock_guard<std::mutex> l(g_stats_mu);
    std::map<std::string, double> r;
    for (auto& kv : g_fallback_ns_by_op) r[kv.first] = kv.second * 1e-9;
    return r;
  });
  m.def("profile", [] {
    ensure_init();
    std::string buf(1 << 16, '\0');
    size_t n = hrt_profile_dump(buf.data(), buf.size());
    buf.resize(std::min(n, buf.size() - 1));
    return buf;
  });
  m.def("coop_caps", [] { return vkt::coop_caps(); });
  m.def("set_coop_enabled", [](bool on) { vkt::set_coop_enabled(on); });
  m.def("set_fused_attention", [](int mode) { vkt::set_fused_attention(mode); });
  m.def("set_coop_range", [](uint64_t lo, uint64_t hi, int kind) { vkt::set_coop_range(lo, hi, kind); });
  m.def("reset_coop_calls", [] { vkt::reset_coop_calls(); });
  m.def("coop_calls", [] { return vkt::coop_calls(); });
  m.def("reset_counts", [] {
    std::lock_guard<std::mutex> l(g_stats_mu);
    g_fallback_counts.clear();
    g_kernel_counts.clear();
  });
  m.def("event_record", [](uint32_t slot) {
    ensure_init();
    hrt_check(hrt_event_record(slot), "event_record");
  });
  m.def("event_elapsed_ms", [](uint32_t a, uint32_t b) { return event_elapsed(a, b); });
}
