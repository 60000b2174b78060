// The vk device itself: runtime access, kernel queueing, memory (device and pinned allocators, storage
// growth), the device guard and accelerator hooks, tensor factories and views, fill, and copies between
// host and device.  Reference interface: csrc/shim.cpp:133-415 (same operators registered, same
// semantics); the organisation below is this runtime's: one storage-growth routine serves both the
// hooks and resize_, and copies are planned by where their two sides live.
//
// Memory model: data_ptr() of a vk tensor is a device address inside an hrt block; every kernel and
// device copy is queued on the runtime's single HIP stream, so the host waits only for downloads and
// explicit synchronisation.
#include "device.h"

#include <ATen/EmptyTensor.h>
#include <ATen/detail/PrivateUse1HooksInterface.h>
#include <ATen/ops/_reshape_alias_native.h>
#include <ATen/ops/as_strided_native.h>
#include <ATen/ops/unfold_native.h>
#include <ATen/ops/view_native.h>
#include <c10/core/impl/DeviceGuardImplInterface.h>

#include <array>
#include <cstring>
#include <mutex>
#include <shared_mutex>
#include <unordered_map>

#include "common.h"

namespace vkt {

// ---- runtime -------------------------------------------------------------------------------------------------
std::string runtime_error_text() {
  std::array<char, 2048> buf{};
  hrt_last_error(buf.data(), buf.size());
  return std::string(buf.data());
}

void expect_ok(int rc, const char* what) {
  if (rc != 0) TORCH_CHECK(false, "vk: ", what, ": ", runtime_error_text());
}

void runtime() {
  static const int rc = hrt_init();  // thread-safe one-time initialisation; hrt_init is idempotent
  expect_ok(rc, "runtime initialisation");
}

// ---- kernels ---------------------------------------------------------------------------------------------------
namespace {
// Kernel ids by name: looked up in the runtime's registry once, then read under a shared lock.
class KernelIds {
 public:
  uint32_t get(std::string_view name) {
    {
      std::shared_lock<std::shared_mutex> r(mu_);
      auto it = ids_.find(std::string(name));
      if (it != ids_.end()) return it->second;
    }
    runtime();
    const std::string key(name);
    const int id = hrt_kernel_index(key.c_str());
    TORCH_CHECK(id >= 0, "vk: libhrt has no kernel named '", key, "'");
    std::unique_lock<std::shared_mutex> w(mu_);
    ids_.emplace(key, static_cast<uint32_t>(id));
    return static_cast<uint32_t>(id);
  }

 private:
  std::shared_mutex mu_;
  std::unordered_map<std::string, uint32_t> ids_;
};
KernelIds& kernel_ids() {
  static KernelIds k;
  return k;
}
}  // namespace

void queue(std::string_view name, const void* args, uint32_t len) {
  const uint32_t id = kernel_ids().get(name);
  if (hrt_dispatch(id, args, len, 0, 0, 0) != 0)
    TORCH_CHECK(false, "vk: kernel ", std::string(name), " rejected the call: ", runtime_error_text());
}

int float_code(at::ScalarType t) {
  return t == at::kFloat ? HRT_F32 : t == at::kBFloat16 ? HRT_BF16 : t == at::kHalf ? HRT_F16 : -1;
}

const char* dtype_suffix(at::ScalarType t) {
  static const char* const names[] = {"f32", "bf16", "f16"};
  const int c = float_code(t);
  return c < 0 ? nullptr : names[c];
}

std::string typed(std::string_view op, at::ScalarType t) {
  const char* s = dtype_suffix(t);
  TORCH_CHECK(s != nullptr, "vk: no kernel variant for dtype ", t);
  std::string n(op);
  n += '_';
  n += s;
  return n;
}

}  // namespace vkt

namespace {

using namespace vkt;

// ---- memory ------------------------------------------------------------------------------------------------
c10::DataPtr wrap(uint64_t addr, c10::DeleterFnPtr del, c10::Device where) {
  void* p = reinterpret_cast<void*>(addr);
  return {p, p, del, where};
}

class DeviceMemory final : public c10::Allocator {
 public:
  static void release(void* p) {
    if (p != nullptr) (void)hrt_free(reinterpret_cast<uint64_t>(p));
  }
  c10::DataPtr allocate(size_t nbytes) override {
    runtime();
    if (nbytes == 0) return wrap(0, &release, c10::Device(kDev, 0));
    const uint64_t a = hrt_alloc(nbytes);
    if (a == 0) TORCH_CHECK(false, "vk: out of device memory (", nbytes, " bytes requested): ", runtime_error_text());
    return wrap(a, &release, c10::Device(kDev, 0));
  }
  c10::DeleterFnPtr raw_deleter() const override { return &release; }
  void copy_data(void* dst, const void* src, std::size_t n) const override {
    expect_ok(hrt_copy_d2d(reinterpret_cast<uint64_t>(dst), reinterpret_cast<uint64_t>(src), n), "device copy");
  }
};

class PinnedMemory final : public c10::Allocator {
 public:
  static void release(void* p) {
    if (p != nullptr) (void)hrt_host_free(reinterpret_cast<uint64_t>(p));  // deferred past in-flight transfers
  }
  c10::DataPtr allocate(size_t nbytes) override {
    runtime();
    if (nbytes == 0) return wrap(0, &release, c10::Device(c10::DeviceType::CPU));
    const uint64_t a = hrt_host_alloc(nbytes);
    if (a == 0) TORCH_CHECK(false, "vk: pinned host allocation of ", nbytes, " bytes failed: ", runtime_error_text());
    return wrap(a, &release, c10::Device(c10::DeviceType::CPU));
  }
  c10::DeleterFnPtr raw_deleter() const override { return &release; }
  void copy_data(void* dst, const void* src, std::size_t n) const override { std::memcpy(dst, src, n); }
};

DeviceMemory g_device_memory;
PinnedMemory g_pinned_memory;

// Give a storage `nbytes` bytes, keeping the leading min(old, new) bytes of its contents.  The new block
// is filled on the device (queued copy), then swapped in; the old block is freed when its DataPtr dies.
void regrow(c10::StorageImpl* s, size_t nbytes) {
  if (s->nbytes() == nbytes) return;
  c10::DataPtr fresh = g_device_memory.allocate(nbytes);
  const size_t kept = std::min(s->nbytes(), nbytes);
  if (kept != 0)
    expect_ok(hrt_copy_d2d(reinterpret_cast<uint64_t>(fresh.get()), reinterpret_cast<uint64_t>(s->data()), kept),
              "storage resize copy");
  s->set_data_ptr_noswap(std::move(fresh));
  s->set_nbytes(nbytes);
}

// ---- guard and hooks: one device, one stream -------------------------------------------------------------
class Guard final : public c10::impl::DeviceGuardImplInterface {
 public:
  c10::DeviceType type() const override { return kDev; }
  c10::Device exchangeDevice(c10::Device) const override { return only(); }
  c10::Device getDevice() const override { return only(); }
  void setDevice(c10::Device) const override {}
  void uncheckedSetDevice(c10::Device) const noexcept override {}
  c10::Stream getStream(c10::Device d) const override { return c10::Stream(c10::Stream::DEFAULT, d); }
  c10::Stream exchangeStream(c10::Stream s) const override { return s; }
  bool queryStream(const c10::Stream&) const override { return true; }
  void synchronizeStream(const c10::Stream&) const override { drain(); }
  void synchronizeDevice(const c10::DeviceIndex) const override { drain(); }
  c10::DeviceIndex deviceCount() const noexcept override { return 1; }

 private:
  static c10::Device only() { return c10::Device(kDev, 0); }
  static void drain() {
    runtime();
    expect_ok(hrt_synchronize(), "synchronize");
  }
};
C10_REGISTER_GUARD_IMPL(PrivateUse1, Guard);

class Hooks final : public at::PrivateUse1HooksInterface {
 public:
  void init() const override { runtime(); }
  bool isBuilt() const override { return true; }
  bool isAvailable() const override { return true; }
  bool hasPrimaryContext(c10::DeviceIndex) const override { return true; }
  at::Device getDeviceFromPtr(void*) const override { return c10::Device(kDev, 0); }
  bool isPinnedPtr(const void* p) const override { return hrt_host_is_pinned(p) == 1; }  // 0 before init
  at::Allocator* getPinnedMemoryAllocator() const override { return &g_pinned_memory; }
  void resizePrivateUse1Bytes(const c10::Storage& storage, size_t newsize) const override {
    regrow(storage.unsafeGetStorageImpl(), newsize);
  }
};
Hooks g_hooks;
const bool g_hooks_registered = [] {
  at::RegisterPrivateUse1HooksInterface(&g_hooks);
  return true;
}();

// ---- copies ---------------------------------------------------------------------------------------------------
// How one copy is carried out, decided from where its two sides live and what they look like.
enum class Route {
  HostOnly,       // neither side on vk: PyTorch's own copy
  Upload,         // host -> vk
  Download,       // vk -> host
  Blit,           // vk -> vk, same dtype and shape, both dense: one device-to-device copy
  DeviceKernel,   // vk -> vk strided / broadcast / converting copy (ew_copy)
  ViaHost,        // vk -> vk dtype pair the device copy does not convert (integer casts)
};

Route route_of(const at::Tensor& dst, const at::Tensor& src) {
  const bool d = on_vk(dst), s = on_vk(src);
  if (!d && !s) return Route::HostOnly;
  if (!s) return Route::Upload;
  if (!d) return Route::Download;
  const bool raw = src.scalar_type() == dst.scalar_type() && src.sizes() == dst.sizes();
  if (raw && src.is_contiguous() && dst.is_contiguous()) return Route::Blit;
  const bool convertible =
      src.scalar_type() == dst.scalar_type() || (float_code(src.scalar_type()) >= 0 && float_code(dst.scalar_type()) >= 0);
  return convertible ? Route::DeviceKernel : Route::ViaHost;
}

// A non_blocking copy can be asynchronous when the host side is dense pinned runtime memory and the
// device side a dense tensor of the same dtype and shape.
bool async_pair(const at::Tensor& host, const at::Tensor& dev) {
  return host.numel() > 0 && host.scalar_type() == dev.scalar_type() && host.sizes() == dev.sizes() &&
         host.is_contiguous() && dev.is_contiguous() && hrt_host_is_pinned(host.data_ptr()) == 1;
}

void upload(const at::Tensor& dst, const at::Tensor& src, bool non_blocking) {
  if (dst.numel() == 0) return;
  if (non_blocking && async_pair(src, dst)) {
    expect_ok(hrt_upload_async(dptr(dst), src.data_ptr(), dst.nbytes()), "asynchronous upload");
    note_gpu("aten::copy_ (async H2D)");
    return;
  }
  // the host side is brought to dst's dtype and shape as one dense block; a strided dst is then filled
  // from a dense device staging copy by the device copy kernel
  const at::Tensor host = src.to(dst.scalar_type()).expand(dst.sizes()).contiguous();
  const at::Tensor landing = dst.is_contiguous() ? dst : at::empty(dst.sizes(), dst.options());
  expect_ok(hrt_upload(dptr(landing), host.data_ptr(), landing.nbytes()), "upload");
  if (!landing.is_same(dst)) TORCH_CHECK(ew_copy(dst, landing), "vk: no device copy into dtype ", dst.scalar_type());
}

at::Tensor to_host(const at::Tensor& src) {
  const at::Tensor packed = src.is_contiguous() ? src : at::empty(src.sizes(), src.options());
  if (!packed.is_same(src)) TORCH_CHECK(ew_copy(packed, src), "vk: no device copy for dtype ", src.scalar_type());
  at::Tensor host = at::empty(packed.sizes(), packed.options().device(at::kCPU));
  if (host.numel() > 0) expect_ok(hrt_download(host.data_ptr(), dptr(packed), host.nbytes()), "download");
  return host;
}

void download(const at::Tensor& dst, const at::Tensor& src, bool non_blocking) {
  if (src.numel() == 0) return;
  if (non_blocking && async_pair(dst, src)) {
    expect_ok(hrt_download_async(dst.data_ptr(), dptr(src), src.nbytes()), "asynchronous download");
    note_gpu("aten::copy_ (async D2H)");
    return;
  }
  dst.copy_(to_host(src));
}

void copy_between(const at::Tensor& dst, const at::Tensor& src, bool non_blocking) {
  switch (route_of(dst, src)) {
    case Route::HostOnly: dst.copy_(src); return;
    case Route::Upload: upload(dst, src, non_blocking); return;
    case Route::Download: download(dst, src, non_blocking); return;
    case Route::Blit:
      if (src.numel() != 0 && dptr(src) != dptr(dst)) expect_ok(hrt_copy_d2d(dptr(dst), dptr(src), dst.nbytes()), "device copy");
      return;
    case Route::DeviceKernel:
      if (ew_copy(dst, src.sizes().equals(dst.sizes()) ? src : src.expand(dst.sizes()))) return;
      [[fallthrough]];  // element sizes the device copy does not move
    case Route::ViaHost: upload(dst, to_host(src), false); return;
  }
}

}  // namespace

namespace vkt {
c10::Allocator* device_allocator() { return &g_device_memory; }
c10::Allocator* pinned_allocator() { return &g_pinned_memory; }
}  // namespace vkt

namespace {

at::Tensor k_copy_from(const at::Tensor& self, const at::Tensor& dst, bool non_blocking) {
  copy_between(dst, self, non_blocking);
  return dst;
}

at::Tensor k_copy_from_and_resize(const at::Tensor& self, const at::Tensor& dst) {
  if (!dst.sizes().equals(self.sizes())) dst.resize_(self.sizes());
  copy_between(dst, self, false);
  return dst;
}

// ---- factories, views, resize_, fill ----------------------------------------------------------------------
const c10::DispatchKeySet kVkKeys(c10::DispatchKey::PrivateUse1);

at::Tensor k_empty(c10::IntArrayRef size, std::optional<at::ScalarType> dtype, std::optional<at::Layout>,
                   std::optional<at::Device>, std::optional<bool>, std::optional<at::MemoryFormat> fmt) {
  return at::detail::empty_generic(size, &g_device_memory, kVkKeys, c10::dtype_or_default(dtype), fmt);
}

at::Tensor k_empty_strided(c10::IntArrayRef size, c10::IntArrayRef stride, std::optional<at::ScalarType> dtype,
                           std::optional<at::Layout>, std::optional<at::Device>, std::optional<bool>) {
  return at::detail::empty_strided_generic(size, stride, &g_device_memory, kVkKeys, c10::dtype_or_default(dtype));
}

// Views share storage with their base, so they are computed here (a CPU fallback would copy).
at::Tensor k_view(const at::Tensor& self, c10::SymIntArrayRef size) {
  return at::native::view(self, C10_AS_INTARRAYREF_SLOW(size));
}
at::Tensor k_as_strided(const at::Tensor& self, c10::SymIntArrayRef size, c10::SymIntArrayRef stride,
                        std::optional<c10::SymInt> offset) {
  std::optional<int64_t> off;
  if (offset) off = offset->guard_int(__FILE__, __LINE__);
  return at::native::as_strided_tensorimpl(self, C10_AS_INTARRAYREF_SLOW(size), C10_AS_INTARRAYREF_SLOW(stride), off);
}
at::Tensor k_reshape_alias(const at::Tensor& self, c10::SymIntArrayRef size, c10::SymIntArrayRef stride) {
  return at::native::_reshape_alias(self, C10_AS_INTARRAYREF_SLOW(size), C10_AS_INTARRAYREF_SLOW(stride));
}
at::Tensor k_unfold(const at::Tensor& self, int64_t dim, int64_t size, int64_t step) {
  return at::native::unfold(self, dim, size, step);
}

// PyTorch's resize_ semantics (same sizes: nothing changes; otherwise contiguous sizes, an optional
// memory-format restride, and storage that only ever grows), with device memory grown by regrow()
// instead of the CPU path's host memcpy.
const at::Tensor& k_resize(const at::Tensor& self, c10::SymIntArrayRef size_sym, std::optional<at::MemoryFormat> fmt) {
  const c10::IntArrayRef size = C10_AS_INTARRAYREF_SLOW(size_sym);
  TORCH_CHECK(!fmt || *fmt != at::MemoryFormat::Preserve, "vk: resize_ does not take memory_format=preserve");
  c10::TensorImpl* t = self.unsafeGetTensorImpl();
  if (!t->sizes().equals(size)) {
    t->set_sizes_contiguous(size);
    if (t->numel() > 0) {
      const size_t need = at::detail::computeStorageNbytesContiguous(size, self.dtype().itemsize(), t->storage_offset());
      c10::StorageImpl* s = self.storage().unsafeGetStorageImpl();
      if (need > s->nbytes()) regrow(s, need);
    }
  }
  if (fmt) t->empty_tensor_restride(*fmt);
  return self;
}

at::Tensor& k_fill(at::Tensor& self, const at::Scalar& value) {
  if (on_vk(self) && ew_fill(self, value)) {
    note_gpu("aten::fill_");
    return self;
  }
  return VKT_CPU(fill__Scalar, self, value);
}

at::Tensor& k_zero(at::Tensor& self) {
  if (on_vk(self) && ew_fill(self, at::Scalar(0))) {
    note_gpu("aten::zero_");
    return self;
  }
  return VKT_CPU(zero_, self);
}

}  // namespace

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("empty.memory_format", &k_empty);
  m.impl("empty_strided", &k_empty_strided);
  m.impl("_copy_from", &k_copy_from);
  m.impl("_copy_from_and_resize", &k_copy_from_and_resize);
  m.impl("view", &k_view);
  m.impl("as_strided", &k_as_strided);
  m.impl("_reshape_alias", &k_reshape_alias);
  m.impl("unfold", &k_unfold);
  m.impl("resize_", &k_resize);
  m.impl("fill_.Scalar", &k_fill);
  m.impl("zero_", &k_zero);
}
