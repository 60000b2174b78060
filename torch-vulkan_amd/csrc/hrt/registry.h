// Kernel registry of the hrt runtime: name -> (argument-block size, launcher).
//
// Each kernel source registers its launchers with a static HRT_REGISTER(...) object; hrt_kernel_index
// looks a name up and hrt_dispatch checks the argument size (as vkrt/src/lib.rs:922-927 checks the
// push-constant size) and calls the launcher.  A launcher validates its arguments, checks every
// operand's byte extent against the allocator through LaunchCtx::check, picks its grid and queues the
// kernel on ctx.stream.  It never synchronizes.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <functional>
#include <string>
#include <vector>

namespace hrt {

struct LaunchCtx {
  hipStream_t stream = nullptr;
  int device = 0;
  std::string error;
  // True when [addr, addr + bytes) lies in one live block; otherwise records an error naming `what`.
  bool (*in_bounds)(uint64_t addr, uint64_t bytes, std::string* err) = nullptr;
  // A device range the launcher owns outside the allocator (a file-scope __device__ scratch array);
  // operands inside it pass check() without an allocator lookup.
  uint64_t own_lo = 0, own_hi = 0;

  bool check(uint64_t addr, uint64_t bytes, const char* what) {
    if (bytes == 0) return true;
    if (addr >= own_lo && addr < own_hi && bytes <= own_hi - addr) return true;
    std::string e;
    if (addr == 0 || !in_bounds(addr, bytes, &e)) {
      error = std::string("operand '") + what + "': " + (addr == 0 ? std::string("null address") : e);
      return false;
    }
    return true;
  }
  bool fail(const std::string& msg) {
    error = msg;
    return false;
  }
};

// Returns true when the kernel was queued; otherwise ctx.error says why.
using LaunchFn = bool (*)(const void* args, const uint32_t grid[3], LaunchCtx& ctx);

struct KernelEntry {
  const char* name;
  uint32_t args_size;
  LaunchFn launch;
  bool raw_grid;  // grid supplied by the caller (only the runtime smoke kernel)
};

std::vector<KernelEntry>& kernel_table();

struct KernelRegistrar {
  KernelRegistrar(const char* name, uint32_t args_size, LaunchFn fn, bool raw_grid = false) {
    kernel_table().push_back(KernelEntry{name, args_size, fn, raw_grid});
  }
};

// Per-device set-up that hrt_init runs once, with the selected device current (for instance resolving
// the address of a file-scope __device__ array).  Returns false and sets *err on failure.
using DeviceInitFn = bool (*)(int device, std::string* err);
std::vector<DeviceInitFn>& device_init_table();
struct DeviceInitRegistrar {
  explicit DeviceInitRegistrar(DeviceInitFn fn) { device_init_table().push_back(fn); }
};

// For entry points other than hrt_dispatch: runs `fn` under the runtime lock with a LaunchCtx on the
// runtime stream.  Returns 0, or -1 with the last error set to "<what>: <ctx.error>" (also when
// hrt_init has not run).
int run_launch(const char* what, const std::function<bool(LaunchCtx&)>& fn);

#define HRT_CAT2(a, b) a##b
#define HRT_CAT(a, b) HRT_CAT2(a, b)
#define HRT_REGISTER(name, ArgsT, fn) static ::hrt::KernelRegistrar HRT_CAT(hrt_reg_, __COUNTER__)(name, sizeof(ArgsT), fn)
#define HRT_REGISTER_DEVICE_INIT(fn) static ::hrt::DeviceInitRegistrar HRT_CAT(hrt_dinit_, __COUNTER__)(fn)
#define HRT_REGISTER_RAW(name, ArgsT, fn) \
  static ::hrt::KernelRegistrar HRT_CAT(hrt_reg_, __COUNTER__)(name, sizeof(ArgsT), fn, true)

// Byte extent touched by a strided view: (1 + sum (size_i - 1) * stride_i) elements, 0 if empty.
inline uint64_t span_bytes(int ndim, const int64_t* sizes, const int64_t* strides, uint64_t elem) {
  uint64_t last = 0;
  for (int i = 0; i < ndim; ++i) {
    if (sizes[i] <= 0) return 0;
    last += uint64_t(sizes[i] - 1) * uint64_t(strides[i]);
  }
  return (last + 1) * elem;
}

inline bool launch_ok(hipError_t e, LaunchCtx& ctx, const char* what) {
  if (e == hipSuccess) return true;
  ctx.error = std::string(what) + ": " + hipGetErrorString(e);
  return false;
}

}  // namespace hrt
