// hrt runtime: the C ABI declared in include/hrt.h, over HIP.
//
// One process-wide Runtime owns the device, ONE HIP stream (default priority) and the slab allocator.
// Kernels and device-to-device copies are queued on that stream and never waited for, so launches
// batch naturally; the host waits only where data must be visible to it (download, synchronize) or
// memory goes back to the driver.  Mirrors the reference runtime's contract (vkrt/src/lib.rs:975-1244):
// 0 / -1 status codes, 0 for failed values, and a last-error string.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cctype>
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../../include/hrt.h"
#include "registry.h"
#include "slab_allocator.h"

namespace hrt {

std::vector<KernelEntry>& kernel_table() {
  static std::vector<KernelEntry> t;
  return t;
}

std::vector<DeviceInitFn>& device_init_table() {
  static std::vector<DeviceInitFn> t;
  return t;
}

namespace {

std::mutex g_err_mu;
std::string g_last_error;

void set_error(const std::string& e) {
  std::lock_guard<std::mutex> l(g_err_mu);
  g_last_error = e;
}

std::atomic<uint64_t> g_stats[8];
std::atomic<uint64_t> g_validation_errors{0};

uint64_t now_ns() {
  return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

struct HipBacking final : Backing {
  hipStream_t stream = nullptr;
  bool capturing = false;
  bool map(uint64_t size, uint64_t* base, std::string* err) override {
    if (capturing) {
      *err = "cannot reserve device memory while a graph is being recorded";
      return false;
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, size);
    if (e != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      *err = "hipMalloc(" + std::to_string(size) + " bytes): " + hipGetErrorString(e);
      return false;
    }
    *base = reinterpret_cast<uint64_t>(p);
    return true;
  }
  void unmap(uint64_t base) override { (void)hipFree(reinterpret_cast<void*>(base)); }
  void drain() override {
    if (stream) (void)hipStreamSynchronize(stream);
  }
};

struct Runtime {
  std::mutex mu;
  int device = 0;
  hipStream_t stream = nullptr;
  std::string name;
  uint64_t total_mem = 0;
  HipBacking backing;
  std::unique_ptr<SlabAllocator> alloc;
  bool profile = false;
  std::map<std::string, std::pair<uint64_t, uint64_t>> prof;  // name -> (ns, count)
  hipEvent_t prof_ev[2] = {nullptr, nullptr};
  static constexpr uint32_t kSlots = 1024;  // timing events (hrt_event_record)
  hipEvent_t slots[kSlots] = {};
  std::vector<hipGraphExec_t> graphs;
  // Asynchronous uploads run on their own stream (default priority) so they overlap kernels.
  hipStream_t copy_stream = nullptr;
  hipEvent_t order_ev = nullptr;      // compute-stream position an upload starts after
  std::vector<hipEvent_t> ev_pool;    // completion events of uploads, reused
  struct Pending {
    uint64_t lo, hi;
    hipEvent_t done;
  };
  std::vector<Pending> pending;       // uploads no later device work has waited for yet
  std::map<uint64_t, uint64_t> pinned;  // live pinned host blocks: base -> bytes
  struct FreedPinned {
    uint64_t base, bytes;
    hipEvent_t after_compute, after_copy;  // reusable once both have completed
  };
  std::vector<FreedPinned> pinned_free;
};

Runtime* g_rt = nullptr;
std::mutex g_init_mu;

hipEvent_t take_event(Runtime* rt) {
  if (!rt->ev_pool.empty()) {
    hipEvent_t e = rt->ev_pool.back();
    rt->ev_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  return e;
}

// Make the compute stream wait for every pending upload into [addr, addr + n) (a wait queued on the
// stream: the host does not block).  After the wait is queued the event may be recorded again.
void wait_pending(Runtime* rt, uint64_t addr, uint64_t n) {
  for (size_t i = 0; i < rt->pending.size();) {
    const Runtime::Pending p = rt->pending[i];
    if (p.lo < addr + n && addr < p.hi) {
      (void)hipStreamWaitEvent(rt->stream, p.done, 0);
      rt->ev_pool.push_back(p.done);
      rt->pending[i] = rt->pending.back();
      rt->pending.pop_back();
    } else {
      ++i;
    }
  }
}

bool in_bounds_locked(uint64_t addr, uint64_t bytes, std::string* err) {
  if (!g_rt->alloc->resolve(addr, bytes, err)) return false;
  if (!g_rt->pending.empty()) wait_pending(g_rt, addr, bytes);
  return true;
}

// Pinned block containing [p, p + n), or pinned.end().
std::map<uint64_t, uint64_t>::const_iterator pinned_of(const Runtime* rt, uint64_t p, uint64_t n) {
  auto it = rt->pinned.upper_bound(p);
  if (it == rt->pinned.begin()) return rt->pinned.end();
  --it;
  if (p >= it->first + it->second || n > it->first + it->second - p) return rt->pinned.end();
  return it;
}

int hip_fail(const char* what, hipError_t e) {
  (void)hipGetLastError();
  set_error(std::string(what) + ": " + hipGetErrorString(e));
  return -1;
}

Runtime* rt_or_error() {
  if (!g_rt) set_error("hrt_init has not been called");
  return g_rt;
}

int init_runtime() {
  auto rt = std::make_unique<Runtime>();
  const char* dev_env = std::getenv("HRT_DEVICE");
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count <= 0) {
    (void)hipGetLastError();
    set_error(std::string("no HIP device available: ") + (e != hipSuccess ? hipGetErrorString(e) : "0 devices"));
    return -1;
  }
  // HRT_DEVICE: a device index, or a case-insensitive substring of a device's name ("name (arch)"), the
  // lowest-numbered match winning (the reference's VKRT_DEVICE rule, vkrt/src/lib.rs:241-262); anything
  // else fails with the list of devices.
  auto display_name = [](int i) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, i) != hipSuccess) {
      (void)hipGetLastError();
      return std::string("?");
    }
    return std::string(p.name) + " (" + p.gcnArchName + ")";
  };
  auto lower = [](std::string t) {
    for (char& c : t) c = (char)std::tolower((unsigned char)c);
    return t;
  };
  int dev = 0;
  std::string sel = dev_env ? dev_env : "";
  while (!sel.empty() && std::isspace((unsigned char)sel.back())) sel.pop_back();
  while (!sel.empty() && std::isspace((unsigned char)sel.front())) sel.erase(sel.begin());
  if (!sel.empty()) {
    int found = -1;
    char* end = nullptr;
    const long v = std::strtol(sel.c_str(), &end, 10);
    if (end != sel.c_str() && *end == '\0') {
      if (v >= 0 && v < count) found = (int)v;
    } else {
      const std::string key = lower(sel);
      for (int i = 0; i < count && found < 0; ++i)
        if (lower(display_name(i)).find(key) != std::string::npos) found = i;
    }
    if (found < 0) {
      std::string names;
      for (int i = 0; i < count; ++i) names += "\n  " + std::to_string(i) + ": " + display_name(i);
      set_error("HRT_DEVICE='" + sel + "' does not name a device; available:" + names);
      return -1;
    }
    dev = found;
  }
  if ((e = hipSetDevice(dev)) != hipSuccess) return hip_fail("hipSetDevice", e);
  for (DeviceInitFn fn : device_init_table()) {  // per-device set-up of the kernel sources, device current
    std::string err;
    if (!fn(dev, &err)) {
      set_error("device set-up: " + err);
      return -1;
    }
  }
  hipDeviceProp_t prop;
  if ((e = hipGetDeviceProperties(&prop, dev)) != hipSuccess) return hip_fail("hipGetDeviceProperties", e);
  rt->device = dev;
  rt->name = std::string(prop.name) + " (" + prop.gcnArchName + ")";
  rt->total_mem = prop.totalGlobalMem;
  if ((e = hipStreamCreateWithFlags(&rt->stream, hipStreamNonBlocking)) != hipSuccess) return hip_fail("hipStreamCreate", e);
  if ((e = hipStreamCreateWithFlags(&rt->copy_stream, hipStreamNonBlocking)) != hipSuccess)
    return hip_fail("hipStreamCreate(copy)", e);
  if ((e = hipEventCreateWithFlags(&rt->order_ev, hipEventDisableTiming)) != hipSuccess) return hip_fail("hipEventCreate", e);
  rt->backing.stream = rt->stream;
  rt->alloc = std::make_unique<SlabAllocator>(&rt->backing, rt->total_mem);
  const char* pe = std::getenv("HRT_PROFILE");
  rt->profile = pe && pe[0] && pe[0] != '0';
  if (rt->profile) {
    for (auto& ev : rt->prof_ev)
      if ((e = hipEventCreate(&ev)) != hipSuccess) return hip_fail("hipEventCreate", e);
  }
  uint64_t t0 = now_ns();
  (void)kernel_table();  // populated by static registration at load time
  g_stats[4] += now_ns() - t0;
  g_rt = rt.release();
  return 0;
}

size_t copy_out(const std::string& s, char* buf, size_t cap) {
  if (buf && cap > 0) {
    size_t n = std::min(s.size(), cap - 1);
    std::memcpy(buf, s.data(), n);
    buf[n] = '\0';
  }
  return s.size();
}

bool checked(Runtime* rt, uint64_t addr, uint64_t n) {
  std::string err;
  if (!rt->alloc->resolve(addr, n, &err)) {
    g_validation_errors++;
    set_error(err);
    return false;
  }
  if (!rt->pending.empty()) wait_pending(rt, addr, n);
  return true;
}

// Record where both streams stand when a pinned block is freed (no stream may be recording a graph).
void mark_freed(Runtime* rt, Runtime::FreedPinned& f) {
  f.after_compute = take_event(rt);
  f.after_copy = take_event(rt);
  if (f.after_compute && f.after_copy) {
    (void)hipEventRecord(f.after_compute, rt->stream);
    (void)hipEventRecord(f.after_copy, rt->copy_stream);
    return;
  }
  (void)hipStreamSynchronize(rt->copy_stream);  // no events: wait for the transfers instead
  (void)hipStreamSynchronize(rt->stream);
  if (f.after_compute) rt->ev_pool.push_back(f.after_compute);
  if (f.after_copy) rt->ev_pool.push_back(f.after_copy);
  f.after_compute = f.after_copy = nullptr;
  (void)hipHostFree(reinterpret_cast<void*>(f.base));
  f.base = 0;
}

// Freed pinned blocks whose transfers have all finished go back to the driver (all: every marked one,
// after the caller has waited for both streams).  Blocks freed while a graph was being recorded wait to
// be marked.
void release_pinned(Runtime* rt, bool all) {
  for (size_t i = 0; i < rt->pinned_free.size();) {
    auto& f = rt->pinned_free[i];
    const bool marked = f.after_compute && f.after_copy;
    const bool done = f.base == 0 || (marked && (all || (hipEventQuery(f.after_compute) == hipSuccess &&
                                                         hipEventQuery(f.after_copy) == hipSuccess)));
    if (done) {
      if (f.base) (void)hipHostFree(reinterpret_cast<void*>(f.base));
      if (f.after_compute) rt->ev_pool.push_back(f.after_compute);
      if (f.after_copy) rt->ev_pool.push_back(f.after_copy);
      rt->pinned_free[i] = rt->pinned_free.back();
      rt->pinned_free.pop_back();
    } else {
      ++i;
    }
  }
  (void)hipGetLastError();  // hipEventQuery reports hipErrorNotReady through the error state
}

}  // namespace

int run_launch(const char* what, const std::function<bool(LaunchCtx&)>& fn) {
  Runtime* rt = rt_or_error();
  if (!rt) return -1;
  uint64_t t0 = now_ns();
  std::lock_guard<std::mutex> l(rt->mu);
  LaunchCtx ctx;
  ctx.stream = rt->stream;
  ctx.device = rt->device;
  ctx.in_bounds = &in_bounds_locked;
  if (!fn(ctx)) {
    if (ctx.error.rfind("operand", 0) == 0) g_validation_errors++;
    set_error(std::string(what) + ": " + ctx.error);
    return -1;
  }
  g_stats[0] += now_ns() - t0;
  g_stats[1]++;
  return 0;
}

}  // namespace hrt

using namespace hrt;

extern "C" {

int hrt_init(void) {
  std::lock_guard<std::mutex> l(g_init_mu);
  if (g_rt) return 0;
  return init_runtime();
}

size_t hrt_last_error(char* buf, size_t cap) {
  std::lock_guard<std::mutex> l(g_err_mu);
  return copy_out(g_last_error, buf, cap);
}

size_t hrt_device_name(char* buf, size_t cap) {
  Runtime* rt = rt_or_error();
  return copy_out(rt ? rt->name : std::string(), buf, cap);
}

uint64_t hrt_max_alloc(void) {
  Runtime* rt = rt_or_error();
  if (!rt) return 0;
  std::lock_guard<std::mutex> l(rt->mu);
  return rt->alloc->max_alloc();
}

uint64_t hrt_live_bytes(void) {
  Runtime* rt = rt_or_error();
  if (!rt) return 0;
  std::lock_guard<std::mutex> l(rt->mu);
  return rt->alloc->live_bytes();
}

int32_t hrt_memory_info(uint64_t* out) {
  Runtime* rt = rt_or_error();
  if (!rt) return -1;
  if (!out) {
    set_error("hrt_memory_info: null output");
    return -1;
  }
  std::lock_guard<std::mutex> l(rt->mu);
  size_t free_b = 0, total_b = 0;
  hipError_t e = hipMemGetInfo(&free_b, &total_b);
  if (e != hipSuccess) return hip_fail("hipMemGetInfo", e);
  out[0] = (uint64_t)free_b + rt->alloc->reserved_bytes();
  if (out[0] > total_b) out[0] = total_b;
  out[1] = (uint64_t)(total_b - free_b);
  out[2] = (uint64_t)total_b;
  return 0;
}

uint64_t hrt_peak_live_bytes(void) {
  Runtime* rt = rt_or_error();
  if (!rt) return 0;
  std::lock_guard<std::mutex> l(rt->mu);
  return rt->alloc->peak_live_bytes();
}

void hrt_reset_peak_live_bytes(void) {
  Runtime* rt = rt_or_error();
  if (!rt) return;
  std::lock_guard<std::mutex> l(rt->mu);
  rt->alloc->reset_peak();
}

void hrt_set_memory_limit(uint64_t bytes) {
  Runtime* rt = rt_or_error();
  if (!rt) return;
  std::lock_guard<std::mutex> l(rt->mu);
  rt->alloc->set_limit(bytes);
}

uint64_t hrt_alloc(uint64_t size) {
  Runtime* rt = rt_or_error();
  if (!rt) return 0;
  std::lock_guard<std::mutex> l(rt->mu);
  std::string err;
  uint64_t a = rt->alloc->alloc(size, &err);
  if (!a) set_error(err);
  return a;
}

int hrt_free(uint64_t addr) {
  Runtime* rt = rt_or_error();
  if (!rt) return -1;
  std::lock_guard<std::mutex> l(rt->mu);
  std::string err;
  if (!rt->pending.empty()) wait_pending(rt, addr, std::max<uint64_t>(rt->alloc->block_bytes(addr), 1));
  if (rt->backing.capturing && !rt->alloc->is_regular_block(addr)) {
    set_error("hrt_free: a dedicated block cannot be released while a graph is being recorded");
    return -1;
  }
  if (!rt->alloc->free(addr, &err)) {
    set_error(err);
    return -1;
  }
  return 0;
}

int hrt_upload(uint64_t dst, const void* src, uint64_t n) {
  Runtime* rt = rt_or_error();
  if (!rt) return -1;
  if (n == 0) return 0;
  uint64_t t0 = now_ns();
  std::lock_guard<std::mutex> l(rt->mu);
  if (!src) {
    set_error("hrt_upload: null source");
    return -1;
  }
  if (rt->backing.capturing) {
    set_error("hrt_upload: not allowed while a graph is being recorded");
    return -1;
  }
  if (!checked(rt, dst, n)) return -1;
  hipError_t e = hipMemcpyAsync(reinterpret_cast<void*>(dst), src, n, hipMemcpyHostToDevice, rt->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);  // the source may be freed on return
  g_stats[2] += now_ns() - t0;
  g_stats[3]++;
  g_stats[5] += n;
  if (e != hipSuccess) return hip_fail("upload", e);
  return 0;
}

int hrt_download(void* dst, uint64_t src, uint64_t n) {
  Runtime* rt = rt_or_error();
  if (!rt) return -1;
  if (n == 0) return 0;
  uint64_t t0 = now_ns();
  std::lock_guard<std::mutex> l(rt->mu);
  if (!dst) {
    set_error("hrt_download: null destination");
    return -1;
  }
  if (rt->backing.capturing) {
    set_error("hrt_download: not allowed while a graph is being recorded");
    return -1;
  }
  if (!checked(rt, src, n)) return -1;
  hipError_t e = hipMemcpyAsync(dst, reinterpret_cast<const void*>(src), n, hipMemcpyDeviceToHost, rt->stream);
  uint64_t tw = now_ns();
  if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);
  g_stats[7] += now_ns() - tw;
  g_stats[2] += now_ns() - t0;
  g_stats[3]++;
  g_stats[6] += n;
  if (e != hipSuccess) return hip_fail("download", e);
  return 0;
}

int hrt_copy_d2d(uint64_t dst, uint64_t src, uint64_t n) {
  Runtime* rt = rt_or_error();
  if (!rt) return -1;
  if (n == 0) return 0;
  std::lock_guard<std::mutex> l(rt->mu);
  if (!checked(rt, dst, n) || !checked(rt, src, n)) return -1;
  hipError_t e =
      hipMemcpyAsync(reinterpret_cast<void*>(dst), reinterpret_cast<const void*>(src), n, hipMemcpyDeviceToDevice, rt->stream);
  if (e != hipSuccess) return hip_fail("copy_d2d", e);
  return 0;
}

uint64_t hrt_host_alloc(uint64_t bytes) {
  Runtime* rt = rt_or_error();
  if (!rt) return 0;
  if (bytes == 0) {
    set_error("hrt_host_alloc: size 0");
    return 0;
  }
  std::lock_guard<std::mutex> l(rt->mu);
  if (!rt->pinned_free.empty()) release_pinned(rt, false);
  void* p = nullptr;
  hipError_t e = hipHostMalloc(&p, bytes, hipHostMallocDefault);
  if (e != hipSuccess || !p) {
    hip_fail("hipHostMalloc", e);
    return 0;
  }
  rt->pinned[reinterpret_cast<uint64_t>(p)] = bytes;
  return reinterpret_cast<uint64_t>(p);
}

int hrt_host_free(uint64_t ptr) {
  Runtime* rt = rt_or_error();
  if (!rt) return -1;
  std::lock_guard<std::mutex> l(rt->mu);
  auto it = rt->pinned.find(ptr);
  if (it == rt->pinned.end()) {
    set_error("hrt_host_free: not a pinned block from hrt_host_alloc");
    return -1;
  }
  Runtime::FreedPinned f{ptr, it->second, nullptr, nullptr};
  rt->pinned.erase(it);
  if (!rt->backing.capturing) mark_freed(rt, f);  // while recording: marked when the recording ends
  rt->pinned_free.push_back(f);
  release_pinned(rt, false);
  return 0;
}

int hrt_host_is_pinned(const void* p) {
  Runtime* rt = g_rt;
  if (!rt || !p) return 0;
  std::lock_guard<std::mutex> l(rt->mu);
  return pinned_of(rt, reinterpret_cast<uint64_t>(p), 1) != rt->pinned.end() ? 1 : 0;
}

int hrt_upload_async(uint64_t dst, const void* src, uint64_t n) {
  Runtime* rt = rt_or_error();
  if (!rt) return -1;
  if (n == 0) return 0;
  uint64_t t0 = now_ns();
  std::lock_guard<std::mutex> l(rt->mu);
  if (rt->backing.capturing) {
    set_error("hrt_upload_async: not allowed while a graph is being recorded");
    return -1;
  }
  if (!src || pinned_of(rt, reinterpret_cast<uint64_t>(src), n) == rt->pinned.end()) {
    set_error("hrt_upload_async: the source is not inside one pinned block from hrt_host_alloc");
    return -1;
  }
  std::string err;
  if (!rt->alloc->resolve(dst, n, &err)) {
    g_validation_errors++;
    set_error(err);
    return -1;
  }
  hipEvent_t done = take_event(rt);
  if (!done) return hip_fail("hipEventCreate", hipErrorOutOfMemory);
  // the copy starts after everything queued so far on the compute stream (no overwrite of data that
  // earlier kernels read) and after earlier uploads (copy stream order)
  hipError_t e = hipEventRecord(rt->order_ev, rt->stream);
  if (e == hipSuccess) e = hipStreamWaitEvent(rt->copy_stream, rt->order_ev, 0);
  if (e == hipSuccess) e = hipMemcpyAsync(reinterpret_cast<void*>(dst), src, n, hipMemcpyHostToDevice, rt->copy_stream);
  if (e == hipSuccess) e = hipEventRecord(done, rt->copy_stream);
  if (e != hipSuccess) {
    rt->ev_pool.push_back(done);
    return hip_fail("upload_async", e);
  }
  rt->pending.push_back({dst, dst + n, done});
  g_stats[2] += now_ns() - t0;
  g_stats[3]++;
  g_stats[5] += n;
  return 0;
}

int hrt_download_async(void* dst, uint64_t src, uint64_t n) {
  Runtime* rt = rt_or_error();
  if (!rt) return -1;
  if (n == 0) return 0;
  uint64_t t0 = now_ns();
  std::lock_guard<std::mutex> l(rt->mu);
  if (rt->backing.capturing) {
    set_error("hrt_download_async: not allowed while a graph is being recorded");
    return -1;
  }
  if (!dst || pinned_of(rt, reinterpret_cast<uint64_t>(dst), n) == rt->pinned.end()) {
    set_error("hrt_download_async: the destination is not inside one pinned block from hrt_host_alloc");
    return -1;
  }
  if (!checked(rt, src, n)) return -1;
  hipError_t e = hipMemcpyAsync(dst, reinterpret_cast<const void*>(src), n, hipMemcpyDeviceToHost, rt->stream);
  g_stats[2] += now_ns() - t0;
  g_stats[3]++;
  g_stats[6] += n;
  if (e != hipSuccess) return hip_fail("download_async", e);
  return 0;
}

int hrt_kernel_index(const char* name) {
  if (!name) return -1;
  const auto& t = kernel_table();
  for (size_t i = 0; i < t.size(); ++i)
    if (std::strcmp(t[i].name, name) == 0) return (int)i;
  return -1;
}

int hrt_dispatch(uint32_t kernel, const void* args, uint32_t len, uint32_t gx, uint32_t gy, uint32_t gz) {
  Runtime* rt = rt_or_error();
  if (!rt) return -1;
  uint64_t t0 = now_ns();
  const auto& t = kernel_table();
  if (kernel >= t.size()) {
    set_error("hrt_dispatch: unknown kernel id " + std::to_string(kernel));
    return -1;
  }
  const KernelEntry& k = t[kernel];
  if (len != k.args_size || !args) {
    set_error(std::string("hrt_dispatch(") + k.name + "): argument block is " + std::to_string(len) + " bytes, expected " +
              std::to_string(k.args_size));
    return -1;
  }
  uint32_t grid[3] = {gx, gy, gz};
  if (k.raw_grid) {
    if (gx == 0 || gy == 0 || gz == 0) {
      set_error(std::string("hrt_dispatch(") + k.name + "): empty grid");
      return -1;
    }
  } else if (gx != 0 || gy != 0 || gz != 0) {
    set_error(std::string("hrt_dispatch(") + k.name + "): this kernel sizes its own grid; pass gx = gy = gz = 0");
    return -1;
  }
  std::lock_guard<std::mutex> l(rt->mu);
  LaunchCtx ctx;
  ctx.stream = rt->stream;
  ctx.device = rt->device;
  ctx.in_bounds = &in_bounds_locked;
  const bool prof = rt->profile && !rt->backing.capturing;
  if (prof) (void)hipEventRecord(rt->prof_ev[0], rt->stream);
  bool ok = k.launch(args, grid, ctx);
  if (!ok) {
    if (ctx.error.rfind("operand", 0) == 0) g_validation_errors++;
    set_error(std::string(k.name) + ": " + ctx.error);
    return -1;
  }
  if (prof) {
    (void)hipEventRecord(rt->prof_ev[1], rt->stream);
    (void)hipEventSynchronize(rt->prof_ev[1]);
    float ms = 0.f;
    (void)hipEventElapsedTime(&ms, rt->prof_ev[0], rt->prof_ev[1]);
    auto& p = rt->prof[k.name];
    p.first += (uint64_t)(ms * 1e6);
    p.second += 1;
  }
  g_stats[0] += now_ns() - t0;
  g_stats[1]++;
  return 0;
}

int hrt_dispatch_batch(const uint32_t* kernels, const void* const* args, const uint32_t* lens, uint32_t n) {
  if (n && (!kernels || !args || !lens)) {
    set_error("hrt_dispatch_batch: null array");
    return -1;
  }
  for (uint32_t i = 0; i < n; ++i)
    if (hrt_dispatch(kernels[i], args[i], lens[i], 0, 0, 0) != 0) return -(int)(i + 1);
  return 0;
}

int hrt_synchronize(void) {
  Runtime* rt = rt_or_error();
  if (!rt) return -1;
  std::lock_guard<std::mutex> l(rt->mu);
  if (rt->backing.capturing) {
    set_error("hrt_synchronize: not allowed while a graph is being recorded");
    return -1;
  }
  uint64_t t0 = now_ns();
  hipError_t e = hipStreamSynchronize(rt->copy_stream);
  if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);
  g_stats[7] += now_ns() - t0;
  if (e != hipSuccess) return hip_fail("synchronize", e);
  if (!rt->pinned_free.empty()) release_pinned(rt, false);
  return 0;
}

size_t hrt_empty_cache(void) {
  Runtime* rt = rt_or_error();
  if (!rt) return 0;
  std::lock_guard<std::mutex> l(rt->mu);
  if (rt->backing.capturing) {
    set_error("hrt_empty_cache: not allowed while a graph is being recorded");
    return 0;
  }
  return rt->alloc->empty_cache();
}

uint64_t hrt_reserved_bytes(void) {
  Runtime* rt = rt_or_error();
  if (!rt) return 0;
  std::lock_guard<std::mutex> l(rt->mu);
  return rt->alloc->reserved_bytes();
}

size_t hrt_live_blocks(void) {
  Runtime* rt = rt_or_error();
  if (!rt) return 0;
  std::lock_guard<std::mutex> l(rt->mu);
  return rt->alloc->live_blocks();
}

size_t hrt_slab_count(void) {
  Runtime* rt = rt_or_error();
  if (!rt) return 0;
  std::lock_guard<std::mutex> l(rt->mu);
  return rt->alloc->slab_count();
}

size_t hrt_validation_errors(void) { return (size_t)g_validation_errors.load(); }

uint64_t hrt_stat(uint32_t i) { return i < 8 ? g_stats[i].load() : 0; }

size_t hrt_profile_dump(char* buf, size_t cap) {
  std::string out;
  if (g_rt) {
    std::lock_guard<std::mutex> l(g_rt->mu);
    std::vector<std::pair<std::string, std::pair<uint64_t, uint64_t>>> v(g_rt->prof.begin(), g_rt->prof.end());
    std::sort(v.begin(), v.end(), [](const auto& a, const auto& b) { return a.second.first > b.second.first; });
    char line[256];
    for (const auto& kv : v) {
      snprintf(line, sizeof(line), "%s\t%.3f\t%llu\n", kv.first.c_str(), kv.second.first * 1e-6,
               (unsigned long long)kv.second.second);
      out += line;
    }
  }
  return copy_out(out, buf, cap);
}

uint32_t hrt_coop_caps(void) {
  Runtime* rt = rt_or_error();
  return rt ? 3u : 0u;
}

int hrt_event_record(uint32_t slot) {
  Runtime* rt = rt_or_error();
  if (!rt) return -1;
  if (slot >= Runtime::kSlots) {
    set_error("hrt_event_record: slot must be < 1024");
    return -1;
  }
  std::lock_guard<std::mutex> l(rt->mu);
  hipError_t e = hipSuccess;
  if (!rt->slots[slot]) e = hipEventCreate(&rt->slots[slot]);
  if (e == hipSuccess) e = hipEventRecord(rt->slots[slot], rt->stream);
  if (e != hipSuccess) return hip_fail("hipEventRecord", e);
  return 0;
}

float hrt_event_elapsed_ms(uint32_t start_slot, uint32_t end_slot) {
  Runtime* rt = rt_or_error();
  if (!rt) return -1.f;
  if (start_slot >= Runtime::kSlots || end_slot >= Runtime::kSlots || !rt->slots[start_slot] || !rt->slots[end_slot]) {
    set_error("hrt_event_elapsed_ms: slot not recorded");
    return -1.f;
  }
  hipError_t e = hipEventSynchronize(rt->slots[end_slot]);
  float ms = -1.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, rt->slots[start_slot], rt->slots[end_slot]);
  if (e != hipSuccess) {
    hip_fail("hipEventElapsedTime", e);
    return -1.f;
  }
  return ms;
}

int hrt_graph_begin(void) {
  Runtime* rt = rt_or_error();
  if (!rt) return -1;
  std::lock_guard<std::mutex> l(rt->mu);
  if (rt->backing.capturing) {
    set_error("hrt_graph_begin: a graph is already being recorded");
    return -1;
  }
  if (!rt->pending.empty()) wait_pending(rt, 0, ~0ull);  // earlier uploads: waited for outside the graph
  hipError_t e = hipStreamBeginCapture(rt->stream, hipStreamCaptureModeRelaxed);
  if (e != hipSuccess) return hip_fail("hipStreamBeginCapture", e);
  rt->backing.capturing = true;
  rt->alloc->set_frozen(true);
  return 0;
}

int64_t hrt_graph_end(void) {
  Runtime* rt = rt_or_error();
  if (!rt) return -1;
  std::lock_guard<std::mutex> l(rt->mu);
  if (!rt->backing.capturing) {
    set_error("hrt_graph_end: no graph is being recorded");
    return -1;
  }
  rt->backing.capturing = false;
  rt->alloc->set_frozen(false);
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(rt->stream, &g);
  for (auto& f : rt->pinned_free)  // pinned blocks freed during the recording
    if (f.base && !f.after_compute) mark_freed(rt, f);
  if (e != hipSuccess) return hip_fail("hipStreamEndCapture", e);
  hipGraphExec_t x = nullptr;
  e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return hip_fail("hipGraphInstantiate", e);
  rt->graphs.push_back(x);
  return (int64_t)rt->graphs.size() - 1;
}

int hrt_graph_launch(int64_t graph) {
  Runtime* rt = rt_or_error();
  if (!rt) return -1;
  std::lock_guard<std::mutex> l(rt->mu);
  if (graph < 0 || graph >= (int64_t)rt->graphs.size() || !rt->graphs[graph]) {
    set_error("hrt_graph_launch: unknown graph id");
    return -1;
  }
  if (rt->backing.capturing) {
    set_error("hrt_graph_launch: not allowed while a graph is being recorded");
    return -1;
  }
  hipError_t e = hipGraphLaunch(rt->graphs[graph], rt->stream);
  if (e != hipSuccess) return hip_fail("hipGraphLaunch", e);
  return 0;
}

int hrt_graph_destroy(int64_t graph) {
  Runtime* rt = rt_or_error();
  if (!rt) return -1;
  std::lock_guard<std::mutex> l(rt->mu);
  if (graph < 0 || graph >= (int64_t)rt->graphs.size() || !rt->graphs[graph]) {
    set_error("hrt_graph_destroy: unknown graph id");
    return -1;
  }
  (void)hipStreamSynchronize(rt->stream);
  (void)hipGraphExecDestroy(rt->graphs[graph]);
  rt->graphs[graph] = nullptr;
  return 0;
}

}  // extern "C"
