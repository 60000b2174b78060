// Python module torch_vulkan_C: what torch_vulkan/__init__.py builds the public API from (the
// reference's pybind surface, csrc/shim.cpp:418-493, plus the pinned-memory, event and fused-linear
// additions).  Runtime queries are bound through `ready<...>`, which initialises the runtime before the
// call.  `stats()` returns the reference's statistics dictionary (same keys and units); Python's
// torch_vulkan.stats() assembles the same dictionary from `runtime_counters()`.
#include <torch/extension.h>

#include <map>
#include <tuple>
#include <vector>

#include "common.h"
#include "device.h"

namespace vkt {
std::map<std::string, int64_t> gpu_counts();
std::map<std::string, int64_t> cpu_counts();
std::map<std::string, double> cpu_seconds_by_op();
void clear_counts();
}  // namespace vkt

namespace {

using namespace vkt;

// A zero-argument C-ABI query or action, with the runtime initialised first.
template <auto Fn>
auto ready() {
  return [] {
    runtime();
    return Fn();
  };
}

std::string text_of(size_t (*fn)(char*, size_t)) {
  std::string s(256, '\0');
  size_t n = fn(s.data(), s.size());
  if (n >= s.size()) {  // the full length is returned: fetch again with room for all of it
    s.assign(n + 1, '\0');
    n = fn(s.data(), s.size());
  }
  s.resize(std::min(n, s.size() - 1));
  return s;
}

at::Tensor pinned_empty(const std::vector<int64_t>& sizes, at::ScalarType dtype) {
  runtime();
  at::globalContext().lazyInitDevice(kDev);  // PyTorch answers is_pinned() only for initialised accelerators
  return at::detail::empty_generic(sizes, pinned_allocator(), c10::DispatchKeySet(c10::DispatchKey::CPU), dtype,
                                   std::nullopt);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("init", &runtime);
  // device and memory
  m.def("device_name", [] {
    runtime();
    return text_of(&hrt_device_name);
  });
  m.def("max_alloc", ready<&hrt_max_alloc>());
  m.def("live_bytes", ready<&hrt_live_bytes>());
  m.def("peak_live_bytes", ready<&hrt_peak_live_bytes>());
  m.def("reset_peak_live_bytes", ready<&hrt_reset_peak_live_bytes>());
  m.def("reserved_bytes", ready<&hrt_reserved_bytes>());
  m.def("live_blocks", ready<&hrt_live_blocks>());
  m.def("slab_count", ready<&hrt_slab_count>());
  m.def("empty_cache", ready<&hrt_empty_cache>());
  m.def("coop_caps", &vkt::coop_caps);
  m.def("validation_errors", &hrt_validation_errors);
  m.def("memory_info", [] {
    runtime();
    uint64_t v[3] = {};
    expect_ok(hrt_memory_info(v), "memory_info");
    return std::make_tuple(v[0], v[1], v[2]);  // budget, usage, heap
  });
  m.def("set_memory_limit", [](uint64_t bytes) {
    runtime();
    hrt_set_memory_limit(bytes);
  });
  m.def("synchronize", [] {
    runtime();
    expect_ok(hrt_synchronize(), "synchronize");
  });
  m.def("empty_pinned", &pinned_empty);
  m.def("is_pinned", [](const at::Tensor& t) { return t.device().is_cpu() && t.numel() > 0 && hrt_host_is_pinned(t.data_ptr()) == 1; });
  // operators without an aten schema
  m.def("dequant_int8", [](const at::Tensor& q, const at::Tensor& s, at::ScalarType dt) {
    runtime();
    return dequant_int8_vk(q, s, dt);
  });
  m.def("dequant_int8_linear",
        [](const at::Tensor& x, const at::Tensor& q, const at::Tensor& s, const std::optional<at::Tensor>& bias) {
          runtime();
          return dequant_int8_linear_vk(x, q, s, bias);
        });
  // accounting and profiling
  m.def("kernel_counts", &gpu_counts);
  m.def("fallback_counts", &cpu_counts);
  m.def("fallback_time_by_op", &cpu_seconds_by_op);
  m.def("reset_counts", &clear_counts);
  m.def("runtime_counters", [] {
    runtime();
    std::vector<uint64_t> c;
    for (uint32_t i = 0; i < 8; ++i) c.push_back(hrt_stat(i));  // the order documented at hrt_stat
    return c;
  });
  m.def("stats", [] {
    runtime();
    // (key, hrt_stat index, unit scale): nanoseconds to seconds, bytes to MiB, counts as they are
    static const std::tuple<const char*, uint32_t, double> keys[] = {
        {"dispatch_s", 0, 1e-9},        {"dispatch_n", 1, 1.0},          {"transfer_s", 2, 1e-9},
        {"transfer_n", 3, 1.0},         {"pipeline_create_s", 4, 1e-9},  {"upload_MB", 5, 1.0 / 1048576.0},
        {"download_MB", 6, 1.0 / 1048576.0}, {"gpu_wait_s", 7, 1e-9}};
    std::map<std::string, double> r;
    for (const auto& [key, i, unit] : keys) r[key] = static_cast<double>(hrt_stat(i)) * unit;
    double fb = 0.0;
    for (const auto& kv : cpu_seconds_by_op()) fb += kv.second;
    r["fallback_s"] = fb;
    return r;
  });
  m.def("profile", [] {
    runtime();
    return text_of(&hrt_profile_dump);
  });
  m.def("event_record", [](uint32_t slot) {
    runtime();
    expect_ok(hrt_event_record(slot), "event_record");
  });
  m.def("event_elapsed_ms", [](uint32_t a, uint32_t b) {
    const float ms = hrt_event_elapsed_ms(a, b);
    if (ms < 0.f) TORCH_CHECK(false, "vk: event timing: ", runtime_error_text());
    return ms;
  });
  // switches
  m.def("set_coop_enabled", &vkt::set_coop_enabled);
  m.def("set_coop_range", &vkt::set_coop_range);
  m.def("reset_coop_calls", &vkt::reset_coop_calls);
  m.def("coop_calls", &vkt::coop_calls);
  m.def("set_fused_attention", &vkt::set_fused_attention);
}
