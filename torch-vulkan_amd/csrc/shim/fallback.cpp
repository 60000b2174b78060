// Operator accounting and the boxed CPU fallback of the vk device.
//
// Behaviour (the reference's contract, csrc/shim.cpp:53-131): every aten operator without a vk kernel
// runs PyTorch's CPU kernel on host copies of its arguments and is counted under its operator name;
// with VKT_TRACE_FALLBACK set, each fallback prints its schema and the device/shape/dtype of its tensor
// arguments, flagging calls that mix vk tensors with non-scalar CPU tensors.  PyTorch's cpu_fallback puts
// results on the device of the first tensor argument, which for `1 - x` is the CPU scalar; here every
// CPU tensor result of a call that had a vk input is moved to vk, so CPU tensors never leak into a vk
// computation.
#include <chrono>
#include <iostream>
#include <map>
#include <mutex>

#include "common.h"

namespace vkt {

namespace {

struct Tally {
  int64_t gpu = 0, cpu = 0;
  uint64_t cpu_ns = 0;
};

class Ledger {
 public:
  void gpu(std::string_view op) {
    std::lock_guard<std::mutex> l(mu_);
    book_[std::string(op)].gpu += 1;
  }
  void cpu(std::string_view op, uint64_t ns) {
    std::lock_guard<std::mutex> l(mu_);
    Tally& t = book_[std::string(op)];
    t.cpu += 1;
    t.cpu_ns += ns;
  }
  template <typename F>
  auto select(F pick) {
    using V = decltype(pick(Tally{}));
    std::map<std::string, V> out;
    std::lock_guard<std::mutex> l(mu_);
    for (const auto& [op, t] : book_) {
      const V v = pick(t);
      if (v != V{}) out.emplace(op, v);
    }
    return out;
  }
  void clear_counts() {
    std::lock_guard<std::mutex> l(mu_);
    for (auto& kv : book_) kv.second.gpu = kv.second.cpu = 0;
  }

 private:
  std::mutex mu_;
  std::map<std::string, Tally> book_;
};

Ledger& ledger() {
  static Ledger l;
  return l;
}

// What the fallback needs to know about the arguments on the stack, gathered in one pass.
struct ArgScan {
  bool vk_input = false;         // a tensor (or tensor-list element) on vk
  bool cpu_nonscalar = false;    // a CPU tensor with at least one dimension
  std::string described;         // for VKT_TRACE_FALLBACK
};

ArgScan scan_arguments(const torch::jit::Stack& stack, size_t nargs, bool describe) {
  ArgScan s;
  auto visit = [&](const at::Tensor& t) {
    if (!t.defined()) return;
    const bool dev = on_vk(t);
    s.vk_input |= dev;
    s.cpu_nonscalar |= !dev && t.dim() > 0;
    if (describe) s.described += c10::str(' ', dev ? "vk" : "cpu", t.sizes(), t.scalar_type());
  };
  for (const c10::IValue& v : torch::jit::last(stack, nargs)) {
    if (v.isTensor()) {
      visit(v.toTensor());
    } else if (v.isTensorList()) {
      for (const at::Tensor& t : v.toTensorList()) visit(t);
    }
  }
  return s;
}

void move_results_to_vk(torch::jit::Stack& stack, size_t nret) {
  const c10::Device vk(kDev, 0);
  for (size_t i = stack.size() - nret; i < stack.size(); ++i) {
    c10::IValue& v = stack[i];
    if (v.isTensor()) {
      const at::Tensor& t = v.toTensor();
      if (t.defined() && !on_vk(t)) v = t.to(vk);
    } else if (v.isTensorList()) {
      c10::List<at::Tensor> list = v.toTensorList();
      for (size_t j = 0; j < list.size(); ++j) {
        const at::Tensor t = list.get(j);
        if (t.defined() && !on_vk(t)) list.set(j, t.to(vk));
      }
    }
  }
}

}  // namespace

void note_gpu(std::string_view op) { ledger().gpu(op); }
void note_cpu(std::string_view op, uint64_t ns) { ledger().cpu(op, ns); }

std::map<std::string, int64_t> gpu_counts() {
  return ledger().select([](const Tally& t) { return t.gpu; });
}
std::map<std::string, int64_t> cpu_counts() {
  return ledger().select([](const Tally& t) { return t.cpu; });
}
std::map<std::string, double> cpu_seconds_by_op() {
  return ledger().select([](const Tally& t) { return t.cpu_ns * 1e-9; });
}
void clear_counts() { ledger().clear_counts(); }

void cpu_fallback_boxed(const c10::OperatorHandle& op, torch::jit::Stack* stack) {
  const auto start = std::chrono::steady_clock::now();
  static const bool trace = std::getenv("VKT_TRACE_FALLBACK") != nullptr;
  const c10::FunctionSchema& schema = op.schema();
  const ArgScan args = scan_arguments(*stack, schema.arguments().size(), trace);
  if (trace) {
    std::cerr << "[vkt fallback] " << schema << "\n[vkt fallback-args]" << args.described << std::endl;
    if (args.vk_input && args.cpu_nonscalar)
      std::cerr << "[vkt MIXED-DEVICE] " << schema.operator_name() << ":" << args.described << std::endl;
  }
  at::native::cpu_fallback(op, stack);
  if (args.vk_input) move_results_to_vk(*stack, schema.returns().size());
  const auto ns = std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - start).count();
  note_cpu(schema.operator_name().name, static_cast<uint64_t>(ns));
}

}  // namespace vkt

TORCH_LIBRARY_IMPL(_, PrivateUse1, m) { m.fallback(torch::CppFunction::makeFromBoxedFunction<&vkt::cpu_fallback_boxed>()); }
