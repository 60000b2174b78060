// mm / bmm / addmm / baddbmm on the vk device (reference: csrc/ops_mm.cpp:1-221).
// Transposed and sliced operands are read in place through their strides (no copies); bias broadcasts
// through stride 0.  bf16/f16 go to the gfx950 matrix-core kernel "mm_mfma_*" unless matrix cores are
// switched off (set_coop_enabled(False) / VKT_NO_COOP), f32 and the switched-off case go to the FMA
// kernel "mm_*".  Anything else (mixed dtypes, empty K, ...) falls back to the CPU like the reference.
#include <ATen/Operators.h>

#include <atomic>
#include <cstdlib>
#include <optional>
#include <string>
#include <vector>

#include "common.h"

namespace {

using namespace vkt;

std::atomic<bool>& coop_flag() {
  static std::atomic<bool> v{std::getenv("VKT_NO_COOP") == nullptr};
  return v;
}

// Debug bisection of matrix-core calls (csrc/ops_mm.cpp:36-39): only calls numbered [lo, hi) use the
// matrix-core kernel; kind 0 = all, 1 = bmm only, 2 = mm only.
std::atomic<uint64_t> g_coop_calls{0}, g_coop_lo{0}, g_coop_hi{~uint64_t(0)};
std::atomic<int> g_coop_kind{0};

std::optional<at::Tensor> try_gemm(const at::Tensor& a, const at::Tensor& b, const at::Tensor* bias, double alpha, double beta,
                                   const char* aten_name) {
  if (!is_vk(a) || !is_vk(b) || a.scalar_type() != b.scalar_type() || a.dim() != b.dim()) return std::nullopt;
  const char* kind = kind_name(a.scalar_type());
  if (!kind) return std::nullopt;
  const bool batched = a.dim() == 3;
  if (!batched && a.dim() != 2) return std::nullopt;
  const int off = batched ? 1 : 0;
  const int64_t batch = batched ? a.size(0) : 1;
  const int64_t M = a.size(off), K = a.size(off + 1), N = b.size(off + 1);
  if ((batched && b.size(0) != batch) || b.size(off) != K) return std::nullopt;
  if (M == 0 || N == 0 || K == 0 || batch == 0) return std::nullopt;

  hrt_mm_args P{};
  P.a_sb = batched ? a.stride(0) : 0;
  P.a_sm = a.stride(off);
  P.a_sk = a.stride(off + 1);
  P.b_sb = batched ? b.stride(0) : 0;
  P.b_sk = b.stride(off);
  P.b_sn = b.stride(off + 1);
  if (P.a_sb < 0 || P.a_sm < 0 || P.a_sk < 0 || P.b_sb < 0 || P.b_sk < 0 || P.b_sn < 0) return std::nullopt;
  const bool use_bias = bias != nullptr && beta != 0.0;
  if (use_bias) {
    if (!is_vk(*bias) || bias->scalar_type() != a.scalar_type()) return std::nullopt;
    // strides of bias broadcast to (batch, M, N)  (csrc/ops_mm.cpp:80-99)
    std::vector<int64_t> full = batched ? std::vector<int64_t>{batch, M, N} : std::vector<int64_t>{M, N};
    if ((int)bias->dim() > (int)full.size()) return std::nullopt;
    std::vector<int64_t> st(full.size(), 0);
    for (size_t i = 0; i < full.size(); ++i) {
      int j = (int)i - ((int)full.size() - (int)bias->dim());
      if (j < 0) continue;
      if (bias->size(j) == full[i])
        st[i] = bias->stride(j);
      else if (bias->size(j) == 1)
        st[i] = 0;
      else
        return std::nullopt;
      if (st[i] < 0) return std::nullopt;
    }
    P.bias = addr_of(*bias);
    P.bias_sb = batched ? st[0] : 0;
    P.bias_sm = st[off];
    P.bias_sn = st[off + 1];
  }
  at::Tensor out = batched ? at::empty({batch, M, N}, a.options()) : at::empty({M, N}, a.options());
  P.a = addr_of(a);
  P.b = addr_of(b);
  P.c = addr_of(out);
  P.M = M;
  P.N = N;
  P.K = K;
  P.batch = batch;
  P.c_sb = M * N;
  P.c_sm = N;
  P.c_sn = 1;
  P.alpha = (float)alpha;
  P.beta = (float)beta;
  P.has_bias = use_bias ? 1u : 0u;

  bool use_mfma = false;
  if (coop_flag().load() && (a.scalar_type() == at::kBFloat16 || a.scalar_type() == at::kHalf)) {
    const int kf = g_coop_kind.load();
    use_mfma = !((kf == 1 && !batched) || (kf == 2 && batched));
    if (use_mfma) {
      const uint64_t idx = g_coop_calls.fetch_add(1);
      use_mfma = idx >= g_coop_lo.load() && idx < g_coop_hi.load();
    }
  }
  // Split-K for products one 64-wide tile across (the rank-16 LoRA factors: M or N = 16 with K = 1024 .. 8192
  // run on 16 - 128 workgroups otherwise; wider products keep one K order, so that e.g. the fused int8 linear
  // stays bit-identical to dequant + mm): the K range is split over the batch
  // dimension of the matrix-core kernel, which writes fp32 partial products into a workspace, and
  // "mm_reduce_*" sums the splits in order (deterministic), applies alpha / beta * bias and rounds once.
  if (use_mfma && !batched && K % 64 == 0 && std::min(M, N) <= 64) {
    const int64_t tiles = ((M + 63) / 64) * ((N + 63) / 64);
    const int64_t kblocks = K / 64;
    int64_t S = 1;
    // up to one workgroup per CU, K slices of at least 128 (more splits measured slower: every split adds a
    // workgroup prologue and an fp32 partial of the output)
    while (tiles * S * 2 <= 256 && kblocks % (S * 2) == 0 && K / (S * 2) >= 128) S *= 2;
    if (S >= 2) {
      at::Tensor ws = at::empty({S, M, N}, a.options().dtype(at::kFloat));
      hrt_mm_reduce_args R{};
      R.ws = addr_of(ws);
      R.c = P.c;
      R.bias = P.bias;
      R.M = M;
      R.N = N;
      R.splits = S;
      R.c_sm = N;
      R.c_sn = 1;
      R.bias_sm = P.bias_sm;
      R.bias_sn = P.bias_sn;
      R.alpha = P.alpha;
      R.beta = P.beta;
      R.has_bias = P.has_bias;
      P.K = K / S;
      P.batch = S;
      P.a_sb = P.K * P.a_sk;
      P.b_sb = P.K * P.b_sk;
      P.c = R.ws;
      P.c_sb = M * N;
      P.has_bias = 0;
      P.bias = 0;
      P.bias_sm = P.bias_sn = 0;
      P.alpha = 1.f;
      P.beta = 0.f;
      P.flags = HRT_MM_F32_OUT;
      launch(std::string("mm_mfma_") + kind, P);
      launch(std::string("mm_reduce_") + kind, R);
      count_kernel(aten_name);
      return out;
    }
  }
  launch(std::string(use_mfma ? "mm_mfma_" : "mm_") + kind, P);
  count_kernel(aten_name);
  return out;
}

at::Tensor k_mm(const at::Tensor& a, const at::Tensor& b) {
  if (auto r = try_gemm(a, b, nullptr, 1.0, 0.0, "aten::mm")) return *r;
  return VKT_FALLBACK(mm, a, b);
}

at::Tensor k_bmm(const at::Tensor& a, const at::Tensor& b) {
  if (auto r = try_gemm(a, b, nullptr, 1.0, 0.0, "aten::bmm")) return *r;
  return VKT_FALLBACK(bmm, a, b);
}

at::Tensor k_addmm(const at::Tensor& self, const at::Tensor& a, const at::Tensor& b, const at::Scalar& beta, const at::Scalar& alpha) {
  if (a.dim() == 2)
    if (auto r = try_gemm(a, b, &self, alpha.toDouble(), beta.toDouble(), "aten::addmm")) return *r;
  return VKT_FALLBACK(addmm, self, a, b, beta, alpha);
}

at::Tensor k_baddbmm(const at::Tensor& self, const at::Tensor& a, const at::Tensor& b, const at::Scalar& beta,
                     const at::Scalar& alpha) {
  if (a.dim() == 3)
    if (auto r = try_gemm(a, b, &self, alpha.toDouble(), beta.toDouble(), "aten::baddbmm")) return *r;
  return VKT_FALLBACK(baddbmm, self, a, b, beta, alpha);
}

}  // namespace

namespace vkt {
void set_coop_enabled(bool on) { coop_flag().store(on); }
bool coop_is_enabled() { return coop_flag().load(); }
uint32_t coop_caps() {
  static uint32_t caps = [] {
    ensure_init();
    return hrt_coop_caps();
  }();
  return caps;
}
void set_coop_range(uint64_t lo, uint64_t hi, int kind) {
  g_coop_lo.store(lo);
  g_coop_hi.store(hi);
  g_coop_kind.store(kind);
}
void reset_coop_calls() { g_coop_calls.store(0); }
uint64_t coop_calls() { return g_coop_calls.load(); }
}  // namespace vkt

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("mm", &k_mm);
  m.impl("bmm", &k_bmm);
  m.impl("addmm", &k_addmm);
  m.impl("baddbmm", &k_baddbmm);
}
