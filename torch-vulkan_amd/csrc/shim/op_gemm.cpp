// Matrix products on the vk device: aten::mm, bmm, addmm, baddbmm (the reference registers the same four,
// csrc/ops_mm.cpp:216-221, with the contract of :61-199: f32/bf16/f16 operands of one dtype, any
// non-negative strides read in place, bias broadcast, alpha/beta, a contiguous result; other calls run
// on the CPU).
//
// A call is planned as one product C[b] = alpha * A[b] @ B[b] + beta * bias[b] over [batch, M, N, K]:
// operands are described by their element strides (transposed and sliced views cost nothing), the bias by
// the strides of its broadcast to the output shape (PyTorch's own expand).  The plan then goes to one of
// three engines: the gfx950 matrix-core kernel "mm_mfma_*" (bf16/f16), the same kernel over split K
// ranges plus the ordered reduction "mm_reduce_*" (products one 64-wide tile across, e.g. rank-16 LoRA
// factors), or the FMA kernel "mm_*" (f32, and bf16/f16 when the matrix cores are switched off).
//
// Debug aids: set_coop_range / VKT_NO_COOP (the matrix-core gate below) and VKT_VERIFY_MM=1, which
// recomputes every matrix-core product with the FMA kernel and reports calls whose results disagree.
#include <atomic>
#include <cstdlib>
#include <iostream>
#include <mutex>

#include "common.h"

namespace {

using namespace vkt;

// ---- the matrix-core gate ----------------------------------------------------------------------------------
// enabled: VKT_NO_COOP unset, or set_coop_enabled(true).  Bisection window: matrix-core-eligible calls of
// the selected kind (0 all, 1 batched only, 2 unbatched only) are numbered from 0; only numbers in
// [lo, hi) use the matrix cores, the rest (and the other kind) the FMA kernel.
class MatrixCoreGate {
 public:
  bool admits(bool batched) {
    if (!enabled_.load(std::memory_order_relaxed)) return false;
    std::lock_guard<std::mutex> l(mu_);
    if ((kind_ == 1 && !batched) || (kind_ == 2 && batched)) return false;
    const uint64_t n = seq_++;
    return n >= lo_ && n < hi_;
  }
  void enable(bool on) { enabled_.store(on); }
  bool enabled() const { return enabled_.load(); }
  void window(uint64_t lo, uint64_t hi, int kind) {
    std::lock_guard<std::mutex> l(mu_);
    lo_ = lo, hi_ = hi, kind_ = kind;
  }
  void restart() {
    std::lock_guard<std::mutex> l(mu_);
    seq_ = 0;
  }
  uint64_t numbered() {
    std::lock_guard<std::mutex> l(mu_);
    return seq_;
  }

 private:
  std::atomic<bool> enabled_{std::getenv("VKT_NO_COOP") == nullptr};
  std::mutex mu_;
  uint64_t lo_ = 0, hi_ = ~uint64_t(0), seq_ = 0;
  int kind_ = 0;
};

MatrixCoreGate& gate() {
  static MatrixCoreGate g;
  return g;
}

// ---- planning -----------------------------------------------------------------------------------------------
struct Plan {
  at::ScalarType dt;
  bool batched;
  int64_t batch, M, N, K;
  hrt_mm_args args{};  // every field but the output address
};

// [batch, rows, cols] strides of a 2-D or 3-D operand (batch stride 0 when 2-D); nullopt if negative.
std::optional<std::array<int64_t, 3>> strides3(const at::Tensor& t) {
  const bool b3 = t.dim() == 3;
  std::array<int64_t, 3> s = {b3 ? t.stride(0) : 0, t.stride(b3 ? 1 : 0), t.stride(b3 ? 2 : 1)};
  for (int64_t v : s)
    if (v < 0) return std::nullopt;
  return s;
}

std::optional<Plan> plan(const at::Tensor& a, const at::Tensor& b, const at::Tensor* bias, double alpha, double beta) {
  if (!on_vk(a) || !on_vk(b) || a.dim() != b.dim() || (a.dim() != 2 && a.dim() != 3)) return std::nullopt;
  if (a.scalar_type() != b.scalar_type() || float_code(a.scalar_type()) < 0) return std::nullopt;
  Plan p{};
  p.dt = a.scalar_type();
  p.batched = a.dim() == 3;
  const int r = p.batched ? 1 : 0;
  p.batch = p.batched ? a.size(0) : 1;
  p.M = a.size(r), p.K = a.size(r + 1), p.N = b.size(r + 1);
  if (b.size(r) != p.K || (p.batched && b.size(0) != p.batch)) return std::nullopt;
  if (p.batch == 0 || p.M == 0 || p.N == 0 || p.K == 0) return std::nullopt;  // empty products: PyTorch's CPU semantics
  const auto sa = strides3(a), sb = strides3(b);
  if (!sa || !sb) return std::nullopt;
  hrt_mm_args& A = p.args;
  A.a = dptr(a), A.b = dptr(b);
  A.M = p.M, A.N = p.N, A.K = p.K, A.batch = p.batch;
  A.a_sb = (*sa)[0], A.a_sm = (*sa)[1], A.a_sk = (*sa)[2];
  A.b_sb = (*sb)[0], A.b_sk = (*sb)[1], A.b_sn = (*sb)[2];
  A.c_sb = p.M * p.N, A.c_sm = p.N, A.c_sn = 1;
  A.alpha = static_cast<float>(alpha);
  A.beta = static_cast<float>(beta);
  if (bias != nullptr && beta != 0.0) {
    if (!on_vk(*bias) || bias->scalar_type() != p.dt) return std::nullopt;
    const std::vector<int64_t> out = p.batched ? std::vector<int64_t>{p.batch, p.M, p.N} : std::vector<int64_t>{p.M, p.N};
    if (!at::is_expandable_to(bias->sizes(), out)) return std::nullopt;
    const auto sc = strides3(bias->expand(out));  // broadcast dimensions get stride 0
    if (!sc) return std::nullopt;
    A.bias = dptr(*bias);
    A.bias_sb = (*sc)[0], A.bias_sm = (*sc)[1], A.bias_sn = (*sc)[2];
    A.has_bias = 1;
  }
  return p;
}

// K-split factor of a matrix-core product (1 = no split; unbatched products only, the slices use the batch
// dimension; K in whole 64-element steps):
//  * products with an output side of at most 16 (a rank-16 LoRA's x A^T, g B, g^T h, dh^T x) run on the
//    narrow-output kernel, one workgroup per 16 rows of the long side P, K split across its wavefronts: S
//    doubles while the P / 16 workgroups times S stay under 256 and every slice keeps >= 1536 of K.  Only
//    long reductions over few rows repay the second launch: measured at 1024 rows, K = 8192 takes 9.1 us
//    at S = 4 against 16.3 unsplit, K = 6144 8.2 against 9.0, but K = 2048 5.8 unsplit against 6.7-7.5.
//  * other narrow products, one 64-wide output tile across (min(M, N) <= 64: rank-16 LoRA factors): S doubles
//    while the grid of 64 x 64 tiles stays within one workgroup per CU (256) and every slice keeps >= 128
//    of K;
//  * wide products whose 128 x 256 (or 256 x 128) tiles alone give fewer than 192 workgroups (1024 x 2048
//    outputs: 64), which would otherwise fall to 64 x 64 tiles that copy three times the bytes per flop:
//    S doubles until S x tiles >= 192, keeping >= 1536 of K per slice; the slices then run on the large
//    tiles.  The fp32 partials cost a write and a read of S x M x N x 4 bytes (32 MB at 1024 x 2048, S = 4),
//    which only long slices repay: measured at 1024 x 2048 outputs, S = 4 takes 51-52 us against 58-65 at
//    K = 8192 and 44 against 47 at K = 6144, but 29.5 against 17-19 at K = 2048 (S = 2 loses everywhere:
//    128 large tiles are too few).  S stays 1 when no split reaches 192 workgroups.
int64_t k_splits(const Plan& p) {
  if (p.batched || p.K % 64 != 0) return 1;
  int64_t s = 1;
  if (std::min(p.M, p.N) <= 16) {
    const int64_t tiles = ((p.N <= 16 ? p.M : p.N) + 15) / 16;
    while (tiles * s < 256 && p.K % (64 * 2 * s) == 0 && p.K / (2 * s) >= 1536) s *= 2;
    return s;
  }
  if (std::min(p.M, p.N) <= 64) {
    const int64_t tiles = ((p.M + 63) / 64) * ((p.N + 63) / 64), steps = p.K / 64;
    while (tiles * (2 * s) <= 256 && steps % (2 * s) == 0 && p.K / (2 * s) >= 128) s *= 2;
    return s;
  }
  const int64_t wide = (p.M % 128 == 0 && p.N % 256 == 0) ? (p.M / 128) * (p.N / 256) : 0;
  const int64_t tall = (p.M % 256 == 0 && p.N % 128 == 0) ? (p.M / 256) * (p.N / 128) : 0;
  const int64_t tiles = std::max(wide, tall);
  if (tiles == 0 || tiles >= 192) return 1;
  while (tiles * s < 192 && p.K % (64 * 2 * s) == 0 && p.K / (2 * s) >= 1536) s *= 2;
  return tiles * s >= 192 ? s : 1;
}

// The split product: slice s of K goes to batch entry s of the matrix-core kernel, which writes unrounded
// fp32 partials [S, M, N]; "mm_reduce_*" adds them in order s = 0, 1, ... (deterministic), applies alpha
// and beta * bias and rounds once into out.
void run_split(const Plan& p, int64_t S, const at::Tensor& out) {
  const at::Tensor partial = at::empty({S, p.M, p.N}, out.options().dtype(at::kFloat));
  hrt_mm_args A = p.args;
  A.K = p.K / S;
  A.batch = S;
  A.a_sb = A.K * A.a_sk;
  A.b_sb = A.K * A.b_sk;
  A.c = dptr(partial);
  A.alpha = 1.f, A.beta = 0.f;
  A.bias = 0, A.has_bias = 0, A.bias_sb = A.bias_sm = A.bias_sn = 0;
  A.flags = HRT_MM_F32_OUT;
  hrt_mm_reduce_args R{};
  R.ws = dptr(partial), R.c = dptr(out), R.bias = p.args.bias;
  R.M = p.M, R.N = p.N, R.splits = S;
  R.c_sm = p.N, R.c_sn = 1;
  R.bias_sm = p.args.bias_sm, R.bias_sn = p.args.bias_sn;
  R.alpha = p.args.alpha, R.beta = p.args.beta, R.has_bias = p.args.has_bias;
  queue(typed("mm_mfma", p.dt), A);
  queue(typed("mm_reduce", p.dt), R);
}

// VKT_VERIFY_MM=1: the FMA kernel recomputes a matrix-core product and the call is reported when more
// than 1% of its elements differ from it by more than 3 ulps of the output dtype, measured at
// max(|ref|, 1e-3 of the largest |ref|).  Both results are rounded once from fp32 sums taken in different
// orders, so a few ulps of difference are normal; an indexing or layout error shows as a large fraction.
void verify_with_fma(const Plan& p, const at::Tensor& out) {
  static std::atomic<int64_t> calls{0}, bad{0};
  at::Tensor ref = at::empty_like(out);
  hrt_mm_args A = p.args;
  A.c = dptr(ref);
  queue(typed("mm", p.dt), A);
  const at::Tensor r = ref.cpu().to(at::kFloat), o = out.cpu().to(at::kFloat);
  const double ulp = p.dt == at::kBFloat16 ? 1.0 / 128 : 1.0 / 1024;  // spacing relative to the value
  const double floor = 1e-3 * r.abs().max().item<double>();
  const double frac = ((o - r).abs() > r.abs().clamp_min(floor) * (3 * ulp)).to(at::kFloat).mean().item<double>();
  const int64_t n = ++calls;
  if (frac > 1e-2) {
    const int64_t nb = ++bad;
    std::cerr << "[vkt VERIFY-MM] " << nb << " of " << n << " checked calls differ: fraction " << frac << " at batch "
              << p.batch << " M " << p.M << " N " << p.N << " K " << p.K << " strides a (" << p.args.a_sb << ","
              << p.args.a_sm << "," << p.args.a_sk << ") b (" << p.args.b_sb << "," << p.args.b_sk << "," << p.args.b_sn
              << ") " << dtype_suffix(p.dt) << std::endl;
  }
}

std::optional<at::Tensor> try_product(const at::Tensor& a, const at::Tensor& b, const at::Tensor* bias, double alpha,
                                      double beta, const char* op) {
  std::optional<Plan> p = plan(a, b, bias, alpha, beta);
  if (!p) return std::nullopt;
  at::Tensor out = p->batched ? at::empty({p->batch, p->M, p->N}, a.options()) : at::empty({p->M, p->N}, a.options());
  const bool matrix_cores = p->dt != at::kFloat && gate().admits(p->batched);
  const int64_t S = matrix_cores ? k_splits(*p) : 1;
  if (S > 1) {
    run_split(*p, S, out);
  } else {
    hrt_mm_args A = p->args;
    A.c = dptr(out);
    queue(typed(matrix_cores ? "mm_mfma" : "mm", p->dt), A);
  }
  static const bool verify = std::getenv("VKT_VERIFY_MM") != nullptr;
  if (verify && matrix_cores) verify_with_fma(*p, out);
  note_gpu(op);
  return out;
}

at::Tensor k_mm(const at::Tensor& a, const at::Tensor& b) {
  if (auto r = try_product(a, b, nullptr, 1.0, 0.0, "aten::mm")) return *r;
  return VKT_CPU(mm, a, b);
}

at::Tensor k_bmm(const at::Tensor& a, const at::Tensor& b) {
  if (auto r = try_product(a, b, nullptr, 1.0, 0.0, "aten::bmm")) return *r;
  return VKT_CPU(bmm, a, b);
}

// addmm takes 2-D factors and baddbmm 3-D ones; the other rank goes to the CPU as PyTorch would reject it.
at::Tensor k_addmm(const at::Tensor& self, const at::Tensor& a, const at::Tensor& b, const at::Scalar& beta,
                   const at::Scalar& alpha) {
  std::optional<at::Tensor> r;
  if (a.dim() == 2) r = try_product(a, b, &self, alpha.toDouble(), beta.toDouble(), "aten::addmm");
  return r ? *r : VKT_CPU(addmm, self, a, b, beta, alpha);
}

at::Tensor k_baddbmm(const at::Tensor& self, const at::Tensor& a, const at::Tensor& b, const at::Scalar& beta,
                     const at::Scalar& alpha) {
  std::optional<at::Tensor> r;
  if (a.dim() == 3) r = try_product(a, b, &self, alpha.toDouble(), beta.toDouble(), "aten::baddbmm");
  return r ? *r : VKT_CPU(baddbmm, self, a, b, beta, alpha);
}

}  // namespace

namespace vkt {
void set_coop_enabled(bool on) { gate().enable(on); }
bool coop_is_enabled() { return gate().enabled(); }
uint32_t coop_caps() {
  runtime();
  return hrt_coop_caps();
}
void set_coop_range(uint64_t lo, uint64_t hi, int kind) { gate().window(lo, hi, kind); }
void reset_coop_calls() { gate().restart(); }
uint64_t coop_calls() { return gate().numbered(); }
}  // namespace vkt

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("mm", &k_mm);
  m.impl("bmm", &k_bmm);
  m.impl("addmm", &k_addmm);
  m.impl("baddbmm", &k_baddbmm);
}
