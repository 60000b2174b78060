// Fused scaled-dot-product attention on the vk device.
//
// PyTorch route (the reference's, csrc/ops_attn.cpp:297-310): the PrivateUse1 `_fused_sdp_choice_stub`
// answers `overrideable` for calls the kernels take and the policy wants, so F.scaled_dot_product_attention
// lands in `_scaled_dot_product_fused_attention_overrideable` and autograd calls its `_backward`; any other
// call takes PyTorch's math path (bmm + softmax on vk).
//
// Taken: 4-D q/k/v [B, H, S, D] of one float dtype on vk, D <= 128, equal B and H, k and v of one length, no
// mask, dropout, causal mask or GQA.  Views are read in place through their (batch, head, seq) strides; only
// a non-unit stride along D costs a copy.  bf16/f16 run the gfx950 matrix-core kernels ("attn_*_mfma_*"),
// f32 (and bf16/f16 with the matrix cores switched off) the FMA kernels ("attn_*_fma_*").
//
// Outputs follow PyTorch's own SDPA: [B, S, H, D]-contiguous memory returned as a [B, H, S, D] view; the
// fp32 logsumexp is [B, H, Sq].  The backward's delta = rowsum(O * dO) is taken from the stored O.  The
// reference keeps an unrounded fp32 copy of O for it, handed over in the `philox_offset` slot
// (csrc/ops_attn.cpp:178-186, 240-248); measured on every parity shape, delta from the bf16 / f16 O moves
// the gradients' rel-L2 against the float64 oracle by at most 3e-4 of 1e-2 (bf16) and 4e-5 of 4e-3 (f16),
// while the copy costs 8 MiB of writes in the forward and 8 MiB of reads in the backward at
// B1 H16 S1024 D128, so the forward writes none.  A backward that is handed an fp32 O in that slot still
// uses it.
#include <ATen/SDPBackend.h>
#include <ATen/native/transformers/attention.h>

#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "common.h"

namespace {

using namespace vkt;

// ---- policy -----------------------------------------------------------------------------------------------
// 0 = never, 1 = whenever the kernels take the call, 2 = auto: always for the matrix-core dtypes, and for
// f32 only when the score matrix the math path would materialise is >= 256 MiB.  Environment at first
// use: VKT_NO_FUSED_ATTN set to anything but "0" means never; VKT_FUSED_ATTN "0" never, other values
// always; neither set: auto.
int initial_mode() {
  auto set = [](const char* v) { return v != nullptr && v[0] != '\0'; };
  const char* off = std::getenv("VKT_NO_FUSED_ATTN");
  if (set(off) && std::strcmp(off, "0") != 0) return 0;
  const char* on = std::getenv("VKT_FUSED_ATTN");
  if (!set(on)) return 2;
  return on[0] == '0' ? 0 : 1;
}

std::atomic<int>& mode() {
  static std::atomic<int> m{initial_mode()};
  return m;
}

bool matrix_cores(at::ScalarType t) { return coop_is_enabled() && (t == at::kBFloat16 || t == at::kHalf); }

struct Dims {
  int64_t B, H, Sq, Sk, D;
};

// The attention shapes the kernels take (sizes only; masks and flags are checked separately).
std::optional<Dims> kernel_dims(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v) {
  for (const at::Tensor* t : {&q, &k, &v})
    if (!on_vk(*t) || t->dim() != 4 || t->scalar_type() != q.scalar_type()) return std::nullopt;
  if (float_code(q.scalar_type()) < 0) return std::nullopt;
  const Dims d{q.size(0), q.size(1), q.size(2), k.size(2), q.size(3)};
  if (d.B < 1 || d.H < 1 || d.Sq < 1 || d.Sk < 1 || d.D < 1 || d.D > 128) return std::nullopt;
  const std::array<int64_t, 3> bhd = {d.B, d.H, d.D};
  for (const at::Tensor* t : {&k, &v})
    if (std::array<int64_t, 3>{t->size(0), t->size(1), t->size(3)} != bhd) return std::nullopt;
  if (v.size(2) != d.Sk) return std::nullopt;
  constexpr int64_t lim = int64_t(1) << 31;  // the kernels index rows and (batch, head) pairs in 32 bits
  if (d.B * d.H >= lim || d.Sq >= lim || d.Sk >= lim) return std::nullopt;
  return d;
}

bool wanted(const Dims& d, at::ScalarType t) {
  switch (mode().load()) {
    case 0: return false;
    case 1: return true;
    default: return matrix_cores(t) || 4.0 * d.B * d.H * d.Sq * d.Sk >= 256.0 * (1 << 20);
  }
}

// The kernels take a positive, finite scale (their running maxima and the backward's exp2 forms scale the
// logits after the max); any other scale goes to the math path.
bool fused_ok(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, bool has_mask, double dropout_p,
              bool is_causal, bool gqa, std::optional<double> scale) {
  if (has_mask || dropout_p != 0.0 || is_causal || gqa) return false;
  if (scale && !(*scale > 0.0 && std::isfinite(*scale))) return false;
  const std::optional<Dims> d = kernel_dims(q, k, v);
  return d && wanted(*d, q.scalar_type());
}

int64_t sdp_choice(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const std::optional<at::Tensor>& mask,
                   double dropout_p, bool is_causal, std::optional<double> scale, bool enable_gqa) {
  const bool fused = fused_ok(q, k, v, present(mask), dropout_p, is_causal, enable_gqa, scale);
  return static_cast<int64_t>(fused ? at::SDPBackend::overrideable : at::SDPBackend::math);
}

// ---- launches -------------------------------------------------------------------------------------------------
at::Tensor unit_d(const at::Tensor& t) { return t.stride(3) == 1 ? t : t.contiguous(); }

// [B, S, H, D] memory viewed as [B, H, S, D].
at::Tensor bshd(const Dims& d, int64_t S, const at::TensorOptions& o) { return at::empty({d.B, S, d.H, d.D}, o).transpose(1, 2); }

void put_operand(int64_t* s3, uint64_t* addr, const at::Tensor& t) {
  *addr = dptr(t);
  s3[0] = t.stride(0), s3[1] = t.stride(1), s3[2] = t.stride(2);
}

hrt_attn_args base_args(const Dims& d, const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                        std::optional<double> scale) {
  hrt_attn_args A{};
  put_operand(&A.q_sb, &A.q, q);
  put_operand(&A.k_sb, &A.k, k);
  put_operand(&A.v_sb, &A.v, v);
  A.B = static_cast<int32_t>(d.B), A.H = static_cast<int32_t>(d.H);
  A.Sq = static_cast<int32_t>(d.Sq), A.Sk = static_cast<int32_t>(d.Sk), A.D = static_cast<int32_t>(d.D);
  A.scale = static_cast<float>(scale.value_or(1.0 / std::sqrt(static_cast<double>(d.D))));
  return A;
}

std::string attn_kernel(const char* op, at::ScalarType t) {
  return typed(std::string("attn_") + op + (matrix_cores(t) ? "_mfma" : "_fma"), t);
}

constexpr const char* kFwdOp = "aten::_scaled_dot_product_fused_attention_overrideable";
constexpr const char* kBwdOp = "aten::_scaled_dot_product_fused_attention_overrideable_backward";

using FwdOut = std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, c10::SymInt, c10::SymInt, at::Tensor, at::Tensor,
                          at::Tensor>;

FwdOut k_sdpa_fwd(const at::Tensor& query, const at::Tensor& key, const at::Tensor& value,
                  const std::optional<at::Tensor>& attn_bias, double dropout_p, bool is_causal, bool /*return_debug_mask*/,
                  std::optional<double> scale) {
  TORCH_CHECK(fused_ok(query, key, value, present(attn_bias), dropout_p, is_causal, false, scale),
              "vk: the fused attention kernels do not take this call");
  runtime();
  const at::Tensor q = unit_d(query), k = unit_d(key), v = unit_d(value);
  const Dims d = *kernel_dims(q, k, v);
  const at::ScalarType dt = q.scalar_type();
  const at::Tensor out = bshd(d, d.Sq, q.options());
  const at::Tensor lse = at::empty({d.B, d.H, d.Sq}, q.options().dtype(at::kFloat));
  hrt_attn_args A = base_args(d, q, k, v, scale);
  A.o = dptr(out);
  A.lse = dptr(lse);
  queue(attn_kernel("fwd", dt), A);
  note_gpu(kFwdOp);
  const at::Tensor none = at::empty({0}, at::TensorOptions().dtype(at::kLong));
  return FwdOut{out, lse, none, none, c10::SymInt(d.Sq), c10::SymInt(d.Sk), none, none,
                at::empty({0}, at::TensorOptions().dtype(dt))};
}

// The forward's fp32 O when it is usable for delta: fp32, on vk, [B, Sq, H, D]-contiguous.
bool usable_o32(const at::Tensor& t, const Dims& d, at::ScalarType dt) {
  return dt != at::kFloat && t.defined() && on_vk(t) && t.scalar_type() == at::kFloat && t.is_contiguous() &&
         t.numel() == d.B * d.Sq * d.H * d.D;
}

using BwdOut = std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor>;

BwdOut k_sdpa_bwd(const at::Tensor& grad_out, const at::Tensor& query, const at::Tensor& key, const at::Tensor& value,
                  const at::Tensor& attn_bias, std::array<bool, 4> need, const at::Tensor& out, const at::Tensor& logsumexp,
                  const at::Tensor&, const at::Tensor&, c10::SymInt, c10::SymInt, double dropout_p, bool is_causal,
                  const at::Tensor&, const at::Tensor& o32, std::optional<double> scale) {
  TORCH_CHECK(fused_ok(query, key, value, attn_bias.defined(), dropout_p, is_causal, false, scale) && on_vk(grad_out) &&
                  on_vk(out) && on_vk(logsumexp),
              "vk: the fused attention kernels do not take this backward call");
  runtime();
  const at::Tensor q = unit_d(query), k = unit_d(key), v = unit_d(value);
  const Dims d = *kernel_dims(q, k, v);
  const at::ScalarType dt = q.scalar_type();
  const at::Tensor dout = unit_d(grad_out.scalar_type() == dt ? grad_out : grad_out.to(dt));
  const at::Tensor lse = dense(logsumexp);
  const at::Tensor delta = at::empty({d.B, d.H, d.Sq}, q.options().dtype(at::kFloat));

  hrt_attn_args A = base_args(d, q, k, v, scale);
  A.lse = dptr(lse);
  A.delta = dptr(delta);
  put_operand(&A.do_sb, &A.dout, dout);
  at::Tensor o_rows;  // keeps a [B, Sq, H, D] copy of the output alive when the fp32 one is missing
  if (usable_o32(o32, d, dt)) {
    A.o = dptr(o32);
    A.flags = HRT_ATTN_O_F32;
  } else {
    o_rows = (out.scalar_type() == dt ? out : out.to(dt)).transpose(1, 2).contiguous();
    A.o = dptr(o_rows);
  }

  // Gradients take their input's layout when q, k and v are all dense (autograd then keeps them as they
  // are; a [B, S, H, D] gradient of a [B, H, S, D]-contiguous leaf would be copied into the leaf's layout),
  // else [B, S, H, D]-contiguous memory viewed as [B, H, S, D].
  const bool like_input = q.is_non_overlapping_and_dense() && k.is_non_overlapping_and_dense() &&
                          v.is_non_overlapping_and_dense();
  auto grad_for = [&](const at::Tensor& in, int64_t S) {
    return like_input ? at::empty_strided(in.sizes(), in.strides(), in.options()) : bshd(d, S, in.options());
  };
  if (like_input) A.flags |= HRT_ATTN_GRAD_LIKE_INPUT;

  // Order: delta (inside the matrix-core dQ kernel, HRT_ATTN_DQ_DELTA, or as its own pass), dQ, dK/dV.
  const bool fold_delta = need[0] && matrix_cores(dt);
  if (!fold_delta) {
    queue(typed("attn_delta", dt), A);
    note_gpu(kBwdOp);
  }
  at::Tensor dq, dk, dv;
  if (need[0]) {
    dq = grad_for(q, d.Sq);
    hrt_attn_args Q = A;
    Q.dq = dptr(dq);
    if (fold_delta) Q.flags |= HRT_ATTN_DQ_DELTA;
    queue(attn_kernel("dq", dt), Q);
    note_gpu(kBwdOp);
  }
  if (need[1] || need[2]) {
    dk = grad_for(k, d.Sk);
    dv = grad_for(v, d.Sk);
    hrt_attn_args KV = A;
    KV.dk = dptr(dk);
    KV.dv = dptr(dv);
    queue(attn_kernel("dkdv", dt), KV);
    note_gpu(kBwdOp);
  }
  return BwdOut{dq, dk, dv, at::Tensor()};
}

}  // namespace

namespace at::native {
REGISTER_PRIVATEUSE1_DISPATCH(_fused_sdp_choice_stub, &sdp_choice);
}

namespace vkt {
void set_fused_attention(int m) { mode().store(m); }
}  // namespace vkt

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("_scaled_dot_product_fused_attention_overrideable", &k_sdpa_fwd);
  m.impl("_scaled_dot_product_fused_attention_overrideable_backward", &k_sdpa_bwd);
}
