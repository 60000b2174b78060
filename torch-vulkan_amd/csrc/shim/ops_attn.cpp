// Fused scaled-dot-product attention on the vk device (reference: csrc/ops_attn.cpp:1-310).
//
// PyTorch route: the PrivateUse1 `_fused_sdp_choice_stub` returns `overrideable` when the call is
// supported and wanted, so F.scaled_dot_product_attention lands in
// `_scaled_dot_product_fused_attention_overrideable` (forward) and its `_backward`; autograd stays in
// PyTorch.  Supported: 4-D [B, H, S, D] with d contiguous (else made contiguous), D <= 128, f32/bf16/f16,
// no mask / dropout / causal / GQA; everything else takes PyTorch's math path (bmm + softmax).
//
// bf16/f16 run the gfx950 matrix-core kernels ("attn_*_mfma_*"), f32 (and bf16/f16 with matrix cores
// switched off) the fp32 FMA kernels ("attn_*_fma_*").  Ragged Sq/Sk and any D <= 128 are handled in the
// kernels, so unlike the reference no zero-padded copies of q/k/v/dO are made.  The unrounded fp32 O
// rides in the `philox_offset` slot from forward to backward so that delta = rowsum(O * dO) matches the
// P the backward recomputes (csrc/ops_attn.cpp:178-186, 240-248).
#include <ATen/Operators.h>
#include <ATen/SDPBackend.h>
#include <ATen/native/transformers/attention.h>

#include <atomic>
#include <cmath>
#include <cstdlib>
#include <optional>
#include <string>
#include <tuple>

#include "common.h"

namespace {

using namespace vkt;

// VKT_FUSED_ATTN: "0" off, "1" on, unset = auto; VKT_NO_FUSED_ATTN=1 equals "0" (csrc/ops_attn.cpp:53-61).
int policy_from_env() {
  const char* n = std::getenv("VKT_NO_FUSED_ATTN");
  if (n && n[0] && n[0] != '0') return 0;
  const char* e = std::getenv("VKT_FUSED_ATTN");
  if (!e || !e[0]) return 2;
  return e[0] == '0' ? 0 : 1;
}
std::atomic<int>& policy_ref() {
  static std::atomic<int> p{policy_from_env()};
  return p;
}

bool use_mfma(at::ScalarType t) { return coop_is_enabled() && (t == at::kBFloat16 || t == at::kHalf); }

// auto: always for the matrix-core dtypes; for f32 only when the score matrix the math path would build
// is large (>= 256 MiB), where the memory saving matters (csrc/ops_attn.cpp:68-77).
bool fused_wanted(const at::Tensor& q, const at::Tensor& k) {
  const int p = policy_ref().load();
  if (p == 0) return false;
  if (p == 1) return true;
  if (use_mfma(q.scalar_type())) return true;
  const double score_bytes = 4.0 * (double)q.size(0) * q.size(1) * q.size(2) * k.size(2);
  return score_bytes >= 256.0 * 1024 * 1024;
}

bool attn_supported(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const std::optional<at::Tensor>& mask,
                    double dropout_p, bool is_causal, bool enable_gqa) {
  if (!is_vk(q) || !is_vk(k) || !is_vk(v)) return false;
  if (q.dim() != 4 || k.dim() != 4 || v.dim() != 4) return false;
  if (mask.has_value() && mask->defined()) return false;
  if (dropout_p != 0.0 || is_causal || enable_gqa) return false;
  if (!kind_name(q.scalar_type()) || k.scalar_type() != q.scalar_type() || v.scalar_type() != q.scalar_type()) return false;
  const int64_t D = q.size(3);
  if (D < 1 || D > 128 || k.size(3) != D || v.size(3) != D) return false;
  if (q.size(0) != k.size(0) || q.size(0) != v.size(0) || q.size(1) != k.size(1) || q.size(1) != v.size(1)) return false;
  if (k.size(2) != v.size(2) || k.size(2) < 1 || q.size(2) < 1 || q.size(0) < 1 || q.size(1) < 1) return false;
  if (q.size(0) * q.size(1) >= (int64_t(1) << 31) || q.size(2) >= (int64_t(1) << 31) || k.size(2) >= (int64_t(1) << 31))
    return false;
  return fused_wanted(q, k);
}

int64_t fused_sdp_choice_vk(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const std::optional<at::Tensor>& mask,
                            double dropout_p, bool is_causal, std::optional<double>, bool enable_gqa) {
  return attn_supported(q, k, v, mask, dropout_p, is_causal, enable_gqa) ? static_cast<int64_t>(at::SDPBackend::overrideable)
                                                                          : static_cast<int64_t>(at::SDPBackend::math);
}

at::Tensor d_contig(const at::Tensor& t) { return t.stride(3) == 1 ? t : t.contiguous(); }

// [B, S, H, D]-contiguous storage viewed as [B, H, S, D], like PyTorch's own SDPA outputs.
at::Tensor alloc_bshd(int64_t B, int64_t H, int64_t S, int64_t D, const at::TensorOptions& opt) {
  return at::empty({B, S, H, D}, opt).permute({0, 2, 1, 3});
}

void set_qkv(hrt_attn_args& P, const at::Tensor& q, const at::Tensor& k, const at::Tensor& v) {
  P.q = addr_of(q);
  P.k = addr_of(k);
  P.v = addr_of(v);
  P.q_sb = q.stride(0), P.q_sh = q.stride(1), P.q_ss = q.stride(2);
  P.k_sb = k.stride(0), P.k_sh = k.stride(1), P.k_ss = k.stride(2);
  P.v_sb = v.stride(0), P.v_sh = v.stride(1), P.v_ss = v.stride(2);
  P.B = (int32_t)q.size(0), P.H = (int32_t)q.size(1), P.Sq = (int32_t)q.size(2), P.Sk = (int32_t)k.size(2);
  P.D = (int32_t)q.size(3);
}

std::string kname(const char* op, at::ScalarType t) {
  return std::string("attn_") + op + (use_mfma(t) ? "_mfma_" : "_fma_") + kind_name(t);
}

using FwdRet = std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, c10::SymInt, c10::SymInt, at::Tensor, at::Tensor, at::Tensor>;

FwdRet k_sdpa_fwd(const at::Tensor& query, const at::Tensor& key, const at::Tensor& value, const std::optional<at::Tensor>& attn_bias,
                  double dropout_p, bool is_causal, bool /*return_debug_mask*/, std::optional<double> scale) {
  TORCH_CHECK(attn_supported(query, key, value, attn_bias, dropout_p, is_causal, false),
              "vk: this attention call is not supported by the fused kernels");
  ensure_init();
  at::Tensor q = d_contig(query), k = d_contig(key), v = d_contig(value);
  const int64_t B = q.size(0), H = q.size(1), Sq = q.size(2), Sk = k.size(2), D = q.size(3);
  const at::ScalarType dt = q.scalar_type();
  at::Tensor out = alloc_bshd(B, H, Sq, D, q.options());
  at::Tensor lse = at::empty({B, H, Sq}, q.options().dtype(at::kFloat));
  at::Tensor o32;
  if (dt != at::kFloat) o32 = at::empty({B, Sq, H, D}, q.options().dtype(at::kFloat));
  hrt_attn_args P{};
  set_qkv(P, q, k, v);
  P.o = addr_of(out);
  P.lse = addr_of(lse);
  P.o32 = o32.defined() ? addr_of(o32) : 0;
  P.scale = (float)scale.value_or(1.0 / std::sqrt((double)D));
  launch(kname("fwd", dt), P);
  count_kernel("aten::_scaled_dot_product_fused_attention_overrideable");
  at::Tensor el = at::empty({0}, at::TensorOptions().dtype(at::kLong));
  return FwdRet{out, lse, el, el, c10::SymInt(Sq), c10::SymInt(Sk), el, o32.defined() ? o32 : el,
                at::empty({0}, at::TensorOptions().dtype(dt))};
}

using BwdRet = std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor>;

BwdRet k_sdpa_bwd(const at::Tensor& grad_out, const at::Tensor& query, const at::Tensor& key, const at::Tensor& value,
                  const at::Tensor& attn_bias, std::array<bool, 4> mask, const at::Tensor& out, const at::Tensor& lse,
                  const at::Tensor&, const at::Tensor&, c10::SymInt, c10::SymInt, double dropout_p, bool is_causal,
                  const at::Tensor&, const at::Tensor& o32_saved, std::optional<double> scale) {
  TORCH_CHECK(attn_supported(query, key, value, attn_bias.defined() ? std::optional<at::Tensor>(attn_bias) : std::nullopt,
                             dropout_p, is_causal, false) &&
                  is_vk(grad_out) && is_vk(out) && is_vk(lse),
              "vk: this attention backward is not supported by the fused kernels");
  ensure_init();
  at::Tensor q = d_contig(query), k = d_contig(key), v = d_contig(value);
  const int64_t B = q.size(0), H = q.size(1), Sq = q.size(2), Sk = k.size(2), D = q.size(3);
  const at::ScalarType dt = q.scalar_type();
  at::Tensor dO = d_contig(grad_out.scalar_type() == dt ? grad_out : grad_out.to(dt));
  at::Tensor lse_c = lse.contiguous();
  at::Tensor delta = at::empty({B, H, Sq}, q.options().dtype(at::kFloat));
  const char* an = "aten::_scaled_dot_product_fused_attention_overrideable_backward";

  hrt_attn_args P{};
  set_qkv(P, q, k, v);
  P.lse = addr_of(lse_c);
  P.delta = addr_of(delta);
  P.dout = addr_of(dO);
  P.do_sb = dO.stride(0), P.do_sh = dO.stride(1), P.do_ss = dO.stride(2);
  P.scale = (float)scale.value_or(1.0 / std::sqrt((double)D));

  // delta = rowsum(O * dO), from the unrounded fp32 O when the forward kept it
  at::Tensor o_bshd;
  if (dt != at::kFloat && o32_saved.defined() && o32_saved.scalar_type() == at::kFloat && is_vk(o32_saved) &&
      o32_saved.numel() == B * Sq * H * D && o32_saved.is_contiguous()) {
    P.o = addr_of(o32_saved);
    P.flags = HRT_ATTN_O_F32;
  } else {
    o_bshd = (out.scalar_type() == dt ? out : out.to(dt)).permute({0, 2, 1, 3}).contiguous();
    P.o = addr_of(o_bshd);
  }
  // The matrix-core dQ kernel computes delta itself (HRT_ATTN_DQ_DELTA), so it runs first and dK/dV
  // reads its delta; otherwise the delta pass runs on its own.
  const std::string dq_name = kname("dq", dt);
  const bool fused_delta = mask[0] && dq_name.find("_mfma_") != std::string::npos;
  if (!fused_delta) {
    launch(std::string("attn_delta_") + kind_name(dt), P);
    count_kernel(an);
  }

  at::Tensor dq, dk, dv;
  if (mask[0]) {
    dq = alloc_bshd(B, H, Sq, D, q.options());
    hrt_attn_args P2 = P;
    P2.dq = addr_of(dq);
    if (fused_delta) P2.flags |= HRT_ATTN_DQ_DELTA;
    launch(dq_name, P2);
    count_kernel(an);
  }
  if (mask[1] || mask[2]) {
    dk = alloc_bshd(B, H, Sk, D, q.options());
    dv = alloc_bshd(B, H, Sk, D, q.options());
    hrt_attn_args P1 = P;
    P1.dk = addr_of(dk);
    P1.dv = addr_of(dv);
    launch(kname("dkdv", dt), P1);
    count_kernel(an);
  }
  return BwdRet{dq, dk, dv, at::Tensor()};
}

}  // namespace

namespace at::native {
REGISTER_PRIVATEUSE1_DISPATCH(_fused_sdp_choice_stub, &fused_sdp_choice_vk);
}

namespace vkt {
void set_fused_attention(int mode) { policy_ref().store(mode); }
}  // namespace vkt

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("_scaled_dot_product_fused_attention_overrideable", &k_sdpa_fwd);
  m.impl("_scaled_dot_product_fused_attention_overrideable_backward", &k_sdpa_bwd);
}
