// conv2d (forward and backward), nearest upsampling and group_norm on the vk device.
// Reference: csrc/ops_conv.cpp:1-228 (conv via im2col + the GEMM, upsample), csrc/ops_norm.cpp:1-148
// (group_norm), csrc/shim.cpp:354-374 (convolution_overrideable).  Same support rules: NCHW, groups 1,
// dilation 1, not transposed, input and weight of one float dtype (f32/bf16/f16); integer upsampling
// factors; other cases run on the CPU and come back.
#include <ATen/Operators.h>

#include <array>
#include <cstdint>
#include <optional>
#include <string>
#include <tuple>
#include <vector>

#include "common.h"

namespace {

using namespace vkt;
using IntVec = std::vector<int64_t>;

IntVec ints(c10::SymIntArrayRef a) {
  IntVec v;
  for (const auto& s : a) v.push_back(s.guard_int(__FILE__, __LINE__));
  return v;
}

at::Tensor contig(const at::Tensor& t) { return t.is_contiguous() ? t : t.contiguous(); }

// ---- conv2d ------------------------------------------------------------------------------------------------
struct Geom {
  int64_t N, C, H, W, Co, KH, KW, SH, SW, PH, PW, OH, OW;
  bool direct;  // 1x1, stride 1, no padding: the input is its own column matrix
  int64_t K() const { return C * KH * KW; }
  int64_t L() const { return OH * OW; }
};

bool conv_geom(const at::Tensor& x, const at::Tensor& w, const IntVec& stride, const IntVec& padding, const IntVec& dilation,
               bool transposed, int64_t groups, Geom& g) {
  if (transposed || groups != 1 || !is_vk(x) || !is_vk(w) || x.dim() != 4 || w.dim() != 4) return false;
  if (float_code(x.scalar_type()) < 0 || x.scalar_type() != w.scalar_type()) return false;
  if (stride.size() != 2 || padding.size() != 2 || dilation.size() != 2 || dilation[0] != 1 || dilation[1] != 1) return false;
  if (stride[0] < 1 || stride[1] < 1 || padding[0] < 0 || padding[1] < 0) return false;
  g.N = x.size(0), g.C = x.size(1), g.H = x.size(2), g.W = x.size(3);
  g.Co = w.size(0), g.KH = w.size(2), g.KW = w.size(3);
  if (w.size(1) != g.C) return false;
  g.SH = stride[0], g.SW = stride[1], g.PH = padding[0], g.PW = padding[1];
  const int64_t oh = g.H + 2 * g.PH - g.KH, ow = g.W + 2 * g.PW - g.KW;
  if (oh < 0 || ow < 0) return false;
  g.OH = oh / g.SH + 1, g.OW = ow / g.SW + 1;
  g.direct = g.KH == 1 && g.KW == 1 && g.SH == 1 && g.SW == 1 && g.PH == 0 && g.PW == 0;
  if (g.N * g.C * g.H * g.W == 0 || g.Co == 0 || g.L() == 0) return false;
  return g.K() <= 65535 && g.N <= 65535 && g.C <= 65535;  // grid limits of the unfolding kernels
}

hrt_im2col_args im2col_args(const Geom& g, const at::Tensor& x, const at::Tensor& cols) {
  hrt_im2col_args A{};
  A.x = addr_of(x);
  A.cols = addr_of(cols);
  A.N = g.N, A.C = g.C, A.H = g.H, A.W = g.W, A.OH = g.OH, A.OW = g.OW;
  A.KH = g.KH, A.KW = g.KW, A.SH = g.SH, A.SW = g.SW, A.PH = g.PH, A.PW = g.PW;
  return A;
}

// The column matrix [N, C*KH*KW, OH*OW] of x (a view of x when the convolution is direct).
at::Tensor cols_of(const at::Tensor& input, const Geom& g) {
  at::Tensor x = contig(input);
  if (g.direct) return x.view({g.N, g.C, g.H * g.W});
  at::Tensor cols = at::empty({g.N, g.K(), g.L()}, x.options());
  launch(std::string("im2col_") + kind_name(x.scalar_type()), im2col_args(g, x, cols));
  return cols;
}

// out[n] = A @ B[n] for A [M, K], B [N, K, L]: one product when N == 1, else bmm with A broadcast.
at::Tensor left_matmul(const at::Tensor& A, const at::Tensor& B) {
  const int64_t N = B.size(0);
  if (N == 1) return at::mm(A, B.select(0, 0)).unsqueeze(0);
  return at::bmm(A.unsqueeze(0).expand({N, A.size(0), A.size(1)}), B);
}

at::Tensor k_convolution_overrideable(const at::Tensor& input, const at::Tensor& weight, const std::optional<at::Tensor>& bias,
                                      c10::SymIntArrayRef stride, c10::SymIntArrayRef padding, c10::SymIntArrayRef dilation,
                                      bool transposed, c10::SymIntArrayRef output_padding, c10::SymInt groups) {
  Geom g;
  const bool has_bias = bias.has_value() && bias->defined();
  if (conv_geom(input, weight, ints(stride), ints(padding), ints(dilation), transposed, groups.guard_int(__FILE__, __LINE__), g) &&
      (!has_bias || (is_vk(*bias) && bias->scalar_type() == input.scalar_type() && bias->numel() == g.Co))) {
    at::Tensor cols = cols_of(input, g);
    at::Tensor out = left_matmul(contig(weight).view({g.Co, g.K()}), cols).view({g.N, g.Co, g.OH, g.OW});
    if (has_bias) out.add_(bias->view({1, g.Co, 1, 1}));
    count_kernel("aten::convolution_overrideable");
    return out;
  }
  // Shapes the kernels do not take (groups, dilation, transposed): PyTorch's CPU convolution, moved back.
  count_fallback("aten::convolution_overrideable");
  std::optional<at::Tensor> b = std::nullopt;
  if (has_bias) b = bias->to(at::kCPU);
  return at::convolution_symint(input.to(at::kCPU), weight.to(at::kCPU), b, stride, padding, dilation, transposed,
                                output_padding, groups)
      .to(input.device());
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> k_convolution_backward_overrideable(
    const at::Tensor& grad_output, const at::Tensor& input, const at::Tensor& weight, c10::SymIntArrayRef stride_,
    c10::SymIntArrayRef padding_, c10::SymIntArrayRef dilation_, bool transposed, c10::SymIntArrayRef output_padding_,
    c10::SymInt groups_, std::array<bool, 3> mask) {
  const IntVec stride = ints(stride_), padding = ints(padding_), dilation = ints(dilation_);
  const int64_t groups = groups_.guard_int(__FILE__, __LINE__);
  Geom g;
  if (!conv_geom(input, weight, stride, padding, dilation, transposed, groups, g) || !is_vk(grad_output) ||
      grad_output.scalar_type() != input.scalar_type() || grad_output.dim() != 4 || grad_output.size(0) != g.N ||
      grad_output.size(1) != g.Co || grad_output.size(2) != g.OH || grad_output.size(3) != g.OW) {
    count_fallback("aten::convolution_backward_overrideable");
    auto r = at::convolution_backward(grad_output.to(at::kCPU), input.to(at::kCPU), weight.to(at::kCPU), std::nullopt, stride,
                                      padding, dilation, transposed, ints(output_padding_), groups, mask);
    auto back = [](const at::Tensor& t, const at::Tensor& like) { return t.defined() ? t.to(like.device()) : at::Tensor(); };
    return {back(std::get<0>(r), input), back(std::get<1>(r), weight), back(std::get<2>(r), weight)};
  }
  at::Tensor go = contig(grad_output);
  at::Tensor G = go.view({g.N, g.Co, g.L()});
  at::Tensor w2 = contig(weight).view({g.Co, g.K()});
  at::Tensor gi, gw, gb;
  if (mask[0]) {
    at::Tensor gcols = contig(left_matmul(w2.t(), G));  // [N, K, L]
    if (g.direct) {
      gi = gcols.view({g.N, g.C, g.H, g.W});
    } else {
      gi = at::empty({g.N, g.C, g.H, g.W}, go.options());
      launch(std::string("col2im_") + kind_name(go.scalar_type()), im2col_args(g, gi, gcols));
    }
  }
  if (mask[1]) {
    at::Tensor cols = cols_of(input, g);
    at::Tensor gw2 = g.N == 1 ? at::mm(G.select(0, 0), cols.select(0, 0).t()) : at::bmm(G, cols.transpose(1, 2)).sum(0);
    gw = gw2.reshape(weight.sizes());
  }
  if (mask[2]) gb = at::sum(go, IntVec{0, 2, 3});
  count_kernel("aten::convolution_backward_overrideable");
  return {gi, gw, gb};
}

// ---- nearest upsampling ------------------------------------------------------------------------------------
bool up_ok(const at::Tensor& t, int64_t H, int64_t W, int64_t OH, int64_t OW) {
  return is_vk(t) && float_code(t.scalar_type()) >= 0 && t.dim() == 4 && H > 0 && W > 0 && OH >= H && OW >= W &&
         OH % H == 0 && OW % W == 0;
}

hrt_upsample_args up_args(const at::Tensor& src, const at::Tensor& dst, int64_t NC, int64_t H, int64_t W, int64_t OH,
                          int64_t OW) {
  hrt_upsample_args A{};
  A.src = addr_of(src);
  A.dst = addr_of(dst);
  A.NC = NC, A.H = H, A.W = W, A.OH = OH, A.OW = OW;
  return A;
}

at::Tensor k_upsample_nearest2d(const at::Tensor& input, c10::SymIntArrayRef output_size, std::optional<double> scales_h,
                                std::optional<double> scales_w) {
  const IntVec os = ints(output_size);
  if (os.size() == 2 && input.dim() == 4 && up_ok(input, input.size(2), input.size(3), os[0], os[1]) && input.numel() > 0) {
    at::Tensor x = contig(input);
    at::Tensor out = at::empty({x.size(0), x.size(1), os[0], os[1]}, x.options());
    launch(std::string("upsample_nearest_fwd_") + kind_name(x.scalar_type()),
           up_args(x, out, x.size(0) * x.size(1), x.size(2), x.size(3), os[0], os[1]));
    count_kernel("aten::upsample_nearest2d");
    return out;
  }
  return VKT_FALLBACK_SYMINT(upsample_nearest2d, input, output_size, scales_h, scales_w);
}

at::Tensor k_upsample_nearest2d_backward(const at::Tensor& grad_output, c10::SymIntArrayRef output_size,
                                         c10::SymIntArrayRef input_size, std::optional<double> scales_h,
                                         std::optional<double> scales_w) {
  const IntVec os = ints(output_size), is = ints(input_size);
  if (os.size() == 2 && is.size() == 4 && grad_output.dim() == 4 && up_ok(grad_output, is[2], is[3], os[0], os[1]) &&
      grad_output.size(2) == os[0] && grad_output.size(3) == os[1] && grad_output.numel() > 0) {
    at::Tensor go = contig(grad_output);
    at::Tensor gx = at::empty({is[0], is[1], is[2], is[3]}, go.options());
    launch(std::string("upsample_nearest_bwd_") + kind_name(go.scalar_type()),
           up_args(go, gx, is[0] * is[1], is[2], is[3], os[0], os[1]));
    count_kernel("aten::upsample_nearest2d_backward");
    return gx;
  }
  return VKT_FALLBACK_SYMINT(upsample_nearest2d_backward, grad_output, output_size, input_size, scales_h, scales_w);
}

// ---- group_norm ------------------------------------------------------------------------------------------
// Affine parameters are read in the input's dtype (converted on the device when they differ).
at::Tensor affine(const std::optional<at::Tensor>& p, const at::Tensor& input, int64_t C, bool& ok) {
  if (!p.has_value() || !p->defined()) return at::Tensor();
  if (!is_vk(*p) || p->numel() != C || float_code(p->scalar_type()) < 0) {
    ok = false;
    return at::Tensor();
  }
  return contig(p->scalar_type() == input.scalar_type() ? *p : p->to(input.scalar_type()));
}

bool gn_ok(const at::Tensor& x, int64_t N, int64_t C, int64_t HW, int64_t G) {
  return is_vk(x) && float_code(x.scalar_type()) >= 0 && N > 0 && C > 0 && HW > 0 && G > 0 && C % G == 0 &&
         x.numel() == N * C * HW && N * G <= 65535 && N * C <= 65535;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> k_native_group_norm(const at::Tensor& input, const std::optional<at::Tensor>& weight,
                                                                   const std::optional<at::Tensor>& bias, c10::SymInt N_,
                                                                   c10::SymInt C_, c10::SymInt HxW_, int64_t group, double eps) {
  const int64_t N = N_.guard_int(__FILE__, __LINE__), C = C_.guard_int(__FILE__, __LINE__),
                HW = HxW_.guard_int(__FILE__, __LINE__);
  bool ok = gn_ok(input, N, C, HW, group);
  at::Tensor w, b;
  if (ok) w = affine(weight, input, C, ok);
  if (ok) b = affine(bias, input, C, ok);
  if (ok) {
    at::Tensor x = contig(input);
    at::Tensor y = at::empty(x.sizes(), x.options());
    at::Tensor mean = at::empty({N, group}, x.options()), rstd = at::empty({N, group}, x.options());
    at::Tensor ws = at::empty({hrt_gn_workspace(N, C, HW, group)}, x.options().dtype(at::kFloat));
    hrt_gn_args A{};
    A.x = addr_of(x), A.y = addr_of(y), A.mean = addr_of(mean), A.rstd = addr_of(rstd), A.ws = addr_of(ws);
    A.w = w.defined() ? addr_of(w) : 0;
    A.b = b.defined() ? addr_of(b) : 0;
    A.N = N, A.C = C, A.HW = HW, A.G = group, A.eps = (float)eps;
    launch(std::string("gn_fwd_") + kind_name(x.scalar_type()), A);
    count_kernel("aten::native_group_norm");
    return {y, mean, rstd};
  }
  return VKT_FALLBACK_SYMINT(native_group_norm, input, weight, bias, N_, C_, HxW_, group, eps);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> k_native_group_norm_backward(
    const at::Tensor& grad_out, const at::Tensor& input, const at::Tensor& mean, const at::Tensor& rstd,
    const std::optional<at::Tensor>& weight, c10::SymInt N_, c10::SymInt C_, c10::SymInt HxW_, int64_t group,
    std::array<bool, 3> mask) {
  const int64_t N = N_.guard_int(__FILE__, __LINE__), C = C_.guard_int(__FILE__, __LINE__),
                HW = HxW_.guard_int(__FILE__, __LINE__);
  bool ok = gn_ok(input, N, C, HW, group) && is_vk(grad_out) && grad_out.scalar_type() == input.scalar_type() &&
            grad_out.numel() == input.numel() && is_vk(mean) && is_vk(rstd) && mean.numel() == N * group &&
            rstd.numel() == N * group && float_code(mean.scalar_type()) >= 0 && float_code(rstd.scalar_type()) >= 0;
  at::Tensor w;
  if (ok) w = affine(weight, input, C, ok);
  if (ok) {
    at::Tensor x = contig(input), g = contig(grad_out);
    auto stat = [&](const at::Tensor& t) { return contig(t.scalar_type() == x.scalar_type() ? t : t.to(x.scalar_type())); };
    at::Tensor mu = stat(mean), rs = stat(rstd);
    at::Tensor ws = at::empty({hrt_gn_workspace(N, C, HW, group)}, x.options().dtype(at::kFloat));
    at::Tensor dx, dw, db;
    const at::ScalarType wdt = (weight.has_value() && weight->defined()) ? weight->scalar_type() : x.scalar_type();
    if (mask[0]) dx = at::empty(x.sizes(), x.options());
    if (mask[1]) dw = at::empty({C}, x.options());
    if (mask[2]) db = at::empty({C}, x.options());
    hrt_gn_args A{};
    A.x = addr_of(x), A.g = addr_of(g), A.mean = addr_of(mu), A.rstd = addr_of(rs), A.ws = addr_of(ws);
    A.w = w.defined() ? addr_of(w) : 0;
    A.dx = mask[0] ? addr_of(dx) : 0;
    A.dw = mask[1] ? addr_of(dw) : 0;
    A.db = mask[2] ? addr_of(db) : 0;
    A.N = N, A.C = C, A.HW = HW, A.G = group;
    if (A.dx || A.dw || A.db) launch(std::string("gn_bwd_") + kind_name(x.scalar_type()), A);
    if (mask[1] && wdt != x.scalar_type()) dw = dw.to(wdt);
    if (mask[2] && wdt != x.scalar_type()) db = db.to(wdt);
    count_kernel("aten::native_group_norm_backward");
    return {dx, dw, db};
  }
  return VKT_FALLBACK_SYMINT(native_group_norm_backward, grad_out, input, mean, rstd, weight, N_, C_, HxW_, group, mask);
}

}  // namespace

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("convolution_overrideable", &k_convolution_overrideable);
  m.impl("convolution_backward_overrideable", &k_convolution_backward_overrideable);
  m.impl("upsample_nearest2d", &k_upsample_nearest2d);
  m.impl("upsample_nearest2d_backward", &k_upsample_nearest2d_backward);
  m.impl("native_group_norm", &k_native_group_norm);
  m.impl("native_group_norm_backward", &k_native_group_norm_backward);
}
