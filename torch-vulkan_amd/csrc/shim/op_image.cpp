// Image operators on the vk device: conv2d forward and backward (convolution_overrideable and its
// backward), nearest upsampling and group_norm.  The reference registers the same operators
// (csrc/ops_conv.cpp:1-228, csrc/ops_norm.cpp:1-148, csrc/shim.cpp:354-374) with the same reach: NCHW,
// one group, no dilation, not transposed, one float dtype; integer upsampling factors; the rest runs on
// the CPU and comes back.  conv2d is an unfolding (im2col, and its adjoint col2im written as a gather)
// around the matrix-core GEMM.
#include <ATen/Operators.h>

#include <algorithm>
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

// ---- conv2d ------------------------------------------------------------------------------------------------
// The convolutions the kernels take: 2-D, NCHW, one group, no dilation, not transposed, input and weight
// of one float dtype, non-negative padding, positive stride; anything else runs on the CPU.
struct ConvShape {
  int64_t N, C, H, W;        // input
  int64_t Co, KH, KW;        // weight [Co, C, KH, KW]
  int64_t SH, SW, PH, PW;    // stride, padding
  int64_t OH, OW;            // output
  int64_t K() const { return C * KH * KW; }  // rows of the column matrix
  int64_t L() const { return OH * OW; }      // columns of the column matrix
  // 1x1, stride 1, no padding: the input already is its column matrix
  bool direct() const { return KH == 1 && KW == 1 && SH == 1 && SW == 1 && PH == 0 && PW == 0; }
};

// Output extent along one axis, or -1 when the kernel does not fit the padded input.
int64_t out_extent(int64_t in, int64_t k, int64_t stride, int64_t pad) {
  const int64_t span = in + 2 * pad - k;
  return span < 0 ? -1 : span / stride + 1;
}

std::optional<ConvShape> conv_shape(const at::Tensor& x, const at::Tensor& w, const IntVec& stride, const IntVec& padding,
                                    const IntVec& dilation, bool transposed, int64_t groups) {
  const bool plain = !transposed && groups == 1 && stride.size() == 2 && padding.size() == 2 && dilation == IntVec{1, 1};
  if (!plain || !on_vk(x) || !on_vk(w) || x.dim() != 4 || w.dim() != 4) return std::nullopt;
  if (x.scalar_type() != w.scalar_type() || float_code(x.scalar_type()) < 0 || w.size(1) != x.size(1)) return std::nullopt;
  if (*std::min_element(stride.begin(), stride.end()) < 1 || *std::min_element(padding.begin(), padding.end()) < 0)
    return std::nullopt;
  ConvShape c{x.size(0), x.size(1), x.size(2), x.size(3), w.size(0), w.size(2), w.size(3),
              stride[0], stride[1], padding[0], padding[1], 0, 0};
  c.OH = out_extent(c.H, c.KH, c.SH, c.PH);
  c.OW = out_extent(c.W, c.KW, c.SW, c.PW);
  if (c.OH < 1 || c.OW < 1 || x.numel() == 0 || c.Co == 0) return std::nullopt;
  if (c.K() > 65535 || c.N > 65535 || c.C > 65535) return std::nullopt;  // grid limits of the unfolding kernels
  return c;
}

hrt_im2col_args im2col_args(const ConvShape& g, const at::Tensor& x, const at::Tensor& cols) {
  hrt_im2col_args A{};
  A.x = dptr(x);
  A.cols = dptr(cols);
  A.N = g.N, A.C = g.C, A.H = g.H, A.W = g.W, A.OH = g.OH, A.OW = g.OW;
  A.KH = g.KH, A.KW = g.KW, A.SH = g.SH, A.SW = g.SW, A.PH = g.PH, A.PW = g.PW;
  return A;
}

// The column matrix [N, C*KH*KW, OH*OW] of x (a view of x when the convolution is direct).
at::Tensor cols_of(const at::Tensor& input, const ConvShape& g) {
  at::Tensor x = dense(input);
  if (g.direct()) return x.view({g.N, g.C, g.H * g.W});
  at::Tensor cols = at::empty({g.N, g.K(), g.L()}, x.options());
  queue(typed("im2col", x.scalar_type()), im2col_args(g, x, cols));
  return cols;
}

// The direct 3x3 kernel ("conv3x3_{dt}": an implicit GEMM over the input rows, no column matrix) takes
// stride 1, padding 1, a matrix-core dtype, input channels in multiples of 16, output channels in multiples of
// 128 and rows of a multiple of 64 pixels (VAE decoder and UNet levels at 64 px and up): at 512 channels
// on 64x64 it runs 44 us against the unfolding + GEMM's 51 us (forward + input gradient 86 against 105).
// VKT_CONV_IM2COL=1 (read on every call) keeps the unfolding.  in_ch / out_ch: the channels the kernel reads
// / writes (swapped for the adjoint).  x, w: the operands the kernel would read, which it takes at 16-byte
// aligned addresses only (a view at an odd offset, e.g. a weight inside a flat parameter buffer, goes to the
// unfolding + GEMM path, which takes any alignment).
bool conv3_ok(const ConvShape& g, at::ScalarType t, int64_t in_ch, int64_t out_ch, const at::Tensor& x, const at::Tensor& w) {
  const char* off = std::getenv("VKT_CONV_IM2COL");
  if (dptr(x) % 16 != 0 || dptr(w) % 16 != 0) return false;
  return !(off != nullptr && off[0] == '1') && coop_is_enabled() && (t == at::kBFloat16 || t == at::kHalf) && g.KH == 3 && g.KW == 3 && g.SH == 1 &&
         g.SW == 1 && g.PH == 1 && g.PW == 1 && in_ch % 16 == 0 && out_ch % 128 == 0 && g.W % 64 == 0 &&
         g.N * g.H * (g.W / 64) * (out_ch / 128) <= 0x7fffffffLL;
}

// y = conv3x3(x) with the weights reordered for the kernel (flip = 0: the forward, w [out_ch, in_ch, 3, 3];
// flip = 1: the input gradient, w [in_ch, out_ch, 3, 3] read as its flipped transpose), plus bias.
at::Tensor conv3_run(const at::Tensor& x, const at::Tensor& w, const at::Tensor* bias, const ConvShape& g,
                     int64_t in_ch, int64_t out_ch, uint32_t flip) {
  const at::Tensor wr = at::empty({hrt_conv3_wr_bytes(out_ch, in_ch) / 2}, x.options());
  hrt_conv3_wprep_args P{};
  P.w = dptr(w), P.wr = dptr(wr), P.O = out_ch, P.I = in_ch, P.flip = flip;
  queue(typed("conv3x3_wprep", x.scalar_type()), P);
  at::Tensor y = at::empty({g.N, out_ch, g.H, g.W}, x.options());
  const int64_t splits = hrt_conv3_splits(g.N, in_ch, out_ch, g.H, g.W);
  at::Tensor ws;  // the splits' fp32 partial sums
  if (splits > 1) ws = at::empty({splits * g.N * out_ch * g.H * g.W}, x.options().dtype(at::kFloat));
  hrt_conv3_args A{};
  A.x = dptr(x), A.wr = dptr(wr), A.y = dptr(y), A.ws = splits > 1 ? dptr(ws) : 0;
  A.N = g.N, A.I = in_ch, A.O = out_ch, A.H = g.H, A.W = g.W, A.splits = (uint32_t)splits;
  if (bias) A.bias = dptr(*bias), A.has_bias = 1;
  queue(typed("conv3x3", x.scalar_type()), A);
  note_gpu("torch_vulkan::conv3x3");  // lets callers and tests see which path ran
  return y;
}

// The weight matrix w2 [M, K] times each image's column matrix cols[n] [K, L] -> [N, M, L]: a plain GEMM for a
// single image, else one batched GEMM whose left operand repeats w2 with a zero batch stride (no copy).
at::Tensor weight_times(const at::Tensor& w2, const at::Tensor& cols) {
  if (cols.size(0) == 1) return at::mm(w2, cols[0]).unsqueeze(0);
  return at::bmm(w2.expand({cols.size(0), w2.size(0), w2.size(1)}), cols);
}

at::Tensor k_convolution_overrideable(const at::Tensor& input, const at::Tensor& weight, const std::optional<at::Tensor>& bias,
                                      c10::SymIntArrayRef stride, c10::SymIntArrayRef padding, c10::SymIntArrayRef dilation,
                                      bool transposed, c10::SymIntArrayRef output_padding, c10::SymInt groups) {
  const bool has_bias = present(bias);
  const std::optional<ConvShape> c = conv_shape(input, weight, ints(stride), ints(padding), ints(dilation), transposed,
                                                groups.guard_int(__FILE__, __LINE__));
  if (c && (!has_bias || (on_vk(*bias) && bias->scalar_type() == input.scalar_type() && bias->numel() == c->Co))) {
    const ConvShape& g = *c;
    const at::Tensor xd = dense(input), wd = dense(weight);
    if (conv3_ok(g, input.scalar_type(), g.C, g.Co, xd, wd)) {
      const at::Tensor b = has_bias ? dense(*bias) : at::Tensor();
      at::Tensor out = conv3_run(xd, wd, has_bias ? &b : nullptr, g, g.C, g.Co, 0);
      note_gpu("aten::convolution_overrideable");
      return out;
    }
    at::Tensor cols = cols_of(input, g);
    at::Tensor out = weight_times(wd.view({g.Co, g.K()}), cols).view({g.N, g.Co, g.OH, g.OW});
    if (has_bias) out.add_(bias->view({1, g.Co, 1, 1}));
    note_gpu("aten::convolution_overrideable");
    return out;
  }
  // Shapes the kernels do not take (groups, dilation, transposed): PyTorch's CPU convolution, moved back.
  note_cpu("aten::convolution_overrideable", 0);
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
  const std::optional<ConvShape> c = conv_shape(input, weight, stride, padding, dilation, transposed, groups);
  const bool grad_ok = c && on_vk(grad_output) && grad_output.scalar_type() == input.scalar_type() &&
                       grad_output.sizes().equals(c10::IntArrayRef{c->N, c->Co, c->OH, c->OW});
  if (!grad_ok) {
    note_cpu("aten::convolution_backward_overrideable", 0);
    auto r = at::convolution_backward(grad_output.to(at::kCPU), input.to(at::kCPU), weight.to(at::kCPU), std::nullopt, stride,
                                      padding, dilation, transposed, ints(output_padding_), groups, mask);
    auto back = [](const at::Tensor& t, const at::Tensor& like) { return t.defined() ? t.to(like.device()) : at::Tensor(); };
    return {back(std::get<0>(r), input), back(std::get<1>(r), weight), back(std::get<2>(r), weight)};
  }
  const ConvShape& g = *c;
  at::Tensor go = dense(grad_output);
  at::Tensor G = go.view({g.N, g.Co, g.L()});
  const at::Tensor wd = dense(weight);
  at::Tensor w2 = wd.view({g.Co, g.K()});
  at::Tensor gi, gw, gb;
  if (mask[0] && conv3_ok(g, go.scalar_type(), g.Co, g.C, go, wd)) {
    gi = conv3_run(go, wd, nullptr, g, g.Co, g.C, 1);  // the adjoint: flipped, transposed kernel
  } else if (mask[0]) {
    at::Tensor gcols = dense(weight_times(w2.t(), G));  // [N, K, L]
    if (g.direct()) {
      gi = gcols.view({g.N, g.C, g.H, g.W});
    } else {
      gi = at::empty({g.N, g.C, g.H, g.W}, go.options());
      queue(typed("col2im", go.scalar_type()), im2col_args(g, gi, gcols));
    }
  }
  if (mask[1]) {
    at::Tensor cols = cols_of(input, g);
    at::Tensor gw2 = g.N == 1 ? at::mm(G.select(0, 0), cols.select(0, 0).t()) : at::bmm(G, cols.transpose(1, 2)).sum(0);
    gw = gw2.reshape(weight.sizes());
  }
  if (mask[2]) gb = at::sum(go, IntVec{0, 2, 3});
  note_gpu("aten::convolution_backward_overrideable");
  return {gi, gw, gb};
}

// ---- nearest upsampling ------------------------------------------------------------------------------------
bool up_ok(const at::Tensor& t, int64_t H, int64_t W, int64_t OH, int64_t OW) {
  return on_vk(t) && float_code(t.scalar_type()) >= 0 && t.dim() == 4 && H > 0 && W > 0 && OH >= H && OW >= W &&
         OH % H == 0 && OW % W == 0;
}

hrt_upsample_args up_args(const at::Tensor& src, const at::Tensor& dst, int64_t NC, int64_t H, int64_t W, int64_t OH,
                          int64_t OW) {
  hrt_upsample_args A{};
  A.src = dptr(src);
  A.dst = dptr(dst);
  A.NC = NC, A.H = H, A.W = W, A.OH = OH, A.OW = OW;
  return A;
}

at::Tensor k_upsample_nearest2d(const at::Tensor& input, c10::SymIntArrayRef output_size, std::optional<double> scales_h,
                                std::optional<double> scales_w) {
  const IntVec os = ints(output_size);
  if (os.size() == 2 && input.dim() == 4 && up_ok(input, input.size(2), input.size(3), os[0], os[1]) && input.numel() > 0) {
    at::Tensor x = dense(input);
    at::Tensor out = at::empty({x.size(0), x.size(1), os[0], os[1]}, x.options());
    queue(typed("upsample_nearest_fwd", x.scalar_type()),
           up_args(x, out, x.size(0) * x.size(1), x.size(2), x.size(3), os[0], os[1]));
    note_gpu("aten::upsample_nearest2d");
    return out;
  }
  return VKT_CPU_SYMINT(upsample_nearest2d, input, output_size, scales_h, scales_w);
}

at::Tensor k_upsample_nearest2d_backward(const at::Tensor& grad_output, c10::SymIntArrayRef output_size,
                                         c10::SymIntArrayRef input_size, std::optional<double> scales_h,
                                         std::optional<double> scales_w) {
  const IntVec os = ints(output_size), is = ints(input_size);
  if (os.size() == 2 && is.size() == 4 && grad_output.dim() == 4 && up_ok(grad_output, is[2], is[3], os[0], os[1]) &&
      grad_output.size(2) == os[0] && grad_output.size(3) == os[1] && grad_output.numel() > 0) {
    at::Tensor go = dense(grad_output);
    at::Tensor gx = at::empty({is[0], is[1], is[2], is[3]}, go.options());
    queue(typed("upsample_nearest_bwd", go.scalar_type()),
           up_args(go, gx, is[0] * is[1], is[2], is[3], os[0], os[1]));
    note_gpu("aten::upsample_nearest2d_backward");
    return gx;
  }
  return VKT_CPU_SYMINT(upsample_nearest2d_backward, grad_output, output_size, input_size, scales_h, scales_w);
}

// ---- group_norm ------------------------------------------------------------------------------------------
// Affine parameters are read in the input's dtype (converted on the device when they differ).
at::Tensor affine(const std::optional<at::Tensor>& p, const at::Tensor& input, int64_t C, bool& ok) {
  if (!p.has_value() || !p->defined()) return at::Tensor();
  if (!on_vk(*p) || p->numel() != C || float_code(p->scalar_type()) < 0) {
    ok = false;
    return at::Tensor();
  }
  return dense(p->scalar_type() == input.scalar_type() ? *p : p->to(input.scalar_type()));
}

bool gn_ok(const at::Tensor& x, int64_t N, int64_t C, int64_t HW, int64_t G) {
  return on_vk(x) && float_code(x.scalar_type()) >= 0 && N > 0 && C > 0 && HW > 0 && G > 0 && C % G == 0 &&
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
    at::Tensor x = dense(input);
    at::Tensor y = at::empty(x.sizes(), x.options());
    at::Tensor mean = at::empty({N, group}, x.options()), rstd = at::empty({N, group}, x.options());
    at::Tensor ws = at::empty({hrt_gn_workspace(N, C, HW, group)}, x.options().dtype(at::kFloat));
    hrt_gn_args A{};
    A.x = dptr(x), A.y = dptr(y), A.mean = dptr(mean), A.rstd = dptr(rstd), A.ws = dptr(ws);
    A.w = w.defined() ? dptr(w) : 0;
    A.b = b.defined() ? dptr(b) : 0;
    A.N = N, A.C = C, A.HW = HW, A.G = group, A.eps = (float)eps;
    queue(typed("gn_fwd", x.scalar_type()), A);
    note_gpu("aten::native_group_norm");
    return {y, mean, rstd};
  }
  return VKT_CPU_SYMINT(native_group_norm, input, weight, bias, N_, C_, HxW_, group, eps);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> k_native_group_norm_backward(
    const at::Tensor& grad_out, const at::Tensor& input, const at::Tensor& mean, const at::Tensor& rstd,
    const std::optional<at::Tensor>& weight, c10::SymInt N_, c10::SymInt C_, c10::SymInt HxW_, int64_t group,
    std::array<bool, 3> mask) {
  const int64_t N = N_.guard_int(__FILE__, __LINE__), C = C_.guard_int(__FILE__, __LINE__),
                HW = HxW_.guard_int(__FILE__, __LINE__);
  bool ok = gn_ok(input, N, C, HW, group) && on_vk(grad_out) && grad_out.scalar_type() == input.scalar_type() &&
            grad_out.numel() == input.numel() && on_vk(mean) && on_vk(rstd) && mean.numel() == N * group &&
            rstd.numel() == N * group && float_code(mean.scalar_type()) >= 0 && float_code(rstd.scalar_type()) >= 0;
  at::Tensor w;
  if (ok) w = affine(weight, input, C, ok);
  if (ok) {
    at::Tensor x = dense(input), g = dense(grad_out);
    auto stat = [&](const at::Tensor& t) { return dense(t.scalar_type() == x.scalar_type() ? t : t.to(x.scalar_type())); };
    at::Tensor mu = stat(mean), rs = stat(rstd);
    at::Tensor ws = at::empty({hrt_gn_workspace(N, C, HW, group)}, x.options().dtype(at::kFloat));
    at::Tensor dx, dw, db;
    const at::ScalarType wdt = (weight.has_value() && weight->defined()) ? weight->scalar_type() : x.scalar_type();
    if (mask[0]) dx = at::empty(x.sizes(), x.options());
    if (mask[1]) dw = at::empty({C}, x.options());
    if (mask[2]) db = at::empty({C}, x.options());
    hrt_gn_args A{};
    A.x = dptr(x), A.g = dptr(g), A.mean = dptr(mu), A.rstd = dptr(rs), A.ws = dptr(ws);
    A.w = w.defined() ? dptr(w) : 0;
    A.dx = mask[0] ? dptr(dx) : 0;
    A.dw = mask[1] ? dptr(dw) : 0;
    A.db = mask[2] ? dptr(db) : 0;
    A.N = N, A.C = C, A.HW = HW, A.G = group;
    if (A.dx || A.dw || A.db) queue(typed("gn_bwd", x.scalar_type()), A);
    if (mask[1] && wdt != x.scalar_type()) dw = dw.to(wdt);
    if (mask[2] && wdt != x.scalar_type()) db = db.to(wdt);
    note_gpu("aten::native_group_norm_backward");
    return {dx, dw, db};
  }
  return VKT_CPU_SYMINT(native_group_norm_backward, grad_out, input, mean, rstd, weight, N_, C_, HxW_, group, mask);
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
