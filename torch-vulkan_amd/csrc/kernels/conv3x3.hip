// Direct 3x3 convolution (stride 1, zero padding 1, no dilation, one group, NCHW) as an implicit GEMM on the
// gfx950 matrix cores: "conv3x3_wprep_{bf16,f16}" and "conv3x3_{bf16,f16}".
//
// The unfolded form (im2col, then a GEMM over the column matrix) writes and reads back a matrix nine times
// the input (37.7 MB for 512 channels of 64 x 64 in bf16) and tiles the GEMM without knowing that neighbouring
// columns of that matrix are the same input pixels.  Here a workgroup owns 128 output channels x two output
// rows x a 64-pixel segment, and walks the input channels in steps of 16:
//  * the weights are reordered once per call ("conv3x3_wprep") into the exact LDS image of a step's weight
//    tile -- [output block of 128][channel block of 16][128 rows of 9 taps x 16 channels + 8 pad] -- so a
//    step's 38 KB tile is one contiguous run of 16-byte pieces;
//  * the four input rows the two output rows need (with the one-pixel halo, zeros outside the image) are
//    stored channel-innermost; the nine taps read their B fragments from that tile at shifted pixel offsets;
//  * both are loaded into registers two steps ahead of their use (two register sets) and written to one of
//    two LDS buffers at the end of the step before it, so each load has two steps of MFMAs to arrive.  (Direct
//    global -> LDS copies for the weights mixed with the register loads of the input rows made the compiler
//    wait for every outstanding load before each LDS store of the rows, as it then treats the counter as
//    out of order);
//  * eight wavefronts (4 along the output channels x the 2 rows) each keep two 32 x 32 accumulators (the
//    row's two 32-pixel halves) with v_mfma_f32_32x32x16: 18 MFMAs per wavefront and step;
//  * the input channels may be split over `splits` workgroups (small images: a 64 x 64 image at 512
//    channels has 128 tiles); each split writes fp32 partial sums and a second kernel, queued by the same
//    call, adds them in split order, adds the bias and rounds once.
// Workgroups are dealt to the eight XCDs in turn; the (output block, split) pair is the fastest-varying
// part of the workgroup index, so with 8 such pairs each XCD's L2 holds one pair's weights.  The input
// gradient of a convolution is the same operator on the output gradient with the flipped, transposed kernel
// (wprep flip = 1).
#include "../hrt/registry.h"
#include "lds_stage.h"

namespace hk {
namespace {

constexpr int C3_CO = 128;                          // output channels per workgroup
constexpr int C3_PX = 64;                           // pixels per output row segment
constexpr int C3_CB = 16;                           // input channels per step
constexpr int C3_ARS = 152;                         // weight tile row: 9 taps x 16 channels + 8 (304 B)
constexpr int C3_ASLAB = C3_CO * C3_ARS * 2;        // bytes of one weight tile: 38912
constexpr int C3_APIECES = C3_ASLAB / 16;            // 16-byte pieces of a weight tile: 2432
constexpr int C3_AREGS = (C3_APIECES + 511) / 512;  // per thread: 5 (the fifth for threads < 384)
constexpr int C3_BPS = 24;                          // LDS slot of one input pixel: 16 channels + 8 (48 B)
constexpr int C3_BCOLS = C3_PX + 2;                 // staged pixels per input row (a halo pixel each side)
constexpr int C3_BTILE = 4 * C3_BCOLS * C3_BPS;     // uint16 elements: four input rows
static_assert(C3_ASLAB == HRT_CONV3_SLAB_BYTES, "weight tile size of the header");

// Workgroup (32-channel output block, input channel block cb) of the weight reordering: the 32 x 16 x 9
// values are read in 16-byte pieces into LDS in their source order (flip 0: w[o][16 cb + i][t], w
// [O][I][3][3]; flip 1: w[16 cb + i][o][t], w [I][O][3][3]) and written as the tile rows
// wr[o / 128][cb][o % 128][9 t + ...] = [t][i] (flip 1: tap 8 - t, the flipped kernel), 16 bytes per store,
// the 8 pad values zero.
__global__ __launch_bounds__(256) void conv3_wprep_k(hrt_conv3_wprep_args a) {
  __shared__ __attribute__((aligned(16))) uint16_t tl[32 * C3_CB * 9];
  const int tid = threadIdx.x;
  const int64_t nb = a.I / C3_CB, o0 = (int64_t)blockIdx.x * 32, cb = blockIdx.y;
  const HK_G uint16_t* w = gcptr<uint16_t>(a.w);
  u32x4 v[3];
#pragma unroll
  for (int j = 0; j < 3; ++j) {  // pieces k = tid + 256 j < 576, all loads issued before the stores
    const int k = tid + 256 * j < 576 ? tid + 256 * j : 575;
    const int64_t src = a.flip ? ((cb * C3_CB + k / 36) * a.O + o0) * 9 + (k % 36) * 8
                               : ((o0 + k / 18) * a.I + cb * C3_CB) * 9 + (k % 18) * 8;
    v[j] = *reinterpret_cast<const HK_G u32x4*>(w + src);
  }
#pragma unroll
  for (int j = 0; j < 3; ++j)
    if (tid + 256 * j < 576) *reinterpret_cast<u32x4*>(tl + (tid + 256 * j) * 8) = v[j];
  __syncthreads();
  for (int k = tid; k < 32 * 19; k += 256) {
    const int o = k / 19, pc = k - o * 19;  // piece pc < 18: tap pc / 2, channels 8 (pc % 2) .. +7; 18: pad
    u32x4 out = {0u, 0u, 0u, 0u};
    if (pc < 18) {
      const int t = pc >> 1, i0 = (pc & 1) * 8;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = i0 + 2 * e;
        const uint32_t lo = a.flip ? tl[i * 288 + o * 9 + 8 - t] : tl[o * 144 + i * 9 + t];
        const uint32_t hi = a.flip ? tl[(i + 1) * 288 + o * 9 + 8 - t] : tl[o * 144 + (i + 1) * 9 + t];
        out[e] = lo | (hi << 16);
      }
    }
    const int64_t og = o0 + o;
    HK_G uint16_t* row = gptr<uint16_t>(a.wr) + (((og / C3_CO) * nb + cb) * C3_CO + og % C3_CO) * C3_ARS;
    *reinterpret_cast<HK_G u32x4*>(row + pc * 8) = out;
  }
}

template <typename T>
__global__ __launch_bounds__(512) void conv3_igemm_k(hrt_conv3_args p) {
  __shared__ __attribute__((aligned(16))) uint8_t a0_raw[C3_ASLAB], a1_raw[C3_ASLAB];
  __shared__ __attribute__((aligned(16))) uint16_t b0_raw[C3_BTILE], b1_raw[C3_BTILE];
  HK_L uint8_t* const A0 = (HK_L uint8_t*)a0_raw;
  HK_L uint8_t* const A1 = (HK_L uint8_t*)a1_raw;
  HK_L uint16_t* const B0 = (HK_L uint16_t*)b0_raw;
  HK_L uint16_t* const B1 = (HK_L uint16_t*)b1_raw;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 3, wr = wave >> 2, l32 = lane & 31, hh = lane >> 5;
  const int64_t H = p.H, W = p.W, I = p.I, O = p.O;
  const int64_t nb = I / C3_CB, S = p.splits, steps = nb / S;
  const int64_t segs = W / C3_PX, rpairs = (H + 1) / 2, ncob = O / C3_CO, combos = ncob * S;
  const uint32_t bid = blockIdx.x;
  const uint32_t combo = bid % (uint32_t)combos, unit = bid / (uint32_t)combos;
  const int64_t cob = combo % ncob, sp = combo / ncob;
  const int64_t n = unit / (segs * rpairs), rs = unit - n * segs * rpairs;
  const int64_t h0 = (rs / segs) * 2, w0 = (rs - (rs / segs) * segs) * C3_PX;
  const int64_t co0 = cob * C3_CO, cb0 = sp * steps;
  const int64_t cstride = (int64_t)C3_CB * H * W;  // elements between channel blocks of x
  const HK_G uint16_t* X = gcptr<uint16_t>(p.x) + n * I * H * W + cb0 * cstride;
  const HK_G uint8_t* WR = gcptr<uint8_t>(p.wr) + (cob * nb + cb0) * (int64_t)C3_ASLAB;

  // this thread's share of a step's loads: weight pieces tid + 512 k (k < 5; past the tile's 2432 pieces the
  // last one is loaded and not stored); vector bv (8 pixels) of input row h0 - 1 + brow of channel bi; the
  // halo pixel hside of row hrow of channel hi (stored by tid < 128).  Every thread issues every load with a
  // clamped address (no branch between loads); out-of-image values are zeroed at the LDS store.
  // Lanes of a wavefront take the 16 channels x 2 vectors x 2 rows of one (vector pair, row pair), so their
  // 2-byte LDS stores (pixel slots 48 bytes apart, channel innermost) fall in four disjoint 8-bank ranges
  // (with 8 vectors x 4 rows x 2 channels per wavefront they met on 8 banks: 4-way conflicts).
  const int bi = lane & 15, bv = 2 * (wave & 3) + ((lane >> 4) & 1), brow = 2 * (wave >> 2) + ((lane >> 5) & 1);
  const int hi = lane & 15, hside = (lane >> 4) & 1, hrow = 2 * (wave & 1) + ((lane >> 5) & 1);
  const int64_t bh = h0 - 1 + brow, hr2 = h0 - 1 + hrow, hw = hside ? w0 + C3_PX : w0 - 1;
  const bool b_ok = bh >= 0 && bh < H, h_ok = hr2 >= 0 && hr2 < H && hw >= 0 && hw < W;
  const int64_t boff = (bi * H + (b_ok ? bh : 0)) * W + w0 + bv * 8;
  const int64_t hoff = (hi * H + (h_ok ? hr2 : 0)) * W + (h_ok ? hw : 0);
  const int bdst = (brow * C3_BCOLS + 1 + bv * 8) * C3_BPS + bi;
  const int hdst = (hrow * C3_BCOLS + (hside ? C3_BCOLS - 1 : 0)) * C3_BPS + hi;

  struct Regs {
    u32x4 a[C3_AREGS];
    u32x4 b;
    uint32_t h;
  };
  auto load = [&](int64_t j, Regs& r) {
    const HK_G uint8_t* wt = WR + j * (int64_t)C3_ASLAB;
#pragma unroll
    for (int k = 0; k < C3_AREGS; ++k) {
      const int pc = tid + 512 * k < C3_APIECES ? tid + 512 * k : C3_APIECES - 1;
      r.a[k] = *reinterpret_cast<const HK_G u32x4*>(wt + pc * 16);
    }
    const HK_G uint16_t* xb = X + j * cstride;
    r.b = *reinterpret_cast<const HK_G u32x4*>(xb + boff);
    r.h = xb[hoff];
  };
  auto store = [&](HK_L uint8_t* At, HK_L uint16_t* Bt, const Regs& r) {
#pragma unroll
    for (int k = 0; k < C3_AREGS; ++k)
      if (tid + 512 * k < C3_APIECES) *reinterpret_cast<HK_L u32x4*>(At + (tid + 512 * k) * 16) = r.a[k];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t v = b_ok ? r.b[j] : 0u;
      Bt[bdst + (2 * j) * C3_BPS] = (uint16_t)(v & 0xffffu);
      Bt[bdst + (2 * j + 1) * C3_BPS] = (uint16_t)(v >> 16);
    }
    if (tid < 128) Bt[hdst] = (uint16_t)(h_ok ? r.h : 0u);
  };

  f32x16 acc0 = zero16(), acc1 = zero16();
  const int aoff = (wm * 32 + l32) * (C3_ARS * 2) + 16 * hh;  // bytes
  const int boff_f = (wr * C3_BCOLS + l32) * C3_BPS + 8 * hh;  // elements
  Regs r0, r1;
  // step i (buffers and register set S = i % 2): the loads of step i + 2 into register set S, the 18 MFMAs
  // of step i from buffers S, then register set 1 - S (step i + 1, loaded during step i - 1) into buffers
  // 1 - S.  Past the last step the loads repeat it (in range, never stored), so every step issues the same
  // 7 loads and the barrier lets exactly those stay in flight.
  auto step = [&](auto sc, int64_t i) {
    constexpr int SB = decltype(sc)::value;
    load(i + 2 < steps ? i + 2 : steps - 1, SB == 0 ? r0 : r1);
    issue_order_fence();  // keeps the loads here, in flight during the MFMAs (else they sink to their use)
    const HK_L uint8_t* At = SB == 0 ? A0 : A1;
    const HK_L uint16_t* Bt = SB == 0 ? B0 : B1;
#pragma unroll
    for (int t = 0; t < 9; ++t) {
      const int kh = t / 3, kw = t - kh * 3;
      const u32x4 a = *reinterpret_cast<const HK_L u32x4*>(At + aoff + t * 32);
      const HK_L uint16_t* bp = Bt + boff_f + (kh * C3_BCOLS + kw) * C3_BPS;
      const u32x4 b0 = *reinterpret_cast<const HK_L u32x4*>(bp);
      const u32x4 b1 = *reinterpret_cast<const HK_L u32x4*>(bp + 32 * C3_BPS);
      acc0 = Mfma32<T>::mac(a, b0, acc0);
      acc1 = Mfma32<T>::mac(a, b1, acc1);
    }
    if (i + 1 < steps) {
      if constexpr (SB == 0) store(A1, B1, r1);
      else store(A0, B0, r0);
    }
    barrier_keep_vm_lds<C3_AREGS + 2>();
  };

  // prologue: step 0 into buffers 0, step 1 into register set 1
  load(0, r0);
  load(steps > 1 ? 1 : 0, r1);
  store(A0, B0, r0);
  barrier_keep_vm_lds<C3_AREGS + 2>();
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  int64_t i = 0;
  for (; i + 2 <= steps; i += 2) {
    step(I0(), i);
    step(I1(), i + 1);
  }
  if (i < steps) step(I0(), i);

  // lane holds out[co0 + wm 32 + 8 j + 4 hh + r][row h0 + wr][pixel w0 + 32 half + l32] in element 4 j + r
  const int64_t row = h0 + wr;
  if (row >= H) return;
  const int64_t HW = H * W, px = row * W + w0 + l32;
  if (S == 1) {
    HK_G uint16_t* Y = gptr<uint16_t>(p.y) + n * O * HW + px;
    float bv2[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) bv2[e] = 0.f;
    if (p.has_bias) {  // all 16 loads issued before the first use
      const HK_G uint16_t* bias = gcptr<uint16_t>(p.bias) + co0 + wm * 32 + 4 * hh;
      uint16_t braw[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) braw[e] = bias[8 * (e >> 2) + (e & 3)];
#pragma unroll
      for (int e = 0; e < 16; ++e) bv2[e] = T::to_f32(braw[e]);
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int64_t co = co0 + wm * 32 + 8 * (e >> 2) + 4 * hh + (e & 3);
      Y[co * HW] = T::from_f32(acc0[e] + bv2[e]);
      Y[co * HW + 32] = T::from_f32(acc1[e] + bv2[e]);
    }
  } else {
    HK_G float* Wp = gptr<float>(p.ws) + (sp * p.N + n) * O * HW + px;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int64_t co = co0 + wm * 32 + 8 * (e >> 2) + 4 * hh + (e & 3);
      Wp[co * HW] = acc0[e];
      Wp[co * HW + 32] = acc1[e];
    }
  }
}

// y = round(sum over splits s, in order, of ws[s] + bias): 8 consecutive outputs per thread (H W is a
// multiple of 64, so they share an output channel), 16-byte loads and store.
template <typename T>
__global__ __launch_bounds__(256) void conv3_reduce_k(hrt_conv3_args p) {
  const int64_t HW = p.H * p.W, total = p.N * p.O * HW;
  const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i0 >= total) return;
  const HK_G float* ws = gcptr<float>(p.ws) + i0;
  f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
  for (int64_t s = 0; s < p.splits; ++s) {
    s0 += *reinterpret_cast<const HK_G f32x4*>(ws + s * total);
    s1 += *reinterpret_cast<const HK_G f32x4*>(ws + s * total + 4);
  }
  float v[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
  if (p.has_bias) {
    const float b = T::to_f32(gcptr<uint16_t>(p.bias)[(i0 / HW) % p.O]);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] += b;
  }
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = pack2<T>(v[2 * e], v[2 * e + 1]);
  *reinterpret_cast<HK_G u32x4*>(gptr<uint16_t>(p.y) + i0) = o;
}

bool conv3_wprep_launch(const void* pp, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_conv3_wprep_args*>(pp);
  if (a.O <= 0 || a.I <= 0 || a.I % C3_CB != 0 || a.O % C3_CO != 0)
    return ctx.fail("O must be a positive multiple of 128 and I of 16");
  if (a.flip > 1) return ctx.fail("flip must be 0 or 1");
  if (a.w % 16 != 0 || a.wr % 16 != 0) return ctx.fail("w and wr must be 16-byte aligned");
  if (a.O / 32 > 0x7fffffffLL || a.I / C3_CB > 65535) return ctx.fail("grid too large");
  if (!ctx.check(a.w, (uint64_t)a.O * a.I * 9 * 2, "w") || !ctx.check(a.wr, (uint64_t)hrt_conv3_wr_bytes(a.O, a.I), "wr"))
    return false;
  hipLaunchKernelGGL(conv3_wprep_k, dim3((uint32_t)(a.O / 32), (uint32_t)(a.I / C3_CB)), dim3(256), 0, ctx.stream, a);
  return hrt::launch_ok(hipGetLastError(), ctx, "conv3x3_wprep");
}

bool conv3_check(const hrt_conv3_args& a, hrt::LaunchCtx& ctx) {
  if (a.N <= 0 || a.H <= 0 || a.W <= 0 || a.I <= 0 || a.O <= 0) return ctx.fail("sizes must be positive");
  if (a.I % C3_CB || a.O % C3_CO || a.W % C3_PX)
    return ctx.fail("I must be a multiple of 16, O of 128 and W of 64");
  if (a.splits < 1 || (a.I / C3_CB) % a.splits) return ctx.fail("splits must divide I / 16");
  if (a.x % 16 || a.wr % 16 || a.y % 16 || (a.has_bias && a.bias % 2) || (a.splits > 1 && a.ws % 16))
    return ctx.fail("misaligned operand");
  const int64_t units = a.N * ((a.H + 1) / 2) * (a.W / C3_PX), combos = (a.O / C3_CO) * a.splits;
  if (units * combos > 0x7fffffffLL) return ctx.fail("grid too large");
  const uint64_t xb = (uint64_t)a.N * a.I * a.H * a.W * 2, yb = (uint64_t)a.N * a.O * a.H * a.W * 2;
  return ctx.check(a.x, xb, "x") && ctx.check(a.y, yb, "y") && ctx.check(a.wr, (uint64_t)hrt_conv3_wr_bytes(a.O, a.I), "wr") &&
         (!a.has_bias || ctx.check(a.bias, (uint64_t)a.O * 2, "bias")) &&
         (a.splits == 1 || ctx.check(a.ws, yb * 2 * a.splits, "ws"));
}

// The convolution, and with splits > 1 the reduction of its partial sums right behind it.
template <typename T>
bool conv3_launch(const void* pp, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_conv3_args*>(pp);
  if (!conv3_check(a, ctx)) return false;
  const int64_t units = a.N * ((a.H + 1) / 2) * (a.W / C3_PX), combos = (a.O / C3_CO) * a.splits;
  hipLaunchKernelGGL(conv3_igemm_k<T>, dim3((uint32_t)(units * combos)), dim3(512), 0, ctx.stream, a);
  if (!hrt::launch_ok(hipGetLastError(), ctx, "conv3x3")) return false;
  if (a.splits == 1) return true;
  const int64_t total = a.N * a.O * a.H * a.W;
  hipLaunchKernelGGL(conv3_reduce_k<T>, dim3((uint32_t)cdiv(total, 2048)), dim3(256), 0, ctx.stream, a);
  return hrt::launch_ok(hipGetLastError(), ctx, "conv3x3_reduce");
}

HRT_REGISTER("conv3x3_wprep_bf16", hrt_conv3_wprep_args, conv3_wprep_launch);
HRT_REGISTER("conv3x3_wprep_f16", hrt_conv3_wprep_args, conv3_wprep_launch);
HRT_REGISTER("conv3x3_bf16", hrt_conv3_args, conv3_launch<BF16>);
HRT_REGISTER("conv3x3_f16", hrt_conv3_args, conv3_launch<F16>);

}  // namespace
}  // namespace hk
