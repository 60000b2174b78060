// Direct 3x3 convolution (stride 1, zero padding 1, no dilation, one group, NCHW) as an implicit GEMM on the
// gfx950 matrix cores: "conv3x3_wprep_{bf16,f16}" and "conv3x3_{bf16,f16}".
//
// The unfolded form (im2col, then a GEMM over the column matrix) writes and reads back a matrix nine times
// the input (37.7 MB for 512 channels of 64 x 64 in bf16) and tiles the GEMM without knowing that neighbouring
// columns of that matrix are the same input pixels.  Here a workgroup owns 128 output channels x one 64-pixel
// segment of an output row.  Per block of 16 input channels it stages the three input rows the segment needs
// (with the one-pixel halo, zeros outside the image) once, channel-innermost in LDS, and the nine taps read
// their B fragments from that tile at shifted pixel offsets: the input is read from L2 once per tap block
// instead of nine times.  The weights are first reordered to [O][I / 16][tap][16] ("conv3x3_wprep"), so the
// A fragment of a tap (8 consecutive input channels of one output channel) is one 16-byte LDS read.  Eight
// wavefronts (4 along the output channels x 2 along the pixels) each accumulate one 32 x 32 tile with
// v_mfma_f32_32x32x16; the next channel block's loads are issued before the current block's MFMAs
// (double-buffered LDS, one barrier per block).  The input gradient of a convolution is the same operator on
// the output gradient with the flipped, transposed kernel (wprep flip = 1).
#include "../hrt/registry.h"
#include "lds_stage.h"

namespace hk {
namespace {

constexpr int C3_CO = 128;  // output channels per workgroup
constexpr int C3_PX = 64;   // output pixels per workgroup (one row segment)
constexpr int C3_CB = 16;   // input channels per block
constexpr int C3_ARS = 152;  // LDS row of the weight tile: 9 taps x 16 channels + 8 (304 B: conflict-free reads)
constexpr int C3_BPS = 24;   // LDS slot of one input pixel: 16 channels + 8 (48 B: conflict-free reads)
constexpr int C3_BCOLS = C3_PX + 2;  // staged pixels per input row (the halo pixel on each side)
constexpr int C3_ATILE = C3_CO * C3_ARS;          // uint16 elements
constexpr int C3_BTILE = 3 * C3_BCOLS * C3_BPS;  // uint16 elements
constexpr int C3_ACHUNKS = C3_CO * 18;            // 16-byte chunks of the weight tile (144 elements per row)
constexpr int C3_AREGS = (C3_ACHUNKS + 511) / 512;

// wr[o][cb][t][i] from w: flip 0: w[o][16 cb + i][t] (w [O][I][3][3]); flip 1: w[16 cb + i][o][8 - t]
// (w [I][O][3][3], the flipped transpose).  flip 0: one thread per (o, cb) reads the contiguous 144 values
// w[o][16 cb .. 16 cb + 15][0..8] in 16-byte pieces and writes the nine 16-channel rows; flip 1: one thread
// per (o, cb, t) gathers its 16 values (rows 9 O elements apart).
__global__ __launch_bounds__(256) void conv3_wprep_k(hrt_conv3_wprep_args a) {
  const int64_t nb = a.I / C3_CB;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const HK_G uint16_t* w = gcptr<uint16_t>(a.w);
  if (!a.flip) {
    if (idx >= a.O * nb) return;
    const int64_t o = idx / nb, cb = idx - o * nb;
    const HK_G u32x4* src = reinterpret_cast<const HK_G u32x4*>(w + (o * a.I + cb * C3_CB) * 9);
    uint16_t v[144];
#pragma unroll
    for (int k = 0; k < 18; ++k) {
      const u32x4 q = src[k];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[8 * k + 2 * e] = (uint16_t)(q[e] & 0xffffu), v[8 * k + 2 * e + 1] = (uint16_t)(q[e] >> 16);
    }
    HK_G u32x4* dst = reinterpret_cast<HK_G u32x4*>(gptr<uint16_t>(a.wr) + idx * 144);
#pragma unroll
    for (int t = 0; t < 9; ++t)
#pragma unroll
      for (int hlf = 0; hlf < 2; ++hlf) {
        uint32_t q[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i0 = 8 * hlf + 2 * e;  // value (channel i, tap t) sits at 9 i + t of the slab
          q[e] = (uint32_t)v[9 * i0 + t] | ((uint32_t)v[9 * (i0 + 1) + t] << 16);
        }
        dst[2 * t + hlf] = u32x4{q[0], q[1], q[2], q[3]};
      }
    return;
  }
  const int64_t total = a.O * nb * 9;
  if (idx >= total) return;
  const int64_t o = idx / (nb * 9), rem = idx - o * nb * 9, cb = rem / 9, t = rem - cb * 9;
  uint32_t v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t i = cb * C3_CB + 2 * j;
    v[j] = (uint32_t)w[(i * a.O + o) * 9 + (8 - t)] | ((uint32_t)w[((i + 1) * a.O + o) * 9 + (8 - t)] << 16);
  }
  HK_G u32x4* dst = reinterpret_cast<HK_G u32x4*>(gptr<uint16_t>(a.wr) + idx * C3_CB);
  dst[0] = u32x4{v[0], v[1], v[2], v[3]};
  dst[1] = u32x4{v[4], v[5], v[6], v[7]};
}

template <typename T>
__global__ __launch_bounds__(512) void conv3_igemm_k(hrt_conv3_args p) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][C3_ATILE];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][C3_BTILE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 3, wn = wave >> 2, l32 = lane & 31, hh = lane >> 5;
  const int64_t H = p.H, W = p.W, I = p.I, O = p.O;
  const int64_t segs = W / C3_PX, units = segs * H * p.N, ncob = O / C3_CO;
  // Workgroups are dealt to the eight XCDs in turn (workgroup b to XCD b % 8), each with its own L2: when the
  // output-channel blocks divide 8 and the row segments split evenly, XCD x serves only block x % ncob, so
  // it holds one block's weights (I x 9 x 128 values: 1.2 MB at 512 channels) instead of all of them
  uint32_t cob, unit;
  const uint32_t bid = blockIdx.x;
  if (8 % ncob == 0 && units % (8 / ncob) == 0) {
    const uint32_t x = bid % 8, loc = bid / 8, per = 8 / (uint32_t)ncob;
    cob = x % (uint32_t)ncob;
    unit = loc * per + x / (uint32_t)ncob;
  } else {
    cob = bid % (uint32_t)ncob;
    unit = bid / (uint32_t)ncob;
  }
  const int64_t n = unit / (segs * H), rs = unit - n * segs * H;
  const int64_t h = rs / segs, w0 = (rs - h * segs) * C3_PX;
  const int64_t co0 = (int64_t)cob * C3_CO;
  const int64_t nb = I / C3_CB;
  const HK_G uint16_t* X = gcptr<uint16_t>(p.x) + n * I * H * W;
  const HK_G uint16_t* WR = gcptr<uint16_t>(p.wr) + co0 * nb * (9 * C3_CB);

  // this thread's share of a block's copies: weight chunks tid + 512 k; one input vector (channel bi, row
  // brow, 8-pixel piece bv; stored by tid < 384); one halo pixel (channel hi, row hrow, side hside; stored by
  // 384 <= tid < 480).  Every thread issues every load with its address clamped in range (a branch between
  // the loads would make the compiler wait for all of them before the MFMAs that follow); out-of-image
  // values are zeroed when the registers go to LDS.
  u32x4 ar[C3_AREGS], br;
  uint32_t hr;
  const int bt = tid % 384, bi = bt / 24, brow = (bt / 8) % 3, bv = bt % 8;
  const int ht = tid % 96, hi = ht / 6, hrow = (ht / 2) % 3, hside = ht & 1;
  const int64_t bh = h - 1 + brow, hh2 = h - 1 + hrow, hw = hside ? w0 + C3_PX : w0 - 1;
  const bool b_ok = bh >= 0 && bh < H, h_ok = hh2 >= 0 && hh2 < H && hw >= 0 && hw < W;
  const int64_t bh_c = b_ok ? bh : h, hh_c = h_ok ? hh2 : h, hw_c = h_ok ? hw : w0;
  auto load = [&](int64_t cb) {
#pragma unroll
    for (int k = 0; k < C3_AREGS; ++k) {
      const int c = tid + 512 * k < C3_ACHUNKS ? tid + 512 * k : C3_ACHUNKS - 1;
      const int row = c / 18, ch = c - row * 18;
      ar[k] = *reinterpret_cast<const HK_G u32x4*>(WR + ((int64_t)row * nb + cb) * (9 * C3_CB) + ch * 8);
    }
    br = *reinterpret_cast<const HK_G u32x4*>(X + ((cb * C3_CB + bi) * H + bh_c) * W + w0 + bv * 8);
    hr = X[((cb * C3_CB + hi) * H + hh_c) * W + hw_c];
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int k = 0; k < C3_AREGS; ++k) {
      const int c = tid + 512 * k;
      if (c < C3_ACHUNKS) {
        const int row = c / 18, ch = c - row * 18;
        *reinterpret_cast<u32x4*>(&As[buf][row * C3_ARS + ch * 8]) = ar[k];
      }
    }
    if (tid < 384) {
      uint16_t* dst = &Bs[buf][(brow * C3_BCOLS + 1 + bv * 8) * C3_BPS + bi];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t v = b_ok ? br[j] : 0u;
        dst[(2 * j) * C3_BPS] = (uint16_t)(v & 0xffffu);
        dst[(2 * j + 1) * C3_BPS] = (uint16_t)(v >> 16);
      }
    } else if (tid < 480) {
      Bs[buf][(hrow * C3_BCOLS + (hside ? C3_BCOLS - 1 : 0)) * C3_BPS + hi] = (uint16_t)(h_ok ? hr : 0u);
    }
  };

  f32x16 acc = zero16();
  const int arow = (wm * 32 + l32) * C3_ARS + 8 * hh;
  const int bpix = wn * 32 + l32;
  load(0);
  store(0);
  __syncthreads();
  for (int64_t cb = 0; cb < nb; ++cb) {
    const int cur = (int)(cb & 1);
    const bool more = cb + 1 < nb;
    load(more ? cb + 1 : cb);  // the last block reloads itself (in range, not stored)
    issue_order_fence();       // keeps the loads here, in flight during the MFMAs (else they sink to their use)
#pragma unroll
    for (int t = 0; t < 9; ++t) {
      const int kh = t / 3, kw = t - kh * 3;
      const u32x4 a = *reinterpret_cast<const u32x4*>(&As[cur][arow + t * C3_CB]);
      const u32x4 b = *reinterpret_cast<const u32x4*>(&Bs[cur][(kh * C3_BCOLS + bpix + kw) * C3_BPS + 8 * hh]);
      acc = Mfma32<T>::mac(a, b, acc);
    }
    if (more) store(cur ^ 1);
    __syncthreads();
  }

  // lane holds y[co0 + wm 32 + 8 j + 4 hh + r][pixel w0 + wn 32 + l32] in element 4 j + r
  HK_G uint16_t* Y = gptr<uint16_t>(p.y) + n * O * H * W + h * W + w0 + bpix;
  const HK_G uint16_t* bias = gcptr<uint16_t>(p.bias);
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int64_t co = co0 + wm * 32 + 8 * (e >> 2) + 4 * hh + (e & 3);
    float v = acc[e];
    if (p.has_bias) v += T::to_f32(bias[co]);
    Y[co * H * W] = T::from_f32(v);
  }
}

bool conv3_wprep_launch(const void* pp, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_conv3_wprep_args*>(pp);
  if (a.O <= 0 || a.I <= 0 || a.I % C3_CB != 0) return ctx.fail("O > 0 and I a positive multiple of 16 required");
  if (a.flip > 1) return ctx.fail("flip must be 0 or 1");
  if (a.wr % 16 != 0) return ctx.fail("wr must be 16-byte aligned");
  const uint64_t bytes = (uint64_t)a.O * a.I * 9 * 2;
  if (!ctx.check(a.w, bytes, "w") || !ctx.check(a.wr, bytes, "wr")) return false;
  const int64_t total = a.flip ? a.O * (a.I / C3_CB) * 9 : a.O * (a.I / C3_CB), blocks = (total + 255) / 256;
  if (blocks > 0x7fffffffLL) return ctx.fail("grid too large");
  hipLaunchKernelGGL(conv3_wprep_k, dim3((uint32_t)blocks), dim3(256), 0, ctx.stream, a);
  return hrt::launch_ok(hipGetLastError(), ctx, "conv3x3_wprep");
}

template <typename T>
bool conv3_launch(const void* pp, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_conv3_args*>(pp);
  if (a.N <= 0 || a.H <= 0 || a.W <= 0 || a.I <= 0 || a.O <= 0) return ctx.fail("sizes must be positive");
  if (a.I % C3_CB || a.O % C3_CO || a.W % C3_PX)
    return ctx.fail("I must be a multiple of 16, O of 128 and W of 64");
  if (a.x % 16 || a.wr % 16 || a.y % 2 || (a.has_bias && a.bias % 2)) return ctx.fail("misaligned operand");
  if (a.N * a.H * (a.W / C3_PX) * (a.O / C3_CO) > 0x7fffffffLL) return ctx.fail("grid too large");
  const uint64_t xb = (uint64_t)a.N * a.I * a.H * a.W * 2, yb = (uint64_t)a.N * a.O * a.H * a.W * 2;
  if (!ctx.check(a.x, xb, "x") || !ctx.check(a.y, yb, "y") || !ctx.check(a.wr, (uint64_t)a.O * a.I * 9 * 2, "wr") ||
      (a.has_bias && !ctx.check(a.bias, (uint64_t)a.O * 2, "bias")))
    return false;
  const dim3 grid((uint32_t)(a.N * a.H * (a.W / C3_PX) * (a.O / C3_CO)));
  hipLaunchKernelGGL(conv3_igemm_k<T>, grid, dim3(512), 0, ctx.stream, a);
  return hrt::launch_ok(hipGetLastError(), ctx, "conv3x3");
}

HRT_REGISTER("conv3x3_wprep_bf16", hrt_conv3_wprep_args, conv3_wprep_launch);
HRT_REGISTER("conv3x3_wprep_f16", hrt_conv3_wprep_args, conv3_wprep_launch);
HRT_REGISTER("conv3x3_bf16", hrt_conv3_args, conv3_launch<BF16>);
HRT_REGISTER("conv3x3_f16", hrt_conv3_args, conv3_launch<F16>);

}  // namespace
}  // namespace hk
