// The image-model operators of the step: conv2d's unfolding (im2col) and its adjoint (col2im), nearest
// upsampling and its backward, and group_norm forward and backward.  Reference: csrc/ops_conv.cpp:31-221,
// csrc/ops_norm.cpp:27-142 with vkrt/shaders/im2col.comp.in, upsample.comp.in, gn.comp.in.
//
// conv2d runs as im2col followed by the MFMA GEMM (the product dominates; the unfolding stages the input
// rows of a block of output rows in LDS once and streams the column matrix out in 16-byte stores).  col2im
// is a gather: each input pixel adds the KH*KW column entries it fed, in a fixed order, so the input
// gradient is deterministic without atomics.  group_norm's statistics are fp32 partial sums over chunks of each group (a group of a VAE
// layer spans up to millions of elements, so one workgroup per group would leave the GPU idle), each
// shifted by the chunk's first element and merged with Chan's formula in a fixed order; applying the
// normalisation and the backward's per-channel sums stream the tensor with coalesced loads.
#include <algorithm>
#include <string>

#include "../hrt/registry.h"
#include "device_common.h"

namespace hk {
namespace {

template <typename T>
__device__ __forceinline__ float ldf(uint64_t p, int64_t i) {
  if constexpr (std::is_same<T, F32>::value) return gcptr<float>(p)[i];
  else return T::to_f32(gcptr<uint16_t>(p)[i]);
}
template <typename T>
__device__ __forceinline__ void stf(uint64_t p, int64_t i, float v) {
  if constexpr (std::is_same<T, F32>::value) gptr<float>(p)[i] = v;
  else gptr<uint16_t>(p)[i] = T::from_f32(v);
}
template <typename T>
constexpr uint64_t esz() {
  return std::is_same<T, F32>::value ? 4 : 2;
}
// Elements per 16-byte access.
template <typename T>
constexpr int vec16() {
  return std::is_same<T, F32>::value ? 4 : 8;
}
// 16 bytes at element i (a multiple of vec16<T>() from a 16-byte aligned base).
template <typename T>
__device__ __forceinline__ void ldv(uint64_t p, int64_t i, float (&v)[vec16<T>()]) {
  if constexpr (std::is_same<T, F32>::value) {
    const f32x4 u = gcptr<f32x4>(p)[i / 4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = u[j];
  } else {
    const u32x4 u = gcptr<u32x4>(p)[i / 8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = lo16<T>(u[j]);
      v[2 * j + 1] = hi16<T>(u[j]);
    }
  }
}
template <typename T>
__device__ __forceinline__ void stv(uint64_t p, int64_t i, const float (&v)[vec16<T>()]) {
  if constexpr (std::is_same<T, F32>::value) {
    gptr<f32x4>(p)[i / 4] = f32x4{v[0], v[1], v[2], v[3]};
  } else {
    u32x4 u;
#pragma unroll
    for (int j = 0; j < 4; ++j) u[j] = pack2<T>(v[2 * j], v[2 * j + 1]);
    gptr<u32x4>(p)[i / 8] = u;
  }
}

// V elements at i: one 16-byte access when V == vec16<T>(), else V single ones.
template <typename T, int V>
__device__ __forceinline__ void ldn(uint64_t p, int64_t i, float (&v)[V]) {
  if constexpr (V == vec16<T>()) {
    ldv<T>(p, i, v);
  } else {
#pragma unroll
    for (int j = 0; j < V; ++j) v[j] = ldf<T>(p, i + j);
  }
}
template <typename T, int V>
__device__ __forceinline__ void stn(uint64_t p, int64_t i, const float (&v)[V]) {
  if constexpr (V == vec16<T>()) {
    stv<T>(p, i, v);
  } else {
#pragma unroll
    for (int j = 0; j < V; ++j) stf<T>(p, i + j, v[j]);
  }
}

// ---- im2col / col2im ----------------------------------------------------------------------------------
// grid (cdiv(L, 256), K, N), K = C*KH*KW, L = OH*OW: block (k, n) writes row k of image n's columns.
template <typename T>
__global__ __launch_bounds__(256) void im2col_k(hrt_im2col_args a) {
  const int64_t L = a.OH * a.OW;
  const int64_t l = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (l >= L) return;
  const int64_t k = blockIdx.y, n = blockIdx.z;
  const int64_t kw = k % a.KW, kh = (k / a.KW) % a.KH, c = k / (a.KW * a.KH);
  const int64_t oh = l / a.OW, ow = l - oh * a.OW;
  const int64_t h = oh * a.SH - a.PH + kh, w = ow * a.SW - a.PW + kw;
  float v = 0.0f;
  if (h >= 0 && h < a.H && w >= 0 && w < a.W) v = ldf<T>(a.x, ((n * a.C + c) * a.H + h) * a.W + w);
  stf<T>(a.cols, (n * (a.C * a.KH * a.KW) + k) * L + l, v);
}

// As im2col_k with vec16 consecutive output pixels per lane (OW a multiple of it: one 16-byte store).
template <typename T>
__global__ __launch_bounds__(256) void im2col_vec_k(hrt_im2col_args a) {
  constexpr int V = vec16<T>();
  const int64_t L = a.OH * a.OW;
  const int64_t l0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * V;
  if (l0 >= L) return;
  const int64_t k = blockIdx.y, n = blockIdx.z;
  const int64_t kw = k % a.KW, kh = (k / a.KW) % a.KH, c = k / (a.KW * a.KH);
  const int64_t oh = l0 / a.OW, ow0 = l0 - oh * a.OW;
  const int64_t h = oh * a.SH - a.PH + kh;
  float v[V];
  const bool row = h >= 0 && h < a.H;
  const int64_t xrow = ((n * a.C + c) * a.H + h) * a.W;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int64_t w = (ow0 + j) * a.SW - a.PW + kw;
    v[j] = (row && w >= 0 && w < a.W) ? ldf<T>(a.x, xrow + w) : 0.0f;
  }
  stv<T>(a.cols, (n * (a.C * a.KH * a.KW) + k) * L + l0, v);
}

// grid (cdiv(H*W, 256), C, N): each input pixel adds the entries im2col copied it to, kh then kw.
template <typename T>
__global__ __launch_bounds__(256) void col2im_k(hrt_im2col_args a) {
  const int64_t HW = a.H * a.W;
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= HW) return;
  const int64_t c = blockIdx.y, n = blockIdx.z;
  const int64_t h = p / a.W, w = p - h * a.W;
  const int64_t L = a.OH * a.OW, K = a.C * a.KH * a.KW;
  float s = 0.0f;
  for (int64_t kh = 0; kh < a.KH; ++kh) {
    const int64_t th = h + a.PH - kh;
    if (th < 0 || th % a.SH) continue;
    const int64_t oh = th / a.SH;
    if (oh >= a.OH) continue;
    for (int64_t kw = 0; kw < a.KW; ++kw) {
      const int64_t tw = w + a.PW - kw;
      if (tw < 0 || tw % a.SW) continue;
      const int64_t ow = tw / a.SW;
      if (ow >= a.OW) continue;
      s += ldf<T>(a.cols, (n * K + (c * a.KH + kh) * a.KW + kw) * L + oh * a.OW + ow);
    }
  }
  stf<T>(a.x, (n * a.C + c) * HW + p, s);
}

// ---- LDS-staged unfolding ------------------------------------------------------------------------------
// Raw element type: values are moved, never converted.
template <typename T>
using raw_t = std::conditional_t<std::is_same<T, F32>::value, uint32_t, uint16_t>;
template <typename T>
__device__ __forceinline__ u32x4 pack_raw(const raw_t<T> (&v)[vec16<T>()]) {
  if constexpr (std::is_same<T, F32>::value) return u32x4{v[0], v[1], v[2], v[3]};
  else
    return u32x4{v[0] | ((uint32_t)v[1] << 16), v[2] | ((uint32_t)v[3] << 16), v[4] | ((uint32_t)v[5] << 16),
                 v[6] | ((uint32_t)v[7] << 16)};
}
template <typename T>
__device__ __forceinline__ float raw_f32(raw_t<T> v) {
  if constexpr (std::is_same<T, F32>::value) return __uint_as_float(v);
  else return T::to_f32(v);
}

// grid (cdiv(OH, RB), C, N): workgroup (row block, c, n) copies the (rb - 1) SH + KH input rows its rb
// output rows read into LDS once, zero-padded (PW columns on each side, rows outside the image zero), then
// writes the KH*KW column rows of channel c for those output rows (a contiguous span of rb*OW elements
// each) from LDS; VEC (OW a multiple of the 16-byte vector, 16-byte aligned cols): one 16-byte store per
// lane and vector.  Input rows are read once per row block, output pixels are written once.
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void im2col_lds_k(hrt_im2col_args a, int RB) {
  using E = raw_t<T>;
  constexpr int V = vec16<T>();
  extern __shared__ __attribute__((aligned(16))) uint8_t im_lds[];
  E* const tile = reinterpret_cast<E*>(im_lds);
  const int OH = (int)a.OH, OW = (int)a.OW, H = (int)a.H, W = (int)a.W, SH = (int)a.SH, SW = (int)a.SW;
  const int PW = (int)a.PW, KH = (int)a.KH, KW = (int)a.KW, KK = KH * KW;
  const int oh0 = (int)blockIdx.x * RB, rb = min(RB, OH - oh0);
  const int c = blockIdx.y;
  const int64_t n = blockIdx.z;
  const int TR = (rb - 1) * SH + KH, TW = W + 2 * PW, h0 = oh0 * SH - (int)a.PH;
  const HK_G E* xs = gcptr<E>(a.x) + (n * a.C + c) * a.H * a.W;
  for (int i = threadIdx.x; i < TR * TW; i += 256) {
    const int r = i / TW, col = i - r * TW;
    const int h = h0 + r, w = col - PW;
    tile[i] = (h >= 0 && h < H && w >= 0 && w < W) ? xs[(int64_t)h * W + w] : (E)0;
  }
  __syncthreads();
  const int64_t K = a.C * KK;
  HK_G E* const cols = gptr<E>(a.cols) + ((n * K + (int64_t)c * KK) * OH + oh0) * (int64_t)OW;
  const int64_t rowlen = (int64_t)OH * OW;  // elements between consecutive k rows
  if constexpr (VEC) {
    const int per = rb * OW / V;  // vectors per k row span (OW % V == 0)
    for (int q = threadIdx.x; q < KK * per; q += 256) {
      const int kk = q / per, e0 = (q - kk * per) * V;
      const int kh = kk / KW, kw = kk - kh * KW;
      const int r = e0 / OW, ow0 = e0 - r * OW;
      const E* src = tile + (r * SH + kh) * TW + ow0 * SW + kw;
      E v[V];
#pragma unroll
      for (int j = 0; j < V; ++j) v[j] = src[j * SW];
      *reinterpret_cast<HK_G u32x4*>(cols + kk * rowlen + e0) = pack_raw<T>(v);
    }
  } else {
    const int span = rb * OW;
    for (int q = threadIdx.x; q < KK * span; q += 256) {
      const int kk = q / span, e = q - kk * span;
      const int kh = kk / KW, kw = kk - kh * KW;
      const int r = e / OW, ow = e - r * OW;
      cols[kk * rowlen + e] = tile[(r * SH + kh) * TW + ow * SW + kw];
    }
  }
}

// grid (cdiv(H, RB), C, N): the adjoint.  For each (kh, kw) the output rows that feed input rows
// [h0, h0 + rb) form a contiguous span of column row (c, kh, kw) (at most RO = (rb - 1) / SH + 1 rows); the
// workgroup copies all KH*KW spans into LDS (16-byte loads when VEC), then each lane sums, for its input
// pixels, the entries it fed in the order kh, then kw (the order of col2im_k, so the two agree bit for
// bit).  S1: unit strides (no divisibility tests).
template <typename T, bool VEC, bool S1>
__global__ __launch_bounds__(256) void col2im_lds_k(hrt_im2col_args a, int RB) {
  using E = raw_t<T>;
  constexpr int V = vec16<T>();
  extern __shared__ __attribute__((aligned(16))) uint8_t im_lds[];
  E* const tile = reinterpret_cast<E*>(im_lds);
  const int OH = (int)a.OH, OW = (int)a.OW, H = (int)a.H, W = (int)a.W, SH = (int)a.SH, SW = (int)a.SW;
  const int PH = (int)a.PH, PW = (int)a.PW, KH = (int)a.KH, KW = (int)a.KW, KK = KH * KW;
  const int h0 = (int)blockIdx.x * RB, rb = min(RB, H - h0);
  const int RO = (RB - 1) / SH + 1;  // LDS rows per (kh, kw)
  const int c = blockIdx.y;
  const int64_t n = blockIdx.z;
  const int64_t K = a.C * KK, rowlen = (int64_t)OH * OW;
  const HK_G E* cs = gcptr<E>(a.cols) + (n * K + (int64_t)c * KK) * rowlen;
  // first output row and row count of kernel row kh for this block
  auto ohlo = [&](int kh) {
    const int t = h0 + PH - kh;
    return t <= 0 ? 0 : (t + SH - 1) / SH;
  };
  auto ohcnt = [&](int kh) {
    const int t = h0 + rb - 1 + PH - kh;
    if (t < 0) return 0;
    const int hi = min(t / SH, OH - 1), lo = ohlo(kh);
    return hi >= lo ? hi - lo + 1 : 0;
  };
  if constexpr (VEC) {
    const int per = RO * OW / V;
    for (int q = threadIdx.x; q < KK * per; q += 256) {
      const int kk = q / per, e0 = (q - kk * per) * V;
      const int kh = kk / KW;
      if (e0 < ohcnt(kh) * OW)
        *reinterpret_cast<u32x4*>(tile + kk * RO * OW + e0) =
            *reinterpret_cast<const HK_G u32x4*>(cs + kk * rowlen + (int64_t)ohlo(kh) * OW + e0);
    }
  } else {
    const int per = RO * OW;
    for (int q = threadIdx.x; q < KK * per; q += 256) {
      const int kk = q / per, e = q - kk * per;
      const int kh = kk / KW;
      if (e < ohcnt(kh) * OW) tile[q] = cs[kk * rowlen + (int64_t)ohlo(kh) * OW + e];
    }
  }
  __syncthreads();
  constexpr int NV = VEC ? V : 1;
  const int per = rb * W / NV;  // VEC: W % V == 0
  for (int q = threadIdx.x; q < per; q += 256) {
    const int e0 = q * NV, r = e0 / W, w0 = e0 - r * W, h = h0 + r;
    float s[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) s[j] = 0.0f;
    for (int kh = 0; kh < KH; ++kh) {
      const int th = h + PH - kh;
      if (th < 0 || (!S1 && th % SH)) continue;
      const int oh = S1 ? th : th / SH;
      if (oh >= OH) continue;
      const E* trow = tile + (kh * KW * RO + (oh - ohlo(kh))) * OW;
      for (int kw = 0; kw < KW; ++kw) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
          const int tw = w0 + j + PW - kw;
          if (tw < 0 || (!S1 && tw % SW)) continue;
          const int ow = S1 ? tw : tw / SW;
          if (ow < OW) s[j] += raw_f32<T>(trow[kw * RO * OW + ow]);
        }
      }
    }
    if constexpr (VEC) stv<T>(a.x, ((n * a.C + c) * a.H + h0) * a.W + e0, s);
    else stf<T>(a.x, ((n * a.C + c) * a.H + h0) * a.W + e0, s[0]);
  }
}

// Row blocks of the LDS-staged kernels: about 1024 output (im2col) or input (col2im) pixels per
// workgroup (faster than 512 or 2048 on a 64x64 image), halved until the staged rows take at most
// 32 KiB; 0 when one row block does not fit 64 KiB (then the per-element kernels run).
int64_t im2col_rows(const hrt_im2col_args& a, uint64_t es, int64_t* lds) {
  const int64_t TW = a.W + 2 * a.PW;
  auto need = [&](int64_t rb) { return ((rb - 1) * a.SH + a.KH) * TW * (int64_t)es; };
  int64_t rb = std::max<int64_t>(1, std::min<int64_t>(a.OH, 1024 / std::max<int64_t>(a.OW, 1)));
  while (rb > 1 && need(rb) > 32768) rb = (rb + 1) / 2;
  *lds = (need(rb) + 15) / 16 * 16;
  return *lds <= 65536 ? rb : 0;
}
int64_t col2im_rows(const hrt_im2col_args& a, uint64_t es, int64_t* lds) {
  auto need = [&](int64_t rb) { return a.KH * a.KW * ((rb - 1) / a.SH + 1) * a.OW * (int64_t)es; };
  int64_t rb = std::max<int64_t>(1, std::min<int64_t>(a.H, 1024 / std::max<int64_t>(a.W, 1)));
  while (rb > 1 && need(rb) > 32768) rb = (rb + 1) / 2;
  *lds = (need(rb) + 15) / 16 * 16;
  return *lds <= 65536 ? rb : 0;
}

bool im2col_check(const hrt_im2col_args& a, hrt::LaunchCtx& ctx, uint64_t es) {
  if (a.N <= 0 || a.C <= 0 || a.H <= 0 || a.W <= 0 || a.KH <= 0 || a.KW <= 0 || a.SH <= 0 || a.SW <= 0 || a.PH < 0 ||
      a.PW < 0)
    return ctx.fail("sizes and strides must be positive, padding non-negative");
  if (a.OH != (a.H + 2 * a.PH - a.KH) / a.SH + 1 || a.OW != (a.W + 2 * a.PW - a.KW) / a.SW + 1 ||
      a.H + 2 * a.PH < a.KH || a.W + 2 * a.PW < a.KW)
    return ctx.fail("OH/OW do not follow from H, W, the kernel, stride and padding");
  if (a.C * a.KH * a.KW > 65535 || a.N > 65535 || a.C > 65535) return ctx.fail("C*KH*KW, C and N must be <= 65535");
  return ctx.check(a.x, (uint64_t)(a.N * a.C * a.H * a.W) * es, "x") &&
         ctx.check(a.cols, (uint64_t)(a.N * a.C * a.KH * a.KW * a.OH * a.OW) * es, "cols");
}

template <typename T>
bool launch_im2col(const void* p, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_im2col_args*>(p);
  if (!im2col_check(a, ctx, esz<T>())) return false;
  constexpr int V = vec16<T>();
  int64_t lds = 0;
  const int64_t rb = im2col_rows(a, esz<T>(), &lds);
  if (rb > 0) {
    const dim3 g((uint32_t)cdiv(a.OH, rb), (uint32_t)a.C, (uint32_t)a.N);
    if (a.OW % V == 0 && a.cols % 16 == 0)
      hipLaunchKernelGGL((im2col_lds_k<T, true>), g, dim3(256), (uint32_t)lds, ctx.stream, a, (int)rb);
    else
      hipLaunchKernelGGL((im2col_lds_k<T, false>), g, dim3(256), (uint32_t)lds, ctx.stream, a, (int)rb);
  } else if (a.OW % V == 0 && a.cols % 16 == 0) {
    const dim3 g((uint32_t)cdiv(a.OH * a.OW / V, 256), (uint32_t)(a.C * a.KH * a.KW), (uint32_t)a.N);
    hipLaunchKernelGGL(im2col_vec_k<T>, g, dim3(256), 0, ctx.stream, a);
  } else {
    const dim3 g((uint32_t)cdiv(a.OH * a.OW, 256), (uint32_t)(a.C * a.KH * a.KW), (uint32_t)a.N);
    hipLaunchKernelGGL(im2col_k<T>, g, dim3(256), 0, ctx.stream, a);
  }
  return hrt::launch_ok(hipGetLastError(), ctx, "im2col");
}
template <typename T>
bool launch_col2im(const void* p, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_im2col_args*>(p);
  if (!im2col_check(a, ctx, esz<T>())) return false;
  constexpr int V = vec16<T>();
  int64_t lds = 0;
  const int64_t rb = col2im_rows(a, esz<T>(), &lds);
  if (rb > 0) {
    const dim3 g((uint32_t)cdiv(a.H, rb), (uint32_t)a.C, (uint32_t)a.N);
    const bool vec = a.OW % V == 0 && a.W % V == 0 && a.cols % 16 == 0 && a.x % 16 == 0;
    const bool s1 = a.SH == 1 && a.SW == 1;
    const uint32_t sh = (uint32_t)lds;
    if (vec && s1) hipLaunchKernelGGL((col2im_lds_k<T, true, true>), g, dim3(256), sh, ctx.stream, a, (int)rb);
    else if (vec) hipLaunchKernelGGL((col2im_lds_k<T, true, false>), g, dim3(256), sh, ctx.stream, a, (int)rb);
    else if (s1) hipLaunchKernelGGL((col2im_lds_k<T, false, true>), g, dim3(256), sh, ctx.stream, a, (int)rb);
    else hipLaunchKernelGGL((col2im_lds_k<T, false, false>), g, dim3(256), sh, ctx.stream, a, (int)rb);
  } else {
    const dim3 g((uint32_t)cdiv(a.H * a.W, 256), (uint32_t)a.C, (uint32_t)a.N);
    hipLaunchKernelGGL(col2im_k<T>, g, dim3(256), 0, ctx.stream, a);
  }
  return hrt::launch_ok(hipGetLastError(), ctx, "col2im");
}
HRT_REGISTER("im2col_f32", hrt_im2col_args, launch_im2col<F32>);
HRT_REGISTER("im2col_bf16", hrt_im2col_args, launch_im2col<BF16>);
HRT_REGISTER("im2col_f16", hrt_im2col_args, launch_im2col<F16>);
HRT_REGISTER("col2im_f32", hrt_im2col_args, launch_col2im<F32>);
HRT_REGISTER("col2im_bf16", hrt_im2col_args, launch_col2im<BF16>);
HRT_REGISTER("col2im_f16", hrt_im2col_args, launch_col2im<F16>);

// ---- nearest upsampling by integer factors ----------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void up_fwd_k(hrt_upsample_args a, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int64_t ow = i % a.OW, t = i / a.OW, oh = t % a.OH, nc = t / a.OH;
  const int64_t fh = a.OH / a.H, fw = a.OW / a.W;
  stf<T>(a.dst, i, ldf<T>(a.src, (nc * a.H + oh / fh) * a.W + ow / fw));
}

// dst [NC, H, W] = block sums of src [NC, OH, OW] (rows of the block in order, then columns).
template <typename T>
__global__ __launch_bounds__(256) void up_bwd_k(hrt_upsample_args a, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int64_t w = i % a.W, t = i / a.W, h = t % a.H, nc = t / a.H;
  const int64_t fh = a.OH / a.H, fw = a.OW / a.W;
  float s = 0.0f;
  for (int64_t y = 0; y < fh; ++y)
    for (int64_t x = 0; x < fw; ++x) s += ldf<T>(a.src, (nc * a.OH + h * fh + y) * a.OW + w * fw + x);
  stf<T>(a.dst, i, s);
}

// One lane per 16-byte output vector of an input row: the vector's source elements are loaded once (one
// 8-byte load when F2, i.e. fw == 2: each source element fills two output slots) and the vector is stored
// to the fh output rows that repeat the input row.  total = NC * H * OW / V vectors; OW % V == 0.
template <typename T, bool F2>
__global__ __launch_bounds__(256) void up_fwd_rows_k(hrt_upsample_args a, int64_t total) {
  constexpr int V = vec16<T>();
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int64_t per = a.OW / V, srow = i / per, ow0 = (i - srow * per) * V;  // srow = nc * H + ih
  const int64_t fh = a.OH / a.H, nc = srow / a.H, ih = srow - nc * a.H;
  u32x4 out;
  if constexpr (F2) {
    const u32x2 u = *reinterpret_cast<const HK_G u32x2*>(gcptr<raw_t<T>>(a.src) + srow * a.W + ow0 / 2);
    if constexpr (std::is_same<T, F32>::value) {
      out = u32x4{u.x, u.x, u.y, u.y};
    } else {
      auto dup = [](uint32_t e) { return (e & 0xffffu) | (e << 16); };
      out = u32x4{dup(u.x & 0xffffu), dup(u.x >> 16), dup(u.y & 0xffffu), dup(u.y >> 16)};
    }
  } else {
    const int64_t fw = a.OW / a.W;
    raw_t<T> v[V];
#pragma unroll
    for (int j = 0; j < V; ++j) v[j] = gcptr<raw_t<T>>(a.src)[srow * a.W + (ow0 + j) / fw];
    out = pack_raw<T>(v);
  }
  HK_G raw_t<T>* dst = gptr<raw_t<T>>(a.dst) + (nc * a.OH + ih * fh) * a.OW + ow0;
  for (int64_t y = 0; y < fh; ++y) *reinterpret_cast<HK_G u32x4*>(dst + y * a.OW) = out;
}

// Backward for fw == 2 and W % V == 0: a lane sums V input pixels; each of the fh source rows gives two
// 16-byte loads (2V columns).  Same order as up_bwd_k: rows, then the two columns of each.
template <typename T>
__global__ __launch_bounds__(256) void up_bwd_vec2_k(hrt_upsample_args a, int64_t total) {
  constexpr int V = vec16<T>();
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * V;
  if (i >= total) return;
  const int64_t row = i / a.W, w0 = i - row * a.W, nc = row / a.H, h = row - nc * a.H;
  const int64_t fh = a.OH / a.H;
  float s[V];
#pragma unroll
  for (int j = 0; j < V; ++j) s[j] = 0.0f;
  for (int64_t y = 0; y < fh; ++y) {
    const int64_t sb = (nc * a.OH + h * fh + y) * a.OW + 2 * w0;
    float u0[V], u1[V];
    ldv<T>(a.src, sb, u0);
    ldv<T>(a.src, sb + V, u1);
#pragma unroll
    for (int j = 0; j < V / 2; ++j) {
      s[j] += u0[2 * j];
      s[j] += u0[2 * j + 1];
      s[V / 2 + j] += u1[2 * j];
      s[V / 2 + j] += u1[2 * j + 1];
    }
  }
  stv<T>(a.dst, i, s);
}

template <typename T, bool FWD>
bool launch_up(const void* p, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_upsample_args*>(p);
  if (a.NC <= 0 || a.H <= 0 || a.W <= 0 || a.OH < a.H || a.OW < a.W || a.OH % a.H || a.OW % a.W)
    return ctx.fail("upsample needs positive sizes and integer factors OH / H, OW / W");
  const uint64_t small = (uint64_t)(a.NC * a.H * a.W) * esz<T>(), big = (uint64_t)(a.NC * a.OH * a.OW) * esz<T>();
  if (!ctx.check(a.src, FWD ? small : big, "src") || !ctx.check(a.dst, FWD ? big : small, "dst")) return false;
  const int64_t total = FWD ? a.NC * a.OH * a.OW : a.NC * a.H * a.W;
  constexpr int V = vec16<T>();
  const int64_t fw = a.OW / a.W;
  if (FWD && a.OW % V == 0 && a.dst % 16 == 0) {
    const int64_t vecs = a.NC * a.H * (a.OW / V);
    const dim3 g((uint32_t)cdiv(vecs, 256));
    if (fw == 2 && a.src % 8 == 0) hipLaunchKernelGGL((up_fwd_rows_k<T, true>), g, dim3(256), 0, ctx.stream, a, vecs);
    else hipLaunchKernelGGL((up_fwd_rows_k<T, false>), g, dim3(256), 0, ctx.stream, a, vecs);
  } else if (!FWD && fw == 2 && a.W % V == 0 && a.src % 16 == 0 && a.dst % 16 == 0)
    hipLaunchKernelGGL(up_bwd_vec2_k<T>, dim3((uint32_t)cdiv(total / V, 256)), dim3(256), 0, ctx.stream, a, total);
  else if (FWD)
    hipLaunchKernelGGL(up_fwd_k<T>, dim3((uint32_t)cdiv(total, 256)), dim3(256), 0, ctx.stream, a, total);
  else
    hipLaunchKernelGGL(up_bwd_k<T>, dim3((uint32_t)cdiv(total, 256)), dim3(256), 0, ctx.stream, a, total);
  return hrt::launch_ok(hipGetLastError(), ctx, "upsample_nearest");
}
HRT_REGISTER("upsample_nearest_fwd_f32", hrt_upsample_args, (launch_up<F32, true>));
HRT_REGISTER("upsample_nearest_fwd_bf16", hrt_upsample_args, (launch_up<BF16, true>));
HRT_REGISTER("upsample_nearest_fwd_f16", hrt_upsample_args, (launch_up<F16, true>));
HRT_REGISTER("upsample_nearest_bwd_f32", hrt_upsample_args, (launch_up<F32, false>));
HRT_REGISTER("upsample_nearest_bwd_bf16", hrt_upsample_args, (launch_up<BF16, false>));
HRT_REGISTER("upsample_nearest_bwd_f16", hrt_upsample_args, (launch_up<F16, false>));

// ---- group_norm ---------------------------------------------------------------------------------------------
struct Wf {
  float n, mean, m2;  // count, mean, sum of squared deviations
};
__device__ __forceinline__ Wf wf_merge(Wf a, Wf b) {
  const float n = a.n + b.n;
  if (n == 0.0f) return a;
  const float d = b.mean - a.mean, f = b.n / n;
  return {n, a.mean + d * f, a.m2 + b.m2 + d * d * a.n * f};
}
__device__ __forceinline__ Wf wf_shfl(Wf v, int m) {
  return {__shfl_xor(v.n, m, 64), __shfl_xor(v.mean, m, 64), __shfl_xor(v.m2, m, 64)};
}
// Workgroup-wide merge of 256 lanes' statistics in a fixed tree order; the result is in lane 0 of wave 0.
__device__ __forceinline__ Wf wf_block(Wf v, Wf* lds) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v = wf_merge(v, wf_shfl(v, m));
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) lds[w] = v;
  __syncthreads();
  return wf_merge(wf_merge(lds[0], lds[1]), wf_merge(lds[2], lds[3]));
}

// Visits e = first, first + step, ... < end in order, calling f(e, v) with v the V elements of p at base
// + e; the loads of four consecutive visits are issued before the first of them is used (one 16-byte load
// in flight per lane leaves HBM latency-bound at these grid sizes).
template <typename T, int V, class F>
__device__ __forceinline__ void visit4(uint64_t p, int64_t base, int64_t first, int64_t end, int64_t step, F&& f) {
  for (int64_t e0 = first; e0 < end; e0 += 4 * step) {
    float v[4][V];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (e0 + u * step < end) ldn<T, V>(p, base + e0 + u * step, v[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (e0 + u * step < end) f(e0 + u * step, v[u]);
  }
}
// The same over two tensors read at the same positions.
template <typename T, int V, class F>
__device__ __forceinline__ void visit4x2(uint64_t p, uint64_t r, int64_t base, int64_t first, int64_t end, int64_t step,
                                         F&& f) {
  for (int64_t e0 = first; e0 < end; e0 += 4 * step) {
    float v[4][V], w[4][V];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (e0 + u * step < end) {
        ldn<T, V>(p, base + e0 + u * step, v[u]);
        ldn<T, V>(r, base + e0 + u * step, w[u]);
      }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (e0 + u * step < end) f(v[u], w[u]);
  }
}

// grid (chunks, N*G): statistics of chunk q of group ng (its elements are contiguous: x is [N, C, HW]),
// each lane summing deviations from the chunk's first element.  V elements per access (V divides HW and
// the chunk size).
template <typename T, int V>
__global__ __launch_bounds__(256) void gn_stats_k(hrt_gn_args a, int64_t chunks, int64_t cs) {
  __shared__ Wf lds[4];
  const int64_t M = (a.C / a.G) * a.HW;
  const int64_t ng = blockIdx.y, q = blockIdx.x;
  const int64_t lo = q * cs, hi = min(M, lo + cs);
  const int64_t base = ng * M;
  const float k = lo < hi ? ldf<T>(a.x, base + lo) : 0.0f;  // an empty last chunk reads nothing
  float s = 0.0f, s2 = 0.0f, cnt = 0.0f;
  visit4<T, V>(a.x, base, lo + (int64_t)threadIdx.x * V, hi, 256 * V, [&](int64_t, const float (&v)[V]) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float d = v[j] - k;
      s += d;
      s2 += d * d;
    }
    cnt += (float)V;
  });
  Wf w = cnt > 0.0f ? Wf{cnt, k + s / cnt, s2 - s * s / cnt} : Wf{0.0f, 0.0f, 0.0f};
  w = wf_block(w, lds);
  if (threadIdx.x == 0) {
    HK_G float* ws = gptr<float>(a.ws) + (ng * chunks + q) * 3;
    ws[0] = w.n;
    ws[1] = w.mean;
    ws[2] = fmaxf(w.m2, 0.0f);
  }
}

// grid (cdiv(M, cs), N*G): merge the group's `chunks` statistics partials, write mean / rstd (block 0),
// normalise elements [q cs, (q + 1) cs) of the group (V consecutive elements share a channel since V
// divides HW).  cs is the apply block (4096), finer than the statistics chunks, so that more workgroups
// are resident to stream the tensor.
template <typename T, int V>
__global__ __launch_bounds__(256) void gn_apply_k(hrt_gn_args a, int64_t chunks, int64_t cs) {
  __shared__ float st[2];
  const int64_t Cg = a.C / a.G, M = Cg * a.HW;
  const int64_t ng = blockIdx.y, q = blockIdx.x;
  if (threadIdx.x < 64) {
    // the group's chunk statistics, merged by wave 0 in a fixed order: lane l takes chunks l, l + 64, ..,
    // then a butterfly in which both partners merge (lower lane, upper lane), so every lane, and every
    // workgroup of the group, ends with the same bits
    const HK_G float* ws = gcptr<float>(a.ws) + ng * chunks * 3;
    Wf v{0.0f, 0.0f, 0.0f};
    for (int64_t i = threadIdx.x; i < chunks; i += 64) v = wf_merge(v, Wf{ws[3 * i], ws[3 * i + 1], ws[3 * i + 2]});
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      const Wf o = wf_shfl(v, m);
      v = (threadIdx.x & m) ? wf_merge(o, v) : wf_merge(v, o);
    }
    if (threadIdx.x == 0) {
      const float var = v.m2 / v.n;
      st[0] = v.mean;
      st[1] = 1.0f / sqrtf(var + a.eps);
      if (q == 0) {
        stf<T>(a.mean, ng, st[0]);
        stf<T>(a.rstd, ng, st[1]);
      }
    }
  }
  __syncthreads();
  const float mean = st[0], rstd = st[1];
  const int64_t g = ng % a.G;
  const int64_t lo = q * cs, hi = min(M, lo + cs), base = ng * M;
  // four vectors per round, with their x, w and b loads all issued before the first store (y may alias w
  // and b as far as the compiler knows, so loads after a store would wait for it)
  constexpr int64_t step = 256 * V;
  for (int64_t e0 = lo + (int64_t)threadIdx.x * V; e0 < hi; e0 += 4 * step) {
    float x[4][V], wc[4], bc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t e = e0 + u * step;
      if (e < hi) {
        ldn<T, V>(a.x, base + e, x[u]);
        const int64_t c = g * Cg + e / a.HW;
        wc[u] = a.w ? ldf<T>(a.w, c) : 1.0f;
        bc[u] = a.b ? ldf<T>(a.b, c) : 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t e = e0 + u * step;
      if (e < hi) {
        float v[V];
#pragma unroll
        for (int j = 0; j < V; ++j) v[j] = (x[u][j] - mean) * rstd * wc[u] + bc[u];
        stn<T, V>(a.y, base + e, v);
      }
    }
  }
}

// grid (N*C): ws[nc] = sum_hw g*x, ws[N*C + nc] = sum_hw g.
template <typename T, int V>
__global__ __launch_bounds__(256) void gn_bwd_sums_k(hrt_gn_args a) {
  __shared__ float red[4];
  const int64_t nc = blockIdx.x, base = nc * a.HW;
  float ds = 0.0f, db = 0.0f;
  visit4x2<T, V>(a.g, a.x, base, (int64_t)threadIdx.x * V, a.HW, 256 * V, [&](const float (&g)[V], const float (&x)[V]) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      ds += g[j] * x[j];
      db += g[j];
    }
  });
  ds = block_sum<4>(ds, red);
  __syncthreads();
  db = block_sum<4>(db, red);
  if (threadIdx.x == 0) {
    gptr<float>(a.ws)[nc] = ds;
    gptr<float>(a.ws)[a.N * a.C + nc] = db;
  }
}

// grid (cdiv(HW / V, 256), N*C): dx = rstd*w*g + c2*x + c3.  c2 and c3 of the channel's group are formed
// by wave 0 from the per-channel sums (lane j takes channels j, j + 64, .. of the group, then a butterfly
// sum; a + b == b + a, so every lane, and every workgroup of the group, gets the same bits) while the
// workgroup's g and x loads are in flight.
template <typename T, int V>
__global__ __launch_bounds__(256) void gn_bwd_dx_k(hrt_gn_args a) {
  __shared__ float cc[2];
  const int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) * V;
  const int64_t nc = blockIdx.y, n = nc / a.C, c = nc % a.C, Cg = a.C / a.G, g = c / Cg, ng = n * a.G + g;
  const bool live = e < a.HW;
  const int64_t i = nc * a.HW + e;
  float gv[V], xv[V];
  if (live) {
    ldn<T, V>(a.g, i, gv);
    ldn<T, V>(a.x, i, xv);
  }
  if (threadIdx.x < 64) {
    const HK_G float* ws = gcptr<float>(a.ws);
    float dsg = 0.0f, dbg = 0.0f;
    for (int64_t j = threadIdx.x; j < Cg; j += 64) {
      const int64_t cj = g * Cg + j;
      const float w = a.w ? ldf<T>(a.w, cj) : 1.0f;
      dsg += ws[n * a.C + cj] * w;
      dbg += ws[a.N * a.C + n * a.C + cj] * w;
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      dsg += __shfl_xor(dsg, m, 64);
      dbg += __shfl_xor(dbg, m, 64);
    }
    if (threadIdx.x == 0) {
      const float mean = ldf<T>(a.mean, ng), rstd = ldf<T>(a.rstd, ng);
      const float s = 1.0f / (float)(Cg * a.HW);
      const float c2 = (dbg * mean - dsg) * rstd * rstd * rstd * s;
      cc[0] = c2;
      cc[1] = -c2 * mean - dbg * rstd * s;
    }
  }
  __syncthreads();
  if (!live) return;
  const float c1 = ldf<T>(a.rstd, ng) * (a.w ? ldf<T>(a.w, c) : 1.0f), c2 = cc[0], c3 = cc[1];
#pragma unroll
  for (int j = 0; j < V; ++j) gv[j] = c1 * gv[j] + c2 * xv[j] + c3;
  stn<T, V>(a.dx, i, gv);
}

// Thread per channel: dw[c] = sum_n (ds - db*mean)*rstd, db[c] = sum_n db, n in order.
template <typename T>
__global__ __launch_bounds__(256) void gn_bwd_wgrad_k(hrt_gn_args a) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= a.C) return;
  const HK_G float* ws = gcptr<float>(a.ws);
  const int64_t g = c / (a.C / a.G);
  float dw = 0.0f, db = 0.0f;
  for (int64_t n = 0; n < a.N; ++n) {
    const float ds = ws[n * a.C + c], dbn = ws[a.N * a.C + n * a.C + c];
    dw += (ds - dbn * ldf<T>(a.mean, n * a.G + g)) * ldf<T>(a.rstd, n * a.G + g);
    db += dbn;
  }
  if (a.dw) stf<T>(a.dw, c, dw);
  if (a.db) stf<T>(a.db, c, db);
}

template <typename T>
bool gn_check(const hrt_gn_args& a, hrt::LaunchCtx& ctx) {
  if (a.N <= 0 || a.C <= 0 || a.HW <= 0 || a.G <= 0 || a.C % a.G) return ctx.fail("need N, C, HW, G > 0 and G dividing C");
  const uint64_t es = esz<T>(), n = (uint64_t)(a.N * a.C * a.HW) * es;
  if (!ctx.check(a.x, n, "x") || !ctx.check(a.ws, (uint64_t)hrt_gn_workspace(a.N, a.C, a.HW, a.G) * 4, "ws")) return false;
  if (!ctx.check(a.mean, (uint64_t)(a.N * a.G) * es, "mean") || !ctx.check(a.rstd, (uint64_t)(a.N * a.G) * es, "rstd"))
    return false;
  if (a.w && !ctx.check(a.w, (uint64_t)a.C * es, "w")) return false;
  return true;
}

template <typename T>
bool launch_gn_fwd(const void* p, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_gn_args*>(p);
  if (!gn_check<T>(a, ctx)) return false;
  if (!ctx.check(a.y, (uint64_t)(a.N * a.C * a.HW) * esz<T>(), "y")) return false;
  if (a.b && !ctx.check(a.b, (uint64_t)a.C * esz<T>(), "b")) return false;
  if (a.N * a.G > 65535) return ctx.fail("N * G must be <= 65535");
  constexpr int V = vec16<T>();
  const bool vec = a.HW % V == 0 && a.x % 16 == 0 && a.y % 16 == 0;
  const int64_t chunks = hrt_gn_chunks(a.C, a.HW, a.G), M = (a.C / a.G) * a.HW;
  const int64_t cs = vec ? cdiv(cdiv(M, chunks), V) * V : cdiv(M, chunks);  // chunks start on a vector
  const dim3 g((uint32_t)chunks, (uint32_t)(a.N * a.G));
  // apply block (a multiple of every V): 16384 elements, each workgroup's merge of its group's statistics
  // then paying for four times the data of 4096 (group_norm of [1, 512, 128, 128] / [1, 256, 256, 256] /
  // [1, 128, 512, 512] bf16: 16.2 -> 15.5, 25.5 -> 22.8, 43.4 -> 38.3-39.2 us; 32768 and 65536 were slower),
  // unless that leaves fewer than 256 workgroups
  const int64_t AS = cdiv(M, 16384) * a.N * a.G >= 256 ? 16384 : 4096;
  const dim3 ga((uint32_t)cdiv(M, AS), (uint32_t)(a.N * a.G));
  if (vec) {
    hipLaunchKernelGGL((gn_stats_k<T, V>), g, dim3(256), 0, ctx.stream, a, chunks, cs);
    hipLaunchKernelGGL((gn_apply_k<T, V>), ga, dim3(256), 0, ctx.stream, a, chunks, AS);
  } else {
    hipLaunchKernelGGL((gn_stats_k<T, 1>), g, dim3(256), 0, ctx.stream, a, chunks, cs);
    hipLaunchKernelGGL((gn_apply_k<T, 1>), ga, dim3(256), 0, ctx.stream, a, chunks, AS);
  }
  return hrt::launch_ok(hipGetLastError(), ctx, "gn_fwd");
}

template <typename T>
bool launch_gn_bwd(const void* p, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_gn_args*>(p);
  if (!gn_check<T>(a, ctx)) return false;
  const uint64_t n = (uint64_t)(a.N * a.C * a.HW) * esz<T>();
  if (!ctx.check(a.g, n, "g") || (a.dx && !ctx.check(a.dx, n, "dx")) ||
      (a.dw && !ctx.check(a.dw, (uint64_t)a.C * esz<T>(), "dw")) || (a.db && !ctx.check(a.db, (uint64_t)a.C * esz<T>(), "db")))
    return false;
  if (a.N * a.C >= ((int64_t)1 << 31)) return ctx.fail("N * C must be < 2^31");
  if (a.dx && a.N * a.C > 65535) return ctx.fail("N * C must be <= 65535 for dx");
  constexpr int V = vec16<T>();
  const bool vec = a.HW % V == 0 && a.x % 16 == 0 && a.g % 16 == 0 && a.dx % 16 == 0;
  if (vec) hipLaunchKernelGGL((gn_bwd_sums_k<T, V>), dim3((uint32_t)(a.N * a.C)), dim3(256), 0, ctx.stream, a);
  else hipLaunchKernelGGL((gn_bwd_sums_k<T, 1>), dim3((uint32_t)(a.N * a.C)), dim3(256), 0, ctx.stream, a);
  if (a.dx) {
    const dim3 g((uint32_t)cdiv(vec ? a.HW / V : a.HW, 256), (uint32_t)(a.N * a.C));
    if (vec) hipLaunchKernelGGL((gn_bwd_dx_k<T, V>), g, dim3(256), 0, ctx.stream, a);
    else hipLaunchKernelGGL((gn_bwd_dx_k<T, 1>), g, dim3(256), 0, ctx.stream, a);
  }
  if (a.dw || a.db) hipLaunchKernelGGL(gn_bwd_wgrad_k<T>, dim3((uint32_t)cdiv(a.C, 256)), dim3(256), 0, ctx.stream, a);
  return hrt::launch_ok(hipGetLastError(), ctx, "gn_bwd");
}
HRT_REGISTER("gn_fwd_f32", hrt_gn_args, launch_gn_fwd<F32>);
HRT_REGISTER("gn_fwd_bf16", hrt_gn_args, launch_gn_fwd<BF16>);
HRT_REGISTER("gn_fwd_f16", hrt_gn_args, launch_gn_fwd<F16>);
HRT_REGISTER("gn_bwd_f32", hrt_gn_args, launch_gn_bwd<F32>);
HRT_REGISTER("gn_bwd_bf16", hrt_gn_args, launch_gn_bwd<BF16>);
HRT_REGISTER("gn_bwd_f16", hrt_gn_args, launch_gn_bwd<F16>);

}  // namespace
}  // namespace hk
