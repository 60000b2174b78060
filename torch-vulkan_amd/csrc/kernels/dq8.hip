// Weight-only int8 dequant (reference: vkrt/shaders/dq8.comp.in:39-62, closed form
// torch_vulkan/__init__.py:203-205):  out[r, c] = round_dt(float(q[r, c]) * float(scale[r, c / 64])).
//
// HBM-bound: 1 byte in + 2 (bf16/f16) or 4 (f32) bytes out per element plus 2 bytes of scale per 64.
// Fast paths (cols % 16 == 0): bf16 / f16 outputs take dq8_vec16 (below: 8-element groups laid out so that
// every store instruction writes 1 KB contiguously).  fp32 outputs: each thread moves 16 int8 with one
// streaming 128-bit load and writes them with 128-bit streaming stores (a 16-element chunk never crosses a
// row or a 64-column scale block); one chunk per thread and many workgroups streams best (measured against
// 1-8 chunks per thread).  The
// chunk's row comes from a double-precision reciprocal of the chunks-per-row count corrected by one step,
// which is exact for every chunk index below 2^40 (the product is then within 2^-12 of ch / cpr, so the
// truncation is off by at most one; no 64-bit integer division).  Any other shape or alignment takes the
// per-element path.  Results are bit-exact: the fp32 product of an int8 and a bf16 is exact, so the only
// rounding is the final RNE store.
#include <type_traits>

#include "../hrt/registry.h"
#include "device_common.h"

namespace hk {
namespace {

constexpr int kChunks = 1;  // 16-element chunks per thread

template <typename T>
__device__ __forceinline__ void store16(typename T::storage* out, int64_t e, const float* v);

template <>
__device__ __forceinline__ void store16<BF16>(uint16_t* out, int64_t e, const float* v) {
  u32x4 w0, w1;
  w0.x = pack2<BF16>(v[0], v[1]);
  w0.y = pack2<BF16>(v[2], v[3]);
  w0.z = pack2<BF16>(v[4], v[5]);
  w0.w = pack2<BF16>(v[6], v[7]);
  w1.x = pack2<BF16>(v[8], v[9]);
  w1.y = pack2<BF16>(v[10], v[11]);
  w1.z = pack2<BF16>(v[12], v[13]);
  w1.w = pack2<BF16>(v[14], v[15]);
  u32x4* o = reinterpret_cast<u32x4*>(out + e);
  __builtin_nontemporal_store(w0, o);
  __builtin_nontemporal_store(w1, o + 1);
}
template <>
__device__ __forceinline__ void store16<F16>(uint16_t* out, int64_t e, const float* v) {
  u32x4 w0, w1;
  w0.x = pack2<F16>(v[0], v[1]);
  w0.y = pack2<F16>(v[2], v[3]);
  w0.z = pack2<F16>(v[4], v[5]);
  w0.w = pack2<F16>(v[6], v[7]);
  w1.x = pack2<F16>(v[8], v[9]);
  w1.y = pack2<F16>(v[10], v[11]);
  w1.z = pack2<F16>(v[12], v[13]);
  w1.w = pack2<F16>(v[14], v[15]);
  u32x4* o = reinterpret_cast<u32x4*>(out + e);
  __builtin_nontemporal_store(w0, o);
  __builtin_nontemporal_store(w1, o + 1);
}
template <>
__device__ __forceinline__ void store16<F32>(float* out, int64_t e, const float* v) {
  f32x4* o = reinterpret_cast<f32x4*>(out + e);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f32x4 w = {v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
    __builtin_nontemporal_store(w, o + i);
  }
}

__device__ __forceinline__ float sbyte(uint32_t w, int i) { return (float)(int8_t)((w >> (8 * i)) & 0xffu); }

template <typename T>
__global__ __launch_bounds__(256) void dq8_vec(const int8_t* __restrict__ q, const uint16_t* __restrict__ scale,
                                               typename T::storage* __restrict__ out, int64_t cols, int64_t nblocks,
                                               int64_t nchunks, double inv_cpr) {
  const int64_t base = (int64_t)blockIdx.x * (256 * kChunks) + threadIdx.x;
  const int64_t cpr = cols >> 4;  // chunks per row
  u32x4 qv[kChunks];
  float sv[kChunks];
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int64_t ch = base + c * 256;
    if (ch < nchunks) {
      qv[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(q + ch * 16));
      int64_t r = (int64_t)((double)ch * inv_cpr);
      if (r * cpr > ch) --r;
      else if ((r + 1) * cpr <= ch) ++r;
      const int64_t col = (ch - r * cpr) << 4;
      sv[c] = bf16_bits_to_f32(scale[r * nblocks + (col >> 6)]);
    }
  }
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int64_t ch = base + c * 256;
    if (ch < nchunks) {
      float v[16];
      const uint32_t w[4] = {qv[c].x, qv[c].y, qv[c].z, qv[c].w};
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = sbyte(w[i >> 2], i & 3) * sv[c];
      store16<T>(out, ch * 16, v);
    }
  }
}

// 16-bit outputs: wavefront w takes elements [1024 w, 1024 w + 1024) as two halves, lane l the 8 elements at
// 8 l of each half, so every load instruction reads 512 contiguous bytes and every store instruction writes
// 1 KB contiguously (with 16 consecutive elements per lane, each store instruction of a wavefront wrote
// every other 16 bytes of a 2 KB span).  bf16: the hardware conversion (v_cvt_pk_bf16_f32, the contract's
// round-to-nearest-even for every non-NaN value) when the group's scale is finite, since an int8 times a
// finite scale is never NaN; the software rounding otherwise (NaN -> 0x7FC0).
template <typename T>
__device__ __forceinline__ u32x4 dq8_group(uint32_t lo, uint32_t hi, float s) {
  float v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = sbyte(lo, i) * s, v[4 + i] = sbyte(hi, i) * s;
  if constexpr (std::is_same<T, BF16>::value) {
    if (__builtin_isfinite(s)) return bf16_pack8_hw(v);
    return bf16_pack8_sw(v);
  } else {
    return u32x4{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3]), pack2<T>(v[4], v[5]), pack2<T>(v[6], v[7])};
  }
}

// ROW: cols % 1024 == 0, so each 1024-element span lies in one row, found once per span (a 32-bit quotient
// through a double reciprocal, exact after one correction), and a wavefront takes two consecutive spans
// (all four loads in flight together: ~2% faster than one span); otherwise a wavefront takes one span and
// each lane finds the row of each of its groups (64-bit, as dq8_vec).  Loads stay nontemporal: cached
// loads measured faster only while the int8 inputs fit the last-level cache, 4% slower beyond it.
template <typename T, bool ROW>
__global__ __launch_bounds__(256) void dq8_vec16(const int8_t* __restrict__ q, const uint16_t* __restrict__ scale,
                                                 typename T::storage* __restrict__ out, int64_t cols, int64_t nblocks,
                                                 int64_t total, double inv_cols, uint32_t spans_per_row,
                                                 double inv_spans_per_row) {
  const int lane = threadIdx.x & 63;
  if constexpr (ROW) {
    const uint32_t s0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 2;  // first of the wavefront's two spans
    const uint32_t ns = (uint32_t)(total >> 10);
    u32x2 qv[4];
    float sv[4];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const uint32_t si = s0 + p < ns ? s0 + p : ns - 1;  // a span past the end loads the last one, stores nothing
      uint32_t r = (uint32_t)((double)si * inv_spans_per_row);
      if (r * spans_per_row > si) --r;
      else if ((r + 1) * spans_per_row <= si) ++r;
      const int64_t e0 = (int64_t)si * 1024 + lane * 8;
      const uint32_t c0 = (si - r * spans_per_row) * 1024 + lane * 8;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        qv[2 * p + h] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(q + e0 + h * 512));
#pragma unroll
      for (int h = 0; h < 2; ++h) sv[2 * p + h] = bf16_bits_to_f32(scale[(int64_t)r * nblocks + ((c0 + h * 512) >> 6)]);
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      if (s0 + p >= ns) break;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        __builtin_nontemporal_store(dq8_group<T>(qv[2 * p + h].x, qv[2 * p + h].y, sv[2 * p + h]),
                                    reinterpret_cast<u32x4*>(out + (int64_t)(s0 + p) * 1024 + lane * 8 + h * 512));
    }
    return;
  }
  const uint32_t wi = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t w0 = (int64_t)wi * 1024 + lane * 8;
  u32x2 qv[2];
  float sv[2];
  {
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // both halves' loads issued before either is used
      const int64_t e = w0 + h * 512;
      const int64_t el = e < total ? e : total - 8;  // a group past the end loads the last one and stores nothing
      qv[h] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(q + el));
      int64_t r = (int64_t)((double)el * inv_cols);
      if (r * cols > el) --r;
      else if ((r + 1) * cols <= el) ++r;
      sv[h] = bf16_bits_to_f32(scale[r * nblocks + ((el - r * cols) >> 6)]);
    }
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t e = w0 + h * 512;
    if (e < total) __builtin_nontemporal_store(dq8_group<T>(qv[h].x, qv[h].y, sv[h]), reinterpret_cast<u32x4*>(out + e));
  }
}

template <typename T>
__global__ __launch_bounds__(256) void dq8_scalar(const int8_t* __restrict__ q, const uint16_t* __restrict__ scale,
                                                  typename T::storage* __restrict__ out, int64_t cols, int64_t nblocks,
                                                  int64_t total) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int64_t r = e / cols, col = e - r * cols;
    const float v = (float)q[e] * bf16_bits_to_f32(scale[r * nblocks + (col >> 6)]);
    out[e] = T::from_f32(v);
  }
}

template <typename T>
bool launch_dq8(const void* p, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_dq8_args*>(p);
  if (a.rows < 0 || a.cols < 0) return ctx.fail("negative shape");
  if (a.nblocks != (a.cols + 63) / 64) return ctx.fail("nblocks must equal ceil(cols / 64)");
  const int64_t total = a.rows * a.cols;
  if (total == 0) return true;
  const uint64_t osz = sizeof(typename T::storage);
  if (!ctx.check(a.q, (uint64_t)total, "q") || !ctx.check(a.scale, (uint64_t)(a.rows * a.nblocks) * 2, "scale") ||
      !ctx.check(a.out, (uint64_t)total * osz, "out"))
    return false;
  const bool vec = a.cols % 16 == 0 && a.q % 16 == 0 && a.out % 16 == 0 && total / 16 < ((int64_t)1 << 40);
  if constexpr (sizeof(typename T::storage) == 2) {
    if (vec && cdiv(total, 4096) <= 0x1fffffffLL) {  // span and wavefront indices stay below 2^31
      const int8_t* q = (const int8_t*)a.q;
      const uint16_t* sc = (const uint16_t*)a.scale;
      auto* out = (typename T::storage*)a.out;
      const uint32_t spr = (uint32_t)(a.cols / 1024);
      if (a.cols % 1024 == 0)  // two 1024-element spans per wavefront
        hipLaunchKernelGGL((dq8_vec16<T, true>), dim3((uint32_t)cdiv(total, 8192)), dim3(256), 0, ctx.stream, q, sc, out,
                           a.cols, a.nblocks, total, 1.0 / (double)a.cols, spr, 1.0 / (double)spr);
      else  // one span per wavefront
        hipLaunchKernelGGL((dq8_vec16<T, false>), dim3((uint32_t)cdiv(total, 4096)), dim3(256), 0, ctx.stream, q, sc, out,
                           a.cols, a.nblocks, total, 1.0 / (double)a.cols, 1u, 1.0);
      return hrt::launch_ok(hipGetLastError(), ctx, "dq8");
    }
  }
  if (vec) {
    const int64_t nchunks = total / 16;
    const int64_t grid = cdiv(nchunks, 256 * kChunks);
    hipLaunchKernelGGL(dq8_vec<T>, dim3((uint32_t)grid), dim3(256), 0, ctx.stream, (const int8_t*)a.q,
                       (const uint16_t*)a.scale, (typename T::storage*)a.out, a.cols, a.nblocks, nchunks,
                       1.0 / (double)(a.cols / 16));
  } else {
    int64_t grid = cdiv(total, 256);
    if (grid > 16384) grid = 16384;
    hipLaunchKernelGGL(dq8_scalar<T>, dim3((uint32_t)grid), dim3(256), 0, ctx.stream, (const int8_t*)a.q,
                       (const uint16_t*)a.scale, (typename T::storage*)a.out, a.cols, a.nblocks, total);
  }
  return hrt::launch_ok(hipGetLastError(), ctx, "dq8");
}

HRT_REGISTER("dq8_f32", hrt_dq8_args, launch_dq8<F32>);
HRT_REGISTER("dq8_bf16", hrt_dq8_args, launch_dq8<BF16>);
HRT_REGISTER("dq8_f16", hrt_dq8_args, launch_dq8<F16>);

}  // namespace
}  // namespace hk
