// Row kernels: softmax forward/backward and layer_norm forward/backward/weight-gradient.
// Reference algorithms: vkrt/shaders/softmax.comp.in:27-50 and vkrt/shaders/ln.comp.in:1-84 (fp32 math,
// max-subtracted softmax, two-pass variance, fp32 statistics).
//
// All of them are HBM-bound (a few flops per byte).  The main path keeps a whole row in registers: one
// 64-lane wavefront per row, 16-byte vector loads (4 fp32 / 8 bf16 per lane per vector), wavefront
// shuffle reductions, so every element is read from HBM exactly once and written once; four rows per
// 256-thread workgroup.  Rows that are too long for registers, misaligned, or softmaxes over a
// non-innermost dimension take a generic multi-pass path.
#include <cmath>
#include <type_traits>

#include "../hrt/registry.h"
#include "device_common.h"

namespace hk {
namespace {

constexpr int kMaxNV = 8;  // 16-byte vectors per lane on the register path
constexpr size_t kLnLds = 128 * 1024;  // LDS bytes the layer_norm backward may stage its chunk's rows in

// Load / store 16 bytes as float values.
template <typename T>
struct Vec;
// 16-byte raw access: rd / wr go through the caches, rd_nt / wr_nt are streaming (nontemporal) accesses
// for data that is touched once; unpack / pack convert between the raw vector and N floats.
__device__ __forceinline__ u32x4 rd(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x4 rd_nt(const void* p) { return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p)); }
__device__ __forceinline__ void wr_nt(void* p, u32x4 w) { __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p)); }

template <>
struct Vec<F32> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void unpack(u32x4 w, float* v) {
    v[0] = __uint_as_float(w.x), v[1] = __uint_as_float(w.y), v[2] = __uint_as_float(w.z), v[3] = __uint_as_float(w.w);
  }
  __device__ __forceinline__ static u32x4 pack(const float* v) {
    return u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
  }
  __device__ __forceinline__ static void load(const float* p, float* v) { unpack(rd(p), v); }
  __device__ __forceinline__ static void store(float* p, const float* v) { *reinterpret_cast<u32x4*>(p) = pack(v); }
};
template <typename T16>
struct Vec16 {
  static constexpr int N = 8;
  __device__ __forceinline__ static void unpack(u32x4 w, float* v) {
    const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = lo16<T16>(a[i]);
      v[2 * i + 1] = hi16<T16>(a[i]);
    }
  }
  __device__ __forceinline__ static u32x4 pack(const float* v) {
    return u32x4{pack2<T16>(v[0], v[1]), pack2<T16>(v[2], v[3]), pack2<T16>(v[4], v[5]), pack2<T16>(v[6], v[7])};
  }
  __device__ __forceinline__ static void load(const uint16_t* p, float* v) { unpack(rd(p), v); }
  __device__ __forceinline__ static void store(uint16_t* p, const float* v) { *reinterpret_cast<u32x4*>(p) = pack(v); }
};
template <>
struct Vec<BF16> : Vec16<BF16> {};
template <>
struct Vec<F16> : Vec16<F16> {};

template <typename T>
__device__ __forceinline__ float ld(const typename T::storage* p, int64_t i) {
  return T::to_f32(p[i]);
}

// ================================ softmax ================================================================
template <typename T, int NV, bool FULL>
__global__ __launch_bounds__(256) void softmax_fwd_reg(const typename T::storage* __restrict__ x,
                                                       typename T::storage* __restrict__ y, int64_t rows, int64_t R,
                                                       uint32_t safe) {
  constexpr int V = Vec<T>::N;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // no block barriers in this kernel
  const typename T::storage* xr = x + row * R;
  float v[NV][V];
  float m = -INFINITY;
  u32x4 raw[NV];
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int64_t col = (int64_t)(c * 64 + lane) * V;
    if ((FULL || col < R)) raw[c] = rd_nt(xr + col);  // every load in flight before the first use
  }
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int64_t col = (int64_t)(c * 64 + lane) * V;
    if ((FULL || col < R)) {
      Vec<T>::unpack(raw[c], v[c]);
#pragma unroll
      for (int e = 0; e < V; ++e) m = fmaxf(m, v[c][e]);
    }
  }
  m = wave_max(m);
  // exp(x - m) = exp2(x log2e - m log2e) in one fma + v_exp_f32; special values behave as exp(x - m):
  // m = -inf (all -inf) or x = m = +inf give NaN, finite x under m = +inf gives 0.  The rounding of
  // m log2e scales every element of the row by the same factor, which the normalisation cancels.
  constexpr float kL2e = 1.4426950408889634f;
  const float nm = -m * kL2e;
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int64_t col = (int64_t)(c * 64 + lane) * V;
    if ((FULL || col < R)) {
#pragma unroll
      for (int e = 0; e < V; ++e) {
        v[c][e] = __builtin_amdgcn_exp2f(fmaf(v[c][e], kL2e, nm));
        s += v[c][e];
      }
    }
  }
  s = wave_sum(s);
  const bool zero = safe && m == -INFINITY;
  const float inv = 1.f / s;
  typename T::storage* yr = y + row * R;
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int64_t col = (int64_t)(c * 64 + lane) * V;
    if ((FULL || col < R)) {
#pragma unroll
      for (int e = 0; e < V; ++e) v[c][e] = zero ? 0.f : v[c][e] * inv;
      wr_nt(yr + col, Vec<T>::pack(v[c]));
    }
  }
}

template <typename T, int NV, bool FULL>
__global__ __launch_bounds__(256) void softmax_bwd_reg(const typename T::storage* __restrict__ y,
                                                       const typename T::storage* __restrict__ g,
                                                       typename T::storage* __restrict__ dx, int64_t rows, int64_t R) {
  constexpr int V = Vec<T>::N;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  float yv[NV][V], gv[NV][V];
  float d = 0.f;
  u32x4 ry[NV], rg[NV];
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int64_t col = (int64_t)(c * 64 + lane) * V;
    if ((FULL || col < R)) {
      ry[c] = rd_nt(y + row * R + col);
      rg[c] = rd_nt(g + row * R + col);
    }
  }
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int64_t col = (int64_t)(c * 64 + lane) * V;
    if ((FULL || col < R)) {
      Vec<T>::unpack(ry[c], yv[c]);
      Vec<T>::unpack(rg[c], gv[c]);
#pragma unroll
      for (int e = 0; e < V; ++e) d += gv[c][e] * yv[c][e];
    }
  }
  d = wave_sum(d);
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int64_t col = (int64_t)(c * 64 + lane) * V;
    if ((FULL || col < R)) {
#pragma unroll
      for (int e = 0; e < V; ++e) yv[c][e] = yv[c][e] * (gv[c][e] - d);
      wr_nt(dx + row * R + col, Vec<T>::pack(yv[c]));
    }
  }
}

// Generic softmax, inner == 1: one workgroup per row, online max/sum pass then a write pass.
template <typename T>
__global__ __launch_bounds__(256) void softmax_fwd_row(const typename T::storage* __restrict__ x,
                                                       typename T::storage* __restrict__ y, int64_t R, uint32_t safe) {
  __shared__ float red[4];
  const int64_t base = (int64_t)blockIdx.x * R;
  float m = -INFINITY, s = 0.f;
  for (int64_t r = threadIdx.x; r < R; r += 256) {
    const float v = ld<T>(x, base + r);
    if (v > m) {
      s = s * expf(m - v) + 1.f;  // m == -inf: expf(-inf) = 0
      m = v;
    } else {
      s += expf(v - m);
    }
  }
  const float mall = block_max<4>(m, red);
  s = (m == -INFINITY) ? 0.f : s * expf(m - mall);
  const float sall = block_sum<4>(s, red);
  const bool zero = safe && mall == -INFINITY;
  for (int64_t r = threadIdx.x; r < R; r += 256) {
    const float v = ld<T>(x, base + r);
    y[base + r] = T::from_f32(zero ? 0.f : expf(v - mall) / sall);
  }
}

// Generic softmax over a non-innermost dimension: one thread per (outer, inner) column; consecutive
// threads read consecutive inner positions, so every pass over R is coalesced.
template <typename T>
__global__ __launch_bounds__(256) void softmax_fwd_col(const typename T::storage* __restrict__ x,
                                                       typename T::storage* __restrict__ y, int64_t outer, int64_t R,
                                                       int64_t inner, uint32_t safe) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= outer * inner) return;
  const int64_t o = t / inner, i = t - o * inner;
  const int64_t base = o * R * inner + i;
  float m = -INFINITY;
  for (int64_t r = 0; r < R; ++r) m = fmaxf(m, ld<T>(x, base + r * inner));
  float s = 0.f;
  for (int64_t r = 0; r < R; ++r) s += expf(ld<T>(x, base + r * inner) - m);
  const bool zero = safe && m == -INFINITY;
  for (int64_t r = 0; r < R; ++r) {
    const float v = ld<T>(x, base + r * inner);
    y[base + r * inner] = T::from_f32(zero ? 0.f : expf(v - m) / s);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void softmax_bwd_generic(const typename T::storage* __restrict__ y,
                                                           const typename T::storage* __restrict__ g,
                                                           typename T::storage* __restrict__ dx, int64_t outer, int64_t R,
                                                           int64_t inner) {
  if (inner == 1) {
    __shared__ float red[4];
    const int64_t base = (int64_t)blockIdx.x * R;
    float d = 0.f;
    for (int64_t r = threadIdx.x; r < R; r += 256) d += ld<T>(g, base + r) * ld<T>(y, base + r);
    d = block_sum<4>(d, red);
    for (int64_t r = threadIdx.x; r < R; r += 256) {
      const float yv = ld<T>(y, base + r);
      dx[base + r] = T::from_f32(yv * (ld<T>(g, base + r) - d));
    }
    return;
  }
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= outer * inner) return;
  const int64_t o = t / inner, i = t - o * inner;
  const int64_t base = o * R * inner + i;
  float d = 0.f;
  for (int64_t r = 0; r < R; ++r) d += ld<T>(g, base + r * inner) * ld<T>(y, base + r * inner);
  for (int64_t r = 0; r < R; ++r) {
    const float yv = ld<T>(y, base + r * inner);
    dx[base + r * inner] = T::from_f32(yv * (ld<T>(g, base + r * inner) - d));
  }
}

template <typename T>
int reg_nv(int64_t R, std::initializer_list<uint64_t> ptrs) {
  constexpr int V = Vec<T>::N;
  if (R % V != 0 || R > 64 * V * kMaxNV) return 0;
  for (uint64_t p : ptrs)
    if (p % 16 != 0) return 0;
  int nv = 1;
  while (64 * V * nv < R) nv *= 2;
  return nv;
}

template <typename T>
bool launch_softmax_fwd(const void* p, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_softmax_args*>(p);
  if (a.outer < 0 || a.R < 0 || a.inner < 0) return ctx.fail("negative shape");
  const int64_t n = a.outer * a.R * a.inner;
  if (n == 0) return true;
  const uint64_t bytes = (uint64_t)n * sizeof(typename T::storage);
  if (!ctx.check(a.x, bytes, "x") || !ctx.check(a.y, bytes, "y")) return false;
  using S = typename T::storage;
  const S* x = (const S*)a.x;
  S* y = (S*)a.y;
  if (a.inner == 1) {
    const int nv = reg_nv<T>(a.R, {a.x, a.y});
  const auto full_row = [&](int v) { return a.R == (int64_t)v * 64 * Vec<T>::N; };  // rows fill every chunk: no column guards
    const dim3 g((uint32_t)cdiv(a.outer, 4));
    switch (nv) {
      case 1: if (full_row(1)) hipLaunchKernelGGL((softmax_fwd_reg<T, 1, true>), g, dim3(256), 0, ctx.stream, x, y, a.outer, a.R, a.safe); else hipLaunchKernelGGL((softmax_fwd_reg<T, 1, false>), g, dim3(256), 0, ctx.stream, x, y, a.outer, a.R, a.safe); break;
      case 2: if (full_row(2)) hipLaunchKernelGGL((softmax_fwd_reg<T, 2, true>), g, dim3(256), 0, ctx.stream, x, y, a.outer, a.R, a.safe); else hipLaunchKernelGGL((softmax_fwd_reg<T, 2, false>), g, dim3(256), 0, ctx.stream, x, y, a.outer, a.R, a.safe); break;
      case 4: if (full_row(4)) hipLaunchKernelGGL((softmax_fwd_reg<T, 4, true>), g, dim3(256), 0, ctx.stream, x, y, a.outer, a.R, a.safe); else hipLaunchKernelGGL((softmax_fwd_reg<T, 4, false>), g, dim3(256), 0, ctx.stream, x, y, a.outer, a.R, a.safe); break;
      case 8: if (full_row(8)) hipLaunchKernelGGL((softmax_fwd_reg<T, 8, true>), g, dim3(256), 0, ctx.stream, x, y, a.outer, a.R, a.safe); else hipLaunchKernelGGL((softmax_fwd_reg<T, 8, false>), g, dim3(256), 0, ctx.stream, x, y, a.outer, a.R, a.safe); break;
      default:
        hipLaunchKernelGGL(softmax_fwd_row<T>, dim3((uint32_t)a.outer), dim3(256), 0, ctx.stream, x, y, a.R, a.safe);
    }
  } else {
    hipLaunchKernelGGL(softmax_fwd_col<T>, dim3((uint32_t)cdiv(a.outer * a.inner, 256)), dim3(256), 0, ctx.stream, x, y,
                       a.outer, a.R, a.inner, a.safe);
  }
  return hrt::launch_ok(hipGetLastError(), ctx, "softmax_fwd");
}

template <typename T>
bool launch_softmax_bwd(const void* p, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_softmax_args*>(p);
  if (a.outer < 0 || a.R < 0 || a.inner < 0) return ctx.fail("negative shape");
  const int64_t n = a.outer * a.R * a.inner;
  if (n == 0) return true;
  const uint64_t bytes = (uint64_t)n * sizeof(typename T::storage);
  if (!ctx.check(a.y, bytes, "y") || !ctx.check(a.g, bytes, "g") || !ctx.check(a.dx, bytes, "dx")) return false;
  using S = typename T::storage;
  const S *y = (const S*)a.y, *g = (const S*)a.g;
  S* dx = (S*)a.dx;
  const int nv = a.inner == 1 ? reg_nv<T>(a.R, {a.y, a.g, a.dx}) : 0;
  const auto full_row = [&](int v) { return a.R == (int64_t)v * 64 * Vec<T>::N; };  // rows fill every chunk: no column guards
  const dim3 g4((uint32_t)cdiv(a.outer, 4));
  switch (nv) {
    case 1: if (full_row(1)) hipLaunchKernelGGL((softmax_bwd_reg<T, 1, true>), g4, dim3(256), 0, ctx.stream, y, g, dx, a.outer, a.R); else hipLaunchKernelGGL((softmax_bwd_reg<T, 1, false>), g4, dim3(256), 0, ctx.stream, y, g, dx, a.outer, a.R); break;
    case 2: if (full_row(2)) hipLaunchKernelGGL((softmax_bwd_reg<T, 2, true>), g4, dim3(256), 0, ctx.stream, y, g, dx, a.outer, a.R); else hipLaunchKernelGGL((softmax_bwd_reg<T, 2, false>), g4, dim3(256), 0, ctx.stream, y, g, dx, a.outer, a.R); break;
    case 4: if (full_row(4)) hipLaunchKernelGGL((softmax_bwd_reg<T, 4, true>), g4, dim3(256), 0, ctx.stream, y, g, dx, a.outer, a.R); else hipLaunchKernelGGL((softmax_bwd_reg<T, 4, false>), g4, dim3(256), 0, ctx.stream, y, g, dx, a.outer, a.R); break;
    case 8: if (full_row(8)) hipLaunchKernelGGL((softmax_bwd_reg<T, 8, true>), g4, dim3(256), 0, ctx.stream, y, g, dx, a.outer, a.R); else hipLaunchKernelGGL((softmax_bwd_reg<T, 8, false>), g4, dim3(256), 0, ctx.stream, y, g, dx, a.outer, a.R); break;
    default: {
      const dim3 grid(a.inner == 1 ? (uint32_t)a.outer : (uint32_t)cdiv(a.outer * a.inner, 256));
      hipLaunchKernelGGL(softmax_bwd_generic<T>, grid, dim3(256), 0, ctx.stream, y, g, dx, a.outer, a.R, a.inner);
    }
  }
  return hrt::launch_ok(hipGetLastError(), ctx, "softmax_bwd");
}

// ================================ layer_norm ============================================================
// Packs NV chunks of V outputs into 16-byte vectors of T.  bf16 goes through the hardware conversion
// (bf16_pack8_hw), which rounds like the contract except for NaN: a NaN among the lane's values makes their
// sum NaN, and then the lane packs with the contract's rounding instead (every NaN -> 0x7FC0).
template <typename T, int NV, int V>
__device__ __forceinline__ void pack_chunks(float (&v)[NV][V], u32x4 (&out)[NV]) {
  if constexpr (std::is_same<T, BF16>::value) {
    float t = 0.f;
#pragma unroll
    for (int c = 0; c < NV; ++c)
#pragma unroll
      for (int e = 0; e < V; ++e) t += v[c][e];
    if (t == t) {
#pragma unroll
      for (int c = 0; c < NV; ++c) out[c] = bf16_pack8_hw(v[c]);
    } else {
#pragma unroll
      for (int c = 0; c < NV; ++c) out[c] = bf16_pack8_sw(v[c]);
    }
  } else {
#pragma unroll
    for (int c = 0; c < NV; ++c) out[c] = Vec<T>::pack(v[c]);
  }
}

// Forward, register path: one wavefront per row (4 rows per workgroup), the row in registers.  HW / HB:
// weight / bias present (compile-time, so the per-element work has no selects).
template <typename T, int NV, bool FULL, bool HW, bool HB>
__global__ __launch_bounds__(256) void ln_fwd_reg(const typename T::storage* __restrict__ x,
                                                  typename T::storage* __restrict__ y, float* __restrict__ mean_out,
                                                  float* __restrict__ rstd_out, const typename T::storage* __restrict__ w,
                                                  const typename T::storage* __restrict__ b, int64_t rows, int64_t D,
                                                  float eps) {
  constexpr int V = Vec<T>::N;
  const int lane = threadIdx.x & 63;
  const int64_t row0 = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const bool live = row0 < rows;
  const int64_t row = live ? row0 : rows - 1;  // a row past the end loads the last row and stores nothing
  // x, w and b of every chunk requested before the first use, with no branch between the loads (a branch
  // there made the compiler wait for the first chunk's loads before issuing the next: two round trips to
  // HBM instead of one).  Lanes past the row load its last vector and do not use it.
  float v[NV][V];
  u32x4 rx[NV], rw[NV], rb[NV];
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int64_t col = (int64_t)(c * 64 + lane) * V;
    const int64_t cl = FULL || col < D ? col : D - V;
    rx[c] = rd_nt(x + row * D + cl);
    if constexpr (HW) rw[c] = rd(w + cl);  // shared by every row: cached
    if constexpr (HB) rb[c] = rd(b + cl);
  }
  // x passes through an empty asm that also uses w and b, right after the loads: without it the compiler
  // sinks the w and b loads to their first use, after the two reductions, where they cost a second round
  // trip.  The row sum needs all of x anyway, so waiting for everything here costs nothing.
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    if constexpr (HW && HB) asm volatile("" : "+v"(rx[c]) : "v"(rw[c]), "v"(rb[c]));
    else if constexpr (HW) asm volatile("" : "+v"(rx[c]) : "v"(rw[c]));
    else if constexpr (HB) asm volatile("" : "+v"(rx[c]) : "v"(rb[c]));
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int64_t col = (int64_t)(c * 64 + lane) * V;
    Vec<T>::unpack(rx[c], v[c]);
    if (FULL || col < D) {
#pragma unroll
      for (int e = 0; e < V; ++e) s += v[c][e];
    }
  }
  const float inv_d = 1.f / (float)D;
  const float mean = wave_sum_dpp(s) * inv_d;
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int64_t col = (int64_t)(c * 64 + lane) * V;
    if (FULL || col < D) {
#pragma unroll
      for (int e = 0; e < V; ++e) {
        v[c][e] -= mean;  // kept centred for the output below
        q += v[c][e] * v[c][e];
      }
    }
  }
  const float var = wave_sum_dpp(q) * inv_d;
  const float rstd = 1.f / sqrtf(var + eps);
  // y = ((x - mean) * rstd) * w + b, the product and sum as one fma
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    float wv[V], bv[V];
    if constexpr (HW) Vec<T>::unpack(rw[c], wv);
    if constexpr (HB) Vec<T>::unpack(rb[c], bv);
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float t = v[c][e] * rstd;
      if constexpr (HW && HB) v[c][e] = fmaf(t, wv[e], bv[e]);
      else if constexpr (HW) v[c][e] = t * wv[e];
      else if constexpr (HB) v[c][e] = t + bv[e];
      else v[c][e] = t;
    }
  }
  u32x4 out[NV];
  pack_chunks<T>(v, out);
  if (live) {
#pragma unroll
    for (int c = 0; c < NV; ++c) {
      const int64_t col = (int64_t)(c * 64 + lane) * V;
      if (FULL || col < D) wr_nt(y + row * D + col, out[c]);
    }
    if (lane == 0) {
      mean_out[row] = mean;
      rstd_out[row] = rstd;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void ln_fwd_row(const typename T::storage* __restrict__ x, typename T::storage* __restrict__ y,
                                                  float* __restrict__ mean_out, float* __restrict__ rstd_out,
                                                  const typename T::storage* __restrict__ w,
                                                  const typename T::storage* __restrict__ b, int64_t D, float eps) {
  __shared__ float red[4];
  const int64_t base = (int64_t)blockIdx.x * D;
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < D; i += 256) s += ld<T>(x, base + i);
  const float mean = block_sum<4>(s, red) / (float)D;
  float q = 0.f;
  for (int64_t i = threadIdx.x; i < D; i += 256) {
    const float d = ld<T>(x, base + i) - mean;
    q += d * d;
  }
  const float var = block_sum<4>(q, red) / (float)D;
  const float rstd = 1.f / sqrtf(var + eps);
  for (int64_t i = threadIdx.x; i < D; i += 256) {
    float o = (ld<T>(x, base + i) - mean) * rstd;
    if (w) o *= ld<T>(w, i);
    if (b) o += ld<T>(b, i);
    y[base + i] = T::from_f32(o);
  }
  if (threadIdx.x == 0) {
    mean_out[blockIdx.x] = mean;
    rstd_out[blockIdx.x] = rstd;
  }
}

// Partial sums go out as streaming stores: read once, by the column reduction (2-4% faster than cached
// stores, whose dirty lines the end of the launch must write back).
__device__ __forceinline__ void ws_store(float* p, f32x4 v) { __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p)); }
// Sum of N consecutive rows of D floats (four positions from b) in a fixed tree: ((r0 + r1) + (r2 + r3)) + ...
template <int N>
__device__ __forceinline__ f32x4 rows_tree(const float* b, int64_t D) {
  if constexpr (N == 1) return *reinterpret_cast<const f32x4*>(b);
  else return rows_tree<N / 2>(b, D) + rows_tree<N / 2>(b + (N / 2) * D, D);
}

// Backward, register path: one chunk of RPC rows per workgroup, one wavefront per row.  dx per row; with
// ws, the chunk's column sums of g*xhat and g (its RPC rows added through LDS: every wavefront stores its
// row, then each thread sums the RPC rows of its columns in a fixed tree) as ws row pair `chunk`.  With
// `both` (2 RPC D floats of LDS) the two quantities are staged together behind one barrier, else one after
// the other (three barriers).  HW: weight present.
template <typename T, int NV, bool FULL, bool HW, int RPC>
__device__ __forceinline__ void ln_bwd_chunk(const typename T::storage* __restrict__ x, const typename T::storage* __restrict__ g,
                                             const float* __restrict__ mean_in, const float* __restrict__ rstd_in,
                                             const typename T::storage* __restrict__ w, typename T::storage* __restrict__ dx,
                                             float* __restrict__ ws, int64_t rows, int64_t D, int64_t chunk, float* part,
                                             bool both) {
  constexpr int V = Vec<T>::N;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row0 = chunk * RPC + wave;
  const bool live = row0 < rows;
  const int64_t row = live ? row0 : rows - 1;  // a row past the end loads the last row; its terms are zeroed
  // every load issued before the first use, with no branch between them, and pinned there by the empty asm
  // (as in ln_fwd_reg); lanes past the row load its last vector and do not use it
  float xh[NV][V], gv[NV][V];
  u32x4 rx[NV], rg[NV], rw[NV];
  float mean = mean_in[row], rstd = rstd_in[row];
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int64_t col = (int64_t)(c * 64 + lane) * V;
    const int64_t cl = FULL || col < D ? col : D - V;
    rx[c] = rd_nt(x + row * D + cl);
    rg[c] = rd_nt(g + row * D + cl);
    if constexpr (HW) rw[c] = rd(w + cl);
  }
  asm volatile("" : "+v"(mean), "+v"(rstd));
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    if constexpr (HW) asm volatile("" : "+v"(rx[c]), "+v"(rg[c]) : "v"(rw[c]));
    else asm volatile("" : "+v"(rx[c]), "+v"(rg[c]));
  }
  // A row past the end or a vector past D contributes nothing: its g is zeroed as loaded (so gw, g * xhat
  // and g vanish; its xhat is that of data the live lanes process anyway, so a non-finite value there makes
  // their sums non-finite as well).  xhat = x rstd - mean rstd (one fma per element).
  const float mr = -mean * rstd;
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int64_t col = (int64_t)(c * 64 + lane) * V;
    const bool ok = live && (FULL || col < D);
    rg[c] = ok ? rg[c] : u32x4{0u, 0u, 0u, 0u};
  }
  float wv[NV][V];
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    Vec<T>::unpack(rx[c], xh[c]);
    Vec<T>::unpack(rg[c], gv[c]);
    if constexpr (HW) Vec<T>::unpack(rw[c], wv[c]);
#pragma unroll
    for (int e = 0; e < V; ++e) {
      xh[c][e] = fmaf(xh[c][e], rstd, mr);
      const float gw = HW ? gv[c][e] * wv[c][e] : gv[c][e];
      s1 += gw;
      s2 = fmaf(gw, xh[c][e], s2);
    }
  }
  const float inv_d = 1.f / (float)D;
  s1 = wave_sum_dpp(s1) * inv_d;
  s2 = wave_sum_dpp(s2) * inv_d;
  if (dx) {
    // dx = rstd (gw - s1 - xhat s2) = rstd gw + (xhat (-rstd s2) + (-rstd s1))
    const float b2 = -rstd * s2, b1 = -rstd * s1;
    float o[NV][V];
#pragma unroll
    for (int c = 0; c < NV; ++c)
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const float gw = HW ? gv[c][e] * wv[c][e] : gv[c][e];
        o[c][e] = fmaf(rstd, gw, fmaf(xh[c][e], b2, b1));
      }
    u32x4 out[NV];
    pack_chunks<T>(o, out);
    if (live) {
#pragma unroll
      for (int c = 0; c < NV; ++c) {
        const int64_t col = (int64_t)(c * 64 + lane) * V;
        if (FULL || col < D) wr_nt(dx + row * D + col, out[c]);
      }
    }
  }
  if (!ws) return;  // uniform across the workgroup: no barrier below is skipped by only some waves
  // rows past the end and lanes past the row hold zeros (xh = gv = 0 above)
  float* out = ws + chunk * 2 * D;
  if (both) {  // part holds [2][RPC rows][D]: both quantities staged, one barrier
#pragma unroll
    for (int c = 0; c < NV; ++c) {
      const int64_t col = (int64_t)(c * 64 + lane) * V;
      if ((FULL || col < D)) {
        float o[V];
#pragma unroll
        for (int e = 0; e < V; ++e) o[e] = gv[c][e] * xh[c][e];
        Vec<F32>::store(part + wave * D + col, o);
        if constexpr (V == 8) Vec<F32>::store(part + wave * D + col + 4, o + 4);
        Vec<F32>::store(part + (RPC + wave) * D + col, gv[c]);
        if constexpr (V == 8) Vec<F32>::store(part + (RPC + wave) * D + col + 4, gv[c] + 4);
      }
    }
    __syncthreads();
    for (int64_t i = (int64_t)threadIdx.x * 4; i < 2 * D; i += 64 * RPC * 4) {  // i: position in the 2D-wide ws row
      const float* b = part + (i < D ? i : (RPC - 1) * D + i);  // quantity 1 starts at RPC D in part, at D in the ws row
      ws_store(out + i, rows_tree<RPC>(b, D));
    }
    return;
  }
#pragma unroll
  for (int qn = 0; qn < 2; ++qn) {  // qn = 0: g * xhat, 1: g
    if (qn) __syncthreads();         // the previous quantity's sums have been read
#pragma unroll
    for (int c = 0; c < NV; ++c) {
      const int64_t col = (int64_t)(c * 64 + lane) * V;
      if ((FULL || col < D)) {
        float o[V];
#pragma unroll
        for (int e = 0; e < V; ++e) o[e] = qn ? gv[c][e] : gv[c][e] * xh[c][e];
        Vec<F32>::store(part + wave * D + col, o);
        if constexpr (V == 8) Vec<F32>::store(part + wave * D + col + 4, o + 4);
      }
    }
    __syncthreads();
    for (int64_t i = (int64_t)threadIdx.x * 4; i < D; i += 64 * RPC * 4)
      ws_store(out + qn * D + i, rows_tree<RPC>(part + i, D));
  }
}

template <typename T, int NV, bool FULL, bool HW, int RPC>
__global__ __launch_bounds__(64 * RPC) void ln_bwd_reg(const typename T::storage* __restrict__ x,
                                                       const typename T::storage* __restrict__ g,
                                                       const float* __restrict__ mean_in, const float* __restrict__ rstd_in,
                                                       const typename T::storage* __restrict__ w,
                                                       typename T::storage* __restrict__ dx, float* __restrict__ ws,
                                                       int64_t rows, int64_t D, bool both) {
  extern __shared__ float part[];  // [RPC rows][D] or [2][RPC rows][D] (both) when ws != nullptr
  ln_bwd_chunk<T, NV, FULL, HW, RPC>(x, g, mean_in, rstd_in, w, dx, ws, rows, D, blockIdx.x, part, both);
}

// Sum over chunks of one column of the per-chunk partial sums (src = the column's value in chunk 0, stride
// = floats between chunks).  Chunk group k of NG takes chunks k, k + NG, ...: eight running sums filled in
// chunk order (sixteen loads in flight per round), then added in a fixed tree, so the result does not
// depend on timing.
template <int NG>
__device__ __forceinline__ float chunk_column_sum(const float* __restrict__ src, int64_t stride, int64_t chunks, int k) {
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int64_t c = k;
  for (; c + 15 * NG < chunks; c += 16 * NG) {  // two rounds of eight at once, added in the same order
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = src[(c + NG * u) * stride];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[u] += v[u];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[u] += v[8 + u];
  }
  for (; c + 7 * NG < chunks; c += 8 * NG) {
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[u] += src[(c + NG * u) * stride];
  }
  for (int u = 0; c < chunks; c += NG, ++u) acc[u & 7] += src[c * stride];
  return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}
// The 16 chunk groups' sums of one column (sp[k * W]) added in a fixed tree.
template <int W>
__device__ __forceinline__ float combine_groups16(const float* sp) {
  float t[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) t[k] = sp[(2 * k) * W] + sp[(2 * k + 1) * W];
  return ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
}

// Backward, generic path: workgroup per chunk of RPC rows; ws accumulated in place (each thread owns its
// columns, so the read-modify-write has no races).
template <typename T, int RPC>
__global__ __launch_bounds__(256) void ln_bwd_row(const typename T::storage* __restrict__ x, const typename T::storage* __restrict__ g,
                                                  const float* __restrict__ mean_in, const float* __restrict__ rstd_in,
                                                  const typename T::storage* __restrict__ w, typename T::storage* __restrict__ dx,
                                                  float* __restrict__ ws, int64_t rows, int64_t D) {
  __shared__ float red[4];
  float* pw = ws ? ws + (int64_t)blockIdx.x * 2 * D : nullptr;
  for (int rr = 0; rr < RPC; ++rr) {
    const int64_t row = (int64_t)blockIdx.x * RPC + rr;
    if (row >= rows) {
      if (pw && rr == 0)
        for (int64_t i = threadIdx.x; i < 2 * D; i += 256) pw[i] = 0.f;
      continue;
    }
    const float mean = mean_in[row], rstd = rstd_in[row];
    const int64_t base = row * D;
    float s1 = 0.f, s2 = 0.f;
    for (int64_t i = threadIdx.x; i < D; i += 256) {
      const float xh = (ld<T>(x, base + i) - mean) * rstd;
      const float gv = ld<T>(g, base + i);
      const float gw = w ? gv * ld<T>(w, i) : gv;
      s1 += gw;
      s2 += gw * xh;
    }
    s1 = block_sum<4>(s1, red) / (float)D;
    s2 = block_sum<4>(s2, red) / (float)D;
    for (int64_t i = threadIdx.x; i < D; i += 256) {
      const float xh = (ld<T>(x, base + i) - mean) * rstd;
      const float gv = ld<T>(g, base + i);
      const float gw = w ? gv * ld<T>(w, i) : gv;
      if (dx) dx[base + i] = T::from_f32(rstd * (gw - s1 - xh * s2));
      if (pw) {
        if (rr == 0) {
          pw[i] = gv * xh;
          pw[D + i] = gv;
        } else {
          pw[i] += gv * xh;
          pw[D + i] += gv;
        }
      }
    }
  }
}

// dw[d] = sum_c ws[c][0][d], db[d] = sum_c ws[c][1][d]: workgroup (column block of 64, quantity) with 16
// chunk groups of 64 threads, each column summed by chunk_column_sum and the groups combined in a fixed
// tree, so the result does not depend on timing.
template <typename T>
__global__ __launch_bounds__(1024) void ln_wgrad_reduce(const float* __restrict__ ws, typename T::storage* __restrict__ dw,
                                                        typename T::storage* __restrict__ db, int64_t chunks, int64_t D) {
  constexpr int NG = 16;
  __shared__ float sp[NG * 64];
  const int cl = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int qn = blockIdx.y;  // 0: dw, 1: db
  typename T::storage* dst = qn ? db : dw;
  if (!dst) return;  // uniform over the workgroup
  const int64_t col = (int64_t)blockIdx.x * 64 + cl;
  sp[grp * 64 + cl] = col < D ? chunk_column_sum<NG>(ws + qn * D + col, 2 * D, chunks, grp) : 0.f;
  __syncthreads();
  if (grp == 0 && col < D) dst[col] = T::from_f32(combine_groups16<64>(sp + cl));
}

// The same sums when D % 16 == 0 and ws is 16-byte aligned, on 2D / 32 workgroups of 512 threads:
// workgroup w owns 32 consecutive positions u of the 2D-wide ws rows (128 bytes, one cache line per chunk
// row, so no line is shared with a workgroup on another XCD; u < D: dw[u], else db[u - D], D % 16 == 0
// keeps a half block on one side); thread t sums the 4 positions of quad t % 8 over chunks t / 8,
// t / 8 + 64, ... in chunk order (16-byte loads, four in flight: one round at 256 chunks), then each
// position's 64 group sums are added in a fixed tree through LDS, so the result does not depend on timing.
template <typename T>
__global__ __launch_bounds__(512) void ln_wgrad_cols32(const float* __restrict__ ws, typename T::storage* __restrict__ dw,
                                                       typename T::storage* __restrict__ db, int64_t chunks, int64_t D) {
  __shared__ float sp[64 * 32];  // [group][position]
  __shared__ float sq[16 * 32];  // [block of 4 groups][position]
  const int t = threadIdx.x, quad = t & 7, grp = t >> 3;
  const int64_t u0 = (int64_t)blockIdx.x * 32;
  const int64_t stride = 2 * D;
  const float* src = ws + u0 + quad * 4;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (u0 + quad * 4 < 2 * D) {  // the last block may cover only 16 positions
    int64_t c = grp;
    for (; c + 192 < chunks; c += 256) {
      const f32x4 v0 = *reinterpret_cast<const f32x4*>(src + c * stride);
      const f32x4 v1 = *reinterpret_cast<const f32x4*>(src + (c + 64) * stride);
      const f32x4 v2 = *reinterpret_cast<const f32x4*>(src + (c + 128) * stride);
      const f32x4 v3 = *reinterpret_cast<const f32x4*>(src + (c + 192) * stride);
      acc += v0;
      acc += v1;
      acc += v2;
      acc += v3;
    }
    if (c < chunks) {  // the last 1-3 chunks of this group: loaded together (indices clamped), added in order
      const int64_t last = chunks - 1;
      f32x4 t0 = *reinterpret_cast<const f32x4*>(src + c * stride);
      f32x4 t1 = *reinterpret_cast<const f32x4*>(src + (c + 64 < last ? c + 64 : last) * stride);
      f32x4 t2 = *reinterpret_cast<const f32x4*>(src + (c + 128 < last ? c + 128 : last) * stride);
      asm volatile("" : "+v"(t0), "+v"(t1), "+v"(t2));  // keeps the loads together, ahead of the branches
      acc += t0;
      if (c + 64 < chunks) acc += t1;
      if (c + 128 < chunks) acc += t2;
    }
  }
  *reinterpret_cast<f32x4*>(sp + grp * 32 + quad * 4) = acc;
  __syncthreads();
  {
    const int v = t & 31, b = t >> 5;  // groups 4b .. 4b + 3 of position v
    sq[b * 32 + v] = (sp[(4 * b) * 32 + v] + sp[(4 * b + 1) * 32 + v]) + (sp[(4 * b + 2) * 32 + v] + sp[(4 * b + 3) * 32 + v]);
  }
  __syncthreads();
  if (t < 32) {
    const int64_t u = u0 + t;
    typename T::storage* dst = u < D ? dw : db;
    if (u < 2 * D && dst) {
      float r[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) r[k] = sq[(2 * k) * 32 + t] + sq[(2 * k + 1) * 32 + t];
      dst[u < D ? u : u - D] = T::from_f32(((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7])));
    }
  }
}

template <typename T>
bool launch_ln_fwd(const void* p, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_ln_args*>(p);
  if (a.rows < 0 || a.D <= 0) return ctx.fail("bad shape");
  if (a.rows == 0) return true;
  using S = typename T::storage;
  const uint64_t bytes = (uint64_t)(a.rows * a.D) * sizeof(S);
  if (!ctx.check(a.x, bytes, "x") || !ctx.check(a.y, bytes, "y") || !ctx.check(a.mean, a.rows * 4, "mean") ||
      !ctx.check(a.rstd, a.rows * 4, "rstd") || (a.w && !ctx.check(a.w, a.D * sizeof(S), "w")) ||
      (a.b && !ctx.check(a.b, a.D * sizeof(S), "b")))
    return false;
  const S *x = (const S*)a.x, *w = (const S*)a.w, *b = (const S*)a.b;
  S* y = (S*)a.y;
  float *mu = (float*)a.mean, *rs = (float*)a.rstd;
  const int nv = reg_nv<T>(a.D, {a.x, a.y, a.w, a.b});
  const auto full_row = [&](int v) { return a.D == (int64_t)v * 64 * Vec<T>::N; };  // rows fill every chunk: no column guards
  const dim3 g4((uint32_t)cdiv(a.rows, 4));
  // one instantiation per (chunks per lane, full rows, weight present, bias present)
  auto go = [&](auto nvc, auto fullc, auto hwc, auto hbc) {
    hipLaunchKernelGGL((ln_fwd_reg<T, decltype(nvc)::value, decltype(fullc)::value, decltype(hwc)::value, decltype(hbc)::value>),
                       g4, dim3(256), 0, ctx.stream, x, y, mu, rs, w, b, a.rows, a.D, a.eps);
  };
  auto by_affine = [&](auto nvc, auto fullc) {
    using Y = std::true_type;
    using N = std::false_type;
    if (w && b) go(nvc, fullc, Y(), Y());
    else if (w) go(nvc, fullc, Y(), N());
    else if (b) go(nvc, fullc, N(), Y());
    else go(nvc, fullc, N(), N());
  };
  auto by_full = [&](auto nvc) {
    if (full_row(decltype(nvc)::value)) by_affine(nvc, std::true_type());
    else by_affine(nvc, std::false_type());
  };
  switch (nv) {
    case 1: by_full(std::integral_constant<int, 1>()); break;
    case 2: by_full(std::integral_constant<int, 2>()); break;
    case 4: by_full(std::integral_constant<int, 4>()); break;
    case 8: by_full(std::integral_constant<int, 8>()); break;
    default:
      hipLaunchKernelGGL(ln_fwd_row<T>, dim3((uint32_t)a.rows), dim3(256), 0, ctx.stream, x, y, mu, rs, w, b, a.D, a.eps);
  }
  return hrt::launch_ok(hipGetLastError(), ctx, "ln_fwd");
}

template <typename T>
bool launch_ln_wgrad(const void* p, const uint32_t*, hrt::LaunchCtx& ctx);

template <typename T>
bool launch_ln_bwd(const void* p, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_ln_args*>(p);
  if (a.rows < 0 || a.D <= 0) return ctx.fail("bad shape");
  if (a.rows == 0) return true;
  // chunks of the partial-sum rule when ws is given; dx alone runs 4-row workgroups (more of them)
  const int rpc = a.ws ? (int)hrt_ln_rows_per_chunk(a.rows, a.D) : 4;
  if (rpc != 4 && rpc != 8 && rpc != 16) return ctx.fail("ln chunking mismatch");
  using S = typename T::storage;
  const uint64_t bytes = (uint64_t)(a.rows * a.D) * sizeof(S);
  const int64_t chunks = hrt_ln_chunks(a.rows, a.D);
  const bool wgrad = a.ws && (a.dw || a.db);
  if ((a.dw || a.db) && !a.ws) return ctx.fail("dw / db need the partial-sum workspace ws");
  if (!ctx.check(a.x, bytes, "x") || !ctx.check(a.g, bytes, "g") || !ctx.check(a.mean, a.rows * 4, "mean") ||
      !ctx.check(a.rstd, a.rows * 4, "rstd") || (a.w && !ctx.check(a.w, a.D * sizeof(S), "w")) ||
      (a.dx && !ctx.check(a.dx, bytes, "dx")) || (a.ws && !ctx.check(a.ws, (uint64_t)(chunks * 2 * a.D) * 4, "ws")) ||
      (a.dw && !ctx.check(a.dw, a.D * sizeof(S), "dw")) || (a.db && !ctx.check(a.db, a.D * sizeof(S), "db")))
    return false;
  const S *x = (const S*)a.x, *g = (const S*)a.g, *w = (const S*)a.w;
  S* dx = (S*)a.dx;
  float* ws = (float*)a.ws;
  const float *mu = (const float*)a.mean, *rs = (const float*)a.rstd;
  int nv = reg_nv<T>(a.D, {a.x, a.g, a.w, a.dx});
  const auto full_row = [&](int v) { return a.D == (int64_t)v * 64 * Vec<T>::N; };  // rows fill every chunk: no column guards
  const bool both = ws && (size_t)(2 * rpc * a.D) * 4 <= kLnLds;
  const size_t lds = ws ? (size_t)((both ? 2 * rpc : rpc) * a.D) * 4 : 0;
  if (lds > kLnLds || a.D % 4) nv = 0;
  const dim3 grid((uint32_t)cdiv(a.rows, rpc));  // = chunks when ws is given
  auto go = [&](auto nvc, auto fullc, auto hwc, auto rpcc) {
    constexpr int RPC = decltype(rpcc)::value, NV = decltype(nvc)::value;
    if constexpr (RPC == 16 && NV * Vec<T>::N > 32)  // D > 2048: 16 rows of D floats exceed kLnLds, never chosen
      hipLaunchKernelGGL((ln_bwd_row<T, 16>), grid, dim3(256), 0, ctx.stream, x, g, mu, rs, w, dx, ws, a.rows, a.D);
    else
      hipLaunchKernelGGL((ln_bwd_reg<T, NV, decltype(fullc)::value, decltype(hwc)::value, RPC>), grid, dim3(64 * RPC), lds,
                         ctx.stream, x, g, mu, rs, w, dx, ws, a.rows, a.D, both);
  };
  auto by_rpc = [&](auto nvc, auto fullc, auto hwc) {
    if (rpc == 4) go(nvc, fullc, hwc, std::integral_constant<int, 4>());
    else if (rpc == 8) go(nvc, fullc, hwc, std::integral_constant<int, 8>());
    else go(nvc, fullc, hwc, std::integral_constant<int, 16>());
  };
  auto by_w = [&](auto nvc, auto fullc) {
    if (w) by_rpc(nvc, fullc, std::true_type());
    else by_rpc(nvc, fullc, std::false_type());
  };
  auto by_full = [&](auto nvc) {
    if (full_row(decltype(nvc)::value)) by_w(nvc, std::true_type());
    else by_w(nvc, std::false_type());
  };
  switch (nv) {
    case 1: by_full(std::integral_constant<int, 1>()); break;
    case 2: by_full(std::integral_constant<int, 2>()); break;
    case 4: by_full(std::integral_constant<int, 4>()); break;
    case 8: by_full(std::integral_constant<int, 8>()); break;
    default:
      if (rpc == 4) hipLaunchKernelGGL((ln_bwd_row<T, 4>), grid, dim3(256), 0, ctx.stream, x, g, mu, rs, w, dx, ws, a.rows, a.D);
      else if (rpc == 8) hipLaunchKernelGGL((ln_bwd_row<T, 8>), grid, dim3(256), 0, ctx.stream, x, g, mu, rs, w, dx, ws, a.rows, a.D);
      else hipLaunchKernelGGL((ln_bwd_row<T, 16>), grid, dim3(256), 0, ctx.stream, x, g, mu, rs, w, dx, ws, a.rows, a.D);
  }
  if (!hrt::launch_ok(hipGetLastError(), ctx, "ln_bwd")) return false;
  // dw / db by the column reduction of the partial sums, queued right behind (ln_wgrad's kernel).  A single
  // launch whose last workgroups wait for the others' partial sums was tried: the waiting workgroups saw
  // the last chunk's count ~12 us after it was made (device- or system-scope counters alike), 23 us in all.
  if (wgrad) {
    static const uint32_t no_grid[3] = {0, 0, 0};
    return launch_ln_wgrad<T>(&a, no_grid, ctx);
  }
  return true;
}

template <typename T>
bool launch_ln_wgrad(const void* p, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_ln_args*>(p);
  if (a.rows <= 0 || a.D <= 0) return ctx.fail("bad shape");
  if (!a.dw && !a.db) return true;
  using S = typename T::storage;
  const int64_t chunks = hrt_ln_chunks(a.rows, a.D);
  if (!ctx.check(a.ws, (uint64_t)(chunks * 2 * a.D) * 4, "ws") || (a.dw && !ctx.check(a.dw, a.D * sizeof(S), "dw")) ||
      (a.db && !ctx.check(a.db, a.D * sizeof(S), "db")))
    return false;
  if (a.D % 16 == 0 && a.ws % 16 == 0 && 2 * a.D / 16 <= 0x7fffffffLL)
    hipLaunchKernelGGL(ln_wgrad_cols32<T>, dim3((uint32_t)cdiv(2 * a.D, 32)), dim3(512), 0, ctx.stream, (const float*)a.ws,
                       (S*)a.dw, (S*)a.db, chunks, a.D);
  else
    hipLaunchKernelGGL(ln_wgrad_reduce<T>, dim3((uint32_t)cdiv(a.D, 64), 2), dim3(1024), 0, ctx.stream, (const float*)a.ws,
                       (S*)a.dw, (S*)a.db, chunks, a.D);
  return hrt::launch_ok(hipGetLastError(), ctx, "ln_wgrad");
}

// ---- allocation-free layer_norm backward (hrt_ln_bwd_noalloc) -------------------------------------------
// The weight-gradient partial sums go to this array instead of a caller workspace.  Host code never uses
// its name as an address: the device address is resolved once per device at hrt_init (device current)
// and kept in ln_scratch_addr.
static __device__ __align__(256) float scratch[HRT_LN_SCRATCH_BYTES / sizeof(float)];
constexpr int kMaxDevices = 64;
uint64_t ln_scratch_addr[kMaxDevices] = {};

bool ln_scratch_setup(int device, std::string* err) {
  if (device < 0 || device >= kMaxDevices) {
    *err = "device index " + std::to_string(device) + " out of range for the layer_norm scratch table";
    return false;
  }
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr) {
    (void)hipGetLastError();
    *err = std::string("hipGetSymbolAddress(layer_norm scratch): ") + hipGetErrorString(e);
    return false;
  }
  ln_scratch_addr[device] = reinterpret_cast<uint64_t>(p);
  return true;
}
HRT_REGISTER_DEVICE_INIT(ln_scratch_setup);

template <typename T>
bool ln_bwd_into_scratch(hrt_ln_args a, hrt::LaunchCtx& ctx) {
  static const uint32_t no_grid[3] = {0, 0, 0};
  const bool wgrad = (a.dw || a.db) && a.rows > 0;
  if (wgrad) {
    const uint64_t cap = HRT_LN_SCRATCH_BYTES, per_chunk = 2 * (uint64_t)a.D * sizeof(float);
    const uint64_t chunks = (uint64_t)hrt_ln_chunks(a.rows, a.D);
    if (per_chunk > cap || chunks > cap / per_chunk)
      return ctx.fail("rows " + std::to_string(a.rows) + " x D " + std::to_string(a.D) + " needs " +
                      std::to_string(chunks) + " x " + std::to_string(per_chunk) +
                      " bytes of weight-gradient partial sums; the scratch array holds " + std::to_string(cap));
    const uint64_t base = ln_scratch_addr[ctx.device];
    if (!base) return ctx.fail("the scratch array is not set up on this device");
    ctx.own_lo = base;
    ctx.own_hi = base + cap;
    a.ws = base;
  }
  return launch_ln_bwd<T>(&a, no_grid, ctx);  // dx, and dw / db from the partial sums, as one entry point
}

HRT_REGISTER("softmax_fwd_f32", hrt_softmax_args, launch_softmax_fwd<F32>);
HRT_REGISTER("softmax_fwd_bf16", hrt_softmax_args, launch_softmax_fwd<BF16>);
HRT_REGISTER("softmax_fwd_f16", hrt_softmax_args, launch_softmax_fwd<F16>);
HRT_REGISTER("softmax_bwd_f32", hrt_softmax_args, launch_softmax_bwd<F32>);
HRT_REGISTER("softmax_bwd_bf16", hrt_softmax_args, launch_softmax_bwd<BF16>);
HRT_REGISTER("softmax_bwd_f16", hrt_softmax_args, launch_softmax_bwd<F16>);
HRT_REGISTER("ln_fwd_f32", hrt_ln_args, launch_ln_fwd<F32>);
HRT_REGISTER("ln_fwd_bf16", hrt_ln_args, launch_ln_fwd<BF16>);
HRT_REGISTER("ln_fwd_f16", hrt_ln_args, launch_ln_fwd<F16>);
HRT_REGISTER("ln_bwd_f32", hrt_ln_args, launch_ln_bwd<F32>);
HRT_REGISTER("ln_bwd_bf16", hrt_ln_args, launch_ln_bwd<BF16>);
HRT_REGISTER("ln_bwd_f16", hrt_ln_args, launch_ln_bwd<F16>);
HRT_REGISTER("ln_wgrad_f32", hrt_ln_args, launch_ln_wgrad<F32>);
HRT_REGISTER("ln_wgrad_bf16", hrt_ln_args, launch_ln_wgrad<BF16>);
HRT_REGISTER("ln_wgrad_f16", hrt_ln_args, launch_ln_wgrad<F16>);

}  // namespace
}  // namespace hk

extern "C" int hrt_ln_bwd_noalloc(const hrt_ln_args* args, int32_t dtype) {
  using namespace hk;
  return hrt::run_launch("hrt_ln_bwd_noalloc", [&](hrt::LaunchCtx& ctx) {
    if (!args) return ctx.fail("null argument block");
    if (args->ws) return ctx.fail("ws must be 0: the partial sums live in the library's scratch array");
    if (args->rows < 0 || args->D <= 0) return ctx.fail("bad shape");
    switch (dtype) {
      case HRT_F32: return ln_bwd_into_scratch<F32>(*args, ctx);
      case HRT_BF16: return ln_bwd_into_scratch<BF16>(*args, ctx);
      case HRT_F16: return ln_bwd_into_scratch<F16>(*args, ctx);
      default: return ctx.fail("dtype must be HRT_F32, HRT_BF16 or HRT_F16");
    }
  });
}
