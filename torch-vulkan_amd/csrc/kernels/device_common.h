// Device-side helpers shared by the gfx950 kernels: element conversions with the reference's rounding
// contract, 64-lane wavefront reductions, and small vector types.
//
// Rounding contract (vkrt/shaders/types.glsl:18-50, identical to torch's CPU `.to()`):
//   f32 -> bf16: round to nearest even, every NaN -> 0x7FC0;
//   f32 -> f16 : round to nearest even including subnormals, overflow -> inf (v_cvt_f16_f32 does this in
//                the default round-to-nearest-even mode with f16 denormals enabled).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../../include/hrt_ops.h"

namespace hk {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Global-memory pointers.  Operand addresses arrive as integers in the argument blocks; casting them to
// address space 1 makes the compiler emit global_load/global_store instead of flat accesses (flat
// accesses also count against the LDS wait counter, which would make every LDS wait drain the
// in-flight global prefetch).
#define HK_G __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ HK_G T* gptr(uint64_t a) {
  return reinterpret_cast<HK_G T*>(a);
}
template <typename T>
__device__ __forceinline__ const HK_G T* gcptr(uint64_t a) {
  return reinterpret_cast<const HK_G T*>(a);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Eight floats to bf16 with the hardware's round-to-nearest-even (v_cvt_pk_bf16_f32), which equals
// f32_to_bf16_bits for every non-NaN input; a NaN keeps its sign and payload there, so the caller uses this
// only when it knows the values hold no NaN (bf16_pack8_checked).
__device__ __forceinline__ u32x4 bf16_pack8_hw(const float* v) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bf16x2 h = {(__bf16)v[2 * i], (__bf16)v[2 * i + 1]};
    r[i] = __builtin_bit_cast(uint32_t, h);
  }
  return r;
}
__device__ __forceinline__ u32x4 bf16_pack8_sw(const float* v) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = f32_to_bf16_bits(v[2 * i]) | (f32_to_bf16_bits(v[2 * i + 1]) << 16);
  return r;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  union {
    uint16_t u;
    _Float16 f;
  } c;
  c.u = (uint16_t)h;
  return (float)c.f;
}

// float -> IEEE half bits: the hardware conversion (round to nearest even, subnormals kept, overflow to
// inf) for every non-NaN value; a NaN keeps its sign and top ten payload bits, quieted (0x200), as the
// reference's f2h does (vkrt/shaders/types.glsl:18-41), where the hardware conversion would not.
__device__ __forceinline__ uint32_t f32_to_f16_bits(float x) {
  union {
    uint16_t u;
    _Float16 f;
  } c;
  c.f = (_Float16)x;
  const uint32_t u = __float_as_uint(x);
  return (u & 0x7fffffffu) > 0x7f800000u ? ((u >> 16) & 0x8000u) | 0x7e00u | ((u >> 13) & 0x3ffu) : (uint32_t)c.u;
}

// Element type tags used as template parameters.
struct F32 {
  using storage = float;
  static constexpr int code = HRT_F32;
  __device__ __forceinline__ static float load(const float* p) { return *p; }
  __device__ __forceinline__ static float to_f32(float v) { return v; }
  __device__ __forceinline__ static float from_f32(float v) { return v; }
};
struct BF16 {
  using storage = uint16_t;
  static constexpr int code = HRT_BF16;
  __device__ __forceinline__ static float to_f32(uint16_t v) { return bf16_bits_to_f32(v); }
  __device__ __forceinline__ static uint16_t from_f32(float v) { return (uint16_t)f32_to_bf16_bits(v); }
};
struct F16 {
  using storage = uint16_t;
  static constexpr int code = HRT_F16;
  __device__ __forceinline__ static float to_f32(uint16_t v) { return f16_bits_to_f32(v); }
  __device__ __forceinline__ static uint16_t from_f32(float v) { return (uint16_t)f32_to_f16_bits(v); }
};

// Pack two floats into one dword of 16-bit elements (low = a).
template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return (uint32_t)T::from_f32(a) | ((uint32_t)T::from_f32(b) << 16);
}
template <typename T>
__device__ __forceinline__ float lo16(uint32_t w) {
  return T::to_f32((uint16_t)(w & 0xffffu));
}
template <typename T>
__device__ __forceinline__ float hi16(uint32_t w) {
  return T::to_f32((uint16_t)(w >> 16));
}

// ---- wavefront (64 lanes) reductions --------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// The same sum without LDS round trips: DPP quad swaps (lane ^ 1, lane ^ 2), the half-row and row mirrors
// (after the quad steps each quad, then each half-row, holds one value, so a mirror pairs it with the other
// half), then the gfx950 16- and 32-lane swaps.  Each step adds a pair of values in both of its lanes, so
// every lane ends with the same bits.  About 20 VALU cycles against ~6 LDS latencies for wave_sum.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141>(v);  // row_half_mirror
  v = dpp_add<0x140>(v);  // row_mirror
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Block-wide reductions for blocks of NW waves; `red` is LDS scratch of at least NW floats.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  if (NW == 1) return v;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < NW; ++i) r += red[i];
  return r;
}
template <int NW>
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  if (NW == 1) return v;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = fmaxf(r, red[i]);
  return r;
}

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Element offset of row (b, h, s) of a gradient output (dq, dk or dv) whose matching input has strides
// (sb, sh, ss): that layout with HRT_ATTN_GRAD_LIKE_INPUT, else [B, S, H, D]-contiguous over S rows.
__device__ __forceinline__ int64_t grad_row(const hrt_attn_args& p, int64_t b, int64_t h, int64_t s, int64_t S, int64_t sb,
                                            int64_t sh, int64_t ss) {
  return (p.flags & HRT_ATTN_GRAD_LIKE_INPUT) ? b * sb + h * sh + s * ss : ((b * S + s) * p.H + h) * p.D;
}

}  // namespace hk
