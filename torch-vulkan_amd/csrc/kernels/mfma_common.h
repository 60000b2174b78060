// Matrix-core helpers for gfx950 (CDNA4): typed wrappers of v_mfma_f32_16x16x32_{bf16,f16} and the
// 8x8 transpose of 16-bit elements used to turn M-/N-contiguous tiles into K-contiguous LDS rows.
//
// Lane layout of v_mfma_f32_16x16x32 (checked on the device): with l = lane (0..63), g = l / 16,
//   A operand (16 x 32, M x K): lane l holds A[l % 16][8 g + i], i = 0..7
//   B operand (32 x 16, K x N): lane l holds B[8 g + i][l % 16]
//   accumulator (16 x 16):      lane l holds D[4 g + i][l % 16], i = 0..3
// so both operands want 8 consecutive K values per lane: every tile is staged in LDS with K contiguous
// and read with one 128-bit ds_read per fragment.
#pragma once

#include <type_traits>

#include "device_common.h"

namespace hk {

template <typename T>
struct Mfma;

template <>
struct Mfma<BF16> {
  __device__ __forceinline__ static f32x4 mac(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma<F16> {
  __device__ __forceinline__ static f32x4 mac(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// in[j] holds row j (8 halves, dword d = cols 2d | 2d+1 << 16); out[m] holds column m (rows 0..7).
__device__ __forceinline__ void transpose8x8(const u32x4 in[8], u32x4 out[8]) {
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    uint32_t w[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t a = in[2 * r][m >> 1], b = in[2 * r + 1][m >> 1];
      w[r] = (m & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
    }
    out[m] = u32x4{w[0], w[1], w[2], w[3]};
  }
}

// Two fp32 -> packed 16-bit of type T with the hardware conversion (round to nearest even; used for
// matrix-core operands and GEMM/attention outputs, where only finite values occur in practice).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
template <typename T>
__device__ __forceinline__ uint32_t cvt2(float a, float b);
template <>
__device__ __forceinline__ uint32_t cvt2<BF16>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}
template <>
__device__ __forceinline__ uint32_t cvt2<F16>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, f16x2_t));
}

// Convert 8 (4) fp32 values to packed 16-bit values of type T with the contract's rounding (round to nearest
// even; bf16: every NaN -> 0x7FC0).  bf16 goes through the hardware conversion (one v_cvt_pk_bf16_f32 per
// pair, bit-identical to the software rounding for every non-NaN value) unless the values' sum is NaN,
// i.e. unless one of them is a NaN (or an inf - inf pair, which the software path rounds the same anyway);
// f16 converts in hardware with its own NaN fix-up.
template <typename T>
__device__ __forceinline__ u32x4 pack8(const float* v) {
  if constexpr (std::is_same<T, BF16>::value) {
    float t = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) t += v[e];
    return t == t ? bf16_pack8_hw(v) : bf16_pack8_sw(v);
  } else {
    return u32x4{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3]), pack2<T>(v[4], v[5]), pack2<T>(v[6], v[7])};
  }
}
template <typename T>
__device__ __forceinline__ u32x2 pack4(const float* v) {
  if constexpr (std::is_same<T, BF16>::value) {
    const float t = (v[0] + v[1]) + (v[2] + v[3]);
    if (t == t) return u32x2{cvt2<T>(v[0], v[1]), cvt2<T>(v[2], v[3])};
  }
  return u32x2{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
}


}  // namespace hk
