// Products with a short reduction dimension (K <= 32): the up-projection of a low-rank adapter, y = h B^T
// (h [M, r], B [N, r]) and its backward dx = dh A (A [r, K_in]), K = the rank.  Their cost is the output
// (M x N written, and read again when accumulated), not the arithmetic, so they are HBM-bound; the matrix
// cores would spend one instruction per 16x16 output block and leave the output to an epilogue through LDS.
// Here every lane owns 8 consecutive outputs of a row (one 16-byte store), keeps its 8 columns of the K x N
// factor in registers as bf16 pairs for the whole launch, and forms each output with K/2 v_dot2 steps whose
// other operand (the row of h, identical across the wavefront) comes from scalar loads.
#pragma once

#include <type_traits>

#include "device_common.h"

namespace hk {
namespace skinny {

// u32 holding two consecutive-k bf16 / f16 values -> fp32 sum of products with another such pair, plus acc.
template <typename T>
__device__ __forceinline__ float dot2(uint32_t x, uint32_t y, float acc);
template <>
__device__ __forceinline__ float dot2<BF16>(uint32_t x, uint32_t y, float acc) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, x), __builtin_bit_cast(b2, y), acc, false);
}
template <>
__device__ __forceinline__ float dot2<F16>(uint32_t x, uint32_t y, float acc) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, x), __builtin_bit_cast(h2, y), acc, false);
}

// Eight outputs to a 16-byte vector of T: bf16 through the hardware conversion unless a value is NaN (then
// the contract's rounding, every NaN -> 0x7FC0), f16 through the hardware conversion.
template <typename T>
__device__ __forceinline__ u32x4 pack8(const float* v) {
  if constexpr (std::is_same<T, BF16>::value) {
    float t = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) t += v[e];
    return t == t ? bf16_pack8_hw(v) : bf16_pack8_sw(v);
  } else {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = pack2<T>(v[2 * i], v[2 * i + 1]);
    return r;
  }
}
template <typename T>
__device__ __forceinline__ void unpack8(u32x4 w, float* v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = lo16<T>(w[i]);
    v[2 * i + 1] = hi16<T>(w[i]);
  }
}

// C[m, n] = alpha * sum_k A[m, k] B[k, n] + beta * X[m, n], X = the bias view (which may be C itself: an
// accumulating product) or nothing.  KP = K / 2 pairs.  BT: B is k-contiguous (B[k, n] at b + n*b_sn + k,
// the transposed view of an [N, K] weight); else n-contiguous rows.  Workgroup = one wavefront: 512 columns
// (8 per lane) of RB rows.  Every load of the workgroup is issued before the first use (one round trip to
// memory): the lane's 8 columns of B, its 8 columns of the RB rows of X, and the RB x K block of A spread
// over the lanes (lane l holds pair l of the block), from which each row's pairs go to scalar registers.
constexpr int kExpandRows = 8;
template <typename T, int KP, bool BT, bool HASX>
__global__ __launch_bounds__(64) void mm_expand(hrt_mm_args a) {
  using S = uint16_t;
  constexpr int RB = kExpandRows, HV = (RB * KP + 63) / 64;
  const int lane = threadIdx.x;
  const int64_t n0 = (int64_t)blockIdx.x * 512 + lane * 8;
  const bool live_n = n0 < a.N;
  const int64_t nl = live_n ? n0 : a.N - 8;  // lanes past the end work on the last 8 columns, store nothing
  const int64_t m0 = (int64_t)blockIdx.y * RB;
  const HK_G S* A = gcptr<S>(a.a);
  const HK_G S* B = gcptr<S>(a.b);
  // the A block: pair p = lane + 64 i is (row p / KP, pair p % KP); rows past the end repeat the last row
  uint32_t hblk[HV];
#pragma unroll
  for (int i = 0; i < HV; ++i) {
    const int p = lane + 64 * i < RB * KP ? lane + 64 * i : RB * KP - 1;
    const int64_t m = m0 + p / KP < a.M ? m0 + p / KP : a.M - 1;
    hblk[i] = reinterpret_cast<const HK_G uint32_t*>(A + m * a.a_sm)[p % KP];
  }
  u32x4 xv[RB];
  if constexpr (HASX) {
    const HK_G S* X = gcptr<S>(a.bias);
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int64_t m = m0 + r < a.M ? m0 + r : a.M - 1;
      xv[r] = *reinterpret_cast<const HK_G u32x4*>(X + m * a.bias_sm + nl);
    }
  }
  uint32_t bw[8][KP];  // bw[c][j] = (B[2j, n+c], B[2j+1, n+c])
  if constexpr (BT) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const HK_G uint32_t* col = reinterpret_cast<const HK_G uint32_t*>(B + (nl + c) * a.b_sn);
#pragma unroll
      for (int j = 0; j < KP; ++j) bw[c][j] = col[j];
    }
  } else {
    u32x4 rows[2 * KP];
#pragma unroll
    for (int k = 0; k < 2 * KP; ++k) rows[k] = *reinterpret_cast<const HK_G u32x4*>(B + k * a.b_sk + nl);
#pragma unroll
    for (int j = 0; j < KP; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // columns 2i, 2i+1: low / high halves of row 2j and 2j+1
        bw[2 * i][j] = (rows[2 * j][i] & 0xffffu) | (rows[2 * j + 1][i] << 16);
        bw[2 * i + 1][j] = (rows[2 * j][i] >> 16) | (rows[2 * j + 1][i] & 0xffff0000u);
      }
  }
  HK_G S* C = gptr<S>(a.c);
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    uint32_t h2[KP];
#pragma unroll
    for (int j = 0; j < KP; ++j) h2[j] = __builtin_amdgcn_readlane(hblk[(r * KP + j) / 64], (r * KP + j) % 64);
    float o[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < KP; ++j) acc = dot2<T>(h2[j], bw[c][j], acc);
      o[c] = a.alpha * acc;
    }
    if constexpr (HASX) {
      float xf[8];
      unpack8<T>(xv[r], xf);
#pragma unroll
      for (int c = 0; c < 8; ++c) o[c] = fmaf(a.beta, xf[c], o[c]);
    }
    const u32x4 out = pack8<T>(o);
    if (live_n && m0 + r < a.M) *reinterpret_cast<HK_G u32x4*>(C + (m0 + r) * a.c_sm + n0) = out;
  }
}

// Queues mm_expand when the product fits it: K even and <= 32, one batch, a 16-byte-aligned output with
// unit column stride, A rows k-contiguous and 4-byte aligned, B either k- or n-contiguous with 16-byte
// aligned vectors, N a multiple of 8, and the bias (if any) a full [M, N] view like C's or a row broadcast.
template <typename T>
bool queue_expand(const hrt_mm_args& a, hipStream_t s) {
  const int64_t K = a.K;
  if (K < 2 || K > 32 || K % 2 || a.batch != 1 || a.M <= 0 || a.N < 8 || a.N % 8) return false;
  if (a.c % 16 || a.c_sn != 1 || a.c_sm % 8) return false;
  if (a.a % 4 || a.a_sk != 1 || a.a_sm % 2) return false;
  const bool bt = a.b_sk == 1 && a.b_sn % 2 == 0 && a.b % 4 == 0;
  const bool bn = a.b_sn == 1 && a.b_sk % 8 == 0 && a.b % 16 == 0;
  if (!bt && !bn) return false;
  const bool hasx = a.has_bias && a.beta != 0.f;
  if (hasx && (a.bias % 16 || a.bias_sn != 1 || (a.bias_sm != 0 && a.bias_sm % 8))) return false;
  if (a.M > 0x7fffffffLL || a.N > 0x7fffffffLL) return false;
  const int64_t nb = (a.N + 511) / 512, mb = (a.M + kExpandRows - 1) / kExpandRows;
  if (mb > 65535) return false;
  const dim3 grid((uint32_t)nb, (uint32_t)mb);
  auto go = [&](auto kp, auto btc, auto hxc) {
    hipLaunchKernelGGL((mm_expand<T, decltype(kp)::value, decltype(btc)::value, decltype(hxc)::value>), grid, dim3(64), 0, s, a);
  };
  auto by_x = [&](auto kp, auto btc) {
    if (hasx) go(kp, btc, std::true_type());
    else go(kp, btc, std::false_type());
  };
  auto by_b = [&](auto kp) {
    if (bt) by_x(kp, std::true_type());
    else by_x(kp, std::false_type());
  };
  switch (K / 2) {
    case 1: by_b(std::integral_constant<int, 1>()); break;
    case 2: by_b(std::integral_constant<int, 2>()); break;
    case 4: by_b(std::integral_constant<int, 4>()); break;
    case 8: by_b(std::integral_constant<int, 8>()); break;
    case 16: by_b(std::integral_constant<int, 16>()); break;
    default: return false;  // other ranks keep the matrix-core path
  }
  return true;
}

}  // namespace skinny
}  // namespace hk
