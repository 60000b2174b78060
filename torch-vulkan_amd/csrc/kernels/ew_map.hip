// "ew_map": the elementwise arithmetic of the training step (bias adds outside addmm, activations and
// their backwards, optimizer updates, where), out = f(a, b, c; s0, s1) over a broadcast, strided index
// space.  Reference: the generated kernel family of vkrt/shaders/ew.comp.in:115-257 (op expressions
// tools/gen_shaders.py:53-92) behind csrc/ops_ew.cpp:76-139.
//
// Layout on MI355X.  These kernels are HBM-bound (a bf16 activation moves 4 bytes per element; the VALU
// has ~20 instructions per element to spare at 8 TB/s), so what matters is that every wavefront issues
// 16-byte loads and stores.  The host merges dimensions first; when the last merged dimension is
// contiguous (stride 1) or broadcast (stride 0) in every operand, the vector kernel moves 8 consecutive
// elements per lane: one 16-byte access per bf16/f16 operand, two per fp32 operand, one broadcast value
// per stride-0 operand.  A leading index (rows of a bias add, say) is decomposed once per 8 elements.
// Everything else (transposed views, odd alignments) takes the per-element kernel.  The op is a template
// parameter; element types are kernel arguments tested with wave-uniform branches, so one instance per
// op covers every dtype combination.
//
// Numerics.  Operands are widened to fp32, f is evaluated in fp32 and the result is rounded once to the
// output type (RNE; bf16 NaN -> 0x7FC0).  Floating-point contraction is off in this file except inside
// the activation formulas: a + s*b is a product and a sum, each rounded, as written, which is what the
// CPU restatement of these formulas computes; division and square root are the correctly rounded IEEE
// operations.
#include <algorithm>
#include <array>
#include <string>
#include <utility>

#include "../hrt/registry.h"
#include "device_common.h"

#pragma clang fp contract(off)

namespace hk {
namespace {

constexpr int EW_VEC = 8;  // elements per lane in the vector kernel

constexpr bool ew_uses_b(int op) {
  return op == HRT_EW_ADD || op == HRT_EW_SUB || op == HRT_EW_MUL || op == HRT_EW_DIV || op == HRT_EW_SILU_BWD ||
         op == HRT_EW_GELU_ERF_BWD || op == HRT_EW_GELU_TANH_BWD || op == HRT_EW_ADDCMUL || op == HRT_EW_ADDCDIV ||
         op == HRT_EW_LERP_S || op == HRT_EW_WHERE;
}
constexpr bool ew_uses_c(int op) { return op == HRT_EW_ADDCMUL || op == HRT_EW_ADDCDIV || op == HRT_EW_WHERE; }

// ---- the scalar functions -------------------------------------------------------------------------
// The activations are evaluated branch-free: with random inputs the library tanhf / erff take different
// branches in neighbouring lanes and the kernel becomes VALU-bound (measured on MI355X at 64 M bf16
// elements: tanh-GELU 61 us with tanhf against 47 us with exp2 + v_rcp, silu 57 us with an IEEE division against
// 41 us with exp2 + v_rcp, the same rate as an add).  Their float32 error stays within a few units in the
// last place (v_exp_f32, v_rcp_f32: 1 ulp; the erfc fit: 1.2e-7 relative), far inside the tolerance
// PyTorch's CPU results are held to (rtol 1e-5).  Inside these forms contraction is allowed.
__device__ __forceinline__ float rcp_f(float x) { return __builtin_amdgcn_rcpf(x); }

__device__ __forceinline__ float sigmoid_f(float x) { return rcp_f(1.0f + __expf(-x)); }

// The tanh-GELU pieces from e = exp(-2|u|) in (0, 1] and r = 1 / (1 + e), without cancellation:
// (1 + tanh u) / 2 = (u < 0 ? e : 1) r and 1 - tanh^2 u = 4 e r^2 (1 - t * t would lose all digits
// where |t| is near 1).  No overflow, no branch.
struct TanhParts {
  float half_one_plus_t, sech2;
};
__device__ __forceinline__ TanhParts tanh_parts(float u) {
#pragma clang fp contract(fast)
  const float e = __expf(-2.0f * fabsf(u));
  const float r = rcp_f(1.0f + e);
  return {(u < 0.0f ? e : 1.0f) * r, 4.0f * e * r * r};
}

// Normal CDF Phi(x) = erfc(-x / sqrt 2) / 2 through the Chebyshev fit of erfc (Numerical Recipes in C,
// 2nd ed., section 6.2, erfcc: relative error < 1.2e-7 for all z >= 0).  Taking erfc of |x| keeps the
// relative accuracy of the negative tail, where 1 + erf(x / sqrt 2) would cancel.
__device__ __forceinline__ float phi_f(float x) {
#pragma clang fp contract(fast)
  const float z = fabsf(x) * 0.70710678118654752440f;
  const float t = rcp_f(fmaf(0.5f, z, 1.0f));
  float q = 0.17087277f;
  q = fmaf(q, t, -0.82215223f);
  q = fmaf(q, t, 1.48851587f);
  q = fmaf(q, t, -1.13520398f);
  q = fmaf(q, t, 0.27886807f);
  q = fmaf(q, t, -0.18628806f);
  q = fmaf(q, t, 0.09678418f);
  q = fmaf(q, t, 0.37409196f);
  q = fmaf(q, t, 1.00002368f);
  q = fmaf(q, t, -1.26551223f);
  const float half_erfc = 0.5f * t * __expf(fmaf(-z, z, q));
  return x < 0.0f ? half_erfc : 1.0f - half_erfc;
}

// torch.pow(x, e) for a scalar exponent: the exponents PyTorch's CPU kernel evaluates by multiplication,
// square root or reciprocal give those results; other exponents use powf (negative bases with integral
// exponents follow C99 pow).
__device__ __forceinline__ float pow_f(float x, float e) {
  if (e == 2.0f) return x * x;
  if (e == 3.0f) return x * x * x;
  if (e == 0.5f) return sqrtf(x);
  if (e == -0.5f) return 1.0f / sqrtf(x);
  if (e == -1.0f) return 1.0f / x;
  if (e == -2.0f) return 1.0f / (x * x);
  return powf(x, e);
}

constexpr float kInvSqrt2Pi = 0.39894228040143267794f;   // 1/sqrt(2 pi)
constexpr float kSqrt2OverPi = 0.79788456080286535588f;  // sqrt(2/pi)
constexpr float kGeluKappa = 0.044715f;

template <int OP>
__device__ __forceinline__ float ew_f(float x, float y, float z, float s0, float s1) {
  if constexpr (OP == HRT_EW_ADD) return x + s0 * y;
  else if constexpr (OP == HRT_EW_SUB) return x - s0 * y;
  else if constexpr (OP == HRT_EW_MUL) return x * y;
  else if constexpr (OP == HRT_EW_DIV) return x / y;
  else if constexpr (OP == HRT_EW_ADD_S) return x + s0;
  else if constexpr (OP == HRT_EW_MUL_S) return x * s0;
  else if constexpr (OP == HRT_EW_DIV_S) return x / s0;
  else if constexpr (OP == HRT_EW_AXPB) return s1 + s0 * x;
  else if constexpr (OP == HRT_EW_RDIV_S) return s0 / x;
  else if constexpr (OP == HRT_EW_POW_S) return pow_f(x, s0);
  else if constexpr (OP == HRT_EW_NEG) return -x;
  else if constexpr (OP == HRT_EW_RSQRT) return 1.0f / sqrtf(x);
  else if constexpr (OP == HRT_EW_RECIP) return 1.0f / x;
  else if constexpr (OP == HRT_EW_EXP) return expf(x);
  else if constexpr (OP == HRT_EW_SIN) return sinf(x);
  else if constexpr (OP == HRT_EW_COS) return cosf(x);
  else if constexpr (OP == HRT_EW_SQRT) return sqrtf(x);
  else if constexpr (OP == HRT_EW_TANH) return tanhf(x);
  else if constexpr (OP == HRT_EW_SIGMOID) return sigmoid_f(x);
  else if constexpr (OP == HRT_EW_RELU) return x < 0.0f ? 0.0f : x;  // NaN stays NaN
  else if constexpr (OP == HRT_EW_SILU) return x * sigmoid_f(x);
  else if constexpr (OP == HRT_EW_GELU_ERF) return x * phi_f(x);
  else if constexpr (OP == HRT_EW_GELU_TANH) {
#pragma clang fp contract(fast)
    return x * tanh_parts(kSqrt2OverPi * (x + kGeluKappa * x * x * x)).half_one_plus_t;
  } else if constexpr (OP == HRT_EW_SILU_BWD) {
#pragma clang fp contract(fast)
    const float s = sigmoid_f(y);  // x = grad, y = input
    return x * s * (1.0f + y * (1.0f - s));
  } else if constexpr (OP == HRT_EW_GELU_ERF_BWD) {
#pragma clang fp contract(fast)
    const float pdf = kInvSqrt2Pi * __expf(-0.5f * y * y);
    return x * (phi_f(y) + y * pdf);
  } else if constexpr (OP == HRT_EW_GELU_TANH_BWD) {
#pragma clang fp contract(fast)
    const float y2 = y * y;
    const TanhParts p = tanh_parts(kSqrt2OverPi * (y + kGeluKappa * y2 * y));
    const float dright = 0.5f * y * p.sech2 * kSqrt2OverPi * (1.0f + 3.0f * kGeluKappa * y2);
    return x * (p.half_one_plus_t + dright);
  } else if constexpr (OP == HRT_EW_ADDCMUL) return x + s0 * y * z;
  else if constexpr (OP == HRT_EW_ADDCDIV) return x + s0 * y / z;
  else if constexpr (OP == HRT_EW_LERP_S) return fabsf(s0) < 0.5f ? x + s0 * (y - x) : y - (y - x) * (1.0f - s0);
  else if constexpr (OP == HRT_EW_WHERE) return z != 0.0f ? x : y;
  else return 0.0f;
}

// ---- typed element access (dtype is wave-uniform) ---------------------------------------------------
__device__ __forceinline__ float ld1(uint64_t base, int dt, int64_t e) {
  if (dt == HRT_F32) return gcptr<float>(base)[e];
  if (dt == HRT_BF16) return bf16_bits_to_f32(gcptr<uint16_t>(base)[e]);
  if (dt == HRT_F16) return f16_bits_to_f32(gcptr<uint16_t>(base)[e]);
  return gcptr<uint8_t>(base)[e] != 0 ? 1.0f : 0.0f;  // HRT_RAW8: bool
}

__device__ __forceinline__ void st1(uint64_t base, int dt, int64_t e, float v) {
  if (dt == HRT_F32) gptr<float>(base)[e] = v;
  else if (dt == HRT_BF16) gptr<uint16_t>(base)[e] = (uint16_t)f32_to_bf16_bits(v);
  else gptr<uint16_t>(base)[e] = (uint16_t)f32_to_f16_bits(v);
}

// 8 consecutive elements starting at element e (a multiple of 8; the base is 16-byte aligned, 8-byte for
// bytes), or one broadcast value when the operand's inner stride is 0.  The streamed operands are read
// and written nontemporally: a flat bf16 add at 64 M elements runs at 6.5 TB/s that way against 5.8 TB/s
// with cached accesses (measured on MI355X).  Loading is split from converting so that every operand's
// load is in flight before the first conversion waits for data.
struct Raw8 {
  u32x4 lo, hi;  // f32: 8 words; 16-bit types: lo; bytes: lo.xy; broadcast: lo.x holds the element's bits
};

__device__ __forceinline__ Raw8 raw_ld8(uint64_t base, int dt, int64_t e, bool bcast) {
  Raw8 r;
  if (bcast) {
    if (dt == HRT_F32) r.lo.x = gcptr<uint32_t>(base)[e];
    else if (dt == HRT_RAW8) r.lo.x = gcptr<uint8_t>(base)[e];
    else r.lo.x = gcptr<uint16_t>(base)[e];
  } else if (dt == HRT_F32) {
    const HK_G u32x4* p = gcptr<u32x4>(base) + e / 4;
    r.lo = __builtin_nontemporal_load(p);
    r.hi = __builtin_nontemporal_load(p + 1);
  } else if (dt == HRT_RAW8) {
    const u32x2 u = __builtin_nontemporal_load(gcptr<u32x2>(base) + e / 8);
    r.lo.x = u.x;
    r.lo.y = u.y;
  } else {
    r.lo = __builtin_nontemporal_load(gcptr<u32x4>(base) + e / 8);
  }
  return r;
}

__device__ __forceinline__ float cvt1(uint32_t bits, int dt) {
  if (dt == HRT_F32) return __uint_as_float(bits);
  if (dt == HRT_BF16) return bf16_bits_to_f32(bits & 0xffffu);
  if (dt == HRT_F16) return f16_bits_to_f32(bits & 0xffffu);
  return (bits & 0xffu) != 0 ? 1.0f : 0.0f;
}

__device__ __forceinline__ void cvt8(float (&v)[EW_VEC], const Raw8& r, int dt, bool bcast) {
  if (bcast) {
    const float s = cvt1(r.lo.x, dt);
#pragma unroll
    for (int i = 0; i < EW_VEC; ++i) v[i] = s;
  } else if (dt == HRT_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = __uint_as_float(r.lo[i]);
      v[4 + i] = __uint_as_float(r.hi[i]);
    }
  } else if (dt == HRT_RAW8) {
#pragma unroll
    for (int i = 0; i < EW_VEC; ++i) v[i] = ((r.lo[i / 4] >> (8 * (i % 4))) & 0xffu) != 0 ? 1.0f : 0.0f;
  } else if (dt == HRT_BF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16_bits_to_f32(r.lo[i] & 0xffffu);
      v[2 * i + 1] = bf16_bits_to_f32(r.lo[i] >> 16);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = f16_bits_to_f32(r.lo[i] & 0xffffu);
      v[2 * i + 1] = f16_bits_to_f32(r.lo[i] >> 16);
    }
  }
}

__device__ __forceinline__ void st8(uint64_t base, int dt, int64_t e, const float (&v)[EW_VEC]) {
  if (dt == HRT_F32) {
    HK_G f32x4* p = gptr<f32x4>(base) + e / 4;
    __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, p);
    __builtin_nontemporal_store(f32x4{v[4], v[5], v[6], v[7]}, p + 1);
  } else {
    u32x4 u;
    if (dt == HRT_BF16) {
#pragma unroll
      for (int i = 0; i < 4; ++i) u[i] = f32_to_bf16_bits(v[2 * i]) | (f32_to_bf16_bits(v[2 * i + 1]) << 16);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) u[i] = f32_to_f16_bits(v[2 * i]) | (f32_to_f16_bits(v[2 * i + 1]) << 16);
    }
    __builtin_nontemporal_store(u, gptr<u32x4>(base) + e / 8);
  }
}

// ---- kernel arguments ---------------------------------------------------------------------------------
struct EwOperand {
  uint64_t p;
  int dt;
  int bcast;  // vector kernel: inner stride 0
};

struct EwKernelArgs {
  EwOperand o[4];  // out, a, b, c
  float s0, s1;
  int ndim;        // merged dimensions (vector kernel: the leading ndim-1 are decomposed per chunk)
  int small;       // every index fits in 32 bits
  int64_t n;       // elements (per-element kernel) or 8-element chunks (vector kernel)
  int64_t n_elems; // vector kernel, ndim == 1: elements (the last chunk may be partial)
  int64_t inner8;  // vector kernel: chunks per inner row
  int64_t sizes[HRT_MAX_DIMS];
  int64_t st[4][HRT_MAX_DIMS];
};

// Offsets of the four operands for index q over dimensions [0, nd) (q's innermost digit is dimension
// nd-1).  I = uint32_t when every index fits, which turns the divisions into the short 32-bit sequence.
template <typename I>
__device__ __forceinline__ void decompose(const EwKernelArgs& p, int nd, int64_t q64, int64_t (&off)[4]) {
  I q = (I)q64;
  off[0] = off[1] = off[2] = off[3] = 0;
  for (int d = nd - 1; d >= 0; --d) {
    const I sz = (I)p.sizes[d];
    const I nq = q / sz;
    const int64_t r = (int64_t)(q - nq * sz);
    q = nq;
#pragma unroll
    for (int k = 0; k < 4; ++k) off[k] += r * p.st[k][d];
  }
}

// Per-element kernel: any strides.
template <int OP>
__global__ __launch_bounds__(256) void ew_any(EwKernelArgs p) {
  const int64_t step = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < p.n; i += step) {
    int64_t off[4];
    if (p.small) decompose<uint32_t>(p, p.ndim, i, off);
    else decompose<uint64_t>(p, p.ndim, i, off);
    const float x = ld1(p.o[1].p, p.o[1].dt, off[1]);
    const float y = ew_uses_b(OP) ? ld1(p.o[2].p, p.o[2].dt, off[2]) : 0.0f;
    const float z = ew_uses_c(OP) ? ld1(p.o[3].p, p.o[3].dt, off[3]) : 0.0f;
    st1(p.o[0].p, p.o[0].dt, off[0], ew_f<OP>(x, y, z, p.s0, p.s1));
  }
}

// Element type of operand k (0 out, 1 a, 2 b, 3 c) in an instance for element type T: all float
// operands are T (the where condition is bytes); T = -1 reads the types from the arguments.
template <int T, int OP>
__device__ __forceinline__ int opdt(const EwKernelArgs& p, int k) {
  if constexpr (T < 0) return p.o[k].dt;
  else return (k == 3 && OP == HRT_EW_WHERE) ? HRT_RAW8 : T;
}

// Vector kernel: the innermost merged dimension has stride 0 or 1 in every operand; each lane handles
// one chunk of 8 consecutive elements of it.  T >= 0: every float operand has element type T, which
// the common training cases satisfy and which compiles to straight-line code; T = -1: mixed types.
template <int OP, int T>
__global__ __launch_bounds__(256) void ew_vec(EwKernelArgs p) {
  const int64_t step = (int64_t)gridDim.x * 256;
  for (int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x; j < p.n; j += step) {
    int64_t off[4];
    int64_t inner;  // first element of the chunk along the innermost dimension
    if (p.ndim <= 1) {
      off[0] = off[1] = off[2] = off[3] = 0;
      inner = j * EW_VEC;
    } else {
      const int64_t row = j / p.inner8;
      inner = (j - row * p.inner8) * EW_VEC;
      if (p.small) decompose<uint32_t>(p, p.ndim - 1, row, off);
      else decompose<uint64_t>(p, p.ndim - 1, row, off);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) off[k] += p.o[k].bcast ? 0 : inner;
    if (p.ndim > 1 || inner + EW_VEC <= p.n_elems) {
      Raw8 ra, rb, rc;
      ra = raw_ld8(p.o[1].p, opdt<T, OP>(p, 1), off[1], p.o[1].bcast);
      if constexpr (ew_uses_b(OP)) rb = raw_ld8(p.o[2].p, opdt<T, OP>(p, 2), off[2], p.o[2].bcast);
      if constexpr (ew_uses_c(OP)) rc = raw_ld8(p.o[3].p, opdt<T, OP>(p, 3), off[3], p.o[3].bcast);
      float x[EW_VEC], y[EW_VEC], z[EW_VEC];
      cvt8(x, ra, opdt<T, OP>(p, 1), p.o[1].bcast);
      if constexpr (ew_uses_b(OP)) cvt8(y, rb, opdt<T, OP>(p, 2), p.o[2].bcast);
      if constexpr (ew_uses_c(OP)) cvt8(z, rc, opdt<T, OP>(p, 3), p.o[3].bcast);
      float r[EW_VEC];
#pragma unroll
      for (int i = 0; i < EW_VEC; ++i)
        r[i] = ew_f<OP>(x[i], ew_uses_b(OP) ? y[i] : 0.0f, ew_uses_c(OP) ? z[i] : 0.0f, p.s0, p.s1);
      st8(p.o[0].p, opdt<T, OP>(p, 0), off[0], r);
    } else {  // the partial last chunk of a 1-D space
      for (int64_t i = 0; i < p.n_elems - inner; ++i) {
        int64_t e[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) e[k] = off[k] + (p.o[k].bcast ? 0 : i);
        const float x = ld1(p.o[1].p, opdt<T, OP>(p, 1), e[1]);
        const float y = ew_uses_b(OP) ? ld1(p.o[2].p, opdt<T, OP>(p, 2), e[2]) : 0.0f;
        const float z = ew_uses_c(OP) ? ld1(p.o[3].p, opdt<T, OP>(p, 3), e[3]) : 0.0f;
        st1(p.o[0].p, opdt<T, OP>(p, 0), e[0], ew_f<OP>(x, y, z, p.s0, p.s1));
      }
    }
  }
}

// Flat kernel: one dimension, every operand contiguous, one element type T.  The most common case of the
// training step (activations and their backwards, residual and LoRA sums, optimizer updates) with the
// least work ahead of the loads: a lane finds its chunk from its index alone and its wave issues the
// loads after one round of argument loads (the general kernels need three, which at one chunk per wave
// cost ~10% of HBM throughput).
struct EwFlatArgs {
  uint64_t out, a, b, c;
  float s0, s1;
  int64_t n;
};

// fp32: a workgroup covers 2048 consecutive elements and a lane takes two groups of 4 that lie 1024
// elements apart, so that each 16-byte load instruction of a wavefront reads one contiguous kilobyte
// (8 consecutive fp32 per lane would leave every other 16-byte piece to a second instruction).
template <int OP>
__device__ __forceinline__ void ew_flat_f32(const EwFlatArgs& p) {
  constexpr bool W = OP == HRT_EW_WHERE;
  const int64_t e0 = (int64_t)blockIdx.x * 2048 + threadIdx.x * 4, e1 = e0 + 1024;
  if ((int64_t)blockIdx.x * 2048 + 2048 <= p.n) {
    const HK_G u32x4* pa = gcptr<u32x4>(p.a);
    const HK_G u32x4* pb = gcptr<u32x4>(p.b);
    const HK_G u32x4* pc = gcptr<u32x4>(p.c);
    u32x4 a0 = __builtin_nontemporal_load(pa + e0 / 4), a1 = __builtin_nontemporal_load(pa + e1 / 4);
    u32x4 b0, b1, c0, c1;
    uint32_t m0 = 0, m1 = 0;
    if constexpr (ew_uses_b(OP)) {
      b0 = __builtin_nontemporal_load(pb + e0 / 4);
      b1 = __builtin_nontemporal_load(pb + e1 / 4);
    }
    if constexpr (W) {
      m0 = __builtin_nontemporal_load(gcptr<uint32_t>(p.c) + e0 / 4);
      m1 = __builtin_nontemporal_load(gcptr<uint32_t>(p.c) + e1 / 4);
    } else if constexpr (ew_uses_c(OP)) {
      c0 = __builtin_nontemporal_load(pc + e0 / 4);
      c1 = __builtin_nontemporal_load(pc + e1 / 4);
    }
    f32x4 r0, r1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float z0 = 0.0f, z1 = 0.0f;
      if constexpr (W) {
        z0 = ((m0 >> (8 * i)) & 0xffu) ? 1.0f : 0.0f;
        z1 = ((m1 >> (8 * i)) & 0xffu) ? 1.0f : 0.0f;
      } else if constexpr (ew_uses_c(OP)) {
        z0 = __uint_as_float(c0[i]);
        z1 = __uint_as_float(c1[i]);
      }
      r0[i] = ew_f<OP>(__uint_as_float(a0[i]), ew_uses_b(OP) ? __uint_as_float(b0[i]) : 0.0f, z0, p.s0, p.s1);
      r1[i] = ew_f<OP>(__uint_as_float(a1[i]), ew_uses_b(OP) ? __uint_as_float(b1[i]) : 0.0f, z1, p.s0, p.s1);
    }
    __builtin_nontemporal_store(r0, gptr<f32x4>(p.out) + e0 / 4);
    __builtin_nontemporal_store(r1, gptr<f32x4>(p.out) + e1 / 4);
  } else {  // the last, partial workgroup
    for (int h = 0; h < 2; ++h) {
      const int64_t e = h ? e1 : e0;
      for (int64_t i = e; i < e + 4 && i < p.n; ++i) {
        const float x = ld1(p.a, HRT_F32, i);
        const float y = ew_uses_b(OP) ? ld1(p.b, HRT_F32, i) : 0.0f;
        const float z = ew_uses_c(OP) ? ld1(p.c, W ? HRT_RAW8 : HRT_F32, i) : 0.0f;
        st1(p.out, HRT_F32, i, ew_f<OP>(x, y, z, p.s0, p.s1));
      }
    }
  }
}

template <int OP, int T>
__global__ __launch_bounds__(256) void ew_flat(EwFlatArgs p) {
  if constexpr (T == HRT_F32) {
    ew_flat_f32<OP>(p);
    return;
  }
  constexpr int TC = OP == HRT_EW_WHERE ? HRT_RAW8 : T;
  const int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) * EW_VEC;
  if (e + EW_VEC <= p.n) {
    Raw8 ra, rb, rc;
    ra = raw_ld8(p.a, T, e, false);
    if constexpr (ew_uses_b(OP)) rb = raw_ld8(p.b, T, e, false);
    if constexpr (ew_uses_c(OP)) rc = raw_ld8(p.c, TC, e, false);
    float x[EW_VEC], y[EW_VEC], z[EW_VEC], r[EW_VEC];
    cvt8(x, ra, T, false);
    if constexpr (ew_uses_b(OP)) cvt8(y, rb, T, false);
    if constexpr (ew_uses_c(OP)) cvt8(z, rc, TC, false);
#pragma unroll
    for (int i = 0; i < EW_VEC; ++i)
      r[i] = ew_f<OP>(x[i], ew_uses_b(OP) ? y[i] : 0.0f, ew_uses_c(OP) ? z[i] : 0.0f, p.s0, p.s1);
    st8(p.out, T, e, r);
  } else {
    for (int64_t i = e; i < p.n; ++i) {
      const float x = ld1(p.a, T, i);
      const float y = ew_uses_b(OP) ? ld1(p.b, T, i) : 0.0f;
      const float z = ew_uses_c(OP) ? ld1(p.c, TC, i) : 0.0f;
      st1(p.out, T, i, ew_f<OP>(x, y, z, p.s0, p.s1));
    }
  }
}

// ---- host side ----------------------------------------------------------------------------------------
uint64_t ew_elem_size(int dt) {
  switch (dt) {
    case HRT_F32: return 4;
    case HRT_BF16:
    case HRT_F16: return 2;
    case HRT_RAW8: return 1;
    default: return 0;
  }
}

bool is_float_code(int dt) { return dt == HRT_F32 || dt == HRT_BF16 || dt == HRT_F16; }

// kind: -2 per-element kernel; -1 vector kernel with mixed types; HRT_F32/BF16/F16 vector kernel with
// one element type; 16 + HRT_F32/BF16/F16 flat kernel.
using EwLaunch = void (*)(int kind, dim3 grid, hipStream_t s, const EwKernelArgs& p, const EwFlatArgs& f);

template <int OP>
void ew_launch_op(int kind, dim3 grid, hipStream_t s, const EwKernelArgs& p, const EwFlatArgs& f) {
  switch (kind) {
    case 16 + HRT_F32: hipLaunchKernelGGL((ew_flat<OP, HRT_F32>), grid, dim3(256), 0, s, f); break;
    case 16 + HRT_BF16: hipLaunchKernelGGL((ew_flat<OP, HRT_BF16>), grid, dim3(256), 0, s, f); break;
    case 16 + HRT_F16: hipLaunchKernelGGL((ew_flat<OP, HRT_F16>), grid, dim3(256), 0, s, f); break;
    case HRT_F32: hipLaunchKernelGGL((ew_vec<OP, HRT_F32>), grid, dim3(256), 0, s, p); break;
    case HRT_BF16: hipLaunchKernelGGL((ew_vec<OP, HRT_BF16>), grid, dim3(256), 0, s, p); break;
    case HRT_F16: hipLaunchKernelGGL((ew_vec<OP, HRT_F16>), grid, dim3(256), 0, s, p); break;
    case -1: hipLaunchKernelGGL((ew_vec<OP, -1>), grid, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL(ew_any<OP>, grid, dim3(256), 0, s, p); break;
  }
}

template <int... OPS>
constexpr std::array<EwLaunch, sizeof...(OPS)> ew_table(std::integer_sequence<int, OPS...>) {
  return {&ew_launch_op<OPS>...};
}
constexpr auto kEwLaunch = ew_table(std::make_integer_sequence<int, HRT_EW_OP_COUNT>{});

bool launch_ew_map(const void* args, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_ew_args*>(args);
  if (a.op < 0 || a.op >= HRT_EW_OP_COUNT) return ctx.fail("unknown elementwise op code");
  if (a.ndim < 0 || a.ndim > HRT_MAX_DIMS) return ctx.fail("ndim out of range");
  const bool ub = ew_uses_b(a.op), uc = ew_uses_c(a.op);
  if (!is_float_code(a.out_dtype) || !is_float_code(a.a_dtype)) return ctx.fail("out and a must be f32, bf16 or f16");
  if (ub && !is_float_code(a.b_dtype)) return ctx.fail("b must be f32, bf16 or f16");
  if (uc && !(a.op == HRT_EW_WHERE ? a.c_dtype == HRT_RAW8 : is_float_code(a.c_dtype)))
    return ctx.fail(a.op == HRT_EW_WHERE ? "where: c must be HRT_RAW8 (bool)" : "c must be f32, bf16 or f16");
  if ((!ub && a.b != 0) || (!uc && a.c != 0)) return ctx.fail("an operand the op does not read has a non-zero address");

  EwKernelArgs p{};
  const uint64_t addr[4] = {a.out, a.a, ub ? a.b : 0, uc ? a.c : 0};
  const int dts[4] = {a.out_dtype, a.a_dtype, a.b_dtype, a.c_dtype};
  const int64_t* strides[4] = {a.out_strides, a.a_strides, a.b_strides, a.c_strides};
  const bool used[4] = {true, true, ub, uc};
  const char* names[4] = {"out", "a", "b", "c"};
  int64_t n = 1;
  for (int d = 0; d < a.ndim; ++d) {
    if (a.sizes[d] < 0) return ctx.fail("negative size");
    n *= a.sizes[d];
  }
  if (n == 0) return true;
  for (int d = 0; d < a.ndim; ++d) {
    if (a.sizes[d] > 1 && a.out_strides[d] == 0) return ctx.fail("out has stride 0 along a dimension of size > 1");
  }
  for (int k = 0; k < 4; ++k) {
    p.o[k].p = used[k] ? addr[k] : 0;
    p.o[k].dt = used[k] ? dts[k] : HRT_F32;
    if (!used[k]) continue;
    for (int d = 0; d < a.ndim; ++d)
      if (strides[k][d] < 0) return ctx.fail(std::string("negative stride in ") + names[k]);
    if (!ctx.check(addr[k], hrt::span_bytes(a.ndim, a.sizes, strides[k], ew_elem_size(dts[k])), names[k])) return false;
  }
  // Canonical index space: size-1 dimensions dropped, neighbours merged where every operand read or
  // written is laid out consecutively across them (the launch then takes the fewest dimensions).
  p.ndim = 0;
  for (int d = 0; d < a.ndim; ++d) {
    if (a.sizes[d] == 1) continue;
    bool merge = p.ndim > 0;
    for (int k = 0; k < 4 && merge; ++k)
      if (used[k]) merge = p.st[k][p.ndim - 1] == strides[k][d] * a.sizes[d];
    const int slot = merge ? p.ndim - 1 : p.ndim++;
    p.sizes[slot] = merge ? p.sizes[slot] * a.sizes[d] : a.sizes[d];
    for (int k = 0; k < 4; ++k) p.st[k][slot] = used[k] ? strides[k][d] : 0;
  }
  p.s0 = a.s0;
  p.s1 = a.s1;

  // Vector form: innermost dimension contiguous or broadcast everywhere, chunk starts aligned.
  bool vec = p.ndim >= 1;
  const int in = p.ndim - 1;
  if (vec) {
    for (int k = 0; k < 4 && vec; ++k) {
      if (!used[k]) continue;
      const int64_t s = p.st[k][in];
      if (s != 0 && s != 1) vec = false;
      if (k == 0 && s != 1) vec = false;
      p.o[k].bcast = s == 0;
      if (s == 1) {
        const uint64_t align = dts[k] == HRT_RAW8 ? 8 : 16;
        if (addr[k] % align) vec = false;
        for (int d = 0; d < in; ++d)
          if (p.st[k][d] % EW_VEC) vec = false;
      }
    }
    if (p.ndim > 1 && p.sizes[in] % EW_VEC) vec = false;
  }
  if (!vec)
    for (int k = 0; k < 4; ++k) p.o[k].bcast = 0;

  // 32-bit index arithmetic when every index and size fits.
  const int64_t lim = (int64_t)1 << 31;
  p.small = n < lim;
  int64_t chunks;
  if (vec) {
    p.n_elems = p.ndim == 1 ? n : 0;
    p.inner8 = p.sizes[in] / EW_VEC;
    chunks = p.ndim == 1 ? cdiv(n, EW_VEC) : n / EW_VEC;
    p.n = chunks;
  } else {
    chunks = n;
    p.n = n;
  }
  int kind = -2;
  if (vec) {
    kind = a.out_dtype;
    for (int k = 1; k < 4; ++k)
      if (used[k] && !(k == 3 && a.op == HRT_EW_WHERE) && dts[k] != a.out_dtype) kind = -1;
  }
  EwFlatArgs f{};
  int64_t blocks = std::min<int64_t>(cdiv(chunks, 256), (int64_t)1 << 20);
  bool flat = kind >= 0 && p.ndim == 1 && cdiv(chunks, 256) < ((int64_t)1 << 31);
  for (int k = 0; k < 4 && flat; ++k)
    if (used[k] && p.o[k].bcast) flat = false;
  if (flat) {  // one chunk per lane, no grid-stride loop
    f = EwFlatArgs{a.out, a.a, ub ? a.b : 0, uc ? a.c : 0, a.s0, a.s1, n};
    blocks = cdiv(chunks, 256);
    kind += 16;
  }
  kEwLaunch[a.op](kind, dim3((uint32_t)blocks), ctx.stream, p, f);
  return hrt::launch_ok(hipGetLastError(), ctx, "ew_map");
}
HRT_REGISTER("ew_map", hrt_ew_args, launch_ew_map);

}  // namespace
}  // namespace hk
