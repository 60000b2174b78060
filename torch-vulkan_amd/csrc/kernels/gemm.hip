// Portable GEMM "mm_{f32,bf16,f16}": c = alpha * a @ b + beta * bias with arbitrary strides, fp32 FMA.
// Serves the f32 path (where fp32 accuracy is required) and bf16/f16 when matrix cores are switched off,
// like the reference's tiled kernel vkrt/shaders/mm.comp.in:90-154 (same math: fp32 accumulate, epilogue
// alpha*acc + beta*bias, one rounding at the store).  64x64 output tile per 256-thread workgroup, 4x4 per
// thread, K in steps of 16 staged through LDS as fp32.
#include "../hrt/registry.h"
#include "device_common.h"

namespace hk {
namespace {

constexpr int BM = 64, BN = 64, BK = 16;

template <typename T>
__device__ __forceinline__ float ldT(const typename T::storage* p) {
  return T::to_f32(*p);
}

template <typename T>
__global__ __launch_bounds__(256) void mm_fma(hrt_mm_args p) {
  using S = typename T::storage;
  __shared__ float As[BK][BM + 4];
  __shared__ float Bs[BK][BN + 4];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int64_t bz = blockIdx.z;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const S* A = reinterpret_cast<const S*>(p.a) + bz * p.a_sb;
  const S* B = reinterpret_cast<const S*>(p.b) + bz * p.b_sb;
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < p.K; k0 += BK) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + i * 256;
      // A tile: consecutive threads walk m when m is the contiguous axis, k otherwise
      int m, k;
      if (p.a_sm == 1) {
        m = e & 63, k = e >> 6;
      } else {
        m = e >> 4, k = e & 15;
      }
      const int64_t gm = m0 + m, gk = k0 + k;
      As[k][m] = (gm < p.M && gk < p.K) ? ldT<T>(A + gm * p.a_sm + gk * p.a_sk) : 0.f;
      int n, kb;
      if (p.b_sk == 1 && p.b_sn != 1) {
        n = e >> 4, kb = e & 15;
      } else {
        n = e & 63, kb = e >> 6;
      }
      const int64_t gn = n0 + n, gkb = k0 + kb;
      Bs[kb][n] = (gn < p.N && gkb < p.K) ? ldT<T>(B + gkb * p.b_sk + gn * p.b_sn) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < BK; ++k) {
      float ra[4], rb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) ra[i] = As[k][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) rb[j] = Bs[k][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(ra[i], rb[j], acc[i][j]);
    }
    __syncthreads();
  }
  S* C = reinterpret_cast<S*>(p.c) + bz * p.c_sb;
  const S* bias = reinterpret_cast<const S*>(p.bias);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t gm = m0 + ty * 4 + i;
    if (gm >= p.M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t gn = n0 + tx * 4 + j;
      if (gn >= p.N) continue;
      float r = p.alpha * acc[i][j];
      if (p.has_bias) r += p.beta * ldT<T>(bias + bz * p.bias_sb + gm * p.bias_sm + gn * p.bias_sn);
      C[gm * p.c_sm + gn * p.c_sn] = T::from_f32(r);
    }
  }
}

}  // namespace

// Shared operand checks of every GEMM launcher (also used by the matrix-core kernels).
bool mm_check_operands(const hrt_mm_args& a, uint64_t elem, hrt::LaunchCtx& ctx) {
  if (a.M <= 0 || a.N <= 0 || a.K <= 0 || a.batch <= 0) return ctx.fail("empty GEMM");
  if (a.batch > 65535) return ctx.fail("batch above 65535");
  if (a.a_sb < 0 || a.a_sm < 0 || a.a_sk < 0 || a.b_sb < 0 || a.b_sk < 0 || a.b_sn < 0 || a.c_sb < 0 || a.c_sm < 0 ||
      a.c_sn < 0 || a.bias_sb < 0 || a.bias_sm < 0 || a.bias_sn < 0)
    return ctx.fail("negative stride");
  const int64_t sa[3] = {a.batch, a.M, a.K}, ta[3] = {a.a_sb, a.a_sm, a.a_sk};
  const int64_t sb[3] = {a.batch, a.K, a.N}, tb[3] = {a.b_sb, a.b_sk, a.b_sn};
  const int64_t sc[3] = {a.batch, a.M, a.N}, tc[3] = {a.c_sb, a.c_sm, a.c_sn};
  const int64_t tbias[3] = {a.bias_sb, a.bias_sm, a.bias_sn};
  if (!ctx.check(a.a, hrt::span_bytes(3, sa, ta, elem), "a") || !ctx.check(a.b, hrt::span_bytes(3, sb, tb, elem), "b") ||
      !ctx.check(a.c, hrt::span_bytes(3, sc, tc, (a.flags & HRT_MM_F32_OUT) ? 4 : elem), "c") ||
      (a.has_bias && !ctx.check(a.bias, hrt::span_bytes(3, sc, tbias, elem), "bias")))
    return false;
  return true;
}

namespace {

template <typename T>
bool launch_mm_fma(const void* p, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_mm_args*>(p);
  if (a.flags != 0) return ctx.fail("the FMA GEMM takes no flags");
  if (!mm_check_operands(a, sizeof(typename T::storage), ctx)) return false;
  if (cdiv(a.M, BM) > 65535) return ctx.fail("M too large for the FMA kernel grid");
  const dim3 grid((uint32_t)cdiv(a.N, BN), (uint32_t)cdiv(a.M, BM), (uint32_t)a.batch);
  hipLaunchKernelGGL(mm_fma<T>, grid, dim3(256), 0, ctx.stream, a);
  return hrt::launch_ok(hipGetLastError(), ctx, "mm_fma");
}

HRT_REGISTER("mm_f32", hrt_mm_args, launch_mm_fma<F32>);
HRT_REGISTER("mm_bf16", hrt_mm_args, launch_mm_fma<BF16>);
HRT_REGISTER("mm_f16", hrt_mm_args, launch_mm_fma<F16>);

}  // namespace
}  // namespace hk
