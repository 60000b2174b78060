// Fused attention with fp32 arithmetic throughout: "attn_{fwd,dkdv,dq}_fma_{f32,bf16,f16}".
//
// The f32 path of the reference (vkrt/shaders/attn.comp.in:256-395, its scalar kernels) and the bf16/f16
// path when matrix cores are switched off: logits, P and dS stay fp32 (no rounding before the second
// products), so f32 inputs meet a 1e-5 relative L2 bound.  Not the performance path: one wavefront of
// 64 lanes per workgroup, one query (forward, dQ) or key (dK/dV) per lane, the streamed operand staged in
// LDS as fp32 and read as broadcasts, the lane's own rows kept in LDS with a +1 padded stride.
#include <cmath>

#include "../hrt/registry.h"
#include "device_common.h"

namespace hk {

bool attn_check(const hrt_attn_args& a, bool fwd, bool dkdv, bool dq, uint64_t elem, hrt::LaunchCtx& ctx);

namespace {

template <typename T>
__device__ __forceinline__ float ldx(const typename T::storage* p, int64_t i) {
  return T::to_f32(p[i]);
}

constexpr int FT = 32;  // streamed rows per tile

template <typename T, int DP>
__global__ __launch_bounds__(64) void attn_fwd_fma(hrt_attn_args p, int nqb) {
  using S = typename T::storage;
  __shared__ float kt[FT][DP], vt[FT][DP];
  const int lane = threadIdx.x;
  const int64_t bh = blockIdx.x / nqb, qb = blockIdx.x % nqb;
  const int64_t b = bh / p.H, hh = bh % p.H;
  const int D = p.D, Sq = p.Sq, Sk = p.Sk;
  const S* Q = reinterpret_cast<const S*>(p.q) + b * p.q_sb + hh * p.q_sh;
  const S* K = reinterpret_cast<const S*>(p.k) + b * p.k_sb + hh * p.k_sh;
  const S* V = reinterpret_cast<const S*>(p.v) + b * p.v_sb + hh * p.v_sh;
  const int64_t q = qb * 64 + lane;
  float qr[DP], o[DP];
#pragma unroll
  for (int d = 0; d < DP; ++d) {
    qr[d] = (q < Sq && d < D) ? ldx<T>(Q, q * p.q_ss + d) : 0.f;
    o[d] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  for (int64_t k0 = 0; k0 < Sk; k0 += FT) {
    __syncthreads();
    for (int e = lane; e < FT * DP; e += 64) {
      const int j = e / DP, d = e % DP;
      const bool ok = k0 + j < Sk && d < D;
      kt[j][d] = ok ? ldx<T>(K, (k0 + j) * p.k_ss + d) : 0.f;
      vt[j][d] = ok ? ldx<T>(V, (k0 + j) * p.v_ss + d) : 0.f;
    }
    __syncthreads();
    float s[FT];
    float mt = -INFINITY;
#pragma unroll
    for (int j = 0; j < FT; ++j) {
      float acc = 0.f;
#pragma unroll
      for (int d = 0; d < DP; ++d) acc = fmaf(qr[d], kt[j][d], acc);
      s[j] = k0 + j < Sk ? acc * p.scale : -INFINITY;
      mt = fmaxf(mt, s[j]);
    }
    const float mn = fmaxf(m, mt);
    const float alpha = m == -INFINITY ? 0.f : expf(m - mn);
    m = mn;
    l *= alpha;
#pragma unroll
    for (int d = 0; d < DP; ++d) o[d] *= alpha;
#pragma unroll
    for (int j = 0; j < FT; ++j) {
      const float pj = s[j] == -INFINITY ? 0.f : expf(s[j] - mn);
      l += pj;
#pragma unroll
      for (int d = 0; d < DP; ++d) o[d] = fmaf(pj, vt[j][d], o[d]);
    }
  }
  if (q >= Sq) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  reinterpret_cast<float*>(p.lse)[bh * Sq + q] = l > 0.f ? m + logf(l) : -INFINITY;
  S* out = reinterpret_cast<S*>(p.o) + ((b * Sq + q) * p.H + hh) * D;
  float* o32 = p.o32 ? reinterpret_cast<float*>(p.o32) + ((b * Sq + q) * p.H + hh) * D : nullptr;
#pragma unroll
  for (int d = 0; d < DP; ++d)
    if (d < D) {
      out[d] = T::from_f32(o[d] * inv);
      if (o32) o32[d] = o[d] * inv;
    }
}

template <typename T, int DP>
__global__ __launch_bounds__(64) void attn_dkdv_fma(hrt_attn_args p, int nkb) {
  using S = typename T::storage;
  constexpr int QT = 16;
  __shared__ float own_k[64][DP + 1], own_v[64][DP + 1];
  __shared__ float qt[QT][DP], dot[QT][DP], lt[QT], dl[QT];
  const int lane = threadIdx.x;
  const int64_t bh = blockIdx.x / nkb, kb = blockIdx.x % nkb;
  const int64_t b = bh / p.H, hh = bh % p.H;
  const int D = p.D, Sq = p.Sq, Sk = p.Sk;
  const S* Q = reinterpret_cast<const S*>(p.q) + b * p.q_sb + hh * p.q_sh;
  const S* K = reinterpret_cast<const S*>(p.k) + b * p.k_sb + hh * p.k_sh;
  const S* V = reinterpret_cast<const S*>(p.v) + b * p.v_sb + hh * p.v_sh;
  const S* dO = reinterpret_cast<const S*>(p.dout) + b * p.do_sb + hh * p.do_sh;
  const float* lse = reinterpret_cast<const float*>(p.lse) + bh * Sq;
  const float* delta = reinterpret_cast<const float*>(p.delta) + bh * Sq;
  const int64_t key = kb * 64 + lane;
  for (int d = 0; d < DP; ++d) {
    own_k[lane][d] = (key < Sk && d < D) ? ldx<T>(K, key * p.k_ss + d) : 0.f;
    own_v[lane][d] = (key < Sk && d < D) ? ldx<T>(V, key * p.v_ss + d) : 0.f;
  }
  float dk[DP], dv[DP];
#pragma unroll
  for (int d = 0; d < DP; ++d) dk[d] = dv[d] = 0.f;
  for (int64_t q0 = 0; q0 < Sq; q0 += QT) {
    __syncthreads();
    for (int e = lane; e < QT * DP; e += 64) {
      const int i = e / DP, d = e % DP;
      const bool ok = q0 + i < Sq && d < D;
      qt[i][d] = ok ? ldx<T>(Q, (q0 + i) * p.q_ss + d) : 0.f;
      dot[i][d] = ok ? ldx<T>(dO, (q0 + i) * p.do_ss + d) : 0.f;
    }
    if (lane < QT) {
      lt[lane] = q0 + lane < Sq ? lse[q0 + lane] : INFINITY;
      dl[lane] = q0 + lane < Sq ? delta[q0 + lane] : 0.f;
    }
    __syncthreads();
    for (int i = 0; i < QT; ++i) {
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int d = 0; d < DP; ++d) {
        s = fmaf(qt[i][d], own_k[lane][d], s);
        dp = fmaf(dot[i][d], own_v[lane][d], dp);
      }
      const float pv = expf(s * p.scale - lt[i]);
      const float ds = pv * (dp - dl[i]);
#pragma unroll
      for (int d = 0; d < DP; ++d) {
        dv[d] = fmaf(pv, dot[i][d], dv[d]);
        dk[d] = fmaf(ds, qt[i][d], dk[d]);
      }
    }
  }
  if (key >= Sk) return;
  S* dK = reinterpret_cast<S*>(p.dk) + grad_row(p, b, hh, key, Sk, p.k_sb, p.k_sh, p.k_ss);
  S* dV = reinterpret_cast<S*>(p.dv) + grad_row(p, b, hh, key, Sk, p.v_sb, p.v_sh, p.v_ss);
#pragma unroll
  for (int d = 0; d < DP; ++d)
    if (d < D) {
      dK[d] = T::from_f32(dk[d] * p.scale);
      dV[d] = T::from_f32(dv[d]);
    }
}

template <typename T, int DP>
__global__ __launch_bounds__(64) void attn_dq_fma(hrt_attn_args p, int nqb) {
  using S = typename T::storage;
  constexpr int KT = 16;
  __shared__ float own_q[64][DP + 1], own_do[64][DP + 1];
  __shared__ float kt[KT][DP], vt[KT][DP];
  const int lane = threadIdx.x;
  const int64_t bh = blockIdx.x / nqb, qb = blockIdx.x % nqb;
  const int64_t b = bh / p.H, hh = bh % p.H;
  const int D = p.D, Sq = p.Sq, Sk = p.Sk;
  const S* Q = reinterpret_cast<const S*>(p.q) + b * p.q_sb + hh * p.q_sh;
  const S* K = reinterpret_cast<const S*>(p.k) + b * p.k_sb + hh * p.k_sh;
  const S* V = reinterpret_cast<const S*>(p.v) + b * p.v_sb + hh * p.v_sh;
  const S* dO = reinterpret_cast<const S*>(p.dout) + b * p.do_sb + hh * p.do_sh;
  const int64_t q = qb * 64 + lane;
  const bool qv = q < Sq;
  for (int d = 0; d < DP; ++d) {
    own_q[lane][d] = (qv && d < D) ? ldx<T>(Q, q * p.q_ss + d) : 0.f;
    own_do[lane][d] = (qv && d < D) ? ldx<T>(dO, q * p.do_ss + d) : 0.f;
  }
  const float lse = qv ? reinterpret_cast<const float*>(p.lse)[bh * Sq + q] : INFINITY;
  const float dlt = qv ? reinterpret_cast<const float*>(p.delta)[bh * Sq + q] : 0.f;
  float dq[DP];
#pragma unroll
  for (int d = 0; d < DP; ++d) dq[d] = 0.f;
  for (int64_t k0 = 0; k0 < Sk; k0 += KT) {
    __syncthreads();
    for (int e = lane; e < KT * DP; e += 64) {
      const int j = e / DP, d = e % DP;
      const bool ok = k0 + j < Sk && d < D;
      kt[j][d] = ok ? ldx<T>(K, (k0 + j) * p.k_ss + d) : 0.f;
      vt[j][d] = ok ? ldx<T>(V, (k0 + j) * p.v_ss + d) : 0.f;
    }
    __syncthreads();
    for (int j = 0; j < KT; ++j) {
      if (k0 + j >= Sk) break;
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int d = 0; d < DP; ++d) {
        s = fmaf(own_q[lane][d], kt[j][d], s);
        dp = fmaf(own_do[lane][d], vt[j][d], dp);
      }
      const float pv = expf(s * p.scale - lse);
      const float ds = pv * (dp - dlt);
#pragma unroll
      for (int d = 0; d < DP; ++d) dq[d] = fmaf(ds, kt[j][d], dq[d]);
    }
  }
  if (!qv) return;
  S* dQ = reinterpret_cast<S*>(p.dq) + grad_row(p, b, hh, q, Sq, p.q_sb, p.q_sh, p.q_ss);
#pragma unroll
  for (int d = 0; d < DP; ++d)
    if (d < D) dQ[d] = T::from_f32(dq[d] * p.scale);
}

template <typename T, int W>
bool launch_fma(const void* pp, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_attn_args*>(pp);
  if (!attn_check(a, W == 0, W == 1, W == 2, sizeof(typename T::storage), ctx)) return false;
  const int nb = ((W == 1 ? a.Sk : a.Sq) + 63) / 64;
  const int64_t total = (int64_t)nb * a.B * a.H;
  if (total > 0x7fffffffLL) return ctx.fail("grid too large");
  const dim3 g((uint32_t)total);
  const int dch = (a.D + 31) / 32;
#define HK_ATTN_FMA(DPV)                                                                         \
  if (W == 0)                                                                                    \
    hipLaunchKernelGGL((attn_fwd_fma<T, DPV>), g, dim3(64), 0, ctx.stream, a, nb);               \
  else if (W == 1)                                                                               \
    hipLaunchKernelGGL((attn_dkdv_fma<T, DPV>), g, dim3(64), 0, ctx.stream, a, nb);              \
  else                                                                                           \
    hipLaunchKernelGGL((attn_dq_fma<T, DPV>), g, dim3(64), 0, ctx.stream, a, nb);
  switch (dch) {
    case 1: HK_ATTN_FMA(32) break;
    case 2: HK_ATTN_FMA(64) break;
    case 3: HK_ATTN_FMA(96) break;
    default: HK_ATTN_FMA(128) break;
  }
#undef HK_ATTN_FMA
  return hrt::launch_ok(hipGetLastError(), ctx, "attn_fma");
}

HRT_REGISTER("attn_fwd_fma_f32", hrt_attn_args, (launch_fma<F32, 0>));
HRT_REGISTER("attn_fwd_fma_bf16", hrt_attn_args, (launch_fma<BF16, 0>));
HRT_REGISTER("attn_fwd_fma_f16", hrt_attn_args, (launch_fma<F16, 0>));
HRT_REGISTER("attn_dkdv_fma_f32", hrt_attn_args, (launch_fma<F32, 1>));
HRT_REGISTER("attn_dkdv_fma_bf16", hrt_attn_args, (launch_fma<BF16, 1>));
HRT_REGISTER("attn_dkdv_fma_f16", hrt_attn_args, (launch_fma<F16, 1>));
HRT_REGISTER("attn_dq_fma_f32", hrt_attn_args, (launch_fma<F32, 2>));
HRT_REGISTER("attn_dq_fma_bf16", hrt_attn_args, (launch_fma<BF16, 2>));
HRT_REGISTER("attn_dq_fma_f16", hrt_attn_args, (launch_fma<F16, 2>));

}  // namespace
}  // namespace hk
