// Flash-attention backward on gfx950 matrix cores, plus the shared host checks of all attention kernels.
//
//   "attn_delta_{f32,bf16,f16}": delta = rowsum(O * dO) (vkrt/shaders/attn.comp.in:210-240), O read as the
//                                unrounded fp32 forward output when available (csrc/ops_attn.cpp:240-248).
//   "attn_dkdv_mfma_{bf16,f16}": per 64-key block, loop over query stages: S = Q K^T, dP = dO V^T,
//                                P = exp(scale S - lse), dS = P (dP - delta), dV += P^T dO, dK += dS^T Q.
//   "attn_dq_mfma_{bf16,f16}":   per 64-query block, loop over key stages: S^T, dP^T, dQ += dS K.
// Same decomposition and numerics as the reference's cooperative-matrix kernels
// (vkrt/shaders/attn_coop.comp.in:213-301): recomputation from lse (no N x N matrix in memory), P and dS
// rounded to the input dtype before their products, fp32 accumulation, dK and dQ scaled at the end.
// CDNA4 mapping (see attn_common.h for the lane layout):
//   * the operand that stays fixed for the workgroup (K, V for dK/dV; Q, dO for dQ) lives in registers
//     as MFMA B fragments; the streamed one is staged per stage through double-buffered LDS twice, as
//     rows and transposed (one set of global loads, an 8x8 register transpose for the second copy), so
//     every MFMA operand is a plain 128-bit or paired 64-bit LDS read;
//   * the first product is laid out so that each lane owns one key (dK/dV) or one query (dQ): P^T / dS^T
//     (resp. dS) go from accumulators directly into the next MFMA's A operand, no LDS round trip;
//   * 4 wavefronts = 2 row groups x 2 halves of every stage, summed through LDS at the end, so all four
//     SIMDs of a CU work on one 64-row block;
//   * workgroups of one head are placed on one XCD.
#include <cmath>

#include "../hrt/registry.h"
#include "attn_common.h"

namespace hk {

bool attn_check(const hrt_attn_args& a, bool fwd, bool dkdv, bool dq, uint64_t elem, hrt::LaunchCtx& ctx) {
  if (a.B < 1 || a.H < 1 || a.Sq < 1 || a.Sk < 1 || a.D < 1 || a.D > 128) return ctx.fail("unsupported attention shape");
  if (!(a.scale > 0.f) || !std::isfinite(a.scale)) return ctx.fail("attention scale must be positive and finite");
  if (a.q_sb < 0 || a.q_sh < 0 || a.q_ss < 0 || a.k_sb < 0 || a.k_sh < 0 || a.k_ss < 0 || a.v_sb < 0 || a.v_sh < 0 ||
      a.v_ss < 0 || a.do_sb < 0 || a.do_sh < 0 || a.do_ss < 0)
    return ctx.fail("negative stride");
  const int64_t qs[4] = {a.B, a.H, a.Sq, a.D}, ks[4] = {a.B, a.H, a.Sk, a.D};
  const int64_t qst[4] = {a.q_sb, a.q_sh, a.q_ss, 1}, kst[4] = {a.k_sb, a.k_sh, a.k_ss, 1}, vst[4] = {a.v_sb, a.v_sh, a.v_ss, 1};
  const int64_t dst[4] = {a.do_sb, a.do_sh, a.do_ss, 1};
  const uint64_t rows_q = (uint64_t)a.B * a.H * a.Sq, rows_k = (uint64_t)a.B * a.H * a.Sk;
  if (!ctx.check(a.q, hrt::span_bytes(4, qs, qst, elem), "q") || !ctx.check(a.k, hrt::span_bytes(4, ks, kst, elem), "k") ||
      !ctx.check(a.v, hrt::span_bytes(4, ks, vst, elem), "v") || !ctx.check(a.lse, rows_q * 4, "lse"))
    return false;
  if (fwd) {
    if (!ctx.check(a.o, rows_q * a.D * elem, "o") || (a.o32 && !ctx.check(a.o32, rows_q * a.D * 4, "o32"))) return false;
  }
  if (dkdv || dq) {
    if (!ctx.check(a.dout, hrt::span_bytes(4, qs, dst, elem), "dout") || !ctx.check(a.delta, rows_q * 4, "delta")) return false;
  }
  const bool like_input = (a.flags & HRT_ATTN_GRAD_LIKE_INPUT) != 0;
  const uint64_t dk_bytes = like_input ? hrt::span_bytes(4, ks, kst, elem) : rows_k * a.D * elem;
  const uint64_t dv_bytes = like_input ? hrt::span_bytes(4, ks, vst, elem) : rows_k * a.D * elem;
  const uint64_t dq_bytes = like_input ? hrt::span_bytes(4, qs, qst, elem) : rows_q * a.D * elem;
  if (dkdv && (!ctx.check(a.dk, dk_bytes, "dk") || !ctx.check(a.dv, dv_bytes, "dv"))) return false;
  if (dq && !ctx.check(a.dq, dq_bytes, "dq")) return false;
  return true;
}

bool attn_vec_ok(const hrt_attn_args& a, bool with_dout) {
  bool ok = a.D % 8 == 0 && a.q % 16 == 0 && a.k % 16 == 0 && a.v % 16 == 0;
  ok = ok && ((a.q_sb | a.q_sh | a.q_ss | a.k_sb | a.k_sh | a.k_ss | a.v_sb | a.v_sh | a.v_ss) % 8 == 0);
  if (with_dout) ok = ok && a.dout % 16 == 0 && ((a.do_sb | a.do_sh | a.do_ss) % 8 == 0);
  return ok;
}

namespace {

// ---- delta ------------------------------------------------------------------------------------------------
template <typename T, bool OF32>
__global__ __launch_bounds__(256) void attn_delta(hrt_attn_args p) {
  const int sub = threadIdx.x & 15;
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);  // = bh * Sq + q
  const int64_t rows = (int64_t)p.B * p.H * p.Sq;
  float acc = 0.f;
  if (row < rows) {
    const int64_t bh = row / p.Sq, q = row % p.Sq, b = bh / p.H, hh = bh % p.H;
    const int64_t oo = ((b * p.Sq + q) * p.H + hh) * p.D;
    const typename T::storage* dO = reinterpret_cast<const typename T::storage*>(p.dout) + b * p.do_sb + hh * p.do_sh + q * p.do_ss;
    for (int d = sub; d < p.D; d += 16) {
      float ov;
      if (OF32)
        ov = reinterpret_cast<const float*>(p.o)[oo + d];
      else
        ov = T::to_f32(reinterpret_cast<const typename T::storage*>(p.o)[oo + d]);
      acc += ov * T::to_f32(dO[d]);
    }
  }
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 16);
  if (row < rows && sub == 0) reinterpret_cast<float*>(p.delta)[row] = acc;
}

template <typename T>
bool launch_delta(const void* pp, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_attn_args*>(pp);
  if (a.B < 1 || a.H < 1 || a.Sq < 1 || a.D < 1 || a.D > 128) return ctx.fail("unsupported attention shape");
  const bool of32 = (a.flags & HRT_ATTN_O_F32) != 0;
  const uint64_t rows = (uint64_t)a.B * a.H * a.Sq;
  const int64_t qs[4] = {a.B, a.H, a.Sq, a.D}, dst[4] = {a.do_sb, a.do_sh, a.do_ss, 1};
  if (a.do_sb < 0 || a.do_sh < 0 || a.do_ss < 0) return ctx.fail("negative stride");
  if (!ctx.check(a.o, rows * a.D * (of32 ? 4 : sizeof(typename T::storage)), "o") ||
      !ctx.check(a.dout, hrt::span_bytes(4, qs, dst, sizeof(typename T::storage)), "dout") ||
      !ctx.check(a.delta, rows * 4, "delta"))
    return false;
  const dim3 g((uint32_t)cdiv((int64_t)rows, 16));
  if (of32)
    hipLaunchKernelGGL((attn_delta<T, true>), g, dim3(256), 0, ctx.stream, a);
  else
    hipLaunchKernelGGL((attn_delta<T, false>), g, dim3(256), 0, ctx.stream, a);
  return hrt::launch_ok(hipGetLastError(), ctx, "attn_delta");
}

HRT_REGISTER("attn_delta_f32", hrt_attn_args, launch_delta<F32>);
HRT_REGISTER("attn_delta_bf16", hrt_attn_args, launch_delta<BF16>);
HRT_REGISTER("attn_delta_f16", hrt_attn_args, launch_delta<F16>);

constexpr int ST = 64;  // rows per LDS stage

// ---- dK / dV -----------------------------------------------------------------------------------------------
template <typename T, int DCH, int LM>
__global__ __launch_bounds__(256) void attn_dkdv_mfma(hrt_attn_args p, int nkb) {
  constexpr int DP = DCH * 32;
  constexpr int NCH = DP / 8;
  constexpr int RLD = DP + 8;  // [q][d] rows (chunks swizzled)
  constexpr int TLD = ST + 8;  // [d][q] rows
  constexpr int STAGE = 2 * ST * RLD + 2 * DP * TLD + 2 * ST * 2;  // Q, dO, Q^T, dO^T (halves), lse2, delta (floats)
  constexpr int RB = ST / 8;
  constexpr int NB = RB * NCH;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * STAGE];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kg = wave & 1, qh = wave >> 1;
  const int rl = lane & 31, hl = lane >> 5;
  const int64_t total = (int64_t)nkb * p.B * p.H;
  int64_t bh, kb;
  xcd_map(blockIdx.x, total, nkb, bh, kb);
  const int64_t b = bh / p.H, hh = bh % p.H;
  const int D = p.D, Sq = p.Sq, Sk = p.Sk;
  using S = uint16_t;
  const HK_G S* Q = gcptr<S>(p.q) + b * p.q_sb + hh * p.q_sh;
  const HK_G S* K = gcptr<S>(p.k) + b * p.k_sb + hh * p.k_sh;
  const HK_G S* V = gcptr<S>(p.v) + b * p.v_sb + hh * p.v_sh;
  const HK_G S* dO = gcptr<S>(p.dout) + b * p.do_sb + hh * p.do_sh;
  const HK_G float* lse = gcptr<float>(p.lse) + bh * Sq;
  const HK_G float* delta = gcptr<float>(p.delta) + bh * Sq;

  // this lane's key: K and V as B fragments (16 d each)
  const int64_t key = kb * 64 + kg * 32 + rl;
  u32x4 kf[2 * DCH], vf[2 * DCH];
#pragma unroll
  for (int ks = 0; ks < 2 * DCH; ++ks) {
    kf[ks] = key < Sk ? load_row8<LM != LD_GATHER>(K + key * p.k_ss, ks * 16 + 8 * hl, D) : u32x4{0, 0, 0, 0};
    vf[ks] = key < Sk ? load_row8<LM != LD_GATHER>(V + key * p.v_ss, ks * 16 + 8 * hl, D) : u32x4{0, 0, 0, 0};
  }

  Block8 blk;
  float sv = 0.f;
  auto load_stage = [&](int64_t q0) {
    const bool full = q0 + ST <= Sq;
    const int bi = threadIdx.x;
    if (bi < 2 * NB) {
      const int t = bi < NB ? bi : bi - NB;
      const int rb = t % RB, dc = t / RB;
      if (bi < NB)
        blk.template load<LM>(Q, p.q_ss, q0 + rb * 8, Sq, dc * 8, D, full);
      else
        blk.template load<LM>(dO, p.do_ss, q0 + rb * 8, Sq, dc * 8, D, full);
    }
    if (threadIdx.x < 2 * ST) {
      const int64_t qq = q0 + (threadIdx.x & (ST - 1));
      if (threadIdx.x < ST)
        sv = qq < Sq ? lse[qq] * kLog2e : INFINITY;
      else
        sv = qq < Sq ? delta[qq] : 0.f;
    }
  };
  auto store_stage = [&](uint16_t* st) {
    const int bi = threadIdx.x;
    if (bi < 2 * NB) {
      const int t = bi < NB ? bi : bi - NB;
      const int rb = t % RB, dc = t / RB;
      uint16_t* rows = st + (bi < NB ? 0 : ST * RLD);
      uint16_t* cols = st + 2 * ST * RLD + (bi < NB ? 0 : DP * TLD);
      blk.template store_rows<NCH>(rows, RLD, rb * 8, dc * 8);
      blk.store_cols(cols, TLD, rb * 8, dc * 8);
    }
    if (threadIdx.x < 2 * ST) reinterpret_cast<float*>(st + 2 * ST * RLD + 2 * DP * TLD)[threadIdx.x] = sv;
  };

  f32x16 dk[DCH], dv[DCH];
#pragma unroll
  for (int n = 0; n < DCH; ++n) dk[n] = dv[n] = zero16();
  const float sl2 = p.scale * kLog2e;
  const int nst = (Sq + ST - 1) / ST;
  load_stage(0);
  store_stage(lds);
  __syncthreads();
  const int row = qh * 32 + rl;  // the query row this lane reads as an A operand
  for (int st = 0; st < nst; ++st) {
    const bool more = st + 1 < nst;
    if (more) load_stage((int64_t)(st + 1) * ST);
    const uint16_t* base = lds + (st & 1) * STAGE;
    const uint16_t* Ql = base;
    const uint16_t* dOl = base + ST * RLD;
    const uint16_t* QTl = base + 2 * ST * RLD;
    const uint16_t* dOTl = QTl + DP * TLD;
    const float* lse2 = reinterpret_cast<const float*>(dOTl + DP * TLD);
    const float* dlt = lse2 + ST;

    f32x16 s = zero16(), dp = zero16();
#pragma unroll
    for (int ks = 0; ks < 2 * DCH; ++ks) {
      const int off = row * RLD + Block8::swz_col<NCH>(row, ks * 16 + 8 * hl);
      s = Mfma32<T>::mac(*reinterpret_cast<const u32x4*>(Ql + off), kf[ks], s);
      dp = Mfma32<T>::mac(*reinterpret_cast<const u32x4*>(dOl + off), vf[ks], dp);
    }
    // element 4j+r: query qh*32 + 8j + 4h + r of the stage, key = this lane's key
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q4 = qh * 32 + 8 * j + 4 * hl;
      const f32x4 l4 = *reinterpret_cast<const f32x4*>(lse2 + q4);
      const f32x4 d4 = *reinterpret_cast<const f32x4*>(dlt + q4);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pv = __builtin_amdgcn_exp2f(fmaf(s[4 * j + r], sl2, -l4[r]));  // lse2 = +inf: padded query
        s[4 * j + r] = pv;
        dp[4 * j + r] = pv * (dp[4 * j + r] - d4[r]);
      }
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const u32x4 pa = pack_slots<T>(s, 2 * c, 2 * c + 1);
      const u32x4 da = pack_slots<T>(dp, 2 * c, 2 * c + 1);
#pragma unroll
      for (int n = 0; n < DCH; ++n) {
        const int off = (n * 32 + rl) * TLD + qh * 32 + c * 16 + 4 * hl;
        dv[n] = Mfma32<T>::mac(pa, lds_pair64(dOTl + off), dv[n]);
        dk[n] = Mfma32<T>::mac(da, lds_pair64(QTl + off), dk[n]);
      }
    }
    if (more) store_stage(lds + ((st + 1) & 1) * STAGE);
    __syncthreads();
  }

  // sum the two query halves: waves qh = 1 hand their accumulators to qh = 0
  float* xch = reinterpret_cast<float*>(lds) + (kg * 64 + lane) * (32 * DCH);
  if (qh == 1) {
#pragma unroll
    for (int n = 0; n < DCH; ++n)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        xch[n * 32 + e] = dk[n][e];
        xch[n * 32 + 16 + e] = dv[n][e];
      }
  }
  __syncthreads();
  if (qh == 1) return;
  HK_G typename T::storage* dK = gptr<typename T::storage>(p.dk);
  HK_G typename T::storage* dV = gptr<typename T::storage>(p.dv);
  // accumulator element 4j+r: key kg*32 + 8j + 4h + r of the block, d = n*32 + lane%32
#pragma unroll
  for (int n = 0; n < DCH; ++n) {
    const int d = n * 32 + rl;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int64_t kk = kb * 64 + kg * 32 + 8 * (e >> 2) + 4 * hl + (e & 3);
      if (kk < Sk && d < D) {
        dK[grad_row(p, b, hh, kk, Sk, p.k_sb, p.k_sh, p.k_ss) + d] = T::from_f32((dk[n][e] + xch[n * 32 + e]) * p.scale);
        dV[grad_row(p, b, hh, kk, Sk, p.v_sb, p.v_sh, p.v_ss) + d] = T::from_f32(dv[n][e] + xch[n * 32 + 16 + e]);
      }
    }
  }
}

// ---- dQ ------------------------------------------------------------------------------------------------------
template <typename T, int DCH, int LM>
__global__ __launch_bounds__(256) void attn_dq_mfma(hrt_attn_args p, int nqb) {
  constexpr int DP = DCH * 32;
  constexpr int NCH = DP / 8;
  constexpr int RLD = DP + 8;
  constexpr int TLD = ST + 8;
  constexpr int STAGE = 2 * ST * RLD + DP * TLD;  // K, V rows (swizzled), K^T
  constexpr int RB = ST / 8;
  constexpr int NB = RB * NCH;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * STAGE];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int qg = wave & 1, kh = wave >> 1;
  const int rl = lane & 31, hl = lane >> 5;
  const int64_t total = (int64_t)nqb * p.B * p.H;
  int64_t bh, qb;
  xcd_map(blockIdx.x, total, nqb, bh, qb);
  const int64_t b = bh / p.H, hh = bh % p.H;
  const int D = p.D, Sq = p.Sq, Sk = p.Sk;
  using S = uint16_t;
  const HK_G S* Q = gcptr<S>(p.q) + b * p.q_sb + hh * p.q_sh;
  const HK_G S* K = gcptr<S>(p.k) + b * p.k_sb + hh * p.k_sh;
  const HK_G S* V = gcptr<S>(p.v) + b * p.v_sb + hh * p.v_sh;
  const HK_G S* dO = gcptr<S>(p.dout) + b * p.do_sb + hh * p.do_sh;

  const int64_t q = qb * 64 + qg * 32 + rl;
  const bool qv = q < Sq;
  u32x4 qf[2 * DCH], df[2 * DCH];
#pragma unroll
  for (int ks = 0; ks < 2 * DCH; ++ks) {
    qf[ks] = qv ? load_row8<LM != LD_GATHER>(Q + q * p.q_ss, ks * 16 + 8 * hl, D) : u32x4{0, 0, 0, 0};
    df[ks] = qv ? load_row8<LM != LD_GATHER>(dO + q * p.do_ss, ks * 16 + 8 * hl, D) : u32x4{0, 0, 0, 0};
  }
  const float nlse2 = qv ? -gcptr<float>(p.lse)[bh * Sq + q] * kLog2e : -INFINITY;
  const float dlt = qv ? gcptr<float>(p.delta)[bh * Sq + q] : 0.f;

  Block8 blk;
  auto load_stage = [&](int64_t k0) {
    const bool full = k0 + ST <= Sk;
    const int bi = threadIdx.x;
    if (bi < 2 * NB) {
      const int t = bi < NB ? bi : bi - NB;
      const int rb = t % RB, dc = t / RB;
      if (bi < NB)
        blk.template load<LM>(K, p.k_ss, k0 + rb * 8, Sk, dc * 8, D, full);
      else
        blk.template load<LM>(V, p.v_ss, k0 + rb * 8, Sk, dc * 8, D, full);
    }
  };
  auto store_stage = [&](uint16_t* st) {
    const int bi = threadIdx.x;
    if (bi < 2 * NB) {
      const int t = bi < NB ? bi : bi - NB;
      const int rb = t % RB, dc = t / RB;
      if (bi < NB) {
        blk.template store_rows<NCH>(st, RLD, rb * 8, dc * 8);
        blk.store_cols(st + 2 * ST * RLD, TLD, rb * 8, dc * 8);
      } else {
        blk.template store_rows<NCH>(st + ST * RLD, RLD, rb * 8, dc * 8);
      }
    }
  };

  f32x16 acc[DCH];
#pragma unroll
  for (int n = 0; n < DCH; ++n) acc[n] = zero16();
  const float sl2 = p.scale * kLog2e;
  const int nst = (Sk + ST - 1) / ST;
  load_stage(0);
  store_stage(lds);
  __syncthreads();
  const int row = kh * 32 + rl;  // the key row this lane reads as an A operand
  for (int st = 0; st < nst; ++st) {
    const bool more = st + 1 < nst;
    if (more) load_stage((int64_t)(st + 1) * ST);
    const uint16_t* Kl = lds + (st & 1) * STAGE;
    const uint16_t* Vl = Kl + ST * RLD;
    const uint16_t* KTl = Kl + 2 * ST * RLD;
    f32x16 s = zero16(), dp = zero16();
#pragma unroll
    for (int ks = 0; ks < 2 * DCH; ++ks) {
      const int off = row * RLD + Block8::swz_col<NCH>(row, ks * 16 + 8 * hl);
      s = Mfma32<T>::mac(*reinterpret_cast<const u32x4*>(Kl + off), qf[ks], s);
      dp = Mfma32<T>::mac(*reinterpret_cast<const u32x4*>(Vl + off), df[ks], dp);
    }
    // element 4j+r: key kh*32 + 8j + 4h + r of the stage, query = this lane's query
    if (st * ST + ST > Sk) {
      const int key0 = st * ST + kh * 32 + 4 * hl;
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (key0 + 8 * (e >> 2) + (e & 3) >= Sk) s[e] = -INFINITY;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float pv = __builtin_amdgcn_exp2f(fmaf(s[e], sl2, nlse2));
      dp[e] = pv * (dp[e] - dlt);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const u32x4 da = pack_slots<T>(dp, 2 * c, 2 * c + 1);
#pragma unroll
      for (int n = 0; n < DCH; ++n)
        acc[n] = Mfma32<T>::mac(da, lds_pair64(KTl + (n * 32 + rl) * TLD + kh * 32 + c * 16 + 4 * hl), acc[n]);
    }
    if (more) store_stage(lds + ((st + 1) & 1) * STAGE);
    __syncthreads();
  }

  float* xch = reinterpret_cast<float*>(lds) + (qg * 64 + lane) * (16 * DCH);
  if (kh == 1) {
#pragma unroll
    for (int n = 0; n < DCH; ++n)
#pragma unroll
      for (int e = 0; e < 16; ++e) xch[n * 16 + e] = acc[n][e];
  }
  __syncthreads();
  if (kh == 1) return;
  HK_G typename T::storage* dQ = gptr<typename T::storage>(p.dq);
  // accumulator element 4j+r: query qg*32 + 8j + 4h + r of the block, d = n*32 + lane%32
#pragma unroll
  for (int n = 0; n < DCH; ++n) {
    const int d = n * 32 + rl;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int64_t qq = qb * 64 + qg * 32 + 8 * (e >> 2) + 4 * hl + (e & 3);
      if (qq < Sq && d < D)
        dQ[grad_row(p, b, hh, qq, Sq, p.q_sb, p.q_sh, p.q_ss) + d] = T::from_f32((acc[n][e] + xch[n * 16 + e]) * p.scale);
    }
  }
}

// ---- dQ fast path: D = 64 or 128, 16-byte aligned rows ------------------------------------------------------
//
// The forward kernel's structure applied to dQ: K and V stages (128 keys) go global -> LDS directly and
// double-buffered; 8 wavefronts, wave (g = w & 1, k = w >> 1) handles query group g (32 rows of the 64-row
// block, this lane's query held as Q^T / dO^T B fragments in registers) against keys 32 k .. +31 of every
// stage.  Per stage: S^T = K Q^T, dP^T = V dO^T (A operands: K / V rows from LDS), P^T = exp2(S^T sl2 -
// lse log2e), dS^T = P^T (dP^T - delta), dQ^T += K^T dS^T with K^T read by ds_read_b64_tr_b16 and dS^T
// packed (rounded to the input dtype, attn_coop.comp.in:283-284) straight from the accumulators.  The four
// key quarters are summed through LDS at the end and dQ is written as coalesced 32-element row pieces.
// With WITH_DELTA the kernel first computes delta = rowsum(O dO) for its rows (one quarter of d per key
// quarter, summed through LDS, vkrt/shaders/attn.comp.in:210-240) and stores it for the dK/dV kernel.
constexpr int KST2 = 128;  // keys per LDS stage

template <typename T, int DCH, bool OF32, bool WITH_DELTA>
__global__ __launch_bounds__(512) void attn_dq_dma(hrt_attn_args p, int nqb) {
  constexpr int NW = 8;
  constexpr int NCH = DCH * 4;
  constexpr int ROWB = NCH * 16;
  constexpr int TILE = KST2 * ROWB;
  constexpr int PIECE = 3 * 16 * 64;
  constexpr int PPT = TILE / (PIECE * 4);
  constexpr int KSQ = DCH / 2;  // 16-wide d chunks per quarter of d
  static_assert(PPT >= 1 && PPT * 4 >= 2 * DCH && 32 * 36 <= PIECE, "merge layout");
  __shared__ __attribute__((aligned(1024))) uint8_t k0_raw[TILE], k1_raw[TILE], v0_raw[TILE], v1_raw[TILE];
  __shared__ float xdel[4][64];
  HK_L uint8_t* const K0 = (HK_L uint8_t*)k0_raw;
  HK_L uint8_t* const K1 = (HK_L uint8_t*)k1_raw;
  HK_L uint8_t* const V0 = (HK_L uint8_t*)v0_raw;
  HK_L uint8_t* const V1 = (HK_L uint8_t*)v1_raw;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = wave & 1, kq = wave >> 1;
  const int ql = lane & 31, hl = lane >> 5;
  uint32_t bh32, qb32;
  xcd_map32(blockIdx.x, (uint32_t)nqb * p.B * p.H, nqb, bh32, qb32);
  const int64_t bh = bh32, qb = qb32, b = bh32 / (uint32_t)p.H, hh = bh32 % (uint32_t)p.H;
  const int Sq = p.Sq, Sk = p.Sk;
  const uint32_t kss = (uint32_t)(p.k_ss * 2), vss = (uint32_t)(p.v_ss * 2);
  const HK_G uint8_t* Kb = reinterpret_cast<const HK_G uint8_t*>(gcptr<uint16_t>(p.k) + b * p.k_sb + hh * p.k_sh);
  const HK_G uint8_t* Vb = reinterpret_cast<const HK_G uint8_t*>(gcptr<uint16_t>(p.v) + b * p.v_sb + hh * p.v_sh);
  const int nst = (Sk + KST2 - 1) / KST2;

  const int j0 = wave * (KST2 * NCH / 64 / NW);
  const DmaLanes klo = dma_lane_offsets<NCH>(kss, lane, j0), vlo = dma_lane_offsets<NCH>(vss, lane, j0);
  // The block's 64 rows of Q and dO go to the stage-1 buffers (free until stage 0 copies into them), copied
  // once for the four wavefronts that share them, ahead of K(0), V(0); rows past Sq hold copies of the last
  // row (P = 0 for them: lse = -inf below)
  const uint32_t qss = (uint32_t)(p.q_ss * 2), oss = (uint32_t)(p.do_ss * 2);
  const int qvalid = (int)(Sq - qb * 64);
  {
    const int jq = wave * (64 * NCH / 64 / NW);
    const HK_G uint8_t* Qblk = reinterpret_cast<const HK_G uint8_t*>(gcptr<uint16_t>(p.q) + b * p.q_sb + hh * p.q_sh) +
                               qb * 64 * (int64_t)qss;
    const HK_G uint8_t* Oblk = reinterpret_cast<const HK_G uint8_t*>(gcptr<uint16_t>(p.dout) + b * p.do_sb + hh * p.do_sh) +
                               qb * 64 * (int64_t)oss;
    dma_tile<NCH, 64, NW>(Qblk, qss, qvalid, K1, wave, lane, dma_lane_offsets<NCH>(qss, lane, jq));
    dma_tile<NCH, 64, NW>(Oblk, oss, qvalid, V1, wave, lane, dma_lane_offsets<NCH>(oss, lane, jq));
  }

  const int64_t q = qb * 64 + g * 32 + ql;
  const bool qv = q < Sq;
  // lse (used after the first barrier: a use here would wait for every copy issued so far)
  const float lse_raw = gcptr<float>(p.lse)[bh * Sq + (qv ? q : 0)];
  // delta: this wave's quarter of d of its row's o (fp32 when OF32), loaded now; dO comes from LDS below
  constexpr int OV = OF32 ? 2 : 1;  // 16-byte pieces of o per 8 elements
  u32x4 oraw[WITH_DELTA ? KSQ * OV : 1];
  if constexpr (WITH_DELTA) {
    const int64_t orow = ((b * Sq + (qv ? q : 0)) * p.H + hh) * p.D;
#pragma unroll
    for (int i = 0; i < KSQ; ++i) {
      const int d0 = (kq * KSQ + i) * 16 + 8 * hl;
      if constexpr (OF32) {
        oraw[2 * i] = *reinterpret_cast<const HK_G u32x4*>(gcptr<float>(p.o) + orow + d0);
        oraw[2 * i + 1] = *reinterpret_cast<const HK_G u32x4*>(gcptr<float>(p.o) + orow + d0 + 4);
      } else {
        oraw[i] = *reinterpret_cast<const HK_G u32x4*>(gcptr<uint16_t>(p.o) + orow + d0);
      }
    }
  }
  float dlt = 0.f;
  if constexpr (!WITH_DELTA) dlt = gcptr<float>(p.delta)[bh * Sq + (qv ? q : 0)];
  issue_order_fence();  // the first barrier counts on K(0), V(0) being the last copies issued
  dma_tile<NCH, KST2, NW>(Kb, kss, Sk, K0, wave, lane, klo);
  dma_tile<NCH, KST2, NW>(Vb, vss, Sk, V0, wave, lane, vlo);

  int koff[2 * DCH], voff[DCH][2];
#pragma unroll
  for (int ks = 0; ks < 2 * DCH; ++ks) koff[ks] = tile_off<NCH>(kq * 32 + ql, 2 * ks + hl);
#pragma unroll
  for (int n = 0; n < DCH; ++n)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int row = kq * 32 + 8 * t + 4 * hl + ((lane & 15) >> 2);
      const int c = 4 * n + 2 * ((lane >> 4) & 1) + ((lane >> 1) & 1);
      voff[n][t] = tile_off<NCH>(row, c) + (lane & 1) * 8;
    }
  f32x16 acc[DCH];
#pragma unroll
  for (int n = 0; n < DCH; ++n) acc[n] = zero16();
  const float sl2 = p.scale * kLog2e;

  // Q and dO rows (and o) landed; K(0), V(0), issued last, may still be in flight
  barrier_keep_vm<2 * (KST2 * NCH / 64 / NW)>();
  const float nlse2 = qv ? -lse_raw * kLog2e : -INFINITY;  // P = 0 for padded rows
  if constexpr (!WITH_DELTA) dlt = qv ? dlt : 0.f;
  u32x4 qf[2 * DCH], df[2 * DCH];
#pragma unroll
  for (int ks = 0; ks < 2 * DCH; ++ks) {
    qf[ks] = *reinterpret_cast<const HK_L u32x4*>(K1 + tile_off<NCH>(g * 32 + ql, 2 * ks + hl));
    df[ks] = *reinterpret_cast<const HK_L u32x4*>(V1 + tile_off<NCH>(g * 32 + ql, 2 * ks + hl));
  }
  if constexpr (WITH_DELTA) {
    float part = 0.f;
#pragma unroll
    for (int ks = 0; ks < 2 * DCH; ++ks) {
      // d = 16 ks + 8 hl .. +7 is this wave's quarter when ks / KSQ == kq (constant indices: a runtime
      // index would move df to scratch memory)
      if (ks / KSQ != kq) continue;
      const int i = ks % KSQ;
      const u32x4 dv = df[ks];
      float ov[8];
      if constexpr (OF32) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          // __uint_as_float: __builtin_bit_cast of a vector element miscompiles here (wrong element read)
          ov[w] = __uint_as_float(oraw[2 * i][w]);
          ov[4 + w] = __uint_as_float(oraw[2 * i + 1][w]);
        }
      } else {
#pragma unroll
        for (int w = 0; w < 4; ++w) ov[2 * w] = lo16<T>(oraw[i][w]), ov[2 * w + 1] = hi16<T>(oraw[i][w]);
      }
#pragma unroll
      for (int w = 0; w < 4; ++w) part += ov[2 * w] * lo16<T>(dv[w]) + ov[2 * w + 1] * hi16<T>(dv[w]);
    }
    part = halfswap_sum(qv ? part : 0.f);
    if (hl == 0) xdel[kq][g * 32 + ql] = part;
  }
  __syncthreads();  // stage 0 in LDS; partial deltas published; Q / dO read out of the stage-1 buffers
  if constexpr (WITH_DELTA) {
    dlt = xdel[0][g * 32 + ql] + xdel[1][g * 32 + ql] + xdel[2][g * 32 + ql] + xdel[3][g * 32 + ql];
    if (kq == 0 && hl == 0 && qv) gptr<float>(p.delta)[bh * Sq + q] = dlt;
  }

  // COPY: stage st + 1 is copied into the other buffers while stage st computes, the copies placed between
  // the MFMAs of S^T / dP^T (the buffers' previous readers passed the last barrier); the last, ragged stage
  // is the window ending at Sk (stage_origin), its keys before the stage masked.  The last stage runs
  // without copies: the tiles are reused as scratch by the merge below, and a copy landing there late has
  // been seen to corrupt LDS written after the closing barrier.
  constexpr int IPW = KST2 * NCH / 64 / NW;
  auto stage = [&](auto bc, auto cc, int st) {
    constexpr int BUF = decltype(bc)::value;
    constexpr bool COPY = decltype(cc)::value;
    const int64_t key0 = (int64_t)st * KST2;
    // buffer resources over the next stage's first rows (scalar row offsets, no 64-bit address arithmetic)
    const __amdgpu_buffer_rsrc_t krs = dma_rsrc(Kb + stage_origin<KST2>(st + 1, nst, Sk) * kss);
    const __amdgpu_buffer_rsrc_t vrs = dma_rsrc(Vb + stage_origin<KST2>(st + 1, nst, Sk) * vss);
    const HK_L uint8_t* Kt = BUF ? K1 : K0;
    const HK_L uint8_t* Vt = BUF ? V1 : V0;
    // S^T, dP^T of d step ks; their A operands (K, V rows) are read RA1 steps ahead into a ring, each step
    // fenced by sched_barrier (the compiler's own order read each operand right before its MFMA)
    f32x16 s = zero16(), dp = zero16();
    constexpr int RA1 = 2;
    u32x4 kr[RA1 + 1], vr[RA1 + 1];
    auto rd1 = [&](int ks) {
      kr[ks % (RA1 + 1)] = *reinterpret_cast<const HK_L u32x4*>(Kt + koff[ks]);
      vr[ks % (RA1 + 1)] = *reinterpret_cast<const HK_L u32x4*>(Vt + koff[ks]);
    };
#pragma unroll
    for (int ks = 0; ks < RA1; ++ks) rd1(ks);
#pragma unroll
    for (int ks = 0; ks < 2 * DCH; ++ks) {
      __builtin_amdgcn_sched_barrier(0);
      if (ks + RA1 < 2 * DCH) rd1(ks + RA1);
      s = Mfma32<T>::mac(kr[ks % (RA1 + 1)], qf[ks], s);
      dp = Mfma32<T>::mac(vr[ks % (RA1 + 1)], df[ks], dp);
      if constexpr (COPY) {
        if (ks < IPW) dma_tile_part_rs<NCH, KST2, NW>(krs, kss, BUF ? K0 : K1, wave, klo, ks);
        else if (ks < 2 * IPW) dma_tile_part_rs<NCH, KST2, NW>(vrs, vss, BUF ? V0 : V1, wave, vlo, ks - IPW);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // element 4j+r: tile row kq*32 + 8j + 4h + r of the stage, query = this lane's
    if (key0 + KST2 > Sk) {
      const int64_t kbase = (nst > 1 ? stage_origin<KST2>(st, nst, Sk) : 0) + kq * 32 + 4 * hl;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t key = kbase + 8 * (e >> 2) + (e & 3);
        if (key < key0 || key >= Sk) s[e] = -INFINITY;
      }
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float pv = __builtin_amdgcn_exp2f(fmaf(s[e], sl2, nlse2));
      dp[e] = pv * (dp[e] - dlt);
    }
    const u32x4 d0 = pack_slots<T>(dp, 0, 1), d1 = pack_slots<T>(dp, 2, 3);
    // dQ^T += K^T dS^T, product i = (n, kc) = (i >> 1, i & 1); its A operand (two column reads of K) is read
    // RA products ahead into a ring
    constexpr int NP = 2 * DCH, RA = 2;
    u32x4 ring[RA + 1];
    auto rd = [&](int i) {
      const int n = i >> 1, kc = i & 1;
      const u32x2 lo = lds_tr4(Kt + voff[n][0] + kc * 16 * ROWB), hi = lds_tr4(Kt + voff[n][1] + kc * 16 * ROWB);
      ring[i % (RA + 1)] = u32x4{lo.x, lo.y, hi.x, hi.y};
    };
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < RA; ++i) rd(i);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      __builtin_amdgcn_sched_barrier(0);
      if (i + RA < NP) rd(i + RA);
      acc[i >> 1] = Mfma32<T>::mac(ring[i % (RA + 1)], (i & 1) ? d1 : d0, acc[i >> 1]);
    }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
  };
  // Pairs of copying stages, the last one or two peeled into straight-line code (the loop body holds one
  // variant per buffer, which keeps the D = 128 kernel within its 256 registers).
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  int st = 0;
  for (; st + 2 < nst; st += 2) {
    stage(B0(), std::true_type(), st);
    stage(B1(), std::true_type(), st + 1);
  }
  if (st + 1 < nst) {
    stage(B0(), std::true_type(), st);
    stage(B1(), std::false_type(), st + 1);
  } else {
    stage(B0(), std::false_type(), st);
  }

  // ---- sum the four key quarters: piece (g, n) = d block n of group g, finished by wavefront (g, k = n)
  auto tile_f = [&](int t) -> float* {
    return reinterpret_cast<float*>(t == 0 ? k0_raw : t == 1 ? k1_raw : t == 2 ? v0_raw : v1_raw);
  };
#pragma unroll
  for (int n = 0; n < DCH; ++n) {
    if (n == kq) continue;
    const int pc = g * DCH + n;
    // [4][64 lanes] 16-byte pieces: acc[n][4 c .. 4 c + 3] of lane l at 4 c * 64 + 4 l (conflict-free)
    f32x4* dst = reinterpret_cast<f32x4*>(tile_f(pc / PPT) + (pc % PPT) * PIECE + ((kq - n - 1) & 3) * 16 * 64) + lane;
#pragma unroll
    for (int c = 0; c < 4; ++c) dst[c * 64] = f32x4{acc[n][4 * c], acc[n][4 * c + 1], acc[n][4 * c + 2], acc[n][4 * c + 3]};
  }
  __syncthreads();
  auto finish = [&](auto nc) {
    constexpr int N = decltype(nc)::value;
    const int pc = g * DCH + N;
    float* const area = tile_f(pc / PPT) + (pc % PPT) * PIECE;
    f32x16 r = acc[N];
#pragma unroll
    for (int sl = 0; sl < 3; ++sl)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const f32x4 x = reinterpret_cast<const f32x4*>(area + sl * 16 * 64)[c * 64 + lane];
#pragma unroll
        for (int w = 0; w < 4; ++w) r[4 * c + w] += x[w];
      }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<f32x4*>(area + ql * 36 + 8 * j + 4 * hl) =
          f32x4{r[4 * j] * p.scale, r[4 * j + 1] * p.scale, r[4 * j + 2] * p.scale, r[4 * j + 3] * p.scale};
    const int c4 = (lane & 7) * 4;
#pragma unroll
    for (int ps = 0; ps < 4; ++ps) {
      const int qq = ps * 8 + (lane >> 3);
      const f32x4 v = *reinterpret_cast<const f32x4*>(area + qq * 36 + c4);
      const int64_t qrow = qb * 64 + g * 32 + qq;
      const float v4[4] = {v[0], v[1], v[2], v[3]};
      if (qrow < Sq)
        *reinterpret_cast<HK_G u32x2*>(gptr<uint16_t>(p.dq) + grad_row(p, b, hh, qrow, Sq, p.q_sb, p.q_sh, p.q_ss) + N * 32 + c4) =
            pack4<T>(v4);
    }
  };
  switch (kq) {
    case 0: finish(std::integral_constant<int, 0>()); break;
    case 1: finish(std::integral_constant<int, 1>()); break;
    case 2: if constexpr (DCH > 2) finish(std::integral_constant<int, 2 % DCH>()); break;
    default: if constexpr (DCH > 3) finish(std::integral_constant<int, 3 % DCH>()); break;
  }
}

constexpr int QST = 128;  // queries per LDS stage of the dK / dV kernel

// ---- dK / dV fast path: D = 64 or 128, 16-byte aligned rows -------------------------------------------------
//
// Per workgroup 64 keys; Q and dO stream through LDS in double-buffered 128-query stages copied global ->
// LDS directly, with that stage's lse and delta rows beside them.  8 wavefronts on v_mfma_f32_32x32x16:
// wave (k = w & 1, q = w >> 1) owns keys 32 k .. +31 of the block and queries 32 q .. +31 of every stage,
// so each wave computes one 32 x 32 tile per stage (lane = key; accumulator element 4 j + r = query
// 8 j + 4 h + r of the wave's 32):
//   S = Q_q K_k^T + (-lse / scale),  dP' = dO_q (-V_k)^T + delta   (A: Q / dO rows from LDS; B: K in
//                                              registers, the negated V rows from the block's LDS tile)
//   P = exp2(S sl2) = exp(scale S_qk - lse),  -dS = P dP' = P (delta - dP)
//   dV += P^T dO, dK += (-dS)^T Q              (A: P^T / -dS^T packed from the accumulators as the 16 k-slots
//                                              of two 8-query groups; B: dO / Q read column-wise with
//                                              ds_read_b64_tr_b16 in the same slot order); dK *= -scale
// Starting the accumulators at -lse / scale and delta (read from LDS) keeps lse and delta out of separate
// registers, and the operands of every product are read ahead into small rings fenced by sched_barrier:
// with 256 registers and the compiler's own order each MFMA waited for the LDS read issued right before it
// (phase timestamps: 37-50% matrix-core use inside the product phases of the 16x16x32 form this replaces).
// The four query quarters of a key group add their dK / dV partials through LDS in query-quarter order
// (deterministic), wave (k, q) finishing d block q (D = 128; D = 64: dK blocks by q = 0, 1, dV blocks by
// q = 2, 3), and store coalesced [key][d] rows.  P and dS are rounded to the input dtype before their
// products, as attn_coop.comp.in:235-236, 283-284.
template <typename T, int DCH>
__global__ __launch_bounds__(512) void attn_dkdv_w32(hrt_attn_args p, int nkb) {
  constexpr int NW = 8;
  constexpr int NCH = DCH * 4;        // 16-byte chunks per row
  constexpr int ROWB = NCH * 16;      // bytes per LDS tile row
  constexpr int TILE = QST * ROWB;    // bytes per Q or dO stage
  constexpr int KSN = 2 * DCH;        // 16-wide d steps of S / dP
  constexpr int IPW = QST * NCH / 64 / NW;  // copy instructions per tile and wavefront
  __shared__ __attribute__((aligned(1024))) uint8_t q0_raw[TILE], q1_raw[TILE], o0_raw[TILE], o1_raw[TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t v_raw[64 * ROWB];
  __shared__ __attribute__((aligned(1024))) float ls_raw[2][2 * QST];  // per stage buffer: lse, then delta
  // Destination of the copies issued during a last stage that has no ragged rows: they are issued (so that
  // no branch splits the stage's instruction stream) but land here, outside the tiles the merge reuses.
  __shared__ __attribute__((aligned(1024))) uint8_t sink_raw[1024];
  HK_L uint8_t* const Q0 = (HK_L uint8_t*)q0_raw;
  HK_L uint8_t* const Q1 = (HK_L uint8_t*)q1_raw;
  HK_L uint8_t* const O0 = (HK_L uint8_t*)o0_raw;
  HK_L uint8_t* const O1 = (HK_L uint8_t*)o1_raw;
  HK_L uint8_t* const VL = (HK_L uint8_t*)v_raw;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kg = wave & 1, qq = wave >> 1;
  const int rl = lane & 31, hl = lane >> 5;
  uint32_t bh32, kb32;
  xcd_map32(blockIdx.x, (uint32_t)nkb * p.B * p.H, nkb, bh32, kb32);
  const int64_t bh = bh32, kb = kb32, b = bh32 / (uint32_t)p.H, hh = bh32 % (uint32_t)p.H;
  const int Sq = p.Sq, Sk = p.Sk;
  const uint32_t qss = (uint32_t)(p.q_ss * 2), oss = (uint32_t)(p.do_ss * 2);
  const HK_G uint8_t* Qb = reinterpret_cast<const HK_G uint8_t*>(gcptr<uint16_t>(p.q) + b * p.q_sb + hh * p.q_sh);
  const HK_G uint8_t* Ob = reinterpret_cast<const HK_G uint8_t*>(gcptr<uint16_t>(p.dout) + b * p.do_sb + hh * p.do_sh);
  const HK_G float* lseb = gcptr<float>(p.lse) + bh * Sq;
  const HK_G float* dltb = gcptr<float>(p.delta) + bh * Sq;
  const int nst = (Sq + QST - 1) / QST;

  const int j0 = wave * IPW;
  // Values that depend only on the lane are re-derived where they are used from an opaque copy of the lane
  // index, so that they are not kept live across the S / dP products (the accumulators, S, dP and the K
  // fragments fill the 256 registers of a two-wavefront-per-SIMD kernel).
  auto opaque = [](int x) {
    asm volatile("" : "+v"(x));
    return x;
  };
  // lse / delta rows of a stage: waves 0..3 each copy 64 floats with one 4-byte-per-lane copy (wave w: rows
  // 64 (w & 1) .. +63 of lse (w < 2) or delta), the rows of a single short stage clamped to Sq - 1
  const __amdgpu_buffer_rsrc_t ls_rs = dma_rsrc(reinterpret_cast<const HK_G uint8_t*>(wave < 2 ? lseb : dltb));
  const int ls_r = nst == 1 && 64 * (wave & 1) + lane >= Sq ? Sq - 1 : 64 * (wave & 1) + lane;
  // (waves 4..7 copy lse rows into the sink instead: every wave issues the same instruction stream)
  auto copy_ls = [&](int st, HK_L void* dst) {
    const int org = nst > 1 ? (int)stage_origin<QST>(st, nst, Sq) : 0;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ls_rs, wave < 4 ? dst : (HK_L void*)sink_raw, 4, ls_r * 4, org * 4, 0, 0);
  };
  auto ls_dst = [&](int buf) { return (HK_L void*)(&ls_raw[buf][(wave >> 1) * QST + 64 * (wave & 1)]); };
  // The block's 64 K rows go to stage-1's Q buffer (free until stage 0 copies into it) and are read into
  // registers; its 64 V rows stay in their own tile for the whole loop (rows past Sk hold copies of the last
  // key; their dK / dV rows are never stored).  Then stage 0.
  {
    const uint32_t kss = (uint32_t)(p.k_ss * 2), vss = (uint32_t)(p.v_ss * 2);
    const int kvalid = (int)(Sk - kb * 64);
    const int jk = wave * (64 * NCH / 64 / NW);
    const HK_G uint8_t* Kblk = reinterpret_cast<const HK_G uint8_t*>(gcptr<uint16_t>(p.k) + b * p.k_sb + hh * p.k_sh) +
                               kb * 64 * (int64_t)kss;
    const HK_G uint8_t* Vblk = reinterpret_cast<const HK_G uint8_t*>(gcptr<uint16_t>(p.v) + b * p.v_sb + hh * p.v_sh) +
                               kb * 64 * (int64_t)vss;
    dma_tile<NCH, 64, NW>(Kblk, kss, kvalid, Q1, wave, lane, dma_lane_offsets<NCH>(kss, lane, jk));
    dma_tile<NCH, 64, NW>(Vblk, vss, kvalid, VL, wave, lane, dma_lane_offsets<NCH>(vss, lane, jk));
  }
  issue_order_fence();  // the first barrier counts on stage 0's copies being the last ones issued
  dma_tile<NCH, QST, NW>(Qb, qss, Sq, Q0, wave, lane, dma_lane_offsets<NCH>(qss, lane, j0));
  dma_tile<NCH, QST, NW>(Ob, oss, Sq, O0, wave, lane, dma_lane_offsets<NCH>(oss, lane, j0));
  copy_ls(0, ls_dst(0));

  // per-lane byte offsets inside a 32-row quarter of a tile of the A-operand rows (row rl, chunk 2 ks + h);
  // the tile rows of a quarter start at 32 q, which keeps the swizzle (it uses row bits 0..3)
  int roff[KSN];
#pragma unroll
  for (int ks = 0; ks < KSN; ++ks) roff[ks] = tile_off<NCH>(rl, 2 * ks + hl);

  f32x16 dk[DCH], dv[DCH];
#pragma unroll
  for (int n = 0; n < DCH; ++n) dk[n] = dv[n] = zero16();
  const float sl2 = p.scale * kLog2e;

  // K and V rows landed (stage 0 may still be in flight; waves 0..3 wait for one of its copies too)
  barrier_keep_vm<2 * IPW>();
  u32x4 kf[KSN];  // this lane's key (column rl of S): K as B fragments, d = 16 ks + 8 h + i
#pragma unroll
  for (int ks = 0; ks < KSN; ++ks) kf[ks] = *reinterpret_cast<const HK_L u32x4*>(Q1 + kg * 32 * ROWB + roff[ks]);
  // V is negated in place (the sign bits of its 16-bit elements), so that dP's accumulator, started at delta,
  // ends at delta - dP = -(dP - delta); the sign of dS is carried into dK's final scale (-scale)
  for (int i = threadIdx.x; i < 64 * ROWB / 16; i += NW * 64) {
    HK_L u32x4* v = reinterpret_cast<HK_L u32x4*>(VL) + i;
    *v = *v ^ u32x4{0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
  }
  __syncthreads();  // stage 0 landed; K fragments read and V negated before stage 1 is copied over K

  const HK_L uint8_t* const Vq = VL + kg * 32 * ROWB;
  // Stage st from buffer BUF.  Its copies of stage st + 1 are placed between the MFMAs of S / dP (a last
  // stage without ragged rows copies its own rows again, into the sink: no branch).  RAGGED (the last stage
  // when Sq % 128 != 0, or a single short stage) issues no copies and gives rows outside [st QST, Sq) P = 0.
  // S's accumulator starts at -lse / scale and dP's at delta (V is negated), so that
  //   P = exp2(acc_S sl2) = exp(scale S - lse),   -dS = P acc_dP = P (delta - dP).
  const float nis = -1.f / p.scale;
  auto stage = [&](auto bc, auto rc, int st) {
    constexpr int BUF = decltype(bc)::value;
    constexpr bool RAGGED = decltype(rc)::value;
    const bool COPY = st + 1 < nst;
    const HK_L uint8_t* Qt = (BUF ? Q1 : Q0) + qq * 32 * ROWB;
    const HK_L uint8_t* Ot = (BUF ? O1 : O0) + qq * 32 * ROWB;
    const float* ls = &ls_raw[BUF][qq * 32 + 4 * hl];
    // element 4 j + r: query 32 q + 8 j + 4 h + r of the stage tile
    f32x16 s, dp;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 l4 = *reinterpret_cast<const f32x4*>(ls + 8 * j);
      const f32x4 d4 = *reinterpret_cast<const f32x4*>(ls + QST + 8 * j);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s[4 * j + r] = l4[r] * nis;
        dp[4 * j + r] = d4[r];
      }
    }
    if constexpr (RAGGED) {
      const int org = nst > 1 ? (int)stage_origin<QST>(st, nst, Sq) : 0;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int qa = org + qq * 32 + 8 * j + 4 * hl + r;
          s[4 * j + r] = qa >= st * QST && qa < Sq ? s[4 * j + r] : -INFINITY;
        }
    }
    const __amdgpu_buffer_rsrc_t qrs = dma_rsrc(Qb + stage_origin<QST>(st + 1, nst, Sq) * qss);
    const __amdgpu_buffer_rsrc_t ors = dma_rsrc(Ob + stage_origin<QST>(st + 1, nst, Sq) * oss);
    HK_L uint8_t* const sink = (HK_L uint8_t*)sink_raw;
    HK_L uint8_t* const qdst = COPY ? (BUF ? Q0 : Q1) + j0 * 1024 : sink;
    HK_L uint8_t* const odst = COPY ? (BUF ? O0 : O1) + j0 * 1024 : sink;
    const int dstep = COPY ? 1024 : 0;
    constexpr int RPI = 64 / NCH;
    // Lane offsets of this stage's copies (dma_lane_offsets, in fewer instructions): j0 is a multiple of the
    // swizzle period (16 rows), and the swizzle is linear in the row bits, so instruction i's offset is
    // rsub ss + ((slot ^ swz(rsub) ^ swz(i RPI)) << 4), the last term a constant
    static_assert((IPW * RPI) % 16 == 0, "copy blocks start on a swizzle period");
    DmaLanes qlo, olo;
    {
      const int ln = opaque(lane);
      const int rsub = ln / NCH;
      const uint32_t x0 = (uint32_t)(((ln % NCH) ^ tile_swz<NCH>(rsub)) << 4);
      const uint32_t bq = (uint32_t)rsub * qss, bo = (uint32_t)rsub * oss;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t x = x0 ^ (uint32_t)(tile_swz<NCH>(i * RPI) << 4);
        qlo.off[i] = bq + x;
        olo.off[i] = bo + x;
      }
    }
    // S and dP products of d step ks; their operands (Q, dO, V rows) are read RA1 steps ahead into a ring,
    // each step fenced by sched_barrier
    constexpr int RA1 = 1;
    u32x4 qr[RA1 + 1], orr[RA1 + 1], vr[RA1 + 1];
    auto rd1 = [&](int ks) {
      qr[ks % (RA1 + 1)] = *reinterpret_cast<const HK_L u32x4*>(Qt + roff[ks]);
      orr[ks % (RA1 + 1)] = *reinterpret_cast<const HK_L u32x4*>(Ot + roff[ks]);
      vr[ks % (RA1 + 1)] = *reinterpret_cast<const HK_L u32x4*>(Vq + roff[ks]);
    };
#pragma unroll
    for (int ks = 0; ks < RA1; ++ks) rd1(ks);
#pragma unroll
    for (int ks = 0; ks < KSN; ++ks) {
      __builtin_amdgcn_sched_barrier(0);
      if (ks + RA1 < KSN) rd1(ks + RA1);
      s = Mfma32<T>::mac(qr[ks % (RA1 + 1)], kf[ks], s);
      dp = Mfma32<T>::mac(orr[ks % (RA1 + 1)], vr[ks % (RA1 + 1)], dp);
      if constexpr (!RAGGED) {
        if (ks < IPW)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(qrs, qdst + ks * dstep, 16, (int)qlo.off[ks % 4],
                                                   (int)((uint32_t)((j0 + ks) * RPI) * qss), 0, 0);
        else if (ks < 2 * IPW)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(ors, odst + (ks - IPW) * dstep, 16, (int)olo.off[(ks - IPW) % 4],
                                                   (int)((uint32_t)((j0 + ks - IPW) * RPI) * oss), 0, 0);
        if (ks == KSN - 1) copy_ls(st + 1, COPY ? ls_dst(BUF ^ 1) : (HK_L void*)sink);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      s[e] = __builtin_amdgcn_exp2f(s[e] * sl2);  // exp2(-inf) = 0 for masked rows
      dp[e] *= s[e];
    }
    // B-operand column reads: rows 4 h + (l16 >> 2) and +8, columns 32 n + 16 ((lane >> 4) & 1) + 4 (l16 & 3)
    // (column block n adds 4 n to a chunk index below 4, which enters the swizzle XOR on bits of its own:
    // block n's offset is block 0's with bits 6-7 flipped by n)
    int toff[DCH][2];
    {
      const int ln = opaque(lane);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int row = 8 * t + 4 * (ln >> 5) + ((ln & 15) >> 2);
        const int c0 = 2 * ((ln >> 4) & 1) + ((ln >> 1) & 1);
        toff[0][t] = tile_off<NCH>(row, c0) + (ln & 1) * 8;
#pragma unroll
        for (int n = 1; n < DCH; ++n) toff[n][t] = toff[0][t] ^ (n << 6);
      }
    }
    const u32x4 pa0 = pack_slots<T>(s, 0, 1), pa1 = pack_slots<T>(s, 2, 3);
    const u32x4 da0 = pack_slots<T>(dp, 0, 1), da1 = pack_slots<T>(dp, 2, 3);
    // dV += P^T dO, dK += (-dS)^T Q: product i = (n, c, dV or dK) in the order n, c, {dV, dK}; its B operand
    // (two column reads) is read RA products ahead into a ring, each step fenced by sched_barrier so that the
    // reads stay ahead of the MFMAs that wait for them
    constexpr int NP = 4 * DCH, RA = 2;
    u32x4 ring[RA + 1];
    auto rd = [&](int i) {
      const int n = i >> 2, c = (i >> 1) & 1;
      const HK_L uint8_t* t = (i & 1) ? Qt : Ot;
      const u32x2 lo = lds_tr4(t + toff[n][0] + c * 16 * ROWB), hi = lds_tr4(t + toff[n][1] + c * 16 * ROWB);
      ring[i % (RA + 1)] = u32x4{lo.x, lo.y, hi.x, hi.y};
    };
#pragma unroll
    for (int i = 0; i < RA; ++i) rd(i);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      __builtin_amdgcn_sched_barrier(0);
      if (i + RA < NP) rd(i + RA);
      const int n = i >> 2, c = (i >> 1) & 1;
      if (i & 1)
        dk[n] = Mfma32<T>::mac(c ? da1 : da0, ring[i % (RA + 1)], dk[n]);
      else
        dv[n] = Mfma32<T>::mac(c ? pa1 : pa0, ring[i % (RA + 1)], dv[n]);
    }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  const int nfull = Sq % QST == 0 ? nst : nst - 1;  // stages without ragged rows
  int st = 0;
  for (; st + 1 < nfull; st += 2) {
    stage(I0(), std::false_type(), st);
    stage(I1(), std::false_type(), st + 1);
  }
  if (st < nfull) {
    stage(I0(), std::false_type(), st);
    ++st;
  }
  if (st < nst) {  // the ragged last stage, in buffer st & 1
    if (st & 1)
      stage(I1(), std::true_type(), st);
    else
      stage(I0(), std::true_type(), st);
  }

  // ---- sum the four query quarters of each key group, dK first, then dV.  Piece (k, n) = d block n of key
  // group k, finished by its owner wave (k, own(n)); the three other waves' partials go to slots 0..2 of
  // the piece's area in query-quarter order, [slot][16 values][64 lanes] (conflict-free 16-byte accesses),
  // and the owner adds all four in query-quarter order.  It then transposes its 32 x 32 block through its
  // own area (rows of 40 floats) and stores 8 d of one key row per lane.
  constexpr int PIECE = 3 * 16 * 64;  // floats
  static_assert(2 * DCH * PIECE * 4 <= 4 * TILE, "the merge areas fit the stage tiles");
  auto area = [&](int k, int n) -> float* {
    const int idx = k * DCH + n;  // PIECE floats each, laid across the four stage tiles
    constexpr int PPT = TILE / (PIECE * 4) > 0 ? TILE / (PIECE * 4) : 1;
    uint8_t* t = idx / PPT == 0 ? q0_raw : idx / PPT == 1 ? q1_raw : idx / PPT == 2 ? o0_raw : o1_raw;
    return reinterpret_cast<float*>(t) + (idx % PPT) * PIECE;
  };
  auto round = [&](auto quant) {
    constexpr int R = decltype(quant)::value;  // 0: dK, 1: dV
    auto own = [](int n) { return DCH == 4 ? n : n + 2 * R; };
    f32x16* acc = R == 0 ? dk : dv;
#pragma unroll
    for (int n = 0; n < DCH; ++n) {
      const int o = own(n);
      if (o == qq) continue;
      f32x4* dst = reinterpret_cast<f32x4*>(area(kg, n) + (qq < o ? qq : qq - 1) * 16 * 64) + lane;
#pragma unroll
      for (int c = 0; c < 4; ++c) dst[c * 64] = f32x4{acc[n][4 * c], acc[n][4 * c + 1], acc[n][4 * c + 2], acc[n][4 * c + 3]};
    }
    // the partials are visible to every wave; the previous round's global stores may stay in flight
    barrier_keep_vm_lds<63>();
#pragma unroll
    for (int n = 0; n < DCH; ++n) {
      if (own(n) != qq) continue;
      float* const ar = area(kg, n);
      f32x16 sum = zero16();
#pragma unroll
      for (int src = 0; src < 4; ++src) {
        if (src == qq) {
#pragma unroll
          for (int e = 0; e < 16; ++e) sum[e] += acc[n][e];
        } else {
          const f32x4* from = reinterpret_cast<const f32x4*>(ar + (src < qq ? src : src - 1) * 16 * 64) + lane;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const f32x4 x = from[c * 64];
#pragma unroll
            for (int w = 0; w < 4; ++w) sum[4 * c + w] += x[w];
          }
        }
      }
      const float mul = R == 0 ? -p.scale : 1.f;  // dK's products used -dS; dV is not scaled (x * 1 == x)
      // element 4 j + r: key 8 j + 4 h + r of the group, d = 32 n + rl; same wavefront wrote and reads the area
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) ar[(8 * j + 4 * hl + r) * 40 + rl] = sum[4 * j + r] * mul;
      const uint64_t dst_base = R == 0 ? p.dk : p.dv;
      const int64_t g_sb = R == 0 ? p.k_sb : p.v_sb, g_sh = R == 0 ? p.k_sh : p.v_sh, g_ss = R == 0 ? p.k_ss : p.v_ss;
#pragma unroll
      for (int ps = 0; ps < 2; ++ps) {
        const int key = ps * 16 + (lane >> 2), c8 = (lane & 3) * 8;
        const f32x4 x = *reinterpret_cast<const f32x4*>(ar + key * 40 + c8);
        const f32x4 y = *reinterpret_cast<const f32x4*>(ar + key * 40 + c8 + 4);
        const int64_t kk = kb * 64 + kg * 32 + key;
        const float o8[8] = {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
        if (kk < Sk)
          *reinterpret_cast<HK_G u32x4*>(gptr<uint16_t>(dst_base) + grad_row(p, b, hh, kk, Sk, g_sb, g_sh, g_ss) + n * 32 + c8) =
              pack8<T>(o8);
      }
    }
  };
  round(I0());
  barrier_keep_vm_lds<63>();  // every owner is done with the areas before the dV partials overwrite them
  round(I1());
}

// The direct-to-LDS paths need D = 64 or 128, 16-byte aligned rows (q, k, v, dout) and per-stage row
// offsets that fit the 32-bit lane offsets of the copies.
bool bwd_dma_ok(const hrt_attn_args& a) {
  if (!(a.D == 64 || a.D == 128) || !attn_vec_ok(a, true)) return false;
  const int64_t lim = (int64_t)1 << 31;
  return a.k_ss * 2 * (KST2 + 1) < lim && a.v_ss * 2 * (KST2 + 1) < lim && a.q_ss * 2 * (KST2 + 1) < lim &&
         a.do_ss * 2 * (KST2 + 1) < lim;
}

template <typename T>
bool launch_dkdv(const void* pp, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_attn_args*>(pp);
  if (!attn_check(a, false, true, false, 2, ctx)) return false;
  const int nkb = (a.Sk + 63) / 64;
  const int64_t total = (int64_t)nkb * a.B * a.H;
  if (total > 0x7fffffffLL) return ctx.fail("grid too large");
  const dim3 g((uint32_t)total);
  if (bwd_dma_ok(a)) {
    if (a.D == 128)
      hipLaunchKernelGGL((attn_dkdv_w32<T, 4>), g, dim3(512), 0, ctx.stream, a, nkb);
    else
      hipLaunchKernelGGL((attn_dkdv_w32<T, 2>), g, dim3(512), 0, ctx.stream, a, nkb);
    return hrt::launch_ok(hipGetLastError(), ctx, "attn_dkdv_w32");
  }
  const int lm = !attn_vec_ok(a, true) ? LD_GATHER : (a.D % 32 == 0 ? LD_FULL : LD_VEC);
#define HK_LAUNCH(DCH)                                                                                   \
  if (lm == LD_FULL)                                                                                \
    hipLaunchKernelGGL((attn_dkdv_mfma<T, DCH, LD_FULL>), g, dim3(256), 0, ctx.stream, a, nkb);        \
  else if (lm == LD_VEC)                                                                            \
    hipLaunchKernelGGL((attn_dkdv_mfma<T, DCH, LD_VEC>), g, dim3(256), 0, ctx.stream, a, nkb);         \
  else                                                                                              \
    hipLaunchKernelGGL((attn_dkdv_mfma<T, DCH, LD_GATHER>), g, dim3(256), 0, ctx.stream, a, nkb);
  switch ((a.D + 31) / 32) {
    case 1: HK_LAUNCH(1) break;
    case 2: HK_LAUNCH(2) break;
    case 3: HK_LAUNCH(3) break;
    default: HK_LAUNCH(4) break;
  }
#undef HK_LAUNCH
  return hrt::launch_ok(hipGetLastError(), ctx, "attn_dkdv_mfma");
}

template <typename T>
bool launch_dq(const void* pp, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_attn_args*>(pp);
  if (!attn_check(a, false, false, true, 2, ctx)) return false;
  const int nqb = (a.Sq + 63) / 64;
  const int64_t total = (int64_t)nqb * a.B * a.H;
  if (total > 0x7fffffffLL) return ctx.fail("grid too large");
  const bool with_delta = (a.flags & HRT_ATTN_DQ_DELTA) != 0;
  const bool of32 = (a.flags & HRT_ATTN_O_F32) != 0;
  const dim3 g((uint32_t)total);
  if (bwd_dma_ok(a)) {
    if (with_delta && !ctx.check(a.o, (uint64_t)a.B * a.H * a.Sq * a.D * (of32 ? 4 : 2), "o")) return false;
#define HK_DQ(DCH)                                                                                          \
  if (!with_delta)                                                                                          \
    hipLaunchKernelGGL((attn_dq_dma<T, DCH, false, false>), g, dim3(512), 0, ctx.stream, a, nqb);            \
  else if (of32)                                                                                            \
    hipLaunchKernelGGL((attn_dq_dma<T, DCH, true, true>), g, dim3(512), 0, ctx.stream, a, nqb);              \
  else                                                                                                      \
    hipLaunchKernelGGL((attn_dq_dma<T, DCH, false, true>), g, dim3(512), 0, ctx.stream, a, nqb);
    if (a.D == 128) {
      HK_DQ(4)
    } else {
      HK_DQ(2)
    }
#undef HK_DQ
    return hrt::launch_ok(hipGetLastError(), ctx, "attn_dq_dma");
  }
  if (with_delta && !launch_delta<T>(pp, nullptr, ctx)) return false;
  const int lm = !attn_vec_ok(a, true) ? LD_GATHER : (a.D % 32 == 0 ? LD_FULL : LD_VEC);
#define HK_LAUNCH(DCH)                                                                                   \
  if (lm == LD_FULL)                                                                                \
    hipLaunchKernelGGL((attn_dq_mfma<T, DCH, LD_FULL>), g, dim3(256), 0, ctx.stream, a, nqb);        \
  else if (lm == LD_VEC)                                                                            \
    hipLaunchKernelGGL((attn_dq_mfma<T, DCH, LD_VEC>), g, dim3(256), 0, ctx.stream, a, nqb);         \
  else                                                                                              \
    hipLaunchKernelGGL((attn_dq_mfma<T, DCH, LD_GATHER>), g, dim3(256), 0, ctx.stream, a, nqb);
  switch ((a.D + 31) / 32) {
    case 1: HK_LAUNCH(1) break;
    case 2: HK_LAUNCH(2) break;
    case 3: HK_LAUNCH(3) break;
    default: HK_LAUNCH(4) break;
  }
#undef HK_LAUNCH
  return hrt::launch_ok(hipGetLastError(), ctx, "attn_dq_mfma");
}

HRT_REGISTER("attn_dkdv_mfma_bf16", hrt_attn_args, launch_dkdv<BF16>);
HRT_REGISTER("attn_dkdv_mfma_f16", hrt_attn_args, launch_dkdv<F16>);
HRT_REGISTER("attn_dq_mfma_bf16", hrt_attn_args, launch_dq<BF16>);
HRT_REGISTER("attn_dq_mfma_f16", hrt_attn_args, launch_dq<F16>);

}  // namespace
}  // namespace hk
