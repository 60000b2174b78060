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
    const HK_G uint8_t* ksrc = Kb + stage_origin<KST2>(st + 1, nst, Sk) * kss;
    const HK_G uint8_t* vsrc = Vb + stage_origin<KST2>(st + 1, nst, Sk) * vss;
    const HK_L uint8_t* Kt = BUF ? K1 : K0;
    const HK_L uint8_t* Vt = BUF ? V1 : V0;
    f32x16 s = zero16(), dp = zero16();
#pragma unroll
    for (int ks = 0; ks < 2 * DCH; ++ks) {
      s = Mfma32<T>::mac(*reinterpret_cast<const HK_L u32x4*>(Kt + koff[ks]), qf[ks], s);
      dp = Mfma32<T>::mac(*reinterpret_cast<const HK_L u32x4*>(Vt + koff[ks]), df[ks], dp);
      if constexpr (COPY) {
        if (ks < IPW) dma_tile_part<NCH, KST2, NW>(ksrc, kss, BUF ? K0 : K1, wave, klo, ks);
        else if (ks < 2 * IPW) dma_tile_part<NCH, KST2, NW>(vsrc, vss, BUF ? V0 : V1, wave, vlo, ks - IPW);
      }
    }
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
#pragma unroll
    for (int n = 0; n < DCH; ++n)
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const u32x2 lo = lds_tr4(Kt + voff[n][0] + kc * 16 * ROWB);
        const u32x2 hi = lds_tr4(Kt + voff[n][1] + kc * 16 * ROWB);
        acc[n] = Mfma32<T>::mac(u32x4{lo.x, lo.y, hi.x, hi.y}, kc ? d1 : d0, acc[n]);
      }
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
      if (qrow < Sq)
        *reinterpret_cast<HK_G u32x2*>(gptr<uint16_t>(p.dq) + grad_row(p, b, hh, qrow, Sq, p.q_sb, p.q_sh, p.q_ss) + N * 32 + c4) =
            u32x2{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
    }
  };
  switch (kq) {
    case 0: finish(std::integral_constant<int, 0>()); break;
    case 1: finish(std::integral_constant<int, 1>()); break;
    case 2: if constexpr (DCH > 2) finish(std::integral_constant<int, 2 % DCH>()); break;
    default: if constexpr (DCH > 3) finish(std::integral_constant<int, 3 % DCH>()); break;
  }
}

// ---- dK / dV fast path: D = 64 or 128, 16-byte aligned rows -------------------------------------------------
//
// Per workgroup 64 keys; Q and dO stream through LDS in double-buffered 128-query stages copied global ->
// LDS directly, each stage computed as two 64-query halves (one barrier per 128 queries).  8 wavefronts on
// v_mfma_f32_16x16x32 (see mfma_common.h for its lane layout): wave (k = w & 3, h = w >> 2) owns keys
// 16 k .. +15 of the block (their K and V rows held as B fragments) and query rows 32 h .. +31 of every
// 64-query half, so its dK/dV partials are 16 keys x D each (64 registers for D = 128) and every LDS
// fragment read is conflict-free.  Per half and 16-query tile t:
//   S_t = Q_t K^T, dP_t = dO_t V^T            (lane = key, 4 queries 4 g + i per tile, g = lane / 16)
//   P = exp2(S sl2 - lse log2e), dS = P (dP - delta)
//   dV += P^T dO, dK += dS^T Q                (A = P^T / dS^T packed from the two tiles' accumulators as
//                                              the 32 k-slots {4 g + i, 16 + 4 g + i}; B = dO / Q read
//                                              column-wise with ds_read_b64_tr_b16 in the same slot order)
// lse and delta of the next half are prefetched into registers.  At the end the two query halves swap
// partials through LDS (wave (k, 1) hands over its dK, wave (k, 0) its dV), so wave (k, 0) writes dK
// (scaled) and wave (k, 1) writes dV, both as coalesced rows.  P and dS are rounded to the input dtype
// before their products, as attn_coop.comp.in:235-236, 283-284.
constexpr int QST = 128;  // queries per LDS stage
constexpr int QHALF = 64;  // queries per computed half

template <typename T, int DCH, bool A4>
__global__ __launch_bounds__(512) void attn_dkdv_dma(hrt_attn_args p, int nkb) {
  constexpr int NW = 8;
  constexpr int NCH = DCH * 4;
  constexpr int ROWB = NCH * 16;
  constexpr int TILE = QST * ROWB;   // bytes per Q or dO stage
  constexpr int NDT = DCH * 2;       // 16-wide d tiles
  constexpr int SW = NCH == 16 ? 1 : 0;  // the 16x16x32 tile layout (conflict-free reads, lds_stage.h)
  __shared__ __attribute__((aligned(1024))) uint8_t q0_raw[TILE], q1_raw[TILE], o0_raw[TILE], o1_raw[TILE];
  HK_L uint8_t* const Q0 = (HK_L uint8_t*)q0_raw;
  HK_L uint8_t* const Q1 = (HK_L uint8_t*)q1_raw;
  HK_L uint8_t* const O0 = (HK_L uint8_t*)o0_raw;
  HK_L uint8_t* const O1 = (HK_L uint8_t*)o1_raw;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kg = wave & 3, qh = wave >> 2;
  const int l16 = lane & 15, g4 = lane >> 4;
  uint32_t bh32, kb32;
  xcd_map32(blockIdx.x, (uint32_t)nkb * p.B * p.H, nkb, bh32, kb32);
  const int64_t bh = bh32, kb = kb32, b = bh32 / (uint32_t)p.H, hh = bh32 % (uint32_t)p.H;
  const int Sq = p.Sq, Sk = p.Sk;
  const uint32_t qss = (uint32_t)(p.q_ss * 2), oss = (uint32_t)(p.do_ss * 2);
  const HK_G uint8_t* Qb = reinterpret_cast<const HK_G uint8_t*>(gcptr<uint16_t>(p.q) + b * p.q_sb + hh * p.q_sh);
  const HK_G uint8_t* Ob = reinterpret_cast<const HK_G uint8_t*>(gcptr<uint16_t>(p.dout) + b * p.do_sb + hh * p.do_sh);
  const int nst = (Sq + QST - 1) / QST;

  const int j0 = wave * (QST * NCH / 64 / NW);
  const DmaLanes qlo = dma_lane_offsets<NCH, SW>(qss, lane, j0), olo = dma_lane_offsets<NCH, SW>(oss, lane, j0);
  // The block's 64 K and V rows go to the stage-1 buffers (free until stage 0 copies into them), copied once
  // for the two wavefronts that share them (rows past Sk hold copies of the last key; their dK / dV rows
  // are never stored), then stage 0 of Q and dO
  {
    const uint32_t kss = (uint32_t)(p.k_ss * 2), vss = (uint32_t)(p.v_ss * 2);
    const int kvalid = (int)(Sk - kb * 64);
    const int jk = wave * (64 * NCH / 64 / NW);
    const HK_G uint8_t* Kblk = reinterpret_cast<const HK_G uint8_t*>(gcptr<uint16_t>(p.k) + b * p.k_sb + hh * p.k_sh) +
                               kb * 64 * (int64_t)kss;
    const HK_G uint8_t* Vblk = reinterpret_cast<const HK_G uint8_t*>(gcptr<uint16_t>(p.v) + b * p.v_sb + hh * p.v_sh) +
                               kb * 64 * (int64_t)vss;
    dma_tile<NCH, 64, NW, SW>(Kblk, kss, kvalid, Q1, wave, lane, dma_lane_offsets<NCH, SW>(kss, lane, jk));
    dma_tile<NCH, 64, NW, SW>(Vblk, vss, kvalid, O1, wave, lane, dma_lane_offsets<NCH, SW>(vss, lane, jk));
  }
  issue_order_fence();  // the first barrier counts on stage 0's copies being the last ones issued
  dma_tile<NCH, QST, NW, SW>(Qb, qss, Sq, Q0, wave, lane, qlo);
  dma_tile<NCH, QST, NW, SW>(Ob, oss, Sq, O0, wave, lane, olo);

  // lse and delta of this lane's 8 queries of a half: tile t, rows 64 half + 32 qh + 16 t + 4 g + i of the
  // stage (i = 0..3, four consecutive floats: one 16-byte load each when A4, i.e. Sq % 4 == 0 and 16-byte
  // aligned arrays)
  const HK_G float* lseb = gcptr<float>(p.lse) + bh * Sq;
  const HK_G float* dltb = gcptr<float>(p.delta) + bh * Sq;
  f32x4 nl[2], dl[2];  // lse, delta
  // Stage st's tile starts at query row origin(st) (stage_origin when there is more than one stage); its
  // rows outside [st QST, Sq) get lse = +inf, so P = dS = 0 for them.
  auto fetch = [&](int st, int half, f32x4* lo, f32x4* dlo) {
    const int64_t org = nst > 1 ? stage_origin<QST>(st, nst, Sq) : 0;
    const int r0 = (int)org + half * QHALF + qh * 32 + 4 * g4;
    if (A4 && st * QST + QST <= Sq) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        lo[t] = *reinterpret_cast<const HK_G f32x4*>(lseb + r0 + 16 * t);
        dlo[t] = *reinterpret_cast<const HK_G f32x4*>(dltb + r0 + 16 * t);
      }
    } else {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int qq = r0 + 16 * t + i;
          const bool ok = qq >= st * QST && qq < Sq;
          lo[t][i] = ok ? lseb[qq] : INFINITY;
          dlo[t][i] = ok ? dltb[qq] : 0.f;
        }
    }
  };
  fetch(0, 0, nl, dl);

  // per-lane byte offsets: A-operand rows (query 32 qh + 16 t + l16, chunk 4 ks + g; t adds 16 rows and the
  // half 64 rows, which keeps the swizzle) and B-operand column reads (rows 32 qh + 4 g + (l16 >> 2) (+16
  // for the second read), columns 16 dt + 4 (l16 & 3))
  int roff[DCH], coff[NDT];
#pragma unroll
  for (int ks = 0; ks < DCH; ++ks) roff[ks] = tile_off<NCH, SW>(qh * 32 + l16, 4 * ks + g4);
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
    coff[dt] = tile_off<NCH, SW>(qh * 32 + 4 * g4 + (l16 >> 2), 2 * dt + ((l16 >> 1) & 1)) + (l16 & 1) * 8;

  f32x4 dk[NDT], dv[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) dk[dt] = dv[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float sl2 = p.scale * kLog2e;

  // K and V rows landed (stage 0 of Q / dO may still be in flight); this lane's key (column l16 of the
  // 16x16 tiles): K and V as B fragments, d = 32 ks + 8 g + i
  barrier_keep_vm<2 * (QST * NCH / 64 / NW)>();
  u32x4 kf[DCH], vf[DCH];
#pragma unroll
  for (int ks = 0; ks < DCH; ++ks) {
    kf[ks] = *reinterpret_cast<const HK_L u32x4*>(Q1 + tile_off<NCH, SW>(kg * 16 + l16, 4 * ks + g4));
    vf[ks] = *reinterpret_cast<const HK_L u32x4*>(O1 + tile_off<NCH, SW>(kg * 16 + l16, 4 * ks + g4));
  }
  __syncthreads();  // stage 0 landed; every wave holds its K / V fragments before stage 1 is copied over them
  // COPY: stage st + 1 is copied while stage st computes (its Q rows during the first half, its dO rows
  // during the second), the copies placed between the MFMAs of S / dP; with more than one stage they are
  // branch-free (stage_origin, as in the other attention kernels).
  constexpr int IPW = QST * NCH / 64 / NW;
  static_assert(IPW <= 2 * DCH, "a half's copies fit between its S / dP products");
  auto half_stage = [&](auto bc, auto hc, auto cc, int st) {
    constexpr int BUF = decltype(bc)::value;
    constexpr int HALF = decltype(hc)::value;
    constexpr bool COPY = decltype(cc)::value;
    const HK_G uint8_t* src = HALF ? Ob + stage_origin<QST>(st + 1, nst, Sq) * oss
                                   : Qb + stage_origin<QST>(st + 1, nst, Sq) * qss;
    const bool more = HALF == 0 || st + 1 < nst;
    f32x4 nn[2], dn[2];
    if (more) fetch(HALF ? st + 1 : st, HALF ^ 1, nn, dn);
    const HK_L uint8_t* Qt = (BUF ? Q1 : Q0) + HALF * QHALF * ROWB;
    const HK_L uint8_t* Ot = (BUF ? O1 : O0) + HALF * QHALF * ROWB;
    f32x4 s[2], dp[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      s[t] = dp[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < DCH; ++ks) {
        s[t] = Mfma<T>::mac(*reinterpret_cast<const HK_L u32x4*>(Qt + roff[ks] + t * 16 * ROWB), kf[ks], s[t]);
        dp[t] = Mfma<T>::mac(*reinterpret_cast<const HK_L u32x4*>(Ot + roff[ks] + t * 16 * ROWB), vf[ks], dp[t]);
        if constexpr (COPY) {
          const int c = t * DCH + ks;
          if (c < IPW) dma_tile_part<NCH, QST, NW>(src, HALF ? oss : qss, HALF ? (BUF ? O0 : O1) : (BUF ? Q0 : Q1),
                                                   wave, HALF ? olo : qlo, c);
        }
      }
    }
    float pv[8], ds[8];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pe = __builtin_amdgcn_exp2f(fmaf(s[t][i], sl2, -nl[t][i] * kLog2e));
        pv[t * 4 + i] = pe;
        ds[t * 4 + i] = pe * (dp[t][i] - dl[t][i]);
      }
    const u32x4 pa = u32x4{cvt2<T>(pv[0], pv[1]), cvt2<T>(pv[2], pv[3]), cvt2<T>(pv[4], pv[5]), cvt2<T>(pv[6], pv[7])};
    const u32x4 da = u32x4{cvt2<T>(ds[0], ds[1]), cvt2<T>(ds[2], ds[3]), cvt2<T>(ds[4], ds[5]), cvt2<T>(ds[6], ds[7])};
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const u32x2 a0 = lds_tr4(Ot + coff[dt]), a1 = lds_tr4(Ot + coff[dt] + 16 * ROWB);
      dv[dt] = Mfma<T>::mac(pa, u32x4{a0.x, a0.y, a1.x, a1.y}, dv[dt]);
      const u32x2 b0 = lds_tr4(Qt + coff[dt]), b1 = lds_tr4(Qt + coff[dt] + 16 * ROWB);
      dk[dt] = Mfma<T>::mac(da, u32x4{b0.x, b0.y, b1.x, b1.y}, dk[dt]);
    }
    if (more) {
      nl[0] = nn[0], nl[1] = nn[1], dl[0] = dn[0], dl[1] = dn[1];
    }
    if constexpr (HALF == 1 && COPY) __syncthreads();
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  // The last stage runs without copies (no stage follows; the tiles are reused as scratch below, and a copy
  // landing there late has been seen to corrupt LDS written after the closing barrier), then one barrier.
  // Pairs of copying stages run in the loop, the last one or two are peeled into straight-line code (one
  // variant per buffer in the loop body keeps the D = 128 kernel within its 256 registers).
  auto full = [&](auto bc, int st) {
    half_stage(bc, I0(), std::true_type(), st);
    half_stage(bc, I1(), std::true_type(), st);
  };
  auto last = [&](auto bc, int st) {
    half_stage(bc, I0(), std::false_type(), st);
    if (nst > 1 || Sq > QHALF) half_stage(bc, I1(), std::false_type(), st);
  };
  int st = 0;
  for (; st + 2 < nst; st += 2) {
    full(I0(), st);
    full(I1(), st + 1);
  }
  if (st + 1 < nst) {
    full(I0(), st);
    last(I1(), st + 1);
  } else {
    last(I0(), st);
  }
  __syncthreads();

  // ---- sum the two query halves through tile k's area: slot 0 takes wave (k, 1)'s dK partials, slot 1 wave
  // (k, 0)'s dV partials (16 bytes per lane and d tile); each wave then reuses its own slot to transpose its
  // result into [key][d] rows for coalesced stores.
  float* const area = reinterpret_cast<float*>(kg == 0 ? q0_raw : kg == 1 ? q1_raw : kg == 2 ? o0_raw : o1_raw);
  constexpr int SLOT = NDT * 64 * 4;  // floats per slot
  static_assert(2 * SLOT * 4 <= TILE && 16 * DCH * 32 == SLOT, "both slots fit a tile; a slot holds 16 rows of D");
  f32x4* const give = reinterpret_cast<f32x4*>(area + (qh == 1 ? 0 : SLOT));
  const f32x4* const take = reinterpret_cast<const f32x4*>(area + (qh == 1 ? SLOT : 0));
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) give[dt * 64 + lane] = qh == 1 ? dk[dt] : dv[dt];
  __syncthreads();
  f32x4 acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc[dt] = take[dt * 64 + lane];  // all reads issued before the first use
  const float mul = qh == 0 ? p.scale : 1.f;                          // dK is scaled, dV not (x * 1 == x)
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[dt][i] = ((qh == 0 ? dk[dt][i] : dv[dt][i]) + acc[dt][i]) * mul;
  // accumulator element i of d tile dt: key 4 g + i, d = 16 dt + l16.  Transposed through this wave's slot
  // (read above, same wavefront, so the reads complete before these writes) into 16 [key][d] rows whose
  // 16-float groups are XOR-permuted by (row / 4) % 4 (conflict-free writes), then stored 8 d per lane.
  constexpr int DP = DCH * 32;
  constexpr int LPR = DCH * 4;  // lanes per row
  float* const tr = reinterpret_cast<float*>(const_cast<f32x4*>(take));
  auto phys = [](int r, int c) { return r * DP + (c ^ (16 * ((r >> 2) & 3))); };
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) tr[phys(4 * g4 + i, 16 * dt + l16)] = acc[dt][i];
  const uint64_t dst_base = qh == 0 ? p.dk : p.dv;
  const int64_t g_sb = qh == 0 ? p.k_sb : p.v_sb, g_sh = qh == 0 ? p.k_sh : p.v_sh, g_ss = qh == 0 ? p.k_ss : p.v_ss;
#pragma unroll
  for (int ps = 0; ps < 16 * LPR / 64; ++ps) {
    const int r = ps * (64 / LPR) + lane / LPR, c8 = (lane % LPR) * 8;
    const f32x4 x = *reinterpret_cast<const f32x4*>(tr + phys(r, c8));
    const f32x4 y = *reinterpret_cast<const f32x4*>(tr + phys(r, c8) + 4);
    const int64_t kk = kb * 64 + kg * 16 + r;
    if (kk < Sk)
      *reinterpret_cast<HK_G u32x4*>(gptr<uint16_t>(dst_base) + grad_row(p, b, hh, kk, Sk, g_sb, g_sh, g_ss) + c8) =
          u32x4{pack2<T>(x[0], x[1]), pack2<T>(x[2], x[3]), pack2<T>(y[0], y[1]), pack2<T>(y[2], y[3])};
  }
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
    const bool a4 = a.Sq % 4 == 0 && a.lse % 16 == 0 && a.delta % 16 == 0;
#define HK_DKDV(DCH)                                                                        \
  if (a4)                                                                                   \
    hipLaunchKernelGGL((attn_dkdv_dma<T, DCH, true>), g, dim3(512), 0, ctx.stream, a, nkb);  \
  else                                                                                      \
    hipLaunchKernelGGL((attn_dkdv_dma<T, DCH, false>), g, dim3(512), 0, ctx.stream, a, nkb);
    if (a.D == 128) {
      HK_DKDV(4)
    } else {
      HK_DKDV(2)
    }
#undef HK_DKDV
    return hrt::launch_ok(hipGetLastError(), ctx, "attn_dkdv_dma");
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
