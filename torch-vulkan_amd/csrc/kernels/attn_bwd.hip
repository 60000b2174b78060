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
  if (dkdv && (!ctx.check(a.dk, rows_k * a.D * elem, "dk") || !ctx.check(a.dv, rows_k * a.D * elem, "dv"))) return false;
  if (dq && !ctx.check(a.dq, rows_q * a.D * elem, "dq")) return false;
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
        const int64_t off = ((b * Sk + kk) * p.H + hh) * D + d;
        dK[off] = T::from_f32((dk[n][e] + xch[n * 32 + e]) * p.scale);
        dV[off] = T::from_f32(dv[n][e] + xch[n * 32 + 16 + e]);
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
      if (qq < Sq && d < D) dQ[((b * Sq + qq) * p.H + hh) * D + d] = T::from_f32((acc[n][e] + xch[n * 16 + e]) * p.scale);
    }
  }
}

template <typename T>
bool launch_dkdv(const void* pp, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_attn_args*>(pp);
  if (!attn_check(a, false, true, false, 2, ctx)) return false;
  const int nkb = (a.Sk + 63) / 64;
  const int64_t total = (int64_t)nkb * a.B * a.H;
  if (total > 0x7fffffffLL) return ctx.fail("grid too large");
  const int lm = !attn_vec_ok(a, true) ? LD_GATHER : (a.D % 32 == 0 ? LD_FULL : LD_VEC);
  const dim3 g((uint32_t)total);
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
  const int lm = !attn_vec_ok(a, true) ? LD_GATHER : (a.D % 32 == 0 ? LD_FULL : LD_VEC);
  const dim3 g((uint32_t)total);
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
