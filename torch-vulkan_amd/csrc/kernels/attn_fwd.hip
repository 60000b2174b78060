// Flash-attention forward on gfx950 matrix cores: "attn_fwd_mfma_{bf16,f16}".
//
// Same algorithm and outputs as the reference's cooperative-matrix kernel
// (vkrt/shaders/attn_coop.comp.in:158-211): logits kept in fp32, online softmax, P rounded to the input
// dtype before P V, out rounded once, lse = max + log(sum) in fp32, and the unrounded fp32 O written for
// the backward's delta.  Mapped onto CDNA4:
//   * a workgroup owns 64 query rows of one (b, h) and streams K/V in stages of 128 keys through
//     double-buffered LDS (K as [key][d], V transposed to [d][key] by 8x8 register transposes while
//     staging), one barrier per stage, next stage's global loads in flight during the MFMAs;
//   * wavefront w handles query rows 32 (w & 1) .. +31 against keys 64 (w >> 1) .. +63 of every stage,
//     so all four SIMDs work on a 64-row block (1024 wavefronts for S=1024, H=16 on 256 CUs) while each
//     LDS fragment feeds a 32x32x16 MFMA; the two key halves are merged (max/sum/O rescale) at the end;
//   * S^T = K Q^T puts one query per lane, so max/sum need one lane swap, the alpha rescale of the
//     O^T = V^T P^T accumulators is per lane, and P^T goes from the S^T accumulators straight into the
//     next MFMA's operand registers (no LDS round trip for S or P);
//   * exp2 with log2(e) folded into the scale;  Q stays in registers for the whole key loop;
//   * workgroups are mapped so that all query blocks of a head run on one XCD (K/V of a head read once
//     into that XCD's L2).
// Ragged Sq / Sk and any D <= 128 are handled by masking (no padded copies).
#include "../hrt/registry.h"
#include "attn_common.h"

namespace hk {

bool attn_check(const hrt_attn_args& a, bool fwd, bool dkdv, bool dq, uint64_t elem, hrt::LaunchCtx& ctx);
bool attn_vec_ok(const hrt_attn_args& a, bool with_dout);

namespace {

constexpr int KST = 128;  // keys per LDS stage

template <typename T, int DCH, int LM>
__global__ __launch_bounds__(256) void attn_fwd_mfma(hrt_attn_args p, int nqb) {
  constexpr int DP = DCH * 32;
  constexpr int NCH = DP / 8;   // 16-byte chunks per K row
  constexpr int KLD = DP + 8;   // K rows [key][d] (chunks swizzled)
  constexpr int VLD = KST + 8;  // V^T rows [d][key]
  constexpr int STAGE = KST * KLD + DP * VLD;
  constexpr int RB = KST / 8;       // row blocks per stage
  constexpr int NB = RB * NCH;      // 8x8 blocks per tensor per stage
  constexpr int BPT = (2 * NB + 255) / 256;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * STAGE];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int qg = wave & 1, kh = wave >> 1;
  const int ql = lane & 31, hl = lane >> 5;
  const int64_t total = (int64_t)nqb * p.B * p.H;
  int64_t bh, qb;
  xcd_map(blockIdx.x, total, nqb, bh, qb);
  const int64_t b = bh / p.H, hh = bh % p.H;
  const int D = p.D, Sq = p.Sq, Sk = p.Sk;

  const HK_G uint16_t* Q = gcptr<uint16_t>(p.q) + b * p.q_sb + hh * p.q_sh;
  const HK_G uint16_t* K = gcptr<uint16_t>(p.k) + b * p.k_sb + hh * p.k_sh;
  const HK_G uint16_t* V = gcptr<uint16_t>(p.v) + b * p.v_sb + hh * p.v_sh;

  // Q^T operand fragments for this lane's query, 16 d per fragment
  const int64_t q = qb * 64 + qg * 32 + ql;
  u32x4 qf[2 * DCH];
#pragma unroll
  for (int ks = 0; ks < 2 * DCH; ++ks)
    qf[ks] = q < Sq ? load_row8<LM != LD_GATHER>(Q + q * p.q_ss, ks * 16 + 8 * hl, D) : u32x4{0, 0, 0, 0};

  Block8 blk[BPT];
  auto load_stage = [&](int64_t key0) {
    const bool full = key0 + KST <= Sk;
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      const int bi = threadIdx.x + i * 256;
      if (bi < 2 * NB) {
        const int t = bi < NB ? bi : bi - NB;
        const int rb = t % RB, dc = t / RB;
        if (bi < NB)
          blk[i].template load<LM>(K, p.k_ss, key0 + rb * 8, Sk, dc * 8, D, full);
        else
          blk[i].template load<LM>(V, p.v_ss, key0 + rb * 8, Sk, dc * 8, D, full);
      }
    }
  };
  auto store_stage = [&](uint16_t* st) {
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      const int bi = threadIdx.x + i * 256;
      if (bi < 2 * NB) {
        const int t = bi < NB ? bi : bi - NB;
        const int rb = t % RB, dc = t / RB;
        if (bi < NB)
          blk[i].template store_rows<NCH>(st, KLD, rb * 8, dc * 8);
        else
          blk[i].store_cols(st + KST * KLD, VLD, rb * 8, dc * 8);
      }
    }
  };

  f32x16 o[DCH];
#pragma unroll
  for (int n = 0; n < DCH; ++n) o[n] = zero16();
  float m = -INFINITY, l = 0.f;  // m in log2 units of the scaled logits
  const float sl2 = p.scale * kLog2e;

  const int nst = (Sk + KST - 1) / KST;
  load_stage(0);
  store_stage(lds);
  __syncthreads();
  const int kb = kh * 64;
  for (int st = 0; st < nst; ++st) {
    const bool more = st + 1 < nst;
    if (more) load_stage((int64_t)(st + 1) * KST);
    const uint16_t* Kl = lds + (st & 1) * STAGE;
    const uint16_t* Vt = Kl + KST * KLD;

    f32x16 s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      s[kt] = zero16();
      const int row = kb + kt * 32 + ql;
#pragma unroll
      for (int ks = 0; ks < 2 * DCH; ++ks) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(Kl + row * KLD + Block8::swz_col<NCH>(row, ks * 16 + 8 * hl));
        s[kt] = Mfma32<T>::mac(a, qf[ks], s[kt]);
      }
    }
    // online softmax for this lane's query over its 32 keys of the stage (the other 32: lane ^ 32)
    if (st * KST + KST > Sk) {  // ragged last stage: keys >= Sk do not exist
      const int key_base = st * KST + kb + 4 * hl;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (key_base + kt * 32 + 8 * (e >> 2) + (e & 3) >= Sk) s[kt][e] = -INFINITY;
    }
    float mx = fmaxf(s[0][0], s[0][1]);
#pragma unroll
    for (int e = 2; e < 16; ++e) mx = fmaxf(mx, s[0][e]);
#pragma unroll
    for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[1][e]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m, mx * sl2);  // scale > 0: max commutes with the scaling
    if (__any(mn != m)) {
      const float alpha = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mn);
      l *= alpha;
#pragma unroll
      for (int n = 0; n < DCH; ++n)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[n][e] *= alpha;
      m = mn;
    }
    const float nm = mn == -INFINITY ? 0.f : -mn;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float pv = __builtin_amdgcn_exp2f(fmaf(s[kt][e], sl2, nm));  // exp2(-inf) = 0 for masked keys
        s[kt][e] = pv;
        l += pv;
      }
    u32x4 pb[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) pb[c] = pack_slots<T>(s[c >> 1], 2 * (c & 1), 2 * (c & 1) + 1);
#pragma unroll
    for (int n = 0; n < DCH; ++n)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4 a = lds_pair64(Vt + (n * 32 + ql) * VLD + kb + c * 16 + 4 * hl);
        o[n] = Mfma32<T>::mac(a, pb[c], o[n]);
      }
    if (more) store_stage(lds + ((st + 1) & 1) * STAGE);
    __syncthreads();
  }

  // merge the two key halves (waves 2,3 -> waves 0,1) through LDS
  float* xch = reinterpret_cast<float*>(lds);
  constexpr int XS = 2 + 16 * DCH;
  float* mine = xch + (qg * 64 + lane) * XS;
  if (kh == 1) {
    mine[0] = m;
    mine[1] = l;
#pragma unroll
    for (int n = 0; n < DCH; ++n)
#pragma unroll
      for (int e = 0; e < 16; ++e) mine[2 + n * 16 + e] = o[n][e];
  }
  __syncthreads();
  if (kh == 1) return;
  const float m2 = mine[0], l2 = mine[1];
  const float mt = fmaxf(m, m2);
  const float a1 = m == -INFINITY ? 0.f : exp2f(m - mt);
  const float a2 = m2 == -INFINITY ? 0.f : exp2f(m2 - mt);
  l = l * a1 + l2 * a2;
  const float lrow = l + __shfl_xor(l, 32, 64);
  const float inv = lrow > 0.f ? 1.f / lrow : 0.f;
  if (q >= Sq) return;
  if (hl == 0) gptr<float>(p.lse)[bh * Sq + q] = lrow > 0.f ? (mt + log2f(lrow)) * kLn2 : -INFINITY;
  HK_G typename T::storage* out = gptr<typename T::storage>(p.o) + ((b * Sq + q) * p.H + hh) * D;
  HK_G float* o32 = p.o32 ? gptr<float>(p.o32) + ((b * Sq + q) * p.H + hh) * D : nullptr;
  const bool vec4 = (D % 4) == 0;
#pragma unroll
  for (int n = 0; n < DCH; ++n)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = n * 32 + 8 * j + 4 * hl;
      if (d >= D) continue;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = (o[n][4 * j + r] * a1 + mine[2 + n * 16 + 4 * j + r] * a2) * inv;
      if (vec4) {
        *reinterpret_cast<HK_G u32x2*>(out + d) = u32x2{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
        if (o32) *reinterpret_cast<HK_G f32x4*>(o32 + d) = f32x4{v[0], v[1], v[2], v[3]};
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (d + r < D) {
            out[d + r] = T::from_f32(v[r]);
            if (o32) o32[d + r] = v[r];
          }
      }
    }
}

template <typename T>
bool launch_fwd(const void* pp, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_attn_args*>(pp);
  if (!attn_check(a, true, false, false, 2, ctx)) return false;
  const int nqb = (a.Sq + 63) / 64;
  const int64_t total = (int64_t)nqb * a.B * a.H;
  if (total > 0x7fffffffLL) return ctx.fail("grid too large");
  const int lm = !attn_vec_ok(a, false) ? LD_GATHER : (a.D % 32 == 0 ? LD_FULL : LD_VEC);
  const dim3 g((uint32_t)total);
#define HK_FWD(DCH)                                                                                      \
  if (lm == LD_FULL)                                                                                     \
    hipLaunchKernelGGL((attn_fwd_mfma<T, DCH, LD_FULL>), g, dim3(256), 0, ctx.stream, a, nqb);          \
  else if (lm == LD_VEC)                                                                                 \
    hipLaunchKernelGGL((attn_fwd_mfma<T, DCH, LD_VEC>), g, dim3(256), 0, ctx.stream, a, nqb);           \
  else                                                                                                   \
    hipLaunchKernelGGL((attn_fwd_mfma<T, DCH, LD_GATHER>), g, dim3(256), 0, ctx.stream, a, nqb);
  switch ((a.D + 31) / 32) {
    case 1: HK_FWD(1) break;
    case 2: HK_FWD(2) break;
    case 3: HK_FWD(3) break;
    default: HK_FWD(4) break;
  }
#undef HK_FWD
  return hrt::launch_ok(hipGetLastError(), ctx, "attn_fwd_mfma");
}

HRT_REGISTER("attn_fwd_mfma_bf16", hrt_attn_args, launch_fwd<BF16>);
HRT_REGISTER("attn_fwd_mfma_f16", hrt_attn_args, launch_fwd<F16>);

}  // namespace
}  // namespace hk
