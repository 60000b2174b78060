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

// ---- fast path: D = 64 or 128, 16-byte aligned rows ---------------------------------------------------------
//
// Differences from the general kernel above:
//   * K and V stages go global -> LDS directly (global_load_lds_dwordx4): no staging registers and no
//     register transposes; V stays row-major and the V^T operand is read with ds_read_b64_tr_b16;
//   * 8 wavefronts, two per SIMD, so that one's softmax overlaps the other's MFMAs: wavefront w handles
//     query group w & 1 (32 rows) against keys 32 (w >> 1) .. +31 of every 128-key stage, with ~150 live
//     registers (the accumulators stay in one register file);
//   * the running max is only raised when a row max exceeds it by more than 2^8 (P values then stay
//     <= 256, far inside the bf16 / f16 / fp32 range), so the O rescale almost never runs;
//   * the four key quarters of a query group are merged at the end through LDS: wavefront (g, k) finishes
//     d block k of group g.
constexpr float kLazy = 8.f;  // log2 of the largest unnormalised P value

template <typename T, int DCH>
__global__ __launch_bounds__(512) void attn_fwd_dma(hrt_attn_args p, int nqb) {
  constexpr int NW = 8;               // wavefronts
  constexpr int NCH = DCH * 4;        // 16-byte chunks per row
  constexpr int ROWB = NCH * 16;      // bytes per LDS tile row
  constexpr int TILE = KST * ROWB;    // bytes per K or V stage
  constexpr int PIECE = 3 * 16 * 64;  // floats: the three partial blocks merged into one (group, d block)
  constexpr int PPT = TILE / (PIECE * 4);
  static_assert(PPT >= 1 && PPT * 4 >= 2 * DCH && PPT * PIECE * 4 + 2 * NW * 64 * 4 <= TILE && 32 * 36 <= PIECE, "merge layout");
  // Four separate LDS objects (not one array), so that the compiler can tell the reads of one buffer from
  // the in-flight copies into the other and does not wait for those copies before every LDS read.
  __shared__ __attribute__((aligned(1024))) uint8_t k0_raw[TILE], k1_raw[TILE], v0_raw[TILE], v1_raw[TILE];
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
  const int nst = (Sk + KST - 1) / KST;

  const int j0 = wave * (KST * NCH / 64 / NW);
  const DmaLanes klo = dma_lane_offsets<NCH>(kss, lane, j0), vlo = dma_lane_offsets<NCH>(vss, lane, j0);
  // The block's 64 Q rows go to V(1)'s buffer (free until stage 0 copies V(1)), copied once for the four
  // wavefronts that share them; then K(0), V(0) and K(1): K streams one stage ahead of V
  const uint32_t qss = (uint32_t)(p.q_ss * 2);
  const HK_G uint8_t* Qblk = reinterpret_cast<const HK_G uint8_t*>(gcptr<uint16_t>(p.q) + b * p.q_sb + hh * p.q_sh) +
                             qb * 64 * (int64_t)qss;
  const int64_t q = qb * 64 + g * 32 + ql;
  u32x4 qf[2 * DCH];  // Q^T operand fragments of this lane's query, read from LDS after the first barrier
  dma_tile<NCH, 64, NW>(Qblk, qss, (int)(Sq - qb * 64), V1, wave, lane,
                        dma_lane_offsets<NCH>(qss, lane, wave * (64 * NCH / 64 / NW)));
  dma_tile<NCH, KST, NW>(Kb, kss, Sk, K0, wave, lane, klo);
  dma_tile<NCH, KST, NW>(Vb, vss, Sk, V0, wave, lane, vlo);
  issue_order_fence();  // the first barrier counts on K(1) being the last copy issued
  if (nst > 1) dma_tile<NCH, KST, NW>(Kb + stage_origin<KST>(1, nst, Sk) * kss, kss, KST, K1, wave, lane, klo);

  // per-lane byte offsets of the A-operand fragments inside a tile
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

  f32x16 o[DCH];
#pragma unroll
  for (int n = 0; n < DCH; ++n) o[n] = zero16();
  float m = -INFINITY, l = 0.f;  // m in log2 units of the scaled logits
  const float sl2 = p.scale * kLog2e;

  // S^T = K Q^T for the wavefront's 32 keys of a stage (its K tile in Kt)
  auto qk = [&](const HK_L uint8_t* Kt) {
    u32x4 kfr[2 * DCH];
#pragma unroll
    for (int ks = 0; ks < 2 * DCH; ++ks) kfr[ks] = *reinterpret_cast<const HK_L u32x4*>(Kt + koff[ks]);
    f32x16 s = zero16();
#pragma unroll
    for (int ks = 0; ks < 2 * DCH; ++ks) s = Mfma32<T>::mac(kfr[ks], qf[ks], s);
    return s;
  };
  // Masking of stage st's tile (keys before the stage, processed already when the last stage's tile was
  // shifted back, and keys >= Sk), then the running max raised when the stage's row max exceeds it by more
  // than 2^kLazy (O and l rescaled; rare after the first stage).  Element 4j+r of s: tile row
  // kq*32 + 8j + 4h + r.
  auto mask_and_max = [&](f32x16& s, int st) {
    const int64_t key0 = (int64_t)st * KST;
    if (key0 + KST > Sk) {
      const int64_t kbase = (nst > 1 ? stage_origin<KST>(st, nst, Sk) : 0) + kq * 32 + 4 * hl;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t key = kbase + 8 * (e >> 2) + (e & 3);
        if (key < key0 || key >= Sk) s[e] = -INFINITY;
      }
    }
    float mx = fmaxf(s[0], s[1]);
#pragma unroll
    for (int e = 2; e < 16; ++e) mx = fmaxf(mx, s[e]);
    const float cand = halfswap_max(mx) * sl2;  // scale > 0: max commutes with the scaling
    const bool up = cand > m + kLazy;           // m = -inf: any finite row max
    if (__any(up)) {
      const float mn = up ? cand : m;
      const float alpha = up ? __builtin_amdgcn_exp2f(m - mn) : 1.f;  // m = -inf: 0, and o, l are 0
      l *= alpha;
#pragma unroll
      for (int n = 0; n < DCH; ++n)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[n][e] *= alpha;
      m = mn;
    }
  };
  // Software pipeline: iteration st computes S(st+1) on the matrix cores while the vector units turn S(st)
  // into P(st), with this iteration's copies (K(st+2), V(st+1)) placed one per MFMA (the three streams
  // interleaved by sched_group_barrier); then O += V(st)^T P(st); then S(st+1) is masked and the running
  // max updated.  K(st) sits in buffer st & 1 and is read one iteration before V(st); the copies go into
  // the buffers the previous iteration finished reading and the closing barrier makes them visible.
  // MODE 2: both copies (st + 2 < nst); 1: V(st+1) only (st + 2 == nst); 0: the last stage, or a single-
  // stage sequence: no copies and no next stage.  No copy is ever issued for a stage past the end: the
  // tiles are reused as scratch by the merge below, and a copy landing there late has been seen to corrupt
  // LDS written after the closing barrier.
  constexpr int IPW = KST * NCH / 64 / NW;  // copy instructions per tile and wavefront
  auto stage = [&](auto bc, auto mc, int st, f32x16& s, f32x16& sn) {
    constexpr int BUF = decltype(bc)::value;
    constexpr int MODE = decltype(mc)::value;
    constexpr bool COPY = MODE > 0;            // there is a next stage
    constexpr int NK = MODE == 2 ? IPW : 0;    // K copies of this stage
    const float nm = m == -INFINITY ? 0.f : -m;
    if constexpr (COPY) {
      // buffer resources over the stages' first rows: a copy then takes its row offset in a scalar register
      // and its lane offset as is, with no per-copy 64-bit address arithmetic
      const __amdgpu_buffer_rsrc_t krs = dma_rsrc(Kb + stage_origin<KST>(st + 2, nst, Sk) * kss);
      const __amdgpu_buffer_rsrc_t vrs = dma_rsrc(Vb + stage_origin<KST>(st + 1, nst, Sk) * vss);
      // S(st+1) with this iteration's copies placed after its MFMAs, one per MFMA, then P(st); the VALU
      // work of P(st) is interleaved with the MFMAs by sched_group_barrier
      const HK_L uint8_t* Kt = BUF ? K0 : K1;
      u32x4 kfr[2 * DCH];
#pragma unroll
      for (int ks = 0; ks < 2 * DCH; ++ks) kfr[ks] = *reinterpret_cast<const HK_L u32x4*>(Kt + koff[ks]);
      sn = zero16();
#pragma unroll
      for (int ks = 0; ks < 2 * DCH; ++ks) {
        sn = Mfma32<T>::mac(kfr[ks], qf[ks], sn);
        if (ks < NK) dma_tile_part_rs<NCH, KST, NW>(krs, kss, BUF ? K1 : K0, wave, klo, ks);
        else if (ks < NK + IPW) dma_tile_part_rs<NCH, KST, NW>(vrs, vss, BUF ? V0 : V1, wave, vlo, ks - NK);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float pv = __builtin_amdgcn_exp2f(fmaf(s[e], sl2, nm));  // exp2(-inf) = 0 for masked keys
        s[e] = pv;
        l += pv;
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * DCH, 0);
#pragma unroll
      for (int i = 0; i < 2 * DCH; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (i < NK + IPW) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 48 / (2 * DCH), 0);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float pv = __builtin_amdgcn_exp2f(fmaf(s[e], sl2, nm));
        s[e] = pv;
        l += pv;
      }
    }
    const HK_L uint8_t* Vt = BUF ? V1 : V0;
    const u32x4 pb0 = pack_slots<T>(s, 0, 1), pb1 = pack_slots<T>(s, 2, 3);
#pragma unroll
    for (int n = 0; n < DCH; ++n)
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const u32x2 lo = lds_tr4(Vt + voff[n][0] + kc * 16 * ROWB);
        const u32x2 hi = lds_tr4(Vt + voff[n][1] + kc * 16 * ROWB);
        o[n] = Mfma32<T>::mac(u32x4{lo.x, lo.y, hi.x, hi.y}, kc ? pb1 : pb0, o[n]);
      }
    if (COPY && st + 1 < nst) mask_and_max(sn, st + 1);
    __syncthreads();  // waits for this wave's copies, then for every wave
  };
  // Q, K(0), V(0) landed (K(1), issued last, may still be in flight)
  if (nst > 1) barrier_keep_vm<KST * NCH / 64 / NW>();
  else __syncthreads();
  // (rows past Sq hold copies of the last row; their results are never stored)
#pragma unroll
  for (int ks = 0; ks < 2 * DCH; ++ks)
    qf[ks] = *reinterpret_cast<const HK_L u32x4*>(V1 + tile_off<NCH>(g * 32 + ql, 2 * ks + hl));
  f32x16 sa = qk(K0), sb;
  mask_and_max(sa, 0);
  __syncthreads();  // every wave is done with K(0) and Q before they are copied over
  using M2 = std::integral_constant<int, 2>;
  using M1 = std::integral_constant<int, 1>;
  using M0 = std::integral_constant<int, 0>;
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  // Pairs of full-copy stages, then the last one to three stages peeled into straight-line code (the loop
  // body holds one variant per buffer, which keeps the D = 128 kernel within its 256 registers).
  int st = 0;
  for (; st + 3 < nst; st += 2) {
    stage(B0(), M2(), st, sa, sb);
    stage(B1(), M2(), st + 1, sb, sa);
  }
  if (st + 2 < nst) {
    stage(B0(), M2(), st, sa, sb);
    stage(B1(), M1(), st + 1, sb, sa);
    stage(B0(), M0(), st + 2, sa, sb);
  } else if (st + 1 < nst) {
    stage(B0(), M1(), st, sa, sb);
    stage(B1(), M0(), st + 1, sb, sa);
  } else {
    stage(B0(), M0(), st, sa, sb);
  }

  // ---- merge the four key quarters of each query group.  Piece (g, n) = d block n of group g, finished by
  // wavefront (g, k = n); its three incoming partial blocks live in tile (g*DCH + n) / PPT as
  // [source slot 0..2][16][64 lanes]; m and l of every wavefront follow the pieces of tile 0.
  auto tile_f = [&](int t) -> float* {
    return reinterpret_cast<float*>(t == 0 ? k0_raw : t == 1 ? k1_raw : t == 2 ? v0_raw : v1_raw);
  };
  float* xml = tile_f(0) + PPT * PIECE;  // [wave][m, l][64 lanes]
  xml[(wave * 2 + 0) * 64 + lane] = m;
  xml[(wave * 2 + 1) * 64 + lane] = halfswap_sum(l);
#pragma unroll
  for (int n = 0; n < DCH; ++n) {
    if (n == kq) continue;
    const int pc = g * DCH + n;
    // [4][64 lanes] 16-byte pieces: o[n][4 c .. 4 c + 3] of lane l at 4 c * 64 + 4 l (conflict-free)
    f32x4* dst = reinterpret_cast<f32x4*>(tile_f(pc / PPT) + (pc % PPT) * PIECE + ((kq - n - 1) & 3) * 16 * 64) + lane;
#pragma unroll
    for (int c = 0; c < 4; ++c) dst[c * 64] = f32x4{o[n][4 * c], o[n][4 * c + 1], o[n][4 * c + 2], o[n][4 * c + 3]};
  }
  __syncthreads();

  auto finish = [&](auto nc) {
    constexpr int N = decltype(nc)::value;
    float mw[4], aw[4];
    float mt = -INFINITY;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      mw[k] = xml[((2 * k + g) * 2 + 0) * 64 + lane];
      mt = fmaxf(mt, mw[k]);
    }
    float L = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      aw[k] = mw[k] == -INFINITY ? 0.f : exp2f(mw[k] - mt);
      L += aw[k] * xml[((2 * k + g) * 2 + 1) * 64 + lane];
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    if (N == 0 && hl == 0 && q < Sq) gptr<float>(p.lse)[bh * Sq + q] = L > 0.f ? (mt + log2f(L)) * kLn2 : -INFINITY;
    const int pc = g * DCH + N;
    float* const area = tile_f(pc / PPT) + (pc % PPT) * PIECE;  // read by this wavefront only
    f32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = o[N][e] * aw[N];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (k == N) continue;
      const f32x4* src = reinterpret_cast<const f32x4*>(area + ((k - N - 1) & 3) * 16 * 64) + lane;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const f32x4 x = src[c * 64];
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[4 * c + r] = fmaf(aw[k], x[r], acc[4 * c + r]);
      }
    }
    // transpose the 32 x 32 block through the same area (rows of 36 floats: conflict-free 16-byte writes),
    // so that 8 lanes store one query's 32 d contiguously (128 bytes of o32, 64 of o) instead of every lane
    // writing 16-byte pieces of 32 different rows
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<f32x4*>(area + ql * 36 + 8 * j + 4 * hl) =
          f32x4{acc[4 * j] * inv, acc[4 * j + 1] * inv, acc[4 * j + 2] * inv, acc[4 * j + 3] * inv};
    const int c4 = (lane & 7) * 4;
#pragma unroll
    for (int ps = 0; ps < 4; ++ps) {
      const int qq = ps * 8 + (lane >> 3);
      const f32x4 v = *reinterpret_cast<const f32x4*>(area + qq * 36 + c4);
      const int64_t qrow = qb * 64 + g * 32 + qq;
      if (qrow < Sq) {
        const int64_t off = ((b * Sq + qrow) * p.H + hh) * p.D + N * 32 + c4;
        const float v4[4] = {v[0], v[1], v[2], v[3]};
        *reinterpret_cast<HK_G u32x2*>(gptr<typename T::storage>(p.o) + off) = pack4<T>(v4);
        if (p.o32) *reinterpret_cast<HK_G f32x4*>(gptr<float>(p.o32) + off) = v;
      }
    }
  };
  switch (kq) {
    case 0: finish(std::integral_constant<int, 0>()); break;
    case 1: finish(std::integral_constant<int, 1>()); break;
    case 2: if constexpr (DCH > 2) finish(std::integral_constant<int, 2 % DCH>()); break;
    default: if constexpr (DCH > 3) finish(std::integral_constant<int, 3 % DCH>()); break;
  }
}

// The direct-to-LDS path needs D = 64 or 128, 16-byte aligned rows, and per-stage row offsets that fit
// the 32-bit lane offsets of the copies.
bool fwd_dma_ok(const hrt_attn_args& a) {
  if (!(a.D == 64 || a.D == 128) || !attn_vec_ok(a, false)) return false;
  const int64_t lim = (int64_t)1 << 31;
  return a.k_ss * 2 * (KST + 1) < lim && a.v_ss * 2 * (KST + 1) < lim && a.q_ss * 2 * (64 + 1) < lim;
}

template <typename T>
bool launch_fwd(const void* pp, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_attn_args*>(pp);
  if (!attn_check(a, true, false, false, 2, ctx)) return false;
  const int nqb = (a.Sq + 63) / 64;
  const int64_t total = (int64_t)nqb * a.B * a.H;
  if (total > 0x7fffffffLL) return ctx.fail("grid too large");
  const dim3 g((uint32_t)total);
  if (fwd_dma_ok(a)) {
    if (a.D == 128)
      hipLaunchKernelGGL((attn_fwd_dma<T, 4>), g, dim3(512), 0, ctx.stream, a, nqb);
    else
      hipLaunchKernelGGL((attn_fwd_dma<T, 2>), g, dim3(512), 0, ctx.stream, a, nqb);
    return hrt::launch_ok(hipGetLastError(), ctx, "attn_fwd_dma");
  }
  const int lm = !attn_vec_ok(a, false) ? LD_GATHER : (a.D % 32 == 0 ? LD_FULL : LD_VEC);
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
