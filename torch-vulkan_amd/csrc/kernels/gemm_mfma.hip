// Matrix-core GEMM "mm_mfma_{bf16,f16}" for gfx950:  c = alpha * a @ b + beta * bias, fp32 accumulate.
//
// Same contract as the reference's cooperative-matrix kernel (vkrt/shaders/mm_coop.comp.in:96-208):
// arbitrary strides (transposes and slices read in place), batched, bias broadcast through strides,
// epilogue alpha*acc + beta*bias with one rounding.  Built for CDNA4 instead of translated:
//   * v_mfma_f32_16x16x32 on 64-wide wavefronts; each wavefront owns a (BM/WM) x (BN/WN) sub-tile held
//     in accumulator registers for the whole K loop;
//   * A and B tiles are staged through LDS with K contiguous (+8 halves of row padding against bank
//     conflicts), double-buffered, one barrier per K step; the next tile's global loads are issued
//     before the current tile's MFMAs so HBM/L2 latency overlaps the math;
//   * global loads are 128-bit along the operand's contiguous axis: a K-contiguous operand goes straight
//     to its LDS row, an M-/N-contiguous one (W for dX = dY W, B of a row-major X @ B) is loaded as 8x8
//     blocks and transposed in registers before the 128-bit LDS store — no copies, no strided LDS writes;
//   * odd shapes / strides / alignments use a per-element gather loader on the same MMA core;
//   * tiles are numbered N-fastest so the default round-robin placement of workgroups over the 8 XCDs
//     gives each XCD a band of N-panels that it reads once into its own L2.
#include <cstring>
#include <type_traits>
#include <utility>

#include "../hrt/registry.h"
#include "gemm_skinny.h"
#include "lds_stage.h"

namespace hk {

bool mm_check_operands(const hrt_mm_args& a, uint64_t elem, hrt::LaunchCtx& ctx);

namespace {

// f(std::integral_constant<int, I>()) for I = 0 .. N - 1, unrolled at compile time (ring buffers are separate
// LDS objects picked by a compile-time index)
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>()), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>());
}

enum LoadMode { KVEC = 0, MNVEC = 1, GATHER = 2 };

constexpr int BK = 64;       // K per LDS stage
constexpr int LDK = BK + 8;  // padded LDS row (halves)

template <int ROWS, int MODE>
struct TileLoader {
  // The ROWS x BK tile of an operand whose element (r, k) is at p[r * s_r + k * s_k]; rows >= nrows and
  // k >= nk read as zero.  load() fills registers, store() writes LDS as [ROWS][LDK] with K contiguous.
  static constexpr int CHUNKS = ROWS * BK / 8;  // 16-byte chunks per tile
  static constexpr int PER_THREAD_V = CHUNKS / 256 > 0 ? CHUNKS / 256 : 1;
  static constexpr int BLOCKS = (ROWS / 8) * (BK / 8);  // 8x8 blocks (MNVEC)
  static constexpr int PER_THREAD_T = BLOCKS / 256 > 0 ? BLOCKS / 256 : 1;
  static constexpr int ELEMS = ROWS * BK / 256;  // GATHER
  static_assert(CHUNKS % 256 == 0 || CHUNKS < 256, "tile/threads mismatch");

  const HK_G uint16_t* p;
  int64_t s_r, s_k, r0, nrows, nk;
  u32x4 v[MODE == KVEC ? PER_THREAD_V : (MODE == MNVEC ? 8 * PER_THREAD_T : 1)];
  uint16_t g[MODE == GATHER ? ELEMS : 1];

  __device__ __forceinline__ void load(int64_t k0) {
    const int t = threadIdx.x;
    if constexpr (MODE == KVEC) {
#pragma unroll
      for (int i = 0; i < PER_THREAD_V; ++i) {
        const int c = t + i * 256;
        const int r = c / (BK / 8), kc = c % (BK / 8);
        const int64_t gr = r0 + r, gk = k0 + kc * 8;
        if (c < CHUNKS && gr < nrows && gk < nk)
          v[i] = *reinterpret_cast<const HK_G u32x4*>(p + gr * s_r + gk);
        else
          v[i] = u32x4{0, 0, 0, 0};
      }
    } else if constexpr (MODE == MNVEC) {
#pragma unroll
      for (int i = 0; i < PER_THREAD_T; ++i) {
        const int b = t + i * 256;
        const int rb = b % (ROWS / 8), kb = b / (ROWS / 8);
        const int64_t gr = r0 + rb * 8;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int64_t gk = k0 + kb * 8 + j;
          if (b < BLOCKS && gr < nrows && gk < nk)
            v[i * 8 + j] = *reinterpret_cast<const HK_G u32x4*>(p + gk * s_k + gr);
          else
            v[i * 8 + j] = u32x4{0, 0, 0, 0};
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < ELEMS; ++i) {
        const int e = t + i * 256;
        const int r = e / BK, k = e % BK;
        const int64_t gr = r0 + r, gk = k0 + k;
        g[i] = (gr < nrows && gk < nk) ? p[gr * s_r + gk * s_k] : (uint16_t)0;
      }
    }
  }

  __device__ __forceinline__ void store(uint16_t* lds) const {
    const int t = threadIdx.x;
    if constexpr (MODE == KVEC) {
#pragma unroll
      for (int i = 0; i < PER_THREAD_V; ++i) {
        const int c = t + i * 256;
        if (c < CHUNKS) {
          const int r = c / (BK / 8), kc = c % (BK / 8);
          *reinterpret_cast<u32x4*>(lds + r * LDK + kc * 8) = v[i];
        }
      }
    } else if constexpr (MODE == MNVEC) {
#pragma unroll
      for (int i = 0; i < PER_THREAD_T; ++i) {
        const int b = t + i * 256;
        if (b < BLOCKS) {
          const int rb = b % (ROWS / 8), kb = b / (ROWS / 8);
          u32x4 o[8];
          transpose8x8(&v[i * 8], o);
#pragma unroll
          for (int m = 0; m < 8; ++m) *reinterpret_cast<u32x4*>(lds + (rb * 8 + m) * LDK + kb * 8) = o[m];
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < ELEMS; ++i) {
        const int e = t + i * 256;
        lds[(e / BK) * LDK + (e % BK)] = g[i];
      }
    }
  }
};

// B tile of the fused int8 linear: rows n of the int8 weight q [N, K] (contiguous), dequantized while
// staging: value = round_T(float(q[n, k]) * float(scale[n, k / 64])) — bit-identical to dq8 — so the
// matrix cores see exactly the weights dequant_int8 would have produced, without them touching HBM.
template <int ROWS, typename T>
struct Dq8Loader {
  static constexpr int CHUNKS = ROWS * BK / 8;  // 8 int8 per chunk
  static constexpr int PT = CHUNKS / 256 > 0 ? CHUNKS / 256 : 1;
  const HK_G int8_t* q;
  const HK_G uint16_t* scale;
  int64_t K, nblocks, r0, nrows;
  u32x2 v[PT];
  float sc[PT];

  __device__ __forceinline__ void load(int64_t k0) {
#pragma unroll
    for (int i = 0; i < PT; ++i) {
      const int c = threadIdx.x + i * 256;
      const int r = c / (BK / 8), kc = c % (BK / 8);
      const int64_t gr = r0 + r, gk = k0 + kc * 8;
      if (c < CHUNKS && gr < nrows && gk < K) {
        v[i] = *reinterpret_cast<const HK_G u32x2*>(q + gr * K + gk);
        sc[i] = bf16_bits_to_f32(scale[gr * nblocks + (gk >> 6)]);
      } else {
        v[i] = u32x2{0, 0};
        sc[i] = 0.f;
      }
    }
  }
  __device__ __forceinline__ void store(uint16_t* lds) const {
#pragma unroll
    for (int i = 0; i < PT; ++i) {
      const int c = threadIdx.x + i * 256;
      if (c < CHUNKS) {
        const int r = c / (BK / 8), kc = c % (BK / 8);
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = (float)(int8_t)(((e < 4 ? v[i].x : v[i].y) >> (8 * (e & 3))) & 0xffu) * sc[i];
        *reinterpret_cast<u32x4*>(lds + r * LDK + kc * 8) = pack8<T>(f);
      }
    }
  }
};

// Main loop shared by the GEMM kernels: K in steps of BK through double-buffered LDS; acc[i][j] is the
// wavefront's (i, j) 16x16 accumulator tile.
template <typename T, int BM, int BN, int WM, int WN, class LA, class LB>
__device__ __forceinline__ void gemm_mainloop(LA& la, LB& lb, int64_t K, uint16_t (*lds)[(BM + BN) * LDK],
                                              f32x4 (&acc)[BM / WM / 16][BN / WN / 16]) {
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 16, TN = WTN / 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int64_t nk = (K + BK - 1) / BK;
  la.load(0);
  lb.load(0);
  la.store(lds[0]);
  lb.store(lds[0] + BM * LDK);
  __syncthreads();
  const int fr = lane & 15, fk = (lane >> 4) * 8;
  for (int64_t kt = 0; kt < nk; ++kt) {
    const bool more = kt + 1 < nk;
    if (more) {
      la.load((kt + 1) * BK);
      lb.load((kt + 1) * BK);
    }
    const uint16_t* As = lds[kt & 1];
    const uint16_t* Bs = As + BM * LDK;
#pragma unroll
    for (int ks = 0; ks < BK; ks += 32) {
      u32x4 af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const u32x4*>(As + (wm * WTM + i * 16 + fr) * LDK + ks + fk);
#pragma unroll
      for (int j = 0; j < TN; ++j) bfr[j] = *reinterpret_cast<const u32x4*>(Bs + (wn * WTN + j * 16 + fr) * LDK + ks + fk);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = Mfma<T>::mac(af[i], bfr[j], acc[i][j]);
    }
    if (more) {
      uint16_t* nxt = lds[(kt + 1) & 1];
      la.store(nxt);
      lb.store(nxt + BM * LDK);
    }
    __syncthreads();
  }
}

// Epilogue: c = alpha * acc + beta * bias, one rounding; lane holds rows 4*(lane/16)+r, column lane%16
// of every 16x16 tile.
// Epilogue: alpha * acc + beta * bias, one rounding (f32out: C is fp32 and takes the unrounded value, the
// split-K partials of HRT_MM_F32_OUT).  Each wavefront's WTM x WTN block goes through LDS in 32-column
// chunks so that a lane writes 8 consecutive outputs of a row (one 16-byte store when C's row is contiguous
// and aligned) instead of 2-byte stores scattered over 4 rows.
constexpr int EPI_RS = 36;  // floats per LDS row of a chunk (conflict-free writes, 16-byte aligned rows)
template <typename T, int BM, int BN, int WM, int WN>
__device__ __forceinline__ void gemm_epilogue(const f32x4 (&acc)[BM / WM / 16][BN / WN / 16], HK_G uint16_t* C, int64_t c_sm,
                                              int64_t c_sn, const HK_G uint16_t* bias, int64_t bias_sm, int64_t bias_sn,
                                              bool has_bias, float alpha, float beta, int64_t m0, int64_t n0, int64_t M,
                                              int64_t N, uint16_t (*lds)[(BM + BN) * LDK], bool f32out = false) {
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 16, TN = WTN / 16;
  static_assert(WTN % 32 == 0 && WM * WN * WTM * EPI_RS * 4 <= 2 * (BM + BN) * LDK * 2, "epilogue chunks fit the tiles");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  float* const area = reinterpret_cast<float*>(&lds[0][0]) + wave * WTM * EPI_RS;
  __syncthreads();  // every wavefront is done with the K loop's tiles
#pragma unroll
  for (int jc = 0; jc < WTN / 32; ++jc) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          area[(i * 16 + (lane >> 4) * 4 + r) * EPI_RS + jj * 16 + (lane & 15)] = acc[i][2 * jc + jj][r];
    // WTM rows x 4 pieces of 8 columns; LDS reads and writes of one wavefront complete in order
#pragma unroll
    for (int ps = 0; ps < WTM / 16; ++ps) {
      const int q = ps * 64 + lane, row = q >> 2, c8 = (q & 3) * 8;
      const f32x4 x = *reinterpret_cast<const f32x4*>(area + row * EPI_RS + c8);
      const f32x4 y = *reinterpret_cast<const f32x4*>(area + row * EPI_RS + c8 + 4);
      const int64_t gm = m0 + wm * WTM + row, gn = n0 + wn * WTN + jc * 32 + c8;
      if (gm >= M || gn >= N) continue;
      float o[8] = {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
      const bool full = gn + 8 <= N;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] *= alpha;
      if (has_bias) {
        const HK_G uint16_t* bp = bias + gm * bias_sm + gn * bias_sn;
        if (full && bias_sn == 1 && ((uint64_t)bp & 15) == 0) {  // one 16-byte load of the bias row
          const u32x4 bv = *reinterpret_cast<const HK_G u32x4*>(bp);
#pragma unroll
          for (int w = 0; w < 4; ++w) o[2 * w] += beta * lo16<T>(bv[w]), o[2 * w + 1] += beta * hi16<T>(bv[w]);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (full || gn + e < N) o[e] += beta * T::to_f32(bp[e * bias_sn]);
        }
      }
      if (f32out) {
        HK_G float* c = reinterpret_cast<HK_G float*>(C) + gm * c_sm + gn * c_sn;
        if (full && c_sn == 1 && ((uint64_t)c & 15) == 0) {
          *reinterpret_cast<HK_G f32x4*>(c) = f32x4{o[0], o[1], o[2], o[3]};
          *reinterpret_cast<HK_G f32x4*>(c + 4) = f32x4{o[4], o[5], o[6], o[7]};
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (gn + e < N) c[e * c_sn] = o[e];
        }
      } else {
        HK_G uint16_t* c = C + gm * c_sm + gn * c_sn;
        if (full && c_sn == 1 && ((uint64_t)c & 15) == 0) {
          *reinterpret_cast<HK_G u32x4*>(c) = pack8<T>(o);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (gn + e < N) c[e * c_sn] = T::from_f32(o[e]);
        }
      }
    }
  }
}

template <typename T, int BM, int BN, int WM, int WN, int AMODE, int BMODE>
__global__ __launch_bounds__(256) void mm_mfma(hrt_mm_args p, int64_t tiles_m, int64_t tiles_n) {
  static_assert(WM * WN == 4, "four wavefronts");
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][(BM + BN) * LDK];
  const int64_t tile = blockIdx.x;
  const int64_t tn = tile % tiles_n, tm = (tile / tiles_n) % tiles_m, bz = tile / (tiles_n * tiles_m);
  const int64_t m0 = tm * BM, n0 = tn * BN;
  // A as rows m with K; B as rows n with K.
  TileLoader<BM, AMODE> la;
  la.p = gcptr<uint16_t>(p.a) + bz * p.a_sb;
  la.s_r = p.a_sm, la.s_k = p.a_sk, la.r0 = m0, la.nrows = p.M, la.nk = p.K;
  TileLoader<BN, BMODE> lb;
  lb.p = gcptr<uint16_t>(p.b) + bz * p.b_sb;
  lb.s_r = p.b_sn, lb.s_k = p.b_sk, lb.r0 = n0, lb.nrows = p.N, lb.nk = p.K;
  f32x4 acc[BM / WM / 16][BN / WN / 16];
  gemm_mainloop<T, BM, BN, WM, WN>(la, lb, p.K, lds, acc);
  const bool f32out = (p.flags & HRT_MM_F32_OUT) != 0;
  HK_G uint16_t* const C = f32out ? reinterpret_cast<HK_G uint16_t*>(gptr<float>(p.c) + bz * p.c_sb)
                                  : gptr<uint16_t>(p.c) + bz * p.c_sb;
  gemm_epilogue<T, BM, BN, WM, WN>(acc, C, p.c_sm, p.c_sn, gcptr<uint16_t>(p.bias) + bz * p.bias_sb, p.bias_sm,
                                   p.bias_sn, p.has_bias != 0, p.alpha, p.beta, m0, n0, p.M, p.N, lds, f32out);
}

template <typename T, int BM, int BN, int WM, int WN, int AMODE>
__global__ __launch_bounds__(256) void mm_dq8_mfma(hrt_mm_dq8_args p, int64_t tiles_m, int64_t tiles_n) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][(BM + BN) * LDK];
  const int64_t tile = blockIdx.x;
  const int64_t tn = tile % tiles_n, tm = tile / tiles_n;
  const int64_t m0 = tm * BM, n0 = tn * BN;
  TileLoader<BM, AMODE> la;
  la.p = gcptr<uint16_t>(p.x);
  la.s_r = p.x_sm, la.s_k = p.x_sk, la.r0 = m0, la.nrows = p.M, la.nk = p.K;
  Dq8Loader<BN, T> lb;
  lb.q = gcptr<int8_t>(p.q);
  lb.scale = gcptr<uint16_t>(p.scale);
  lb.K = p.K, lb.nblocks = p.nblocks, lb.r0 = n0, lb.nrows = p.N;
  f32x4 acc[BM / WM / 16][BN / WN / 16];
  gemm_mainloop<T, BM, BN, WM, WN>(la, lb, p.K, lds, acc);
  gemm_epilogue<T, BM, BN, WM, WN>(acc, gptr<uint16_t>(p.y), p.N, 1, gcptr<uint16_t>(p.bias), 0,
                                   1, p.has_bias != 0, p.alpha, p.beta, m0, n0, p.M, p.N, lds);
}

// ---- fast path: tile-aligned GEMMs, operands copied global -> LDS directly ------------------------------------
//
// C tile BM x BN per workgroup of (BM / WM) x (BN / WN) wavefronts; each wavefront owns a WM x WN sub-tile as
// (WM / 32) x (WN / 32) v_mfma_f32_32x32x16 accumulators.  Shapes: 128 x 256 or 256 x 128 tiles of 64 x 64
// sub-tiles (8 wavefronts, two per SIMD) for problems that fill the GPU with them, else 64 x 64 tiles of
// 32 x 32 sub-tiles (4 wavefronts, several workgroups per CU), so that a 1024 x 1024 product still spreads
// over 256 workgroups (measured faster than 128 x 128 tiles of 64 x 64 at 1024 x {1024, 2048, 8192} x N).
// K advances in steps of 64
// through a ring of RING LDS buffers (three; two or up to six for the plain GEMM) filled by
// global_load_lds_dwordx4 copies of the operands' raw rows: the copies of step kt + RING - 1 are spread over
// the MFMAs of step kt, so a copy has RING - 1 steps to land (one step of compute is shorter than the L2
// latency plus the transfer of a 48 KiB step), one barrier per step.  An operand whose K axis is contiguous (A [M][K],
// or B given as [N][K]) is staged as [row][k] and read with 128-bit row reads; an operand contiguous along
// M or N (A given as [K][M], B as [K][N]) is staged as [k][row] and read with ds_read_b64_tr_b16 column
// reads, so all four layouts need no register transposes.  Epilogue: alpha * acc + beta * bias in fp32,
// one rounding, transposed through LDS so that C is written as 16-byte row pieces.
//
// DQ8 (the fused int8 linear y = x deq(q)^T + bias): B is int8 q [N][K] with one bf16 scale per row and
// 64-column block, so a K step covers exactly one scale block.  The raw int8 rows of step kt + 3 are copied
// global -> LDS during step kt (a ring of three int8 tiles: a copy still has two steps to land before it
// is converted); during step kt every thread converts 8-element pieces of step kt + 1's tile to
// deq = round(float(q) * float(scale)) in the input dtype (the exact product, one RNE rounding,
// as the standalone dequant) and writes it into the swizzled B tile of step kt + 1 (two such tiles), which
// the MFMAs then read exactly as a copied B tile.  The step barrier also waits for these LDS writes.
constexpr int GBK = 64;

template <typename T, int BM, int BN, int WM, int WN, bool ATR, bool BTR, bool DQ8, int RING = 3, bool F32OUT = false>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void mm_dma(hrt_mm_args p, int tiles_m, int tiles_n, int xbm,
                                                                   uint64_t dq_scale, int64_t dq_nblocks) {
  static_assert(!DQ8 || !BTR, "int8 B is staged as [n][k] rows");
  static_assert(!(DQ8 && F32OUT), "the fused int8 linear writes its own dtype");
  static_assert(RING == 3 || (RING >= 2 && RING <= 6 && !DQ8), "three-buffer ring, or 2 to 6 buffers for the plain GEMM");
  constexpr int WNN = BN / WN;         // wavefronts along n
  constexpr int NW = (BM / WM) * WNN;  // wavefronts
  constexpr int FM = WM / 32, FN = WN / 32;  // 32 x 32 accumulators per wavefront along m, n
  static_assert(BM % WM == 0 && BN % WN == 0 && WM % 32 == 0 && WN % 32 == 0 && NW >= 4, "tile shape");
  constexpr int A_ROWS = ATR ? GBK : BM, A_NCH = ATR ? BM / 8 : GBK / 8;
  constexpr int B_ROWS = BTR ? GBK : BN, B_NCH = BTR ? BN / 8 : GBK / 8;
  constexpr int A_ROWB = A_NCH * 16, B_ROWB = B_NCH * 16;
  constexpr int A_TILE = A_ROWS * A_ROWB, B_TILE = B_ROWS * B_ROWB;
  constexpr int IPA = A_ROWS * A_NCH / 64 / NW, IPB = B_ROWS * B_NCH / 64 / NW;  // copies per wavefront
  static_assert(IPA >= 1 && IPB >= 1 && IPA * NW * 64 == A_ROWS * A_NCH && IPB * NW * 64 == B_ROWS * B_NCH &&
                    IPA + IPB <= 16, "copy split");
  constexpr int RS = 40;                  // epilogue row stride (floats): conflict-free half-wave writes
  constexpr int AREA = WM * RS * 4;       // one wavefront's epilogue area (bytes)
  constexpr int PA = A_TILE / AREA, PB = B_TILE / AREA;  // epilogue areas per A / B tile
  static_assert(2 * PA + 2 * PB >= NW, "epilogue areas fit the tiles");
  // DQ8: int8 tiles of BN rows x 64 bytes (4 chunks, unswizzled); each thread converts CPT 8-element pieces
  // per step, piece c = row c / 8, bf16 chunk c % 8
  constexpr int Q_TILE = DQ8 ? BN * GBK : 16, IPQ = DQ8 ? BN * 4 / 64 / NW : 1, CPT = DQ8 ? BN * 8 / (NW * 64) : 1;
  static_assert(!DQ8 || (IPQ >= 1 && IPA + IPQ <= 16 && CPT * NW * 64 == BN * 8), "int8 copy split");
  // separate LDS objects per buffer, so that reads of one are known not to alias copies into another
  __shared__ __attribute__((aligned(1024))) uint8_t a0_raw[A_TILE], a1_raw[A_TILE], a2_raw[RING >= 3 ? A_TILE : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t b0_raw[B_TILE], b1_raw[B_TILE];
  __shared__ __attribute__((aligned(1024))) uint8_t b2_raw[DQ8 ? Q_TILE : RING >= 3 ? B_TILE : 16];  // DQ8: int8 tile 0
  __shared__ __attribute__((aligned(1024))) uint8_t a3_raw[RING >= 4 ? A_TILE : 16], b3_raw[RING >= 4 ? B_TILE : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t a4_raw[RING >= 5 ? A_TILE : 16], b4_raw[RING >= 5 ? B_TILE : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t a5_raw[RING >= 6 ? A_TILE : 16], b5_raw[RING >= 6 ? B_TILE : 16];
  __shared__ __attribute__((aligned(DQ8 ? 1024 : 16))) uint8_t q1_raw[Q_TILE], q2_raw[Q_TILE];
  HK_L uint8_t* const A0 = (HK_L uint8_t*)a0_raw;
  HK_L uint8_t* const A1 = (HK_L uint8_t*)a1_raw;
  HK_L uint8_t* const A2 = (HK_L uint8_t*)a2_raw;
  HK_L uint8_t* const B0 = (HK_L uint8_t*)b0_raw;
  HK_L uint8_t* const B1 = (HK_L uint8_t*)b1_raw;
  HK_L uint8_t* const B2 = (HK_L uint8_t*)b2_raw;
  auto abuf = [&](auto ic) {
    constexpr int I = decltype(ic)::value;
    return (HK_L uint8_t*)(I == 0 ? a0_raw : I == 1 ? a1_raw : I == 2 ? a2_raw : I == 3 ? a3_raw : I == 4 ? a4_raw : a5_raw);
  };
  auto bbuf = [&](auto ic) {
    constexpr int I = decltype(ic)::value;
    return (HK_L uint8_t*)(I == 0 ? b0_raw : I == 1 ? b1_raw : I == 2 ? b2_raw : I == 3 ? b3_raw : I == 4 ? b4_raw : b5_raw);
  };
  HK_L uint8_t* const Q0 = (HK_L uint8_t*)b2_raw;
  HK_L uint8_t* const Q1 = (HK_L uint8_t*)q1_raw;
  HK_L uint8_t* const Q2 = (HK_L uint8_t*)q2_raw;
  auto qbuf = [&](auto ic) { constexpr int I = decltype(ic)::value; return I == 0 ? Q0 : I == 1 ? Q1 : Q2; };

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WNN, wn = wave % WNN;
  const int l32 = lane & 31, h = lane >> 5, s16 = lane & 15, g2 = (lane >> 4) & 1;
  // Workgroups are dealt to the eight XCDs in turn (workgroup i to XCD i % 8), and each XCD has its own L2.
  // xbm > 0 (a batch of 1, 2, 4 or 8 products whose tile count per product divides into 8 / batch blocks):
  // XCD x takes product x / (8 / batch) and, of its tile grid, one xbm x (count / (8 / batch) / xbm) block,
  // the block shape the launcher chose to minimise the A and B panel bytes each XCD reads (a split-K
  // product's K slices are its batch).  xbm = 0: tiles numbered n-fastest, products one after another.
  const uint32_t tile = blockIdx.x;
  uint32_t tn = tile % (uint32_t)tiles_n, tm = (tile / (uint32_t)tiles_n) % (uint32_t)tiles_m;
  uint32_t bz = tile / ((uint32_t)tiles_n * (uint32_t)tiles_m);
  if (xbm > 0) {
    const uint32_t G = 8 / (uint32_t)p.batch;  // XCDs per product
    const uint32_t bnw = (uint32_t)tiles_m * (uint32_t)tiles_n / G / (uint32_t)xbm, nbn = (uint32_t)tiles_n / bnw;
    const uint32_t x = tile % 8, loc = tile / 8, sub = x % G;
    bz = x / G;
    tm = (sub / nbn) * (uint32_t)xbm + loc / bnw;
    tn = (sub % nbn) * bnw + loc % bnw;
  }
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int nk = (int)(p.K / GBK);

  // copy sources (bytes) of K step 0 and the per-step advance
  const HK_G uint8_t* Ab = reinterpret_cast<const HK_G uint8_t*>(gcptr<uint16_t>(p.a) + bz * p.a_sb +
                                                                 (ATR ? m0 : m0 * p.a_sm));
  // (DQ8: B = q, strides in bytes, one byte per element)
  constexpr int BEL = DQ8 ? 1 : 2;
  const HK_G uint8_t* Bb = DQ8 ? gcptr<uint8_t>(p.b) + n0 * p.b_sn
                               : reinterpret_cast<const HK_G uint8_t*>(gcptr<uint16_t>(p.b) + bz * p.b_sb +
                                                                       (BTR ? n0 : n0 * p.b_sn));
  const uint32_t ass = (uint32_t)((ATR ? p.a_sk : p.a_sm) * 2), bss = (uint32_t)((BTR ? p.b_sk : p.b_sn) * BEL);
  const int64_t astep = ATR ? (int64_t)GBK * p.a_sk * 2 : GBK * 2;
  const int64_t bstep = BTR ? (int64_t)GBK * p.b_sk * BEL : GBK * BEL;
  const DmaLanes alo = dma_lane_offsets<A_NCH>(ass, lane, wave * IPA);
  const DmaLanes blo = DQ8 ? dma_lane_offsets<4>(bss, lane, wave * IPQ) : dma_lane_offsets<B_NCH>(bss, lane, wave * IPB);

  // fragment offsets inside a tile for m (n) sub-tile i (j) and 16-wide K slice kk; a transposed operand
  // uses two column reads per fragment (rows 16 kk + 8 h + 4 t + (s >> 2), t = 0, 1: entries kk = 0, 1)
  int aoff[FM][4], boff[FN][4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      if constexpr (!ATR) {
        aoff[i][kk] = tile_off<A_NCH>(wm * WM + i * 32 + l32, 2 * kk + h);
      } else {
        const int col = wm * WM + i * 32 + 16 * g2 + 4 * (s16 & 3);
        aoff[i][kk] = kk < 2 ? tile_off<A_NCH>(8 * h + 4 * (kk & 1) + (s16 >> 2), col >> 3) + (s16 & 1) * 8 : 0;
      }
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      if constexpr (!BTR) {
        boff[j][kk] = tile_off<B_NCH>(wn * WN + j * 32 + l32, 2 * kk + h);
      } else {
        const int col = wn * WN + j * 32 + 16 * g2 + 4 * (s16 & 3);
        boff[j][kk] = kk < 2 ? tile_off<B_NCH>(8 * h + 4 * (kk & 1) + (s16 >> 2), col >> 3) + (s16 & 1) * 8 : 0;
      }
    }
  }
  auto afrag = [&](const HK_L uint8_t* At, int i, int kk) -> u32x4 {
    if constexpr (!ATR) {
      return *reinterpret_cast<const HK_L u32x4*>(At + aoff[i][kk]);
    } else {
      const u32x2 lo = lds_tr4(At + aoff[i][0] + kk * 16 * A_ROWB), hi = lds_tr4(At + aoff[i][1] + kk * 16 * A_ROWB);
      return u32x4{lo.x, lo.y, hi.x, hi.y};
    }
  };
  auto bfrag = [&](const HK_L uint8_t* Bt, int j, int kk) -> u32x4 {
    if constexpr (!BTR) {
      return *reinterpret_cast<const HK_L u32x4*>(Bt + boff[j][kk]);
    } else {
      const u32x2 lo = lds_tr4(Bt + boff[j][0] + kk * 16 * B_ROWB), hi = lds_tr4(Bt + boff[j][1] + kk * 16 * B_ROWB);
      return u32x4{lo.x, lo.y, hi.x, hi.y};
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = zero16();

  // DQ8 conversion: chunk u of this thread in the int8 tile of K step ks (buffer Qt) -> B tile Bt
  const HK_G uint16_t* scl = gcptr<uint16_t>(dq_scale) + (DQ8 ? n0 * dq_nblocks : 0);
  auto dq_scales = [&](int ks, float* sv) {
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int row = (u * NW * 64 + (int)threadIdx.x) >> 3;
      sv[u] = bf16_bits_to_f32(scl[row * dq_nblocks + ks]);
    }
  };
  // 8 int8 -> 8 values of T per piece: the 8 lanes of a group write the 8 chunks of one 128-byte B row
  // (LDS writes are conflict-free when each group of 8 consecutive lanes stays inside one 128-byte row,
  // measured), and the int8 reads are contiguous 8-byte pieces.
  auto dq_convert = [&](const HK_L uint8_t* Qt, HK_L uint8_t* Bt, const float* sv) {
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int c = u * NW * 64 + (int)threadIdx.x, row = c >> 3, ch = c & 7;
      const u32x2 w = *reinterpret_cast<const HK_L u32x2*>(Qt + c * 8);
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = (float)(int8_t)(((i < 4 ? w.x : w.y) >> (8 * (i & 3))) & 0xffu) * sv[u];
      // round to the input dtype: the hardware pack (RNE) when the products are finite, which they are
      // unless the scale is inf or NaN; then the software rounding, which maps NaN to 0x7FC0 like dq8_*
      const u32x4 h = __builtin_isfinite(sv[u]) ? u32x4{cvt2<T>(v[0], v[1]), cvt2<T>(v[2], v[3]), cvt2<T>(v[4], v[5]), cvt2<T>(v[6], v[7])}
                                                 : u32x4{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3]), pack2<T>(v[4], v[5]), pack2<T>(v[6], v[7])};
      *reinterpret_cast<HK_L u32x4*>(Bt + tile_off<B_NCH>(row, ch)) = h;
    }
  };
  const int k1 = nk > 1 ? 1 : 0, k2 = nk > 2 ? 2 : nk - 1;
  float svq[CPT];  // DQ8: scales of the int8 tile that the next step converts (loaded a step ahead)
  if constexpr (!DQ8 && RING == 2) {
    // step 0; each step then copies the next one into the other buffer and waits for it at its end
#pragma unroll
    for (int c = 0; c < IPA; ++c) dma_tile_part<A_NCH, A_ROWS, NW>(Ab, ass, A0, wave, alo, c);
#pragma unroll
    for (int c = 0; c < IPB; ++c) dma_tile_part<B_NCH, B_ROWS, NW>(Bb, bss, B0, wave, blo, c);
    __syncthreads();
  } else if constexpr (!DQ8) {
    // steps 0 .. RING - 2 into buffers 0 .. RING - 2 (step min(s, nk - 1): a short K re-copies its last step
    // into buffers nobody reads)
    static_for<RING - 1>([&](auto ic) {
      constexpr int S = decltype(ic)::value;
      const int ks = S < nk ? S : nk - 1;
#pragma unroll
      for (int c = 0; c < IPA; ++c) dma_tile_part<A_NCH, A_ROWS, NW>(Ab + ks * astep, ass, abuf(ic), wave, alo, c);
#pragma unroll
      for (int c = 0; c < IPB; ++c) dma_tile_part<B_NCH, B_ROWS, NW>(Bb + ks * bstep, bss, bbuf(ic), wave, blo, c);
      issue_order_fence();
    });
    barrier_keep_vm<(RING - 2) * (IPA + IPB)>();  // step 0 landed everywhere, steps 1 .. RING - 2 in flight
  } else {
    // int8 steps 0, 1, 2 and A steps 0, 1; step 0's int8 tile converted before the loop
    float sv[CPT];
    dq_scales(0, sv);
#pragma unroll
    for (int c = 0; c < IPQ; ++c) dma_tile_part<4, BN, NW>(Bb, bss, Q0, wave, blo, c);
#pragma unroll
    for (int c = 0; c < IPA; ++c) dma_tile_part<A_NCH, A_ROWS, NW>(Ab, ass, A0, wave, alo, c);
    issue_order_fence();
#pragma unroll
    for (int c = 0; c < IPA; ++c) dma_tile_part<A_NCH, A_ROWS, NW>(Ab + k1 * astep, ass, A1, wave, alo, c);
#pragma unroll
    for (int c = 0; c < IPQ; ++c) dma_tile_part<4, BN, NW>(Bb + k1 * bstep, bss, Q1, wave, blo, c);
#pragma unroll
    for (int c = 0; c < IPQ; ++c) dma_tile_part<4, BN, NW>(Bb + k2 * bstep, bss, Q2, wave, blo, c);
    barrier_keep_vm<IPA + 2 * IPQ>();  // int8 step 0 and A step 0 landed everywhere
    dq_scales(k1, svq);
    dq_convert(Q0, B0, sv);
    __syncthreads();  // B tile 0 written; the other copies landed
  }

  // K step kt: MFMAs from buffer kt % 3, copies of step min(kt + 2, nk - 1) into buffer (kt + 2) % 3 (read
  // by step kt - 1, whose readers all passed the previous barrier) placed after the first MFMAs; no copy is
  // issued for steps past the end.  Before the barrier that ends
  // the step each wavefront waits for its copies of the previous step only, so step kt + 1's buffer is
  // complete after the barrier while the copies of step kt + 2 stay in flight.  DQ8: B tiles alternate
  // (kt % 2), int8 step min(kt + 3, nk - 1) is copied into int8 buffer kt % 3 (converted during step
  // kt - 1) and int8 step kt + 1 (buffer (kt + 1) % 3, landed at the last barrier) is converted into B
  // tile (kt + 1) % 2 (last read in step kt - 1); steps past the end convert a repeat nobody reads.
  auto step = [&](auto bc, auto bq, int kt) {
    constexpr int BUF = decltype(bc)::value;
    constexpr int NXT = DQ8 ? (BUF + 2) % 3 : (BUF + RING - 1) % RING;
    constexpr int BB = decltype(bq)::value;  // DQ8: B tile kt % 2
    constexpr int AHEAD = RING - 1;          // steps between a copy and its use
    const int kn = kt + AHEAD < nk ? kt + AHEAD : nk - 1;
    const HK_G uint8_t* an = Ab + kn * astep;
    const HK_L uint8_t* At = abuf(bc);
    const HK_L uint8_t* Bt = DQ8 ? bbuf(bq) : bbuf(bc);
    const int kq = DQ8 ? (kt + 3 < nk ? kt + 3 : nk - 1) : kn;
    const HK_G uint8_t* bn = Bb + kq * bstep;
    // No copies past the last K step: the ring buffers they would fill are the epilogue's staging areas.
    // (DQ8: A runs AHEAD = 2 steps ahead, the int8 tiles 3.)
    const bool more_a = kt + AHEAD < nk, more_b = DQ8 ? kt + 3 < nk : more_a;
    float sv[CPT];
    if constexpr (DQ8) {
#pragma unroll
      for (int u = 0; u < CPT; ++u) sv[u] = svq[u];
      dq_scales(kt + 2 < nk ? kt + 2 : nk - 1, svq);
    }
    // Sub-tiles of at least two accumulators: the fragments of K slice kk + 1 are read while slice kk's
    // MFMAs run (two register sets, each slice fenced by sched_barrier: in the compiler's own order every
    // slice waited for its reads; 1024 x 2048 x 8192 -3%, the fused int8 linear -3%, the DiT stack -2%).
    // 64 x 64 tiles (one MFMA per slice) keep the compiler's order, which measured faster for them.
    constexpr bool AHEAD1 = FM * FN >= 2;
    u32x4 af[2][FM], bf[2][FN];
    auto rdk = [&](int kk) {
#pragma unroll
      for (int i = 0; i < FM; ++i) af[kk & 1][i] = afrag(At, i, kk);
#pragma unroll
      for (int j = 0; j < FN; ++j) bf[kk & 1][j] = bfrag(Bt, j, kk);
    };
    if constexpr (AHEAD1) rdk(0);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if constexpr (AHEAD1) {
        __builtin_amdgcn_sched_barrier(0);
        if (kk + 1 < 4) rdk(kk + 1);
      } else {
        rdk(kk);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = Mfma32<T>::mac(af[kk & 1][i], bf[kk & 1][j], acc[i][j]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c = kk * 4 + q;
        if (c < IPA) {
          if (more_a) dma_tile_part<A_NCH, A_ROWS, NW>(an, ass, abuf(std::integral_constant<int, NXT>()), wave, alo, c);
        } else if constexpr (!DQ8) {
          if (c < IPA + IPB && more_b)
            dma_tile_part<B_NCH, B_ROWS, NW>(bn, bss, bbuf(std::integral_constant<int, NXT>()), wave, blo, c - IPA);
        } else {
          if (c < IPA + IPQ && more_b)
            dma_tile_part<4, BN, NW>(bn, bss, qbuf(std::integral_constant<int, BUF>()), wave, blo, c - IPA);
        }
      }
      if constexpr (DQ8) {
        if (kk == 1) dq_convert(qbuf(std::integral_constant<int, (BUF + 1) % 3>()), bbuf(std::integral_constant<int, BB ^ 1>()), sv);
      }
    }
    if constexpr (AHEAD1) __builtin_amdgcn_sched_barrier(0);
    // each wavefront lets exactly the copies it issued in this step stay in flight
    if constexpr (DQ8) {
      if (more_b) barrier_keep_vm_lds<IPA + IPQ>();
      else if (more_a) barrier_keep_vm_lds<IPA>();
      else barrier_keep_vm_lds<0>();
    } else if constexpr (RING >= 3) {
      // step kt + 1's copies (issued RING - 1 steps before it) must have landed; those of steps kt + 2 ..
      // min(kt + RING - 1, nk - 1), issued after them, may stay in flight (a count below the true one only
      // waits longer)
      const int last = kt + RING - 1 < nk - 1 ? kt + RING - 1 : nk - 1;
      const int fly = last - (kt + 1) > 0 ? last - (kt + 1) : 0;
      static_for<RING - 1>([&](auto ic) {
        constexpr int F = decltype(ic)::value;
        if (fly == F || (F == RING - 2 && fly > F)) barrier_keep_vm<F * (IPA + IPB)>();
      });
    } else {
      __syncthreads();  // the next step's copies, issued in this one, have landed everywhere
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  if constexpr (!DQ8 && RING == 2) {
    int kt = 0;
    for (; kt + 2 <= nk; kt += 2) {
      step(I0(), I0(), kt);
      step(I1(), I0(), kt + 1);
    }
    if (kt < nk) step(I0(), I0(), kt);
  } else if constexpr (!DQ8) {
    int kt = 0;
    for (; kt + RING <= nk; kt += RING) static_for<RING>([&](auto ic) { step(ic, I0(), kt + decltype(ic)::value); });
    static_for<RING - 1>([&](auto ic) {
      if (kt + decltype(ic)::value < nk) step(ic, I0(), kt + decltype(ic)::value);
    });
  } else {
    // A and int8 buffers rotate by 3, B tiles by 2: blocks of 6 steps, leaving after any step
    for (int kt = 0;; kt += 6) {
      step(I0(), I0(), kt);
      if (kt + 1 >= nk) break;
      step(I1(), I1(), kt + 1);
      if (kt + 2 >= nk) break;
      step(I2(), I0(), kt + 2);
      if (kt + 3 >= nk) break;
      step(I0(), I1(), kt + 3);
      if (kt + 4 >= nk) break;
      step(I1(), I0(), kt + 4);
      if (kt + 5 >= nk) break;
      step(I2(), I1(), kt + 5);
      if (kt + 6 >= nk) break;
    }
  }
  __syncthreads();  // the last copies have landed before the epilogue reuses the tiles

  // ---- epilogue: per n sub-tile j, the WM x 32 fp32 block goes through this wavefront's area as [m][n]
  float* const area = reinterpret_cast<float*>(wave < PA            ? a0_raw + wave * AREA
                                              : wave < 2 * PA        ? a1_raw + (wave - PA) * AREA
                                              : wave < 2 * PA + PB   ? b0_raw + (wave - 2 * PA) * AREA
                                                                     : b1_raw + (wave - 2 * PA - PB) * AREA);
  const bool has_bias = p.has_bias != 0;
  const HK_G uint16_t* bias = gcptr<uint16_t>(p.bias) + bz * p.bias_sb;
  HK_G uint16_t* C = gptr<uint16_t>(p.c) + bz * p.c_sb;
  HK_G float* C32 = gptr<float>(p.c) + bz * p.c_sb;  // F32OUT: unrounded fp32 results (split-K partials)
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t gn = n0 + wn * WN + j * 32 + l32;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      float bv[16];  // beta * bias, all 16 loads in flight together
      if (has_bias) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
          bv[e] = p.beta * T::to_f32(bias[(m0 + wm * WM + r) * p.bias_sm + gn * p.bias_sn]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) bv[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
        area[r * RS + l32] = p.alpha * acc[i][j][e] + bv[e];
      }
    }
    // 4 lanes per 32-wide row, 8 floats each: 16 rows per pass
#pragma unroll
    for (int ps = 0; ps < WM / 16; ++ps) {
      const int r = ps * 16 + (lane >> 2), c8 = (lane & 3) * 8;
      const f32x4 x = *reinterpret_cast<const f32x4*>(area + r * RS + c8);
      const f32x4 y = *reinterpret_cast<const f32x4*>(area + r * RS + c8 + 4);
      const int64_t off = (m0 + wm * WM + r) * p.c_sm + n0 + wn * WN + j * 32 + c8;
      if constexpr (F32OUT) {
        *reinterpret_cast<HK_G f32x4*>(C32 + off) = x;
        *reinterpret_cast<HK_G f32x4*>(C32 + off + 4) = y;
      } else {
        const float o8[8] = {x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
        *reinterpret_cast<HK_G u32x4*>(C + off) = pack8<T>(o8);
      }
    }
  }
}

// The fast path applies to tile-aligned problems whose operands are contiguous along one axis with 16-byte
// aligned rows, a row-contiguous C, and per-tile row offsets that fit the copies' 32-bit lane offsets.
bool mm_dma_ok(const hrt_mm_args& a, int BM, int BN, bool& atr, bool& btr) {
  if (a.M % BM || a.N % BN || a.K % GBK || a.K < GBK) return false;
  const auto al = [](uint64_t x) { return x % 16 == 0; };
  if (!al(a.a) || !al(a.b) || !al(a.c) || a.c_sn != 1 || a.c_sm % 8 || (a.batch > 1 && (a.a_sb % 8 || a.b_sb % 8 || a.c_sb % 8)))
    return false;
  if (a.a_sk == 1 && a.a_sm % 8 == 0) atr = false;
  else if (a.a_sm == 1 && a.a_sk % 8 == 0) atr = true;
  else return false;
  if (a.b_sk == 1 && a.b_sn % 8 == 0) btr = false;
  else if (a.b_sn == 1 && a.b_sk % 8 == 0) btr = true;
  else return false;
  const int64_t lim = (int64_t)1 << 31;
  const int64_t arows = atr ? GBK : BM, brows = btr ? GBK : BN;
  return (atr ? a.a_sk : a.a_sm) * 2 * (arows + 1) < lim && (btr ? a.b_sk : a.b_sn) * 2 * (brows + 1) < lim;
}

// The XCD block of mm_dma for a tm x tn tile grid of each of `batch` products (batch 1, 2, 4 or 8; a
// split-K product's slices): the rows xbm of the block shape xbm x bn (xbm | tm, bn | tn, 8 / batch blocks
// per product, one per XCD) with the fewest panel bytes per XCD, xbm * a_panel + bn * b_panel (a_panel /
// b_panel: bytes of one BM-row A panel / BN-row B panel over K); 0 (n-fastest order) when the grid does not
// split so, or K < 2048 (one product) / 1536 (slices).  For the four K slices of a 1024 x 2048 output on
// 128 x 256 tiles each XCD then reads one slice's A panels and half its B panels instead of every slice's
// A panels: 2.6-4.6% faster (K = 6144 and 8192, slices + reduction 42.2 -> 41.1, 49.9 -> 48.5 us).
// The block order is used only where it reads at least 10% fewer panel bytes than the n-fastest order (which,
// with tn a multiple of 8, gives each XCD tn / 8 B panels and every A panel): where the two read the same,
// as at 1024 x 2048 x 8192 on 128 x 256 tiles, the block order measured ~1.5% slower.  Measured:
// 1024 x 2048 x 2048 on 64 x 64 tiles 15.4-16.1 us against 16.6-18.1 n-fastest (41.9 -> 33.6 MB of panels
// read), 4096 x 2048 x 8192 1.5% faster; but 1024^3 6.65 against 6.45 us although it reads 12.6 instead of
// 18.9 MB, so short reductions keep the n-fastest order.
int xcd_block_rows(int64_t tm, int64_t tn, int64_t batch, int64_t K, double a_panel, double b_panel) {
  if (batch < 1 || batch > 8 || 8 % batch != 0 || tn % 8 != 0) return 0;
  if (K < (batch == 1 ? 2048 : 1536)) return 0;
  const int64_t G = 8 / batch;  // XCDs per product
  if ((tm * tn) % G != 0) return 0;
  const int64_t per = tm * tn / G;
  int best = 0;
  double cost = 0.0;
  for (int64_t bm = 1; bm <= tm; ++bm) {
    if (tm % bm || per % bm) continue;
    const int64_t bn = per / bm;
    if (tn % bn) continue;
    const double c = bm * a_panel + bn * b_panel;
    if (best == 0 || c < cost) best = (int)bm, cost = c;
  }
  // n-fastest order: every XCD reads all A panels and tn / 8 B panels of every product
  const double n_fastest = batch * (tm * a_panel + (tn / 8) * b_panel);
  return best > 0 && cost <= 0.9 * n_fastest ? best : 0;
}

template <typename T, int BM, int BN, int WM, int WN, int RING = 3, bool F32OUT = false>
bool queue_dma(const hrt_mm_args& a, hipStream_t s) {
  bool atr = false, btr = false;
  if (!mm_dma_ok(a, BM, BN, atr, btr)) return false;
  const int tm = (int)(a.M / BM), tn = (int)(a.N / BN);
  const int xbm = xcd_block_rows(tm, tn, a.batch, a.K, (double)BM * a.K * 2, (double)BN * a.K * 2);
  const dim3 g((uint32_t)((int64_t)tm * tn * a.batch)), blk((BM / WM) * (BN / WN) * 64);
  const uint64_t ns = 0;
  if (!atr && !btr) hipLaunchKernelGGL((mm_dma<T, BM, BN, WM, WN, false, false, false, RING, F32OUT>), g, blk, 0, s, a, tm, tn, xbm, ns, 0);
  else if (!atr && btr) hipLaunchKernelGGL((mm_dma<T, BM, BN, WM, WN, false, true, false, RING, F32OUT>), g, blk, 0, s, a, tm, tn, xbm, ns, 0);
  else if (atr && !btr) hipLaunchKernelGGL((mm_dma<T, BM, BN, WM, WN, true, false, false, RING, F32OUT>), g, blk, 0, s, a, tm, tn, xbm, ns, 0);
  else hipLaunchKernelGGL((mm_dma<T, BM, BN, WM, WN, true, true, false, RING, F32OUT>), g, blk, 0, s, a, tm, tn, xbm, ns, 0);
  return true;
}

// The same for 128 x 192 tiles (eight wavefronts of 32 x 96 sub-tiles), whose 24-chunk rows the LDS swizzle
// supports only for a B operand laid out along K (B given as [N][K]: x W^T); false for the other layouts.
template <typename T>
bool queue_dma_192(const hrt_mm_args& a, hipStream_t s) {
  constexpr int BM = 128, BN = 192, WM = 32, WN = 96;
  bool atr = false, btr = false;
  if (!mm_dma_ok(a, BM, BN, atr, btr) || btr) return false;
  const int tm = (int)(a.M / BM), tn = (int)(a.N / BN);
  const int xbm = xcd_block_rows(tm, tn, a.batch, a.K, (double)BM * a.K * 2, (double)BN * a.K * 2);
  const dim3 g((uint32_t)((int64_t)tm * tn * a.batch)), blk((BM / WM) * (BN / WN) * 64);
  const uint64_t ns = 0;
  if (!atr) hipLaunchKernelGGL((mm_dma<T, BM, BN, WM, WN, false, false, false>), g, blk, 0, s, a, tm, tn, xbm, ns, 0);
  else hipLaunchKernelGGL((mm_dma<T, BM, BN, WM, WN, true, false, false>), g, blk, 0, s, a, tm, tn, xbm, ns, 0);
  return true;
}

// The fused int8 linear on the fast path: y = alpha x deq(q)^T + beta bias as the GEMM A = x [M][K] (either
// layout), B = q read as [N][K] int8 rows with the per-64 scales, C = y [M][N].
template <typename T, int BM, int BN, int WM, int WN>
bool queue_dma_dq8(const hrt_mm_dq8_args& d, hipStream_t s) {
  if (d.K % GBK || d.q % 16 || d.scale % 2) return false;
  hrt_mm_args a{};
  a.a = d.x, a.b = d.q, a.c = d.y, a.bias = d.bias;
  a.M = d.M, a.N = d.N, a.K = d.K, a.batch = 1;
  a.a_sm = d.x_sm, a.a_sk = d.x_sk, a.b_sk = 1, a.b_sn = d.K, a.c_sm = d.N, a.c_sn = 1, a.bias_sn = 1;
  a.alpha = d.alpha, a.beta = d.beta, a.has_bias = d.has_bias;
  bool atr = false, btr = false;
  if (!mm_dma_ok(a, BM, BN, atr, btr) || btr) return false;
  const int tm = (int)(a.M / BM), tn = (int)(a.N / BN);
  const dim3 g((uint32_t)((int64_t)tm * tn)), blk((BM / WM) * (BN / WN) * 64);
  const int xbm = xcd_block_rows(tm, tn, 1, a.K, (double)BM * a.K * 2, (double)BN * a.K);
  if (!atr) hipLaunchKernelGGL((mm_dma<T, BM, BN, WM, WN, false, false, true>), g, blk, 0, s, a, tm, tn, xbm, d.scale, d.nblocks);
  else hipLaunchKernelGGL((mm_dma<T, BM, BN, WM, WN, true, false, true>), g, blk, 0, s, a, tm, tn, xbm, d.scale, d.nblocks);
  return true;
}

// Which loader an operand can use.  rows = M (A) or N (B); s_r / s_k its strides.
int pick_mode(uint64_t ptr, int64_t s_b, int64_t s_r, int64_t s_k, int64_t rows, int64_t K, int64_t batch) {
  const bool aligned = ptr % 16 == 0 && (batch == 1 || s_b % 8 == 0);
  if (aligned && s_k == 1 && K % 8 == 0 && (rows == 1 || s_r % 8 == 0)) return KVEC;
  if (aligned && s_r == 1 && rows % 8 == 0 && (K == 1 || s_k % 8 == 0)) return MNVEC;
  return GATHER;
}

template <typename T, int BM, int BN, int WM, int WN, int AM, int BMd>
void queue(const hrt_mm_args& a, hipStream_t s) {
  const int64_t tm = cdiv(a.M, BM), tn = cdiv(a.N, BN);
  hipLaunchKernelGGL((mm_mfma<T, BM, BN, WM, WN, AM, BMd>), dim3((uint32_t)(tm * tn * a.batch)), dim3(256), 0, s, a, tm, tn);
}

template <typename T, int BM, int BN, int WM, int WN>
void dispatch_modes(const hrt_mm_args& a, int am, int bm, hipStream_t s) {
  switch (am * 3 + bm) {
    case KVEC * 3 + KVEC: queue<T, BM, BN, WM, WN, KVEC, KVEC>(a, s); break;
    case KVEC * 3 + MNVEC: queue<T, BM, BN, WM, WN, KVEC, MNVEC>(a, s); break;
    case MNVEC * 3 + KVEC: queue<T, BM, BN, WM, WN, MNVEC, KVEC>(a, s); break;
    case MNVEC * 3 + MNVEC: queue<T, BM, BN, WM, WN, MNVEC, MNVEC>(a, s); break;
    default: break;
  }
}

template <typename T>
void dispatch_gather(const hrt_mm_args& a, int am, int bm, hipStream_t s) {
  switch (am * 3 + bm) {
    case KVEC * 3 + KVEC: queue<T, 64, 64, 2, 2, KVEC, KVEC>(a, s); break;
    case KVEC * 3 + MNVEC: queue<T, 64, 64, 2, 2, KVEC, MNVEC>(a, s); break;
    case KVEC * 3 + GATHER: queue<T, 64, 64, 2, 2, KVEC, GATHER>(a, s); break;
    case MNVEC * 3 + KVEC: queue<T, 64, 64, 2, 2, MNVEC, KVEC>(a, s); break;
    case MNVEC * 3 + MNVEC: queue<T, 64, 64, 2, 2, MNVEC, MNVEC>(a, s); break;
    case MNVEC * 3 + GATHER: queue<T, 64, 64, 2, 2, MNVEC, GATHER>(a, s); break;
    case GATHER * 3 + KVEC: queue<T, 64, 64, 2, 2, GATHER, KVEC>(a, s); break;
    case GATHER * 3 + MNVEC: queue<T, 64, 64, 2, 2, GATHER, MNVEC>(a, s); break;
    default: queue<T, 64, 64, 2, 2, GATHER, GATHER>(a, s); break;
  }
}

template <typename T>
bool launch_mm_mfma(const void* pp, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_mm_args*>(pp);
  if (!mm_check_operands(a, 2, ctx)) return false;
  if (a.flags & ~HRT_MM_F32_OUT) return ctx.fail("unknown GEMM flags");
  const bool f32out = (a.flags & HRT_MM_F32_OUT) != 0;
  const int am = pick_mode(a.a, a.a_sb, a.a_sm, a.a_sk, a.M, a.K, a.batch);
  const int bm = pick_mode(a.b, a.b_sb, a.b_sn, a.b_sk, a.N, a.K, a.batch);
  const int64_t big = cdiv(a.M, 128) * cdiv(a.N, 256) * a.batch;
  const int64_t med = cdiv(a.M, 128) * cdiv(a.N, 128) * a.batch;
  const int64_t small = cdiv(a.M, 64) * cdiv(a.N, 64) * a.batch;
  if (small > 0x7fffffffLL) return ctx.fail("GEMM grid too large");
  // a short reduction (K <= 32, a low-rank adapter's up-projection): bound by the output, not the matrix cores
  if (!f32out && a.K <= 32 && skinny::queue_expand<T>(a, ctx.stream)) return hrt::launch_ok(hipGetLastError(), ctx, "mm_expand");
  // a narrow output (M or N <= 16, a low-rank adapter's down-projection and factor gradients, also the
  // fp32 slices of such a product split along K)
  if ((a.M <= 16 || a.N <= 16) && skinny::queue_narrow<T>(a, ctx.stream))
    return hrt::launch_ok(hipGetLastError(), ctx, "mm_narrow");
  // fast path: the largest tile that still gives enough workgroups.  256 x 256 tiles (two-buffer ring) copy a
  // third fewer bytes per flop than 128 x 256 (the copies, not the MFMAs, bound these kernels once the grid
  // fills the chip) but wait a whole step for each copy: measured 3% faster at K = 2048 (M = 2048, 4096 and
  // N = 8192), 5% slower at 8192^3.  Both run one workgroup per CU, so a grid runs in rounds of 256 tiles;
  // 256 x 256 is taken only when its rounds are as full as those of the 128 x 256 / 256 x 128 tiling (the
  // convolution's input-gradient product 4608 x 4096 x 512: 288 tiles fill 56% of two rounds, 576 half-size
  // tiles 75% of three, measured 41.9 against 36.2-37.2 us).
  auto round_fill = [](int64_t t) { return t > 0 ? (double)t / (double)(((t + 255) / 256) * 256) : 0.0; };
  const int64_t t256 = a.M % 256 == 0 && a.N % 256 == 0 ? a.batch * (a.M / 256) * (a.N / 256) : 0;
  const int64_t t_wide = a.M % 128 == 0 && a.N % 256 == 0 ? a.batch * (a.M / 128) * (a.N / 256) : 0;
  const int64_t t_tall = a.M % 256 == 0 && a.N % 128 == 0 ? a.batch * (a.M / 256) * (a.N / 128) : 0;
  if (!f32out && a.K <= 4096 && t256 >= 256 && round_fill(t256) >= round_fill(std::max(t_wide, t_tall)) &&
      queue_dma<T, 256, 256, 64, 128, 2>(a, ctx.stream))
    return hrt::launch_ok(hipGetLastError(), ctx, "mm_dma");
  // 128 x 192 tiles where they fill the rounds better than 128 x 256 (1024 x 2048 x 6144 x W^T: 256 tiles
  // against 192 half-empty-round ones, 32.1 -> 29.9 us)
  const int64_t t192 = a.M % 128 == 0 && a.N % 192 == 0 ? a.batch * (a.M / 128) * (a.N / 192) : 0;
  if (!f32out && t192 >= 192 && round_fill(t192) > round_fill(std::max(t_wide, t_tall)) && queue_dma_192<T>(a, ctx.stream))
    return hrt::launch_ok(hipGetLastError(), ctx, "mm_dma");
  if (!f32out && a.batch * (a.M / 128) * (a.N / 256) >= 192 && queue_dma<T, 128, 256, 64, 64>(a, ctx.stream))
    return hrt::launch_ok(hipGetLastError(), ctx, "mm_dma");
  if (!f32out && a.batch * (a.M / 256) * (a.N / 128) >= 192 && queue_dma<T, 256, 128, 64, 64>(a, ctx.stream))
    return hrt::launch_ok(hipGetLastError(), ctx, "mm_dma");
  // 64 x 128 tiles (four wavefronts of 32 x 64: a third fewer LDS bytes per MFMA than 32 x 32 ones) where they
  // still give a few hundred workgroups: 2048^3 34.5 -> 24.8 us, 1024 x 512 x 4096 10.3 -> 9.1 us, 1024 x 2048
  // x 2048 unchanged (the 64 x 64 grid's second round there costs what the larger tiles save)
  if (!f32out && a.M % 64 == 0 && a.N % 128 == 0 && a.batch * (a.M / 64) * (a.N / 128) >= 192 &&
      queue_dma<T, 64, 128, 32, 64>(a, ctx.stream))
    return hrt::launch_ok(hipGetLastError(), ctx, "mm_dma");
  // 64 x 64 tiles, whose steps (4 MFMAs per wavefront) are far shorter than a copy's latency: a ring of four
  // buffers (copies three steps ahead) for long reductions, 64 KiB per workgroup, still two per CU
  // (1024 x 4096 x 1024 NT / NN 28.5 / 25.5 -> 24.0 us, 512 x 4096 x 2048 28.4 -> 23.7 us; at K <= 2048 the
  // fourth buffer measured -4% to +9%, so shorter reductions keep three)
  const int64_t t64 = a.batch * (a.M / 64) * (a.N / 64);
  if (!f32out && t64 >= 128 &&
      (a.K >= 4096 && t64 <= 512 ? queue_dma<T, 64, 64, 32, 32, 4>(a, ctx.stream) : queue_dma<T, 64, 64, 32, 32>(a, ctx.stream)))
    return hrt::launch_ok(hipGetLastError(), ctx, "mm_dma");
  // fp32 partials of a split-K product whose slices (the batch) fill the GPU with the large tiles
  if (f32out && a.batch * (a.M / 128) * (a.N / 256) >= 192 && queue_dma<T, 128, 256, 64, 64, 3, true>(a, ctx.stream))
    return hrt::launch_ok(hipGetLastError(), ctx, "mm_dma");
  if (f32out && a.batch * (a.M / 256) * (a.N / 128) >= 192 && queue_dma<T, 256, 128, 64, 64, 3, true>(a, ctx.stream))
    return hrt::launch_ok(hipGetLastError(), ctx, "mm_dma");
  if (am == GATHER || bm == GATHER) {
    dispatch_gather<T>(a, am, bm, ctx.stream);
  } else if (big >= 240) {
    dispatch_modes<T, 128, 256, 2, 2>(a, am, bm, ctx.stream);
  } else if (med >= 240) {
    dispatch_modes<T, 128, 128, 2, 2>(a, am, bm, ctx.stream);
  } else {
    dispatch_modes<T, 64, 64, 2, 2>(a, am, bm, ctx.stream);
  }
  return hrt::launch_ok(hipGetLastError(), ctx, "mm_mfma");
}

template <typename T, int BM, int BN, int AM>
void queue_dq8(const hrt_mm_dq8_args& a, hipStream_t s) {
  const int64_t tm = cdiv(a.M, BM), tn = cdiv(a.N, BN);
  hipLaunchKernelGGL((mm_dq8_mfma<T, BM, BN, 2, 2, AM>), dim3((uint32_t)(tm * tn)), dim3(256), 0, s, a, tm, tn);
}

// Smallest M at which the fused int8 linear dequantizes into the caller's workspace first: the fused kernel
// converts every weight once per 256-row block of x, which costs more than one standalone dequant pass
// beyond a few blocks (M = 4096: 222 us fused vs ~157 us dequant + GEMM for 8192 x 2048 weights).
constexpr int64_t kDq8WsMinM = 2048;

template <typename T>
bool launch_mm_dq8(const void* pp, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_mm_dq8_args*>(pp);
  if (a.M <= 0 || a.N <= 0 || a.K <= 0) return ctx.fail("empty GEMM");
  if (a.nblocks != (a.K + 63) / 64) return ctx.fail("nblocks must equal ceil(K / 64)");
  if (a.x_sm < 0 || a.x_sk < 0) return ctx.fail("negative stride");
  if (a.K % 8 != 0 || a.q % 8 != 0) return ctx.fail("the fused int8 linear needs K % 8 == 0 and an 8-byte aligned q");
  const int64_t xs[2] = {a.M, a.K}, xt[2] = {a.x_sm, a.x_sk};
  if (!ctx.check(a.x, hrt::span_bytes(2, xs, xt, 2), "x") || !ctx.check(a.q, (uint64_t)(a.N * a.K), "q") ||
      !ctx.check(a.scale, (uint64_t)(a.N * a.nblocks) * 2, "scale") || !ctx.check(a.y, (uint64_t)(a.M * a.N) * 2, "y") ||
      (a.has_bias && !ctx.check(a.bias, (uint64_t)a.N * 2, "bias")))
    return false;
  // large M with a workspace: dequantize once (the dq8 kernel), then the fast GEMM on the bf16 / f16 weights
  if (a.ws && a.M >= kDq8WsMinM && a.K % GBK == 0 && a.ws % 16 == 0) {
    hrt_mm_args m{};
    m.a = a.x, m.b = a.ws, m.c = a.y, m.bias = a.bias;
    m.M = a.M, m.N = a.N, m.K = a.K, m.batch = 1;
    m.a_sm = a.x_sm, m.a_sk = a.x_sk, m.b_sk = 1, m.b_sn = a.K, m.c_sm = a.N, m.c_sn = 1, m.bias_sn = 1;
    m.alpha = a.alpha, m.beta = a.beta, m.has_bias = a.has_bias;
    bool atr = false, btr = false;
    if (mm_dma_ok(m, 128, 256, atr, btr) && (a.M / 128) * (a.N / 256) >= 192) {
      if (!ctx.check(a.ws, (uint64_t)(a.N * a.K) * 2, "ws")) return false;
      hrt_dq8_args d{};
      d.q = a.q, d.scale = a.scale, d.out = a.ws, d.rows = a.N, d.cols = a.K, d.nblocks = a.nblocks;
      const char* dq = sizeof(typename T::storage) == 2 && std::is_same<T, BF16>::value ? "dq8_bf16" : "dq8_f16";
      for (auto& e : hrt::kernel_table())
        if (!strcmp(e.name, dq)) {
          if (!e.launch(&d, nullptr, ctx)) return false;
          if (queue_dma<T, 128, 256, 64, 64>(m, ctx.stream)) return hrt::launch_ok(hipGetLastError(), ctx, "mm_dq8_ws");
        }
      return ctx.fail("mm_dq8: workspace path unavailable");
    }
  }
  // fast path (tile-aligned, K % 64 == 0): dequant fused into the direct-to-LDS GEMM
  if ((a.M / 256) * (a.N / 128) >= 192 && queue_dma_dq8<T, 256, 128, 64, 64>(a, ctx.stream))
    return hrt::launch_ok(hipGetLastError(), ctx, "mm_dq8_dma");
  if ((a.M / 128) * (a.N / 256) >= 192 && queue_dma_dq8<T, 128, 256, 64, 64>(a, ctx.stream))
    return hrt::launch_ok(hipGetLastError(), ctx, "mm_dq8_dma");
  if ((a.M / 64) * (a.N / 64) >= 128 && queue_dma_dq8<T, 64, 64, 32, 32>(a, ctx.stream))
    return hrt::launch_ok(hipGetLastError(), ctx, "mm_dq8_dma");
  const int am = pick_mode(a.x, 0, a.x_sm, a.x_sk, a.M, a.K, 1);
  const int64_t big = cdiv(a.M, 128) * cdiv(a.N, 256);
  if (big >= 240) {
    if (am == KVEC) queue_dq8<T, 128, 256, KVEC>(a, ctx.stream);
    else if (am == MNVEC) queue_dq8<T, 128, 256, MNVEC>(a, ctx.stream);
    else queue_dq8<T, 64, 64, GATHER>(a, ctx.stream);
  } else {
    if (am == KVEC) queue_dq8<T, 64, 64, KVEC>(a, ctx.stream);
    else if (am == MNVEC) queue_dq8<T, 64, 64, MNVEC>(a, ctx.stream);
    else queue_dq8<T, 64, 64, GATHER>(a, ctx.stream);
  }
  return hrt::launch_ok(hipGetLastError(), ctx, "mm_dq8");
}

// ---- split-K reduction: c = round(alpha * sum_s ws[s] + beta * bias), splits summed in order ---------------
// Four consecutive outputs (of the flattened [M, N]) per thread, read as 16-byte pieces of each split when
// M N is a multiple of 4; the loads of up to 16 splits are in flight together (the outputs are small: one
// memory round trip per 16 splits bounds the kernel), then summed in split order.
template <typename T>
__global__ __launch_bounds__(256) void mm_reduce(hrt_mm_reduce_args p) {
  const int64_t total = p.M * p.N;
  const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i0 >= total) return;
  const HK_G float* w = gcptr<float>(p.ws);
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  if (total % 4 == 0) {
    for (int64_t k = 0; k < p.splits; k += 16) {
      f32x4 v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u)  // splits past the end re-read the last one (in range) and are not added
        v[u] = *reinterpret_cast<const HK_G f32x4*>(w + (k + u < p.splits ? k + u : p.splits - 1) * total + i0);
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (k + u < p.splits) s += v[u];
    }
  } else {
    for (int64_t k = 0; k < p.splits; ++k)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (i0 + e < total) s[e] += w[k * total + i0 + e];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t i = i0 + e;
    if (i >= total) break;
    const int64_t m = i / p.N, n = i % p.N;
    float o = p.alpha * s[e];
    if (p.has_bias) o += p.beta * T::to_f32(gcptr<uint16_t>(p.bias)[m * p.bias_sm + n * p.bias_sn]);
    gptr<uint16_t>(p.c)[m * p.c_sm + n * p.c_sn] = T::from_f32(o);
  }
}

// Vector form of mm_reduce for the common layout (N % 8 == 0, C rows contiguous and 16-byte aligned, the bias
// absent or with contiguous rows): a thread takes 8 consecutive outputs of one row (one division for the
// row), loads exactly the S slices' two 16-byte pieces (four slices' loads in flight at a time), adds them in
// slice order 0, 1, ... exactly as mm_reduce does (bit-identical results) and writes one 16-byte store.
template <typename T>
__global__ __launch_bounds__(256) void mm_reduce_vec(hrt_mm_reduce_args p, int64_t nvec) {
  const int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (v >= nvec) return;
  const int64_t i0 = v * 8, total = p.M * p.N;
  const int64_t m = i0 / p.N, n = i0 - m * p.N;
  const HK_G f32x4* w = gcptr<f32x4>(p.ws) + i0 / 4;
  const int64_t st = total / 4;  // 16-byte pieces per slice
  f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
  int64_t k = 0;
  for (; k + 4 <= p.splits; k += 4) {
    f32x4 a[4], b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) a[u] = w[(k + u) * st], b[u] = w[(k + u) * st + 1];
#pragma unroll
    for (int u = 0; u < 4; ++u) s0 += a[u], s1 += b[u];
  }
  for (; k < p.splits; ++k) s0 += w[k * st], s1 += w[k * st + 1];
  float o[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = p.alpha * s0[e], o[4 + e] = p.alpha * s1[e];
  if (p.has_bias) {
    const u32x4 bb = *reinterpret_cast<const HK_G u32x4*>(gcptr<uint16_t>(p.bias) + m * p.bias_sm + n);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[2 * e] += p.beta * T::to_f32((uint16_t)(bb[e] & 0xffffu));
      o[2 * e + 1] += p.beta * T::to_f32((uint16_t)(bb[e] >> 16));
    }
  }
  u32x4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = (uint32_t)T::from_f32(o[2 * e]) | ((uint32_t)T::from_f32(o[2 * e + 1]) << 16);
  *reinterpret_cast<HK_G u32x4*>(gptr<uint16_t>(p.c) + m * p.c_sm + n) = r;
}

template <typename T>
bool launch_mm_reduce(const void* pp, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_mm_reduce_args*>(pp);
  if (a.M <= 0 || a.N <= 0 || a.splits <= 0) return ctx.fail("empty split-K reduction");
  if (a.c_sm < 0 || a.c_sn < 0 || a.bias_sm < 0 || a.bias_sn < 0) return ctx.fail("negative stride");
  const int64_t total = a.M * a.N;
  if (cdiv(total, 1024) > 0x7fffffffLL) return ctx.fail("reduction grid too large");
  const int64_t sw[3] = {a.splits, a.M, a.N}, tw[3] = {a.M * a.N, a.N, 1};
  const int64_t sc[2] = {a.M, a.N}, tc[2] = {a.c_sm, a.c_sn}, tb[2] = {a.bias_sm, a.bias_sn};
  if (!ctx.check(a.ws, hrt::span_bytes(3, sw, tw, 4), "ws") || !ctx.check(a.c, hrt::span_bytes(2, sc, tc, 2), "c") ||
      (a.has_bias && !ctx.check(a.bias, hrt::span_bytes(2, sc, tb, 2), "bias")))
    return false;
  const bool vec = a.N % 8 == 0 && a.c_sn == 1 && a.c % 16 == 0 && a.c_sm % 8 == 0 && a.ws % 16 == 0 &&
                   (!a.has_bias || (a.bias_sn == 1 && a.bias % 16 == 0 && a.bias_sm % 8 == 0));
  if (vec) {
    const int64_t nvec = total / 8;
    hipLaunchKernelGGL(mm_reduce_vec<T>, dim3((uint32_t)cdiv(nvec, 256)), dim3(256), 0, ctx.stream, a, nvec);
  } else {
    hipLaunchKernelGGL(mm_reduce<T>, dim3((uint32_t)cdiv(total, 1024)), dim3(256), 0, ctx.stream, a);
  }
  return hrt::launch_ok(hipGetLastError(), ctx, "mm_reduce");
}

HRT_REGISTER("mm_mfma_bf16", hrt_mm_args, launch_mm_mfma<BF16>);
HRT_REGISTER("mm_reduce_bf16", hrt_mm_reduce_args, launch_mm_reduce<BF16>);
HRT_REGISTER("mm_reduce_f16", hrt_mm_reduce_args, launch_mm_reduce<F16>);
HRT_REGISTER("mm_mfma_f16", hrt_mm_args, launch_mm_mfma<F16>);
HRT_REGISTER("mm_dq8_bf16", hrt_mm_dq8_args, launch_mm_dq8<BF16>);
HRT_REGISTER("mm_dq8_f16", hrt_mm_dq8_args, launch_mm_dq8<F16>);

}  // namespace
}  // namespace hk
