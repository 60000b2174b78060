// Shared pieces of the gfx950 flash-attention kernels (forward, dK/dV, dQ).
//
// They use v_mfma_f32_32x32x16_{bf16,f16}.  Lane layout (checked on the device), l = lane, h = l / 32:
//   A operand (32 x 16, M x K): lane l holds A[l % 32][8 h + i], i = 0..7
//   B operand (16 x 32, K x N): lane l holds B[8 h + i][l % 32]
//   accumulator (32 x 32):      lane l holds D[8 j + 4 h + r][l % 32] in element 4 j + r (j, r = 0..3)
// A product whose rows are the "fixed" index of a lane (S^T = K Q^T: lane = one query column) therefore
// leaves every lane with 16 of the 32 keys of its query, and the two half-waves together hold the row,
// so a row reduction is a 16-value local reduction plus one lane swap (xor 32).  The same 16 values,
// regrouped as keys {16c + 4h + r} and {16c + 8 + 4h + r}, are directly the 8-value B operand of the next
// product over a 16-key chunk c, provided the other operand is read with the same key order — which is
// why the second operand is staged transposed ([d][key]) in LDS and read as two 64-bit halves.
#pragma once

#include "mfma_common.h"

namespace hk {

template <typename T>
struct Mfma32;
template <>
struct Mfma32<BF16> {
  __device__ __forceinline__ static f32x16 mac(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma32<F16> {
  __device__ __forceinline__ static f32x16 mac(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// 8 consecutive 16-bit elements of one row starting at column d0; zero beyond D.  VEC: one 16-byte load
// (requires D % 8 == 0 and 16-byte aligned rows).
template <bool VEC>
__device__ __forceinline__ u32x4 load_row8(const HK_G uint16_t* row, int d0, int D) {
  if constexpr (VEC) {
    if (d0 < D) return *reinterpret_cast<const HK_G u32x4*>(row + d0);
    return u32x4{0, 0, 0, 0};
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = (d0 + 2 * i < D) ? row[d0 + 2 * i] : 0u;
      const uint32_t hi = (d0 + 2 * i + 1 < D) ? row[d0 + 2 * i + 1] : 0u;
      w[i] = lo | (hi << 16);
    }
    return u32x4{w[0], w[1], w[2], w[3]};
  }
}

// Operand load modes: GATHER = element loads (D % 8 != 0 or unaligned rows); VEC = 16-byte loads with
// columns >= D zeroed; FULL = 16-byte loads, D equals the padded width (no column mask).
enum { LD_GATHER = 0, LD_VEC = 1, LD_FULL = 2 };

// An 8-row x 8-column block of a [rows, D] operand (rows at `row_stride` elements apart), rows >= nrows
// and columns >= D read as zero.  Stored either as rows ([row][d]) or transposed ([d][row]) into LDS.
//
// Staging layout rules that keep the LDS stores conflict-free: blocks are assigned to threads with the
// row-block index fastest, so the 16-byte column stores of one instruction (store_cols) land side by side
// in one LDS row; the row stores (store_rows) then hit rows 8 apart, so row copies XOR-swizzle their
// 16-byte chunk position with (row / 8) (readers use swz()).
struct Block8 {
  u32x4 r[8];
  template <int LM>
  __device__ __forceinline__ void load(const HK_G uint16_t* base, int64_t row_stride, int64_t row0, int64_t nrows, int d0,
                                       int D, bool full_rows) {
    if constexpr (LM != LD_GATHER) {
      if (full_rows && (LM == LD_FULL || d0 < D)) {
        const HK_G uint16_t* p = base + row0 * row_stride + d0;
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = *reinterpret_cast<const HK_G u32x4*>(p + j * row_stride);
        return;
      }
      // ragged stage: clamp to a valid row, then zero (no divergent branches around the loads)
      const bool dok = LM == LD_FULL || d0 < D;
      const int dd = dok ? d0 : 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t rr = row0 + j < nrows ? row0 + j : nrows - 1;
        const u32x4 v = *reinterpret_cast<const HK_G u32x4*>(base + rr * row_stride + dd);
        const bool ok = dok && row0 + j < nrows;
        r[j] = ok ? v : u32x4{0, 0, 0, 0};
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (row0 + j < nrows)
          r[j] = load_row8<false>(base + (row0 + j) * row_stride, d0, D);
        else
          r[j] = u32x4{0, 0, 0, 0};
      }
    }
  }
  // rows (lr0 .. lr0+7) x cols (d0 .. d0+7) into lds[row * ld + col], chunk position swizzled by swz(row)
  template <int NCH>
  __device__ __forceinline__ void store_rows(uint16_t* lds, int ld, int lr0, int d0) const {
#pragma unroll
    for (int j = 0; j < 8; ++j) *reinterpret_cast<u32x4*>(lds + (lr0 + j) * ld + swz_col<NCH>(lr0 + j, d0)) = r[j];
  }
  // transposed: lds[col * ld + row]
  __device__ __forceinline__ void store_cols(uint16_t* lds, int ld, int lr0, int d0) const {
    u32x4 t[8];
    transpose8x8(r, t);
#pragma unroll
    for (int m = 0; m < 8; ++m) *reinterpret_cast<u32x4*>(lds + (d0 + m) * ld + lr0) = t[m];
  }
  // Column (in elements) where the 16-byte chunk starting at column c of `row` is stored, for a row of
  // NCH chunks: chunk index XOR (row / 8), kept inside the row.
  template <int NCH>
  __device__ __forceinline__ static int swz_col(int row, int c) {
    return (((c >> 3) ^ ((row >> 3) & (NCH - 1) & 7)) << 3) | (c & 7);
  }
};

// Two 64-bit LDS reads forming the 8 k-slots {k0 .. k0+3, k0+8 .. k0+11} of an A/B operand.
__device__ __forceinline__ u32x4 lds_pair64(const uint16_t* p) {
  const u32x2 a = *reinterpret_cast<const u32x2*>(p);
  const u32x2 b = *reinterpret_cast<const u32x2*>(p + 8);
  return u32x4{a.x, a.y, b.x, b.y};
}

// Pack accumulator elements 4j0+r (r < 4) then 4j1+r into the 8 k-slots of an operand.
template <typename T>
__device__ __forceinline__ u32x4 pack_slots(const f32x16& s, int j0, int j1) {
  return u32x4{cvt2<T>(s[4 * j0], s[4 * j0 + 1]), cvt2<T>(s[4 * j0 + 2], s[4 * j0 + 3]), cvt2<T>(s[4 * j1], s[4 * j1 + 1]),
               cvt2<T>(s[4 * j1 + 2], s[4 * j1 + 3])};
}

// Workgroup -> (bh, block) so that the blocks of a head land on the same XCD (workgroups are placed on
// the 8 XCDs round-robin by id): each XCD's L2 then holds the K/V (or Q/dO) of only its own heads.
__device__ __forceinline__ void xcd_map(int64_t id, int64_t total, int64_t nblk, int64_t& bh, int64_t& blk) {
  int64_t logical = id;
  if (total % 8 == 0) logical = (id % 8) * (total / 8) + id / 8;
  bh = logical / nblk;
  blk = logical % nblk;
}

// The same mapping in 32-bit arithmetic (grids are below 2^31 workgroups; 64-bit division is a long
// instruction sequence).
__device__ __forceinline__ void xcd_map32(uint32_t id, uint32_t total, uint32_t nblk, uint32_t& bh, uint32_t& blk) {
  uint32_t logical = id;
  if (total % 8 == 0) logical = (id % 8) * (total / 8) + id / 8;
  bh = logical / nblk;
  blk = logical % nblk;
}

// Natural-log constants for the exp2 formulation.
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---- direct global -> LDS staging (gfx950 global_load_lds_dwordx4) -----------------------------------------
//
// One instruction copies 16 bytes per lane and lane i's bytes land at lds_base + 16 i (checked on the
// device), so the LDS layout of a wave's 1 KiB is fixed and any swizzle is applied by choosing which
// global chunk each lane fetches.  Tiles of 16-bit [row][d] data with NCH 16-byte chunks per row are stored
// with chunk c of `row` in slot c ^ swz(row).  swz is chosen so that every reader is conflict-free on the
// 64 x 4-byte LDS banks (a 256-byte bank line; 16 lanes of a 128-bit read, 32 lanes of a 64-bit read per
// cycle):
//   * 128-bit row reads (MFMA A operand, 16 lanes = 16 consecutive rows at one chunk): swz is a bijection
//     on every aligned group of 16 rows (NCH = 16) or of 8 same-parity rows (NCH = 8, two rows per bank line);
//   * ds_read_b64_tr_b16 column reads of the 32x32x16 kernels (4 aligned rows x 4 aligned chunks per 32
//     lanes): the 4 rows differ in swz bits 2..3 (NCH = 16) or, per row parity, in bit 2 (NCH = 8);
//   * ds_read_b64_tr_b16 column reads of the 16x16x32 kernels (8 aligned rows x 2 aligned chunks per 32
//     lanes): the 8 rows differ in swz bits 1..3 (NCH = 16) or, per row parity, in bits 1..2 (NCH = 8).
#define HK_L __attribute__((address_space(3)))

template <int NCH>
__device__ __forceinline__ int tile_swz(int row);
// NCH = 16 (256-byte rows, one row per bank line): slot bits (3, 2, 1, 0) = row bits (1, 0, 2, 3).
template <>
__device__ __forceinline__ int tile_swz<16>(int row) {
  return ((row & 3) << 2) | (((row >> 2) & 1) << 1) | ((row >> 3) & 1);
}
// NCH = 8 (128-byte rows, row bit 0 selects the half bank line): slot bits (2, 1, 0) = row bits (1, 2, 3).
template <>
__device__ __forceinline__ int tile_swz<8>(int row) {
  return (((row >> 1) & 1) << 2) | (((row >> 2) & 1) << 1) | ((row >> 3) & 1);
}

__device__ __forceinline__ void dma16(const HK_G uint8_t* src, HK_L uint8_t* lds_base) {
  __builtin_amdgcn_global_load_lds(reinterpret_cast<HK_G void*>(const_cast<HK_G uint8_t*>(src)), lds_base, 16, 0, 0);
}

// Copy rows [row0, row0 + ROWS) of a 16-bit operand with NCH * 8 columns (row stride `ss` bytes, row0's
// address `src`) into the swizzled LDS tile `tile` (ROWS x NCH chunks), using the 4 wavefronts of the
// workgroup.  Rows at or beyond `valid` are clamped to row valid - 1 (the caller masks their results; the
// duplicated row is real, finite-or-not data that is used anyway).  `lane_off` must not exceed 32 bits,
// which the launchers check.
//
// The wavefront-uniform part of each address (row0 + the instruction's first row) is kept in scalar
// registers.  The per-lane part depends only on the lane and on the instruction index modulo the swizzle
// period (swz uses row bits 0..3 and an instruction covers 64 / NCH rows, so the pattern repeats every
// 16 NCH / 64 instructions, a divisor of 4); full tiles use those loop-invariant lane offsets
// (dma_lane_offsets), ragged tiles recompute clamped offsets.
struct DmaLanes {
  uint32_t off[4];
};
// Lane offsets of instructions j0 .. j0 + 3 (j0 = the wavefront's first instruction index in the tile).
template <int NCH>
__device__ __forceinline__ DmaLanes dma_lane_offsets(uint32_t ss, int lane, int j0) {
  constexpr int RPI = 64 / NCH;
  const int rsub = lane / NCH, slot = lane % NCH;
  DmaLanes d;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = (j0 + i) * RPI + rsub;
    d.off[i] = (uint32_t)rsub * ss + (uint32_t)((slot ^ tile_swz<NCH>(row)) << 4);
  }
  return d;
}
// `lo` must come from dma_lane_offsets with j0 = wave * (ROWS * NCH / 64 / NW).
template <int NCH, int ROWS, int NW>
__device__ __forceinline__ void dma_tile(const HK_G uint8_t* src, uint32_t ss, int valid, HK_L uint8_t* tile, int wave,
                                         int lane, const DmaLanes& lo) {
  constexpr int RPI = 64 / NCH;               // rows per instruction
  constexpr int IPW = ROWS * NCH / 64 / NW;   // instructions per wavefront
  constexpr int PERIOD = 16 / RPI;            // swizzle period in instructions
  static_assert(IPW * NW * 64 == ROWS * NCH && 4 % PERIOD == 0, "tile / wavefront split");
  if (valid >= ROWS) {
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      const int j = wave * IPW + i;
      dma16(src + (uint32_t)(j * RPI) * ss + lo.off[i % 4], tile + j * 1024);
    }
  } else {
    const int rsub = lane / NCH, slot = lane % NCH;
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      const int j = wave * IPW + i;
      const int row = j * RPI + rsub;
      const int r = row < valid ? row : valid - 1;
      dma16(src + ((uint32_t)r * ss + (uint32_t)((slot ^ tile_swz<NCH>(row)) << 4)), tile + j * 1024);
    }
  }
}

// Instruction i (0 .. IPW-1) of this wavefront's share of a full tile copy: rows [0, ROWS) at `src` all
// exist (no clamping, no branch), so a caller can place the copies one by one between its MFMAs instead of
// issuing the whole tile in one burst (a burst of 1 KiB copies from every wavefront stalls each of them at
// issue until the address unit has drained the others).
template <int NCH, int ROWS, int NW>
__device__ __forceinline__ void dma_tile_part(const HK_G uint8_t* src, uint32_t ss, HK_L uint8_t* tile, int wave,
                                              const DmaLanes& lo, int i) {
  constexpr int RPI = 64 / NCH;
  constexpr int IPW = ROWS * NCH / 64 / NW;
  const int j = wave * IPW + i;
  dma16(src + (uint32_t)(j * RPI) * ss + lo.off[i % 4], tile + j * 1024);
}

// First row of the tile that stage st copies when the sequence has more than one stage (len > ROWS): stage
// st covers rows [st ROWS, (st + 1) ROWS); the last, ragged stage copies the full window that ends at row
// len - 1 instead (origin len - ROWS), so no copy reads past the sequence, and its rows below st ROWS
// (processed by the previous stage) are masked by the caller.  Stages past the end repeat the last one.
template <int ROWS>
__device__ __forceinline__ int64_t stage_origin(int st, int nst, int64_t len) {
  const int s = st < nst ? st : nst - 1;
  const int64_t o = (int64_t)s * ROWS;
  return o + ROWS <= len ? o : len - ROWS;
}

// 16 bytes of a swizzled tile at (row, chunk c), as a byte offset.
template <int NCH>
__device__ __forceinline__ int tile_off(int row, int c) {
  return row * (NCH * 16) + ((c ^ tile_swz<NCH>(row)) << 4);
}

// ds_read_b64_tr_b16 on 16-bit data: within each group of 16 lanes, if lane s addresses row k0 + (s >> 2),
// columns n0 + 4 (s & 3) .. +3 of a row-major matrix X, lane j receives X[k0 + e][n0 + j] for e = 0..3
// (checked on the device) -- a column read of 4 consecutive rows.
typedef short i16x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 lds_tr4(const HK_L uint8_t* p) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((HK_L i16x4_t*)p));
}

// Max of the two half-waves' values (lane and lane ^ 32) without an LDS round trip.
__device__ __forceinline__ float halfswap_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halfswap_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace hk
