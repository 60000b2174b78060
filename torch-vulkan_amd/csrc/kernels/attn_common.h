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

#include "lds_stage.h"

namespace hk {

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

}  // namespace hk
