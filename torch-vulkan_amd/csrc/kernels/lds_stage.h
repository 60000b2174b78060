// LDS staging and matrix-core fragment helpers shared by the gfx950 attention and GEMM kernels:
// v_mfma_f32_32x32x16 wrappers, direct global -> LDS tile copies with a bank swizzle, transpose reads.
//
// v_mfma_f32_32x32x16_{bf16,f16} lane layout (checked on the device), l = lane, h = l / 32:
//   A operand (32 x 16, M x K): lane l holds A[l % 32][8 h + i], i = 0..7
//   B operand (16 x 32, K x N): lane l holds B[8 h + i][l % 32]
//   accumulator (32 x 32):      lane l holds D[8 j + 4 h + r][l % 32] in element 4 j + r (j, r = 0..3)
#pragma once

#include <type_traits>

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

// SW = 0: the layouts above.  SW = 1 (NCH = 16 only): the layout of the 16x16x32 kernels' tiles (dK/dV),
// whose 128-bit A-operand reads (16 rows x 4 chunks per wavefront) are 2-way conflicted under SW = 0 on the
// device although that layout gives every 16 consecutive lanes distinct banks; slot = chunk ^ (row bits
// 0..3 -> 2, 8, 14, 13), found by measuring 200 XOR maps on the device (SQ_LDS_BANK_CONFLICT): zero
// conflicts for those reads and for the kernels' transpose reads (8 rows x 2 chunks per 32 lanes) at every
// chunk offset.
template <int NCH, int SW = 0>
__device__ __forceinline__ int tile_swz(int row) {
  static_assert(SW == 0 || NCH == 16, "the second layout exists for 256-byte rows only");
  if constexpr (NCH == 16 && SW == 1) {
    return (-(row & 1) & 2) ^ (-((row >> 1) & 1) & 8) ^ (-((row >> 2) & 1) & 14) ^ (-((row >> 3) & 1) & 13);
  } else if constexpr (NCH == 16) {
    // 256-byte rows, one row per bank line: slot bits (3, 2, 1, 0) = row bits (1, 0, 2, 3)
    return ((row & 3) << 2) | (((row >> 2) & 1) << 1) | ((row >> 3) & 1);
  } else if constexpr (NCH == 8) {
    // 128-byte rows, row bit 0 selects the half bank line: slot bits (2, 1, 0) = row bits (1, 2, 3)
    return (((row >> 1) & 1) << 2) | (((row >> 2) & 1) << 1) | ((row >> 3) & 1);
  } else if constexpr (NCH == 32) {
    // 512-byte rows (two bank lines per row), read only column-wise by the 32x32x16 transpose reads
    // (4 aligned rows x 4 aligned chunks per 32 lanes): slot bits (3, 2) = row bits (1, 0)
    return (row & 3) << 2;
  } else {
    static_assert(NCH == 4, "tile width");
    return 0;  // 64-byte rows of int8 staging tiles, read linearly
  }
}
// Rows after which tile_swz repeats.
template <int NCH>
constexpr int swz_period_rows() {
  return NCH == 32 ? 4 : 16;
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
template <int NCH, int SW = 0>
__device__ __forceinline__ DmaLanes dma_lane_offsets(uint32_t ss, int lane, int j0) {
  constexpr int RPI = 64 / NCH;
  const int rsub = lane / NCH, slot = lane % NCH;
  DmaLanes d;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = (j0 + i) * RPI + rsub;
    d.off[i] = (uint32_t)rsub * ss + (uint32_t)((slot ^ tile_swz<NCH, SW>(row)) << 4);
  }
  return d;
}
// `lo` must come from dma_lane_offsets with j0 = wave * (ROWS * NCH / 64 / NW).
template <int NCH, int ROWS, int NW, int SW = 0>
__device__ __forceinline__ void dma_tile(const HK_G uint8_t* src, uint32_t ss, int valid, HK_L uint8_t* tile, int wave,
                                         int lane, const DmaLanes& lo) {
  constexpr int RPI = 64 / NCH;               // rows per instruction
  constexpr int IPW = ROWS * NCH / 64 / NW;   // instructions per wavefront
  constexpr int PERIOD = swz_period_rows<NCH>() / RPI > 0 ? swz_period_rows<NCH>() / RPI : 1;  // in instructions
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
      dma16(src + ((uint32_t)r * ss + (uint32_t)((slot ^ tile_swz<NCH, SW>(row)) << 4)), tile + j * 1024);
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

// The same copy through a raw buffer resource (buffer_load_dwordx4 ... lds, same LDS layout: lane i's 16
// bytes at the instruction's LDS base + 16 i, checked on the device): the resource holds the 64-bit base in
// scalar registers and the wavefront-uniform row offset goes in the scalar offset, so a copy needs no
// per-lane 64-bit address arithmetic, only the 32-bit lane offsets of dma_lane_offsets.  The range check
// is disabled (num_records = 2^32 - 1): callers copy only rows that exist.  Word 3 = 0x00020000 selects the
// 32-bit data format used for raw byte-addressed buffers on CDNA.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dma_rsrc(const HK_G uint8_t* base) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)(base), (short)0, -1, 0x00020000);
}
template <int NCH, int ROWS, int NW>
__device__ __forceinline__ void dma_tile_part_rs(__amdgpu_buffer_rsrc_t rs, uint32_t ss, HK_L uint8_t* tile, int wave,
                                                 const DmaLanes& lo, int i) {
  constexpr int RPI = 64 / NCH;
  constexpr int IPW = ROWS * NCH / 64 / NW;
  const int j = wave * IPW + i;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, tile + j * 1024, 16, (int)lo.off[i % 4], (int)((uint32_t)(j * RPI) * ss), 0, 0);
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
template <int NCH, int SW = 0>
__device__ __forceinline__ int tile_off(int row, int c) {
  return row * (NCH * 16) + ((c ^ tile_swz<NCH, SW>(row)) << 4);
}

// ds_read_b64_tr_b16 on 16-bit data: within each group of 16 lanes, if lane s addresses row k0 + (s >> 2),
// columns n0 + 4 (s & 3) .. +3 of a row-major matrix X, lane j receives X[k0 + e][n0 + j] for e = 0..3
// (checked on the device) -- a column read of 4 consecutive rows.
typedef short i16x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 lds_tr4(const HK_L uint8_t* p) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((HK_L i16x4_t*)p));
}

// Workgroup barrier that lets the N most recently issued vector-memory operations of this wavefront (the
// copies of a later stage) stay in flight: waits until at most N are outstanding, then joins the barrier.
// __syncthreads() would wait for all of them (its release fence waits for every outstanding load).  The
// wait is the s_waitcnt builtin (vmcnt in bits 3:0 and 15:14, expcnt 7 and lgkmcnt 15 = no wait), which
// the compiler's wait-insertion pass takes into account: reads of a stage whose copies it has seen
// complete get no further wait.  The barrier is an asm statement with a memory clobber, so the compiler
// moves no memory access across it.
template <int N>
__device__ __forceinline__ void barrier_keep_vm() {
  static_assert(N >= 0 && N < 64, "the vmcnt field holds 0..63");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("s_barrier" ::: "memory");
}

// The same, also waiting for this wavefront's LDS accesses (for stages that write LDS with ds_write before
// the barrier that publishes them).
template <int N>
__device__ __forceinline__ void barrier_keep_vm_lds() {
  static_assert(N >= 0 && N < 64, "the vmcnt field holds 0..63");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
  asm volatile("s_barrier" ::: "memory");
}

// Keeps the compiler from moving memory accesses (copies included) across this point, so that the copies
// before it are issued before those after it, as barrier_keep_vm's count assumes.
__device__ __forceinline__ void issue_order_fence() { asm volatile("" ::: "memory"); }

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
