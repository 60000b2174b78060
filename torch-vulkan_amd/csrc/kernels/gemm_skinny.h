// Products of a low-rank adapter (rank r <= 32) that the tiled GEMM serves badly.
//
// 1. A short reduction dimension (K <= 32): the up-projection of a low-rank adapter, y = h B^T
// (h [M, r], B [N, r]) and its backward dx = dh A (A [r, K_in]), K = the rank.  Their cost is the output
// (M x N written, and read again when accumulated), not the arithmetic, so they are HBM-bound; the matrix
// cores would spend one instruction per 16x16 output block and leave the output to an epilogue through LDS.
// Here every lane owns 8 consecutive outputs of a row (one 16-byte store), keeps its 8 columns of the K x N
// factor in registers as bf16 pairs for the whole launch, and forms each output with K/2 v_dot2 steps whose
// other operand (the row of h, identical across the wavefront) comes from scalar loads.
#pragma once

#include <type_traits>

#include "lds_stage.h"
#include "mfma_common.h"

namespace hk {
namespace skinny {

// u32 holding two consecutive-k bf16 / f16 values -> fp32 sum of products with another such pair, plus acc.
template <typename T>
__device__ __forceinline__ float dot2(uint32_t x, uint32_t y, float acc);
template <>
__device__ __forceinline__ float dot2<BF16>(uint32_t x, uint32_t y, float acc) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, x), __builtin_bit_cast(b2, y), acc, false);
}
template <>
__device__ __forceinline__ float dot2<F16>(uint32_t x, uint32_t y, float acc) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, x), __builtin_bit_cast(h2, y), acc, false);
}

template <typename T>
__device__ __forceinline__ void unpack8(u32x4 w, float* v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = lo16<T>(w[i]);
    v[2 * i + 1] = hi16<T>(w[i]);
  }
}

// C[m, n] = alpha * sum_k A[m, k] B[k, n] + beta * X[m, n], X = the bias view (which may be C itself: an
// accumulating product) or nothing.  KP = K / 2 pairs.  BT: B is k-contiguous (B[k, n] at b + n*b_sn + k,
// the transposed view of an [N, K] weight); else n-contiguous rows.  Workgroup = four wavefronts over the
// same 512 columns (8 per lane), RB rows each.  Every load of a wavefront is issued before the first use
// (one round trip to memory): its lane's 8 columns of B, its 8 columns of the RB rows of X, and the RB x K
// block of A spread over the lanes (lane l holds pair l of the block), from which each row's pairs go to
// scalar registers.  B laid out along k (K a multiple of 8) is read once per workgroup in coalesced 16-byte
// chunks and handed to the lanes through LDS (a lane's 8 columns are 16 K contiguous bytes: read per lane,
// each 16-byte load would touch 64 cache lines); the chunks of a lane's row are XOR-swizzled so that the
// lanes' 128-bit reads of one chunk index fall on distinct banks.
constexpr int kExpandRows = 8, kExpandWaves = 4;
template <typename T, int KP, bool BT, bool HASX>
__global__ __launch_bounds__(kExpandWaves * 64) void mm_expand(hrt_mm_args a) {
  using S = uint16_t;
  constexpr int RB = kExpandRows, HV = (RB * KP + 63) / 64, K = 2 * KP;
  constexpr bool SHARED = BT && K % 8 == 0;   // B through LDS
  constexpr int CPC = K / 8, CPR = K;         // 16-byte chunks per column / per lane's 8 columns
  constexpr int CPT = SHARED ? 64 * CPR / (kExpandWaves * 64) : 1;  // chunks loaded per thread
  __shared__ __attribute__((aligned(16))) u32x4 fl[SHARED ? 64 * CPR : 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t nb0 = (int64_t)blockIdx.x * 512, n0 = nb0 + lane * 8;
  const bool live_n = n0 < a.N;
  const int64_t nl = live_n ? n0 : a.N - 8;  // lanes past the end work on the last 8 columns, store nothing
  const int64_t m0 = ((int64_t)blockIdx.y * kExpandWaves + wave) * RB;
  const HK_G S* A = gcptr<S>(a.a);
  const HK_G S* B = gcptr<S>(a.b);
  uint32_t bw[8][KP];  // bw[c][j] = (B[2j, n+c], B[2j+1, n+c])
  u32x4 fc[CPT];
  if constexpr (SHARED) {  // chunk t of the block: column t / CPC, k = 8 (t % CPC) .. +7
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int t = tid + kExpandWaves * 64 * i;
      const int64_t n = nb0 + t / CPC < a.N ? nb0 + t / CPC : a.N - 1;
      fc[i] = *reinterpret_cast<const HK_G u32x4*>(B + n * a.b_sn + 8 * (t % CPC));
    }
    issue_order_fence();
  }
  // the A block: pair p = lane + 64 i is (row p / KP, pair p % KP); rows past the end repeat the last row
  uint32_t hblk[HV];
#pragma unroll
  for (int i = 0; i < HV; ++i) {
    const int p = lane + 64 * i < RB * KP ? lane + 64 * i : RB * KP - 1;
    const int64_t m = m0 + p / KP < a.M ? m0 + p / KP : a.M - 1;
    hblk[i] = reinterpret_cast<const HK_G uint32_t*>(A + m * a.a_sm)[p % KP];
  }
  u32x4 xv[RB];
  if constexpr (HASX) {
    const HK_G S* X = gcptr<S>(a.bias);
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int64_t m = m0 + r < a.M ? m0 + r : a.M - 1;
      xv[r] = *reinterpret_cast<const HK_G u32x4*>(X + m * a.bias_sm + nl);
    }
  }
  if constexpr (SHARED) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int t = tid + kExpandWaves * 64 * i;
      const int c = t / CPC, L = c / 8, sl = (c % 8) * CPC + t % CPC;
      fl[L * CPR + (sl ^ (L & (CPR - 1)))] = fc[i];
    }
    barrier_keep_vm_lds<HV + (HASX ? RB : 0)>();  // the chunks are in LDS; the row loads stay in flight
#pragma unroll
    for (int sl = 0; sl < CPR; ++sl) {
      const u32x4 v = fl[lane * CPR + (sl ^ (lane & (CPR - 1)))];
#pragma unroll
      for (int e = 0; e < 4; ++e) bw[sl / CPC][4 * (sl % CPC) + e] = v[e];
    }
  } else if constexpr (BT) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const HK_G uint32_t* col = reinterpret_cast<const HK_G uint32_t*>(B + (nl + c) * a.b_sn);
#pragma unroll
      for (int j = 0; j < KP; ++j) bw[c][j] = col[j];
    }
  } else {
    u32x4 rows[2 * KP];
#pragma unroll
    for (int k = 0; k < 2 * KP; ++k) rows[k] = *reinterpret_cast<const HK_G u32x4*>(B + k * a.b_sk + nl);
#pragma unroll
    for (int j = 0; j < KP; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // columns 2i, 2i+1: low / high halves of row 2j and 2j+1
        bw[2 * i][j] = (rows[2 * j][i] & 0xffffu) | (rows[2 * j + 1][i] << 16);
        bw[2 * i + 1][j] = (rows[2 * j][i] >> 16) | (rows[2 * j + 1][i] & 0xffff0000u);
      }
  }
  HK_G S* C = gptr<S>(a.c);
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    uint32_t h2[KP];
#pragma unroll
    for (int j = 0; j < KP; ++j) h2[j] = __builtin_amdgcn_readlane(hblk[(r * KP + j) / 64], (r * KP + j) % 64);
    float o[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < KP; ++j) acc = dot2<T>(h2[j], bw[c][j], acc);
      o[c] = a.alpha * acc;
    }
    if constexpr (HASX) {
      float xf[8];
      unpack8<T>(xv[r], xf);
#pragma unroll
      for (int c = 0; c < 8; ++c) o[c] = fmaf(a.beta, xf[c], o[c]);
    }
    const u32x4 out = pack8<T>(o);
    if (live_n && m0 + r < a.M) *reinterpret_cast<HK_G u32x4*>(C + (m0 + r) * a.c_sm + n0) = out;
  }
}

// Queues mm_expand when the product fits it: K even and <= 32, one batch, a 16-byte-aligned output with
// unit column stride, A rows k-contiguous and 4-byte aligned, B either k- or n-contiguous with 16-byte
// aligned vectors, N a multiple of 8, and the bias (if any) a full [M, N] view like C's or a row broadcast.
template <typename T>
bool queue_expand(const hrt_mm_args& a, hipStream_t s) {
  const int64_t K = a.K;
  if (K < 2 || K > 32 || K % 2 || a.batch != 1 || a.M <= 0 || a.N < 8 || a.N % 8) return false;
  if (a.c % 16 || a.c_sn != 1 || a.c_sm % 8) return false;
  if (a.a % 4 || a.a_sk != 1 || a.a_sm % 2) return false;
  // k-contiguous B: 4-byte pairs per column; with K a multiple of 8 the 16-byte chunks read through LDS
  const bool bt = a.b_sk == 1 && a.b_sn % 2 == 0 && a.b % 4 == 0 && (K % 8 != 0 || (a.b_sn % 8 == 0 && a.b % 16 == 0));
  const bool bn = a.b_sn == 1 && a.b_sk % 8 == 0 && a.b % 16 == 0;
  if (!bt && !bn) return false;
  const bool hasx = a.has_bias && a.beta != 0.f;
  if (hasx && (a.bias % 16 || a.bias_sn != 1 || (a.bias_sm != 0 && a.bias_sm % 8))) return false;
  if (a.M > 0x7fffffffLL || a.N > 0x7fffffffLL) return false;
  const int64_t nb = (a.N + 511) / 512, mb = (a.M + kExpandRows * kExpandWaves - 1) / (kExpandRows * kExpandWaves);
  if (mb > 65535) return false;
  const dim3 grid((uint32_t)nb, (uint32_t)mb);
  auto go = [&](auto kp, auto btc, auto hxc) {
    hipLaunchKernelGGL((mm_expand<T, decltype(kp)::value, decltype(btc)::value, decltype(hxc)::value>), grid, dim3(kExpandWaves * 64), 0, s, a);
  };
  auto by_x = [&](auto kp, auto btc) {
    if (hasx) go(kp, btc, std::true_type());
    else go(kp, btc, std::false_type());
  };
  auto by_b = [&](auto kp) {
    if (bt) by_x(kp, std::true_type());
    else by_x(kp, std::false_type());
  };
  switch (K / 2) {
    case 1: by_b(std::integral_constant<int, 1>()); break;
    case 2: by_b(std::integral_constant<int, 2>()); break;
    case 4: by_b(std::integral_constant<int, 4>()); break;
    case 8: by_b(std::integral_constant<int, 8>()); break;
    case 16: by_b(std::integral_constant<int, 16>()); break;
    default: return false;  // other ranks keep the matrix-core path
  }
  return true;
}

// 2. A narrow output (one of M, N <= 16): the down-projection h = x A^T, and the backward products
// dh = g B, dB = g^T h, dA = dh^T x.  They read one large matrix once and write a thin one, so they are
// bound by that read; the 64-wide tiles of the general kernel spend three quarters of the matrix-core work
// on padding and copy the small factor through LDS per tile.  Here the product is normalised to
// Out[P x R] = X[P x Q] Y[Q x R] with R <= 16 (the narrow side): a workgroup of eight wavefronts owns 16
// rows of Out, the wavefronts split the reduction (32 values of Q per step, wavefront w taking steps w,
// w + 8, ...), each accumulates one 16 x 16 v_mfma_f32_16x16x32 tile, and the eight tiles are added through
// LDS in wavefront order (deterministic).  Operand fragments hold 8 consecutive Q per lane: an operand
// contiguous along Q loads straight from memory in 16-byte vectors; one contiguous along P or R (g^T, x^T,
// h, B) loads as [32 q x 16] blocks of 16-byte vectors and is transposed through a wavefront-private LDS
// tile; other layouts of the small factor load as 2-byte gathers.  The loads of kNarrowUnroll steps are
// issued before their matrix-core work.  The batch index (blockIdx.y) lets the caller split Q across
// workgroups (batch entry s = slice s of Q) with fp32 partial outputs that a second kernel adds in order.
struct NarrowArgs {
  uint64_t x, y, c, bias;
  int64_t P, Q, R;
  int64_t x_sb, x_sp, x_sq, y_sb, y_sq, y_sr, c_sb, c_sp, c_sr, b_sb, b_sp, b_sr;
  float alpha, beta;
  uint32_t has_bias, f32out;
};
constexpr int kNarrowWaves = 8, kNarrowUnroll = 4, kNarrowLdsRow = 24;  // LDS row: 16 values + 8 pad (48 B)
enum NarrowLayout { kAlongQ = 0, kBlocked = 1, kGather = 2 };

// 16-byte load of 8 values at base + off, zeros where !ok: the address falls back to base itself (always
// valid) and the value is selected afterwards, so the loads of a step carry no branches between them.
__device__ __forceinline__ u32x4 narrow_load(const HK_G uint16_t* base, int64_t off, bool ok) {
  const u32x4 v = *reinterpret_cast<const HK_G u32x4*>(base + (ok ? off : 0));
  return ok ? v : u32x4{0, 0, 0, 0};
}

// Fragment of 8 consecutive q (rows 8g .. 8g+7 of a [32][kNarrowLdsRow] tile) for column i, packed in pairs.
__device__ __forceinline__ u32x4 narrow_lds_fragment(const uint16_t* t, int i, int g) {
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    w[k] = (uint32_t)t[(8 * g + 2 * k) * kNarrowLdsRow + i] | ((uint32_t)t[(8 * g + 2 * k + 1) * kNarrowLdsRow + i] << 16);
  return u32x4{w[0], w[1], w[2], w[3]};
}

// One [32 q x 16] block through the wavefront's LDS tile: lane l wrote row l/2, columns 8 (l & 1) .. +7; the
// tile is reused for the next block right away (a wavefront's LDS accesses complete in issue order, and
// the empty asm statements with a memory clobber keep the compiler from moving them across each other).
__device__ __forceinline__ u32x4 narrow_transpose(uint16_t* t, u32x4 v, int lane, int i, int g) {
  asm volatile("" ::: "memory");
  *reinterpret_cast<u32x4*>(t + (lane >> 1) * kNarrowLdsRow + 8 * (lane & 1)) = v;
  asm volatile("" ::: "memory");
  const u32x4 f = narrow_lds_fragment(t, i, g);
  asm volatile("" ::: "memory");
  return f;
}

template <typename T, int XL, int YL, bool F32>
__global__ __launch_bounds__(kNarrowWaves * 64) void mm_narrow(NarrowArgs n) {
  constexpr int NW = kNarrowWaves, U = kNarrowUnroll, LR = kNarrowLdsRow;
  constexpr bool TILE = XL == kBlocked || YL == kBlocked;
  __shared__ __attribute__((aligned(16))) uint16_t lt[TILE ? NW * 32 * LR : 8];
  __shared__ __attribute__((aligned(16))) f32x4 red[NW][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, g = lane >> 4;
  // XCD-aware order: workgroups are dealt to the eight XCDs in turn, so consecutive tiles (which share the
  // cache lines of an operand laid out along P) are given to one XCD when the row count allows
  const uint32_t nb = gridDim.x, bx = blockIdx.x;
  const uint32_t tile = nb % 8 == 0 ? (bx % 8) * (nb / 8) + bx / 8 : bx;
  const int64_t p0 = (int64_t)tile * 16, z = blockIdx.y;
  const int64_t nsteps = (n.Q + 31) / 32;
  const HK_G uint16_t* X = gcptr<uint16_t>(n.x) + z * n.x_sb;
  const HK_G uint16_t* Y = gcptr<uint16_t>(n.y) + z * n.y_sb;
  uint16_t* const tw = lt + (TILE ? wave * 32 * LR : 0);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int64_t s0 = wave; s0 < nsteps; s0 += NW * U) {
    u32x4 xa[U], yb[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t q = (s0 + (int64_t)u * NW) * 32;  // q >= Q for steps past the end: zeros
      if constexpr (XL == kAlongQ) {
        const int64_t p = p0 + i, qq = q + 8 * g;
        xa[u] = narrow_load(X, p * n.x_sp + qq, p < n.P && qq < n.Q);
      } else {  // X^T row q + lane/2, P columns 8 (lane & 1) .. +7
        const int64_t qr = q + (lane >> 1), pp = p0 + 8 * (lane & 1);
        xa[u] = narrow_load(X, qr * n.x_sq + pp, qr < n.Q && pp < n.P);
      }
      if constexpr (YL == kAlongQ) {
        const int64_t qq = q + 8 * g;
        yb[u] = narrow_load(Y, i * n.y_sr + qq, i < n.R && qq < n.Q);
      } else if constexpr (YL == kBlocked) {  // Y row q + lane/2, R columns 8 (lane & 1) .. +7 (R a multiple of 8)
        const int64_t qr = q + (lane >> 1);
        const int r = 8 * (lane & 1);
        yb[u] = narrow_load(Y, qr * n.y_sq + r, qr < n.Q && r < n.R);
      } else {
        uint32_t w[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int64_t qa = q + 8 * g + 2 * t;
          const uint32_t lo = i < n.R && qa < n.Q ? Y[qa * n.y_sq + i * n.y_sr] : 0u;
          const uint32_t hi = i < n.R && qa + 1 < n.Q ? Y[(qa + 1) * n.y_sq + i * n.y_sr] : 0u;
          w[t] = lo | (hi << 16);
        }
        yb[u] = u32x4{w[0], w[1], w[2], w[3]};
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (XL == kBlocked) xa[u] = narrow_transpose(tw, xa[u], lane, i, g);
      if constexpr (YL == kBlocked) yb[u] = narrow_transpose(tw, yb[u], lane, i, g);
      acc = Mfma<T>::mac(xa[u], yb[u], acc);
    }
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  f32x4 sum = red[0][lane];
#pragma unroll
  for (int w = 1; w < NW; ++w) sum += red[w][lane];
  if (i >= n.R) return;
  const HK_G uint16_t* Bs = gcptr<uint16_t>(n.bias) + z * n.b_sb;
#pragma unroll
  for (int r = 0; r < 4; ++r) {  // lane holds Out[p0 + 4g + r][i]
    const int64_t p = p0 + 4 * g + r;
    if (p >= n.P) continue;
    float o = n.alpha * sum[r];
    if (n.has_bias) o += n.beta * T::to_f32(Bs[p * n.b_sp + i * n.b_sr]);
    if constexpr (F32) gptr<float>(n.c)[z * n.c_sb + p * n.c_sp + i * n.c_sr] = o;
    else gptr<uint16_t>(n.c)[z * n.c_sb + p * n.c_sp + i * n.c_sr] = T::from_f32(o);
  }
}

// Queues mm_narrow when the product fits it: one of M, N <= 16 (the other side is P), X contiguous along Q
// or along P with 16-byte aligned vectors (any batch, fp32 or rounded output).  Returns false otherwise.
template <typename T>
bool queue_narrow(const hrt_mm_args& a, hipStream_t s) {
  if (a.batch <= 0 || a.batch > 65535 || a.M <= 0 || a.N <= 0 || a.K <= 0) return false;
  NarrowArgs n{};
  if (a.N <= 16) {  // Out = C, X = A, Y = B
    n.x = a.a, n.y = a.b, n.P = a.M, n.R = a.N;
    n.x_sb = a.a_sb, n.x_sp = a.a_sm, n.x_sq = a.a_sk, n.y_sb = a.b_sb, n.y_sq = a.b_sk, n.y_sr = a.b_sn;
    n.c_sp = a.c_sm, n.c_sr = a.c_sn, n.b_sp = a.bias_sm, n.b_sr = a.bias_sn;
  } else if (a.M <= 16) {  // Out = C^T, X = B^T, Y = A^T
    n.x = a.b, n.y = a.a, n.P = a.N, n.R = a.M;
    n.x_sb = a.b_sb, n.x_sp = a.b_sn, n.x_sq = a.b_sk, n.y_sb = a.a_sb, n.y_sq = a.a_sk, n.y_sr = a.a_sm;
    n.c_sp = a.c_sn, n.c_sr = a.c_sm, n.b_sp = a.bias_sn, n.b_sr = a.bias_sm;
  } else {
    return false;
  }
  n.c = a.c, n.c_sb = a.c_sb, n.b_sb = a.bias_sb, n.Q = a.K, n.bias = a.bias;
  n.alpha = a.alpha, n.beta = a.beta, n.has_bias = a.has_bias && a.beta != 0.f;
  n.f32out = (a.flags & HRT_MM_F32_OUT) != 0;
  auto vec = [](uint64_t base, int64_t sb, int64_t batch) { return base % 16 == 0 && (batch == 1 || sb % 8 == 0); };
  const bool xv = vec(n.x, n.x_sb, a.batch), yv = vec(n.y, n.y_sb, a.batch);
  int xl, yl;
  if (xv && n.x_sq == 1 && n.x_sp % 8 == 0 && n.Q % 8 == 0) xl = kAlongQ;
  else if (xv && n.x_sp == 1 && n.x_sq % 8 == 0 && n.P % 8 == 0) xl = kBlocked;
  else return false;
  if (yv && n.y_sq == 1 && n.y_sr % 8 == 0 && n.Q % 8 == 0) yl = kAlongQ;
  else if (yv && n.y_sr == 1 && n.y_sq % 8 == 0 && n.R % 8 == 0) yl = kBlocked;
  else yl = kGather;
  const int64_t blocks = (n.P + 15) / 16;
  if (blocks > 0x7fffffffLL) return false;
  const dim3 grid((uint32_t)blocks, (uint32_t)a.batch), blk(kNarrowWaves * 64);
  const int key = (xl * 3 + yl) * 2 + (n.f32out ? 1 : 0);
  switch (key) {
#define HK_NARROW_CASE(XL, YL, F)                                                      \
  case (XL * 3 + YL) * 2 + F:                                                          \
    hipLaunchKernelGGL((mm_narrow<T, XL, YL, F != 0>), grid, blk, 0, s, n);            \
    return true;
    HK_NARROW_CASE(0, 0, 0) HK_NARROW_CASE(0, 1, 0) HK_NARROW_CASE(0, 2, 0)
    HK_NARROW_CASE(1, 0, 0) HK_NARROW_CASE(1, 1, 0) HK_NARROW_CASE(1, 2, 0)
    HK_NARROW_CASE(0, 0, 1) HK_NARROW_CASE(0, 1, 1) HK_NARROW_CASE(0, 2, 1)
    HK_NARROW_CASE(1, 0, 1) HK_NARROW_CASE(1, 1, 1) HK_NARROW_CASE(1, 2, 1)
#undef HK_NARROW_CASE
    default: return false;
  }
}

}  // namespace skinny
}  // namespace hk
