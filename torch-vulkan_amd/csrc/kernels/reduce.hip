// "reduce_sum": sum and mean over any subset of the dimensions of a strided view (bias gradients,
// losses, statistics).  Reference: try_reduce csrc/ops_rows.cpp:183-270 with
// vkrt/shaders/reduce.comp.in:1-45 (one 256-thread workgroup per output, strided loads).
//
// Layout on MI355X.  Reductions are HBM-bound (every input element is read once), so the kernel is chosen
// by which dimension of x is contiguous, so that a wavefront always reads consecutive memory:
//   * columns (the contiguous dimension is kept: a bias gradient sum over rows): lanes own consecutive
//     outputs, V of them each, and walk the reduced coordinates with 16-byte loads, 16 in flight; the
//     four wavefronts of a workgroup take quarters of the coordinates and add up through LDS;
//   * rows (the contiguous dimension is reduced: row sums, full sums): a wavefront per output for short
//     rows, else a workgroup per output (and split) streaming 16-byte loads, 4 in flight;
//   * any other layout: the column kernel with one output per lane.
// When there are too few outputs to fill the GPU, the reduced range is split over up to 1024 workgroups;
// each writes fp32 partial sums and a second pass adds them in split order, so results never depend on
// scheduling.  Accumulation is fp32; the result is divided by `div` and rounded once.
#include <algorithm>
#include <string>

#include "../hrt/registry.h"
#include "device_common.h"

namespace hk {
namespace {

enum { RED_COLS = 0, RED_ROWS = 1 };

struct RedPlan {
  int mode = RED_COLS, V = 1;
  int nk = 0, nr = 0;
  int64_t ksz[HRT_MAX_DIMS], kst[HRT_MAX_DIMS], rsz[HRT_MAX_DIMS], rst[HRT_MAX_DIMS];
  int64_t n_out = 1, n_red = 1, splits = 1, per_split = 0;
};

struct RedKArgs {
  uint64_t x, out, ws;
  int odt, nk, nr, pad;
  int64_t ksz[HRT_MAX_DIMS], kst[HRT_MAX_DIMS], rsz[HRT_MAX_DIMS], rst[HRT_MAX_DIMS];
  int64_t n_out, n_red, per_split, splits;
  float div;
};

uint64_t esize(int dt) { return dt == HRT_F32 ? 4 : 2; }
bool is_float_dt(int dt) { return dt == HRT_F32 || dt == HRT_BF16 || dt == HRT_F16; }

// Drop size-1 dimensions and merge neighbours that are consecutive in memory.
int merge(int n, const int64_t* sz, const int64_t* st, int64_t* osz, int64_t* ost) {
  int m = 0;
  for (int d = 0; d < n; ++d) {
    if (sz[d] == 1) continue;
    if (m > 0 && ost[m - 1] == st[d] * sz[d]) {
      osz[m - 1] *= sz[d];
      ost[m - 1] = st[d];
    } else {
      osz[m] = sz[d];
      ost[m] = st[d];
      ++m;
    }
  }
  return m;
}

bool plan_reduce(const hrt_reduce_args& a, RedPlan& P, std::string& err) {
  if (a.ndim < 0 || a.ndim > HRT_MAX_DIMS) return err = "ndim out of range", false;
  if (!is_float_dt(a.x_dtype) || !is_float_dt(a.out_dtype)) return err = "x and out must be f32, bf16 or f16", false;
  if (a.ndim < 32 && (a.reduce_mask >> a.ndim) != 0) return err = "reduce_mask names a dimension >= ndim", false;
  int64_t ks[HRT_MAX_DIMS], kt[HRT_MAX_DIMS], rs[HRT_MAX_DIMS], rt[HRT_MAX_DIMS];
  int nk = 0, nr = 0;
  for (int d = 0; d < a.ndim; ++d) {
    if (a.sizes[d] < 0 || a.strides[d] < 0) return err = "negative size or stride", false;
    if ((a.reduce_mask >> d) & 1u) {
      rs[nr] = a.sizes[d];
      rt[nr++] = a.strides[d];
    } else {
      ks[nk] = a.sizes[d];
      kt[nk++] = a.strides[d];
    }
  }
  P.n_out = 1;
  P.n_red = 1;
  for (int d = 0; d < nk; ++d) P.n_out *= ks[d];
  for (int d = 0; d < nr; ++d) P.n_red *= rs[d];
  P.nk = merge(nk, ks, kt, P.ksz, P.kst);
  P.nr = merge(nr, rs, rt, P.rsz, P.rst);
  if (P.n_red == 0) {
    P.nr = 0;  // empty sums: every output is 0 / div
  } else if (P.nr == 0) {
    P.nr = 1;  // only size-1 dimensions reduced: a one-element sum
    P.rsz[0] = 1;
    P.rst[0] = 0;
  }
  const int V16 = (int)(16 / esize(a.x_dtype));
  const bool kept_inner = P.nk > 0 && P.kst[P.nk - 1] == 1;
  const bool red_inner = P.nr > 0 && P.rst[P.nr - 1] == 1;
  P.mode = (!kept_inner && red_inner) ? RED_ROWS : RED_COLS;
  bool vec = a.x % 16 == 0;
  if (P.mode == RED_COLS && kept_inner) {
    vec = vec && P.ksz[P.nk - 1] % V16 == 0;
    for (int d = 0; d + 1 < P.nk; ++d) vec = vec && P.kst[d] % V16 == 0;
    for (int d = 0; d < P.nr; ++d) vec = vec && P.rst[d] % V16 == 0;
  } else if (P.mode == RED_ROWS) {
    vec = vec && P.rsz[P.nr - 1] % V16 == 0;
    for (int d = 0; d < P.nk; ++d) vec = vec && P.kst[d] % V16 == 0;
    for (int d = 0; d + 1 < P.nr; ++d) vec = vec && P.rst[d] % V16 == 0;
  } else {
    vec = false;
  }
  P.V = vec ? V16 : 1;
  // Splits of the reduced range: enough workgroups to fill 256 CUs a few times over, each split long
  // enough that its partial sum is worth a round trip.
  int64_t S;
  if (P.mode == RED_COLS) {  // workgroups of 64 * V outputs; each of their 4 wavefronts >= 16 coordinates
    const int64_t tiles = cdiv(P.n_out, 64 * (int64_t)P.V);
    S = std::min<int64_t>(cdiv(512, std::max<int64_t>(tiles, 1)), std::max<int64_t>(1, P.n_red / 64));
  } else {  // a workgroup per (output, split) of >= 16 K elements
    S = std::min<int64_t>(cdiv(1024, std::max<int64_t>(P.n_out, 1)), std::max<int64_t>(1, P.n_red / 16384));
  }
  S = std::max<int64_t>(1, std::min<int64_t>(S, 1024));
  P.per_split = cdiv(P.n_red, S);
  if (P.mode == RED_ROWS) P.per_split = cdiv(P.per_split, P.V) * P.V;  // splits start on a vector
  P.splits = P.per_split > 0 ? cdiv(P.n_red, P.per_split) : 1;
  return true;
}

// ---- device side --------------------------------------------------------------------------------------
template <int XT>
__device__ __forceinline__ float ldx(uint64_t x, int64_t e) {
  if constexpr (XT == HRT_F32) return gcptr<float>(x)[e];
  else if constexpr (XT == HRT_BF16) return bf16_bits_to_f32(gcptr<uint16_t>(x)[e]);
  else return f16_bits_to_f32(gcptr<uint16_t>(x)[e]);
}

// V consecutive elements at element e (16-byte aligned when V > 1), added into acc.
template <int XT, int V>
__device__ __forceinline__ void addv(float (&acc)[V], uint64_t x, int64_t e) {
  if constexpr (V == 1) {
    acc[0] += ldx<XT>(x, e);
  } else if constexpr (XT == HRT_F32) {
    const f32x4 u = __builtin_nontemporal_load(gcptr<f32x4>(x) + e / 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] += u[i];
  } else {
    const u32x4 u = __builtin_nontemporal_load(gcptr<u32x4>(x) + e / 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] += XT == HRT_BF16 ? bf16_bits_to_f32(u[i] & 0xffffu) : f16_bits_to_f32(u[i] & 0xffffu);
      acc[2 * i + 1] += XT == HRT_BF16 ? bf16_bits_to_f32(u[i] >> 16) : f16_bits_to_f32(u[i] >> 16);
    }
  }
}

__device__ __forceinline__ void store_out(uint64_t out, int dt, int64_t o, float v) {
  if (dt == HRT_F32) gptr<float>(out)[o] = v;
  else if (dt == HRT_BF16) gptr<uint16_t>(out)[o] = (uint16_t)f32_to_bf16_bits(v);
  else gptr<uint16_t>(out)[o] = (uint16_t)f32_to_f16_bits(v);
}

// Element offset of index q over dimensions [0, n) of (sz, st), the last dimension varying fastest.
__device__ __forceinline__ int64_t offset_of(int64_t q, int n, const int64_t* sz, const int64_t* st) {
  int64_t off = 0;
  for (int d = n - 1; d >= 0; --d) {
    const int64_t nq = q / sz[d];
    off += (q - nq * sz[d]) * st[d];
    q = nq;
  }
  return off;
}

// Final value or partial sum of output o.
__device__ __forceinline__ void emit(const RedKArgs& p, int64_t o, float acc) {
  if (p.splits == 1) store_out(p.out, p.odt, o, acc / p.div);
  else gptr<float>(p.ws)[blockIdx.y * p.n_out + o] = acc;
}

// Columns: a workgroup owns 64 * V consecutive outputs (lane l: outputs o0 .. o0 + V - 1); its four
// wavefronts take consecutive quarters of split blockIdx.y's reduced coordinates and their sums are added
// through LDS in wavefront order.  Each lane keeps up to 16 loads in flight (one wavefront per SIMD
// needs ~64 KB in flight per CU to cover HBM latency).
template <int XT, int V>
__global__ __launch_bounds__(256) void red_cols(RedKArgs p) {
  __shared__ float part[3][64 * V];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t o0 = ((int64_t)blockIdx.x * 64 + lane) * V;
  const bool live = o0 < p.n_out;
  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.0f;
  const int64_t s0 = (int64_t)blockIdx.y * p.per_split;
  const int64_t s1 = min(p.n_red, s0 + p.per_split);
  const int64_t q4 = cdiv(s1 - s0, 4);
  const int64_t r0 = min(s1, s0 + w * q4), r1 = min(s1, r0 + q4);
  if (live && p.nr > 0 && r0 < r1) {
    const int64_t base = offset_of(o0, p.nk, p.ksz, p.kst);
    // The reduced range as rows of the innermost reduced dimension (stride rin): a row's offset is
    // recomputed only when the row ends.
    const int64_t rsz_in = p.rsz[p.nr - 1], rin = p.rst[p.nr - 1];
    int64_t q = r0 / rsz_in, i = r0 - q * rsz_in;
    int64_t row = base + offset_of(q, p.nr - 1, p.rsz, p.rst);
    for (int64_t r = r0; r < r1;) {
      const int64_t n = min(rsz_in - i, r1 - r);  // elements left in this row and range
      int64_t e = row + i * rin;
      int64_t k = 0;
      for (; k + 16 <= n; k += 16, e += 16 * rin) {
#pragma unroll
        for (int u = 0; u < 16; ++u) addv<XT, V>(acc, p.x, e + u * rin);
      }
      for (; k + 8 <= n; k += 8, e += 8 * rin) {
#pragma unroll
        for (int u = 0; u < 8; ++u) addv<XT, V>(acc, p.x, e + u * rin);
      }
      for (; k < n; ++k, e += rin) addv<XT, V>(acc, p.x, e);
      r += n;
      ++q;
      i = 0;
      if (r < r1) row = base + offset_of(q, p.nr - 1, p.rsz, p.rst);
    }
  }
  if (w > 0) {
#pragma unroll
    for (int j = 0; j < V; ++j) part[w - 1][lane * V + j] = acc[j];
  }
  __syncthreads();
  if (w == 0 && live) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float t = ((acc[j] + part[0][lane * V + j]) + part[1][lane * V + j]) + part[2][lane * V + j];
      emit(p, o0 + j, t);
    }
  }
}

// Rows: workgroup (output blockIdx.x, split blockIdx.y) streams the split's reduced elements, the
// innermost reduced dimension being contiguous; V elements per load, 4 loads in flight per lane.
template <int XT, int V>
__device__ __forceinline__ int64_t rows_elem(const RedKArgs& p, int64_t base, int64_t r, int64_t rsz_in) {
  if (p.nr == 1) return base + r;
  const int64_t q = r / rsz_in;
  return base + offset_of(q, p.nr - 1, p.rsz, p.rst) + (r - q * rsz_in);
}

template <int XT, int V>
__global__ __launch_bounds__(256) void red_rows(RedKArgs p) {
  __shared__ float red[4];
  const int64_t o = blockIdx.x;
  const int64_t base = offset_of(o, p.nk, p.ksz, p.kst);
  const int64_t r0 = (int64_t)blockIdx.y * p.per_split;
  const int64_t r1 = min(p.n_red, r0 + p.per_split);
  const int64_t rsz_in = p.rsz[p.nr - 1];
  float acc[4][V];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int i = 0; i < V; ++i) acc[u][i] = 0.0f;
  constexpr int64_t STEP = 256 * V;
  int64_t r = r0 + (int64_t)threadIdx.x * V;
  for (; r + 3 * STEP < r1; r += 4 * STEP) {
#pragma unroll
    for (int u = 0; u < 4; ++u) addv<XT, V>(acc[u], p.x, rows_elem<XT, V>(p, base, r + u * STEP, rsz_in));
  }
  for (; r < r1; r += STEP) addv<XT, V>(acc[0], p.x, rows_elem<XT, V>(p, base, r, rsz_in));
  float s = 0.0f;
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int i = 0; i < V; ++i) s += acc[u][i];
  s = block_sum<4>(s, red);
  if (threadIdx.x == 0) emit(p, o, s);
}

// Short rows (at most 64 * V * 16 reduced elements, one split): one wavefront per output, no LDS.
template <int XT, int V>
__global__ __launch_bounds__(256) void red_rows_wave(RedKArgs p) {
  const int64_t o = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (o >= p.n_out) return;
  const int lane = threadIdx.x & 63;
  const int64_t base = offset_of(o, p.nk, p.ksz, p.kst);
  const int64_t rsz_in = p.rsz[p.nr - 1];
  float acc[4][V];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int i = 0; i < V; ++i) acc[u][i] = 0.0f;
  constexpr int64_t STEP = 64 * V;
  int64_t r = (int64_t)lane * V;
  for (; r + 3 * STEP < p.n_red; r += 4 * STEP) {
#pragma unroll
    for (int u = 0; u < 4; ++u) addv<XT, V>(acc[u], p.x, rows_elem<XT, V>(p, base, r + u * STEP, rsz_in));
  }
  for (; r < p.n_red; r += STEP) addv<XT, V>(acc[0], p.x, rows_elem<XT, V>(p, base, r, rsz_in));
  float s = 0.0f;
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int i = 0; i < V; ++i) s += acc[u][i];
  s = wave_sum(s);
  if (lane == 0) emit(p, o, s);
}

// Second pass: out[o] = (sum of ws[s][o] over the splits, in a fixed order) / div.
__global__ __launch_bounds__(256) void red_finish(RedKArgs p) {
  const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (o >= p.n_out) return;
  // split k goes to accumulator k % 8 (8 loads in flight); the accumulators are added in a fixed order
  // (16 loads issued together per round, and the last round's loads too, with clamped indices: a loop of
  // 8 loads per iteration waited for each iteration's loads before issuing the next)
  const HK_G float* ws = gcptr<float>(p.ws);
  float a[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  int64_t k = 0;
  for (; k + 16 <= p.splits; k += 16) {
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = ws[(k + u) * p.n_out + o];
#pragma unroll
    for (int u = 0; u < 16; u += 4) asm volatile("" : "+v"(v[u]), "+v"(v[u + 1]), "+v"(v[u + 2]), "+v"(v[u + 3]));
#pragma unroll
    for (int u = 0; u < 16; ++u) a[u & 7] += v[u];
  }
  if (k < p.splits) {
    const int64_t last = p.splits - 1;
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = ws[(k + u < last ? k + u : last) * p.n_out + o];
#pragma unroll
    for (int u = 0; u < 16; u += 4) asm volatile("" : "+v"(v[u]), "+v"(v[u + 1]), "+v"(v[u + 2]), "+v"(v[u + 3]));
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (k + u < p.splits) a[u & 7] += v[u];
  }
  const float s = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
  store_out(p.out, p.odt, o, s / p.div);
}

// Second pass for few outputs and many splits: a workgroup per output; thread t adds splits t, t + 256,
// ... in order, then the workgroup's fixed reduction tree combines the threads.
__global__ __launch_bounds__(256) void red_finish_wide(RedKArgs p) {
  __shared__ float red[4];
  const int64_t o = blockIdx.x;
  const HK_G float* ws = gcptr<float>(p.ws);
  // thread t adds splits t, t + 256, ... in order, four loads issued together per round (a loop of one
  // load per iteration made a round trip per split it added)
  float a = 0.0f;
  int64_t k = threadIdx.x;
  for (; k + 768 < p.splits; k += 1024) {
    float v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = ws[(k + 256 * u) * p.n_out + o];
    asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]));
#pragma unroll
    for (int u = 0; u < 4; ++u) a += v[u];
  }
  if (k < p.splits) {
    const int64_t last = p.splits - 1;
    float v[3];
#pragma unroll
    for (int u = 0; u < 3; ++u) v[u] = ws[(k + 256 * u < last ? k + 256 * u : last) * p.n_out + o];
    asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]));
    a += v[0];
    if (k + 256 < p.splits) a += v[1];
    if (k + 512 < p.splits) a += v[2];
  }
  a = block_sum<4>(a, red);
  if (threadIdx.x == 0) store_out(p.out, p.odt, o, a / p.div);
}

template <int XT>
void launch_pass1(const RedPlan& P, const RedKArgs& k, hipStream_t s) {
  constexpr int V16 = XT == HRT_F32 ? 4 : 8;
  const dim3 blk(256);
  if (P.mode == RED_ROWS && P.splits == 1 && P.n_red <= 64 * (int64_t)P.V * 16) {
    const dim3 g((uint32_t)cdiv(P.n_out, 4));
    if (P.V > 1) hipLaunchKernelGGL((red_rows_wave<XT, V16>), g, blk, 0, s, k);
    else hipLaunchKernelGGL((red_rows_wave<XT, 1>), g, blk, 0, s, k);
  } else if (P.mode == RED_ROWS) {
    const dim3 g((uint32_t)P.n_out, (uint32_t)P.splits);
    if (P.V > 1) hipLaunchKernelGGL((red_rows<XT, V16>), g, blk, 0, s, k);
    else hipLaunchKernelGGL((red_rows<XT, 1>), g, blk, 0, s, k);
  } else {
    const dim3 g((uint32_t)cdiv(P.n_out, 64 * (int64_t)P.V), (uint32_t)P.splits);
    if (P.V > 1) hipLaunchKernelGGL((red_cols<XT, V16>), g, blk, 0, s, k);
    else hipLaunchKernelGGL((red_cols<XT, 1>), g, blk, 0, s, k);
  }
}

bool launch_reduce(const void* args, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_reduce_args*>(args);
  RedPlan P;
  std::string err;
  if (!plan_reduce(a, P, err)) return ctx.fail(err);
  if (P.n_out == 0) return true;
  if (P.mode == RED_ROWS && P.n_out >= ((int64_t)1 << 31)) return ctx.fail("too many outputs for one launch");
  if (!ctx.check(a.x, hrt::span_bytes(a.ndim, a.sizes, a.strides, esize(a.x_dtype)), "x") ||
      !ctx.check(a.out, (uint64_t)P.n_out * esize(a.out_dtype), "out"))
    return false;
  if (P.splits > 1 && !ctx.check(a.ws, (uint64_t)(P.splits * P.n_out) * 4, "ws")) return false;
  RedKArgs k{};
  k.x = a.x;
  k.out = a.out;
  k.ws = a.ws;
  k.odt = a.out_dtype;
  k.nk = P.nk;
  k.nr = P.nr;
  for (int d = 0; d < HRT_MAX_DIMS; ++d) {
    k.ksz[d] = d < P.nk ? P.ksz[d] : 1;
    k.kst[d] = d < P.nk ? P.kst[d] : 0;
    k.rsz[d] = d < P.nr ? P.rsz[d] : 1;
    k.rst[d] = d < P.nr ? P.rst[d] : 0;
  }
  k.n_out = P.n_out;
  k.n_red = P.n_red;
  k.per_split = P.per_split;
  k.splits = P.splits;
  k.div = a.div;
  switch (a.x_dtype) {
    case HRT_F32: launch_pass1<HRT_F32>(P, k, ctx.stream); break;
    case HRT_BF16: launch_pass1<HRT_BF16>(P, k, ctx.stream); break;
    default: launch_pass1<HRT_F16>(P, k, ctx.stream); break;
  }
  if (P.splits > 1 && P.n_out < 256 && P.splits >= 64)
    hipLaunchKernelGGL(red_finish_wide, dim3((uint32_t)P.n_out), dim3(256), 0, ctx.stream, k);
  else if (P.splits > 1)
    hipLaunchKernelGGL(red_finish, dim3((uint32_t)cdiv(P.n_out, 256)), dim3(256), 0, ctx.stream, k);
  return hrt::launch_ok(hipGetLastError(), ctx, "reduce_sum");
}
HRT_REGISTER("reduce_sum", hrt_reduce_args, launch_reduce);

}  // namespace
}  // namespace hk

extern "C" int64_t hrt_reduce_workspace(const hrt_reduce_args* args) {
  if (!args) return -1;
  hk::RedPlan P;
  std::string err;
  if (!hk::plan_reduce(*args, P, err)) return -1;
  return P.splits > 1 ? P.splits * P.n_out : 0;
}
