// Support kernels of the boundary: the runtime smoke kernel, strided copy/cast and fill.
// The hot-path adapters call `.contiguous()`, `.to(dtype)` and `at::zeros`; without these the data
// would round-trip through the host (reference: csrc/ops_ew.cpp:382-392, 495-506; csrc/shim.cpp:257-276).
#include "../hrt/registry.h"
#include "device_common.h"

namespace hk {
namespace {

// ---- add_f32: raw-grid smoke kernel (vkrt/tests/basic.rs:53-76) -----------------------------------
__global__ __launch_bounds__(256) void add_f32_kernel(const float* a, const float* b, float* c, uint64_t n) {
  uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) c[i] = a[i] + b[i];
}

bool launch_add_f32(const void* p, const uint32_t grid[3], hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_add_f32_args*>(p);
  const uint64_t cover = (uint64_t)grid[0] * grid[1] * grid[2] * 256;
  const uint64_t n = a.n < cover ? a.n : cover;
  if (!ctx.check(a.a, n * 4, "a") || !ctx.check(a.b, n * 4, "b") || !ctx.check(a.c, n * 4, "c")) return false;
  if (grid[1] != 1 || grid[2] != 1) return ctx.fail("add_f32 uses a 1-D grid");
  hipLaunchKernelGGL(add_f32_kernel, dim3(grid[0]), dim3(256), 0, ctx.stream, (const float*)a.a, (const float*)a.b,
                     (float*)a.c, n);
  return hrt::launch_ok(hipGetLastError(), ctx, "add_f32");
}
HRT_REGISTER_RAW("add_f32", hrt_add_f32_args, launch_add_f32);

// ---- element access by type code --------------------------------------------------------------------
template <int CODE>
struct Elem;
template <>
struct Elem<HRT_F32> {
  using S = float;
  __device__ static float get(const S* p) { return *p; }
  __device__ static void put(S* p, float v) { *p = v; }
};
template <>
struct Elem<HRT_BF16> {
  using S = uint16_t;
  __device__ static float get(const S* p) { return bf16_bits_to_f32(*p); }
  __device__ static void put(S* p, float v) { *p = (uint16_t)f32_to_bf16_bits(v); }
};
template <>
struct Elem<HRT_F16> {
  using S = uint16_t;
  __device__ static float get(const S* p) { return f16_bits_to_f32(*p); }
  __device__ static void put(S* p, float v) { *p = (uint16_t)f32_to_f16_bits(v); }
};

template <int CODE>
struct Raw;
template <>
struct Raw<HRT_RAW8> {
  using S = uint8_t;
};
template <>
struct Raw<HRT_RAW16> {
  using S = uint16_t;
};
template <>
struct Raw<HRT_RAW32> {
  using S = uint32_t;
};
template <>
struct Raw<HRT_RAW64> {
  using S = uint64_t;
};

struct Shape {
  int ndim;
  int64_t sizes[HRT_MAX_DIMS];
  int64_t s0[HRT_MAX_DIMS];  // dst strides
  int64_t s1[HRT_MAX_DIMS];  // src strides
};

__device__ __forceinline__ void offsets(const Shape& sh, int64_t i, int64_t& o0, int64_t& o1) {
  o0 = 0;
  o1 = 0;
  for (int d = sh.ndim - 1; d >= 0; --d) {
    int64_t sz = sh.sizes[d];
    int64_t q = i / sz;
    int64_t r = i - q * sz;
    o0 += r * sh.s0[d];
    o1 += r * sh.s1[d];
    i = q;
  }
}

template <int DC, int SC>
__global__ __launch_bounds__(256) void cast_nd(void* dst, const void* src, Shape sh, int64_t n) {
  using DS = typename Elem<DC>::S;
  using SS = typename Elem<SC>::S;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    int64_t od, os;
    offsets(sh, i, od, os);
    Elem<DC>::put((DS*)dst + od, Elem<SC>::get((const SS*)src + os));
  }
}

// Contiguous 1-D cast, 4 elements per thread per step.
template <int DC, int SC>
__global__ __launch_bounds__(256) void cast_1d(void* dst, const void* src, int64_t n) {
  using DS = typename Elem<DC>::S;
  using SS = typename Elem<SC>::S;
  const SS* s = (const SS*)src;
  DS* d = (DS*)dst;
  for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4; i < n; i += (int64_t)gridDim.x * 256 * 4) {
    if (i + 4 <= n) {
      float v0 = Elem<SC>::get(s + i), v1 = Elem<SC>::get(s + i + 1), v2 = Elem<SC>::get(s + i + 2),
            v3 = Elem<SC>::get(s + i + 3);
      Elem<DC>::put(d + i, v0);
      Elem<DC>::put(d + i + 1, v1);
      Elem<DC>::put(d + i + 2, v2);
      Elem<DC>::put(d + i + 3, v3);
    } else {
      for (int64_t j = i; j < n; ++j) Elem<DC>::put(d + j, Elem<SC>::get(s + j));
    }
  }
}

// Contiguous same-type copy of 16-byte chunks: one chunk per thread, streaming loads and stores (one
// chunk per thread over many workgroups measured fastest on MI355X: 6.5 TB/s for a 512 MiB copy).
__global__ __launch_bounds__(256) void ew_copy_vec16(u32x4* __restrict__ dst, const u32x4* __restrict__ src, int64_t n16) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n16) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// Same-type copy whose innermost dimension is contiguous on both sides and whole 16-byte chunks long,
// with 16-byte aligned rows (a slice of a concatenation, a sliced view made contiguous): one chunk per
// thread, the row found once per chunk.  Sizes and strides of sh are in bytes here; its last dimension
// is the row (stride 1 chunk).
__global__ __launch_bounds__(256) void copy_rows16(uint8_t* dst, const uint8_t* src, Shape sh, int64_t row16,
                                                   int64_t n16) {
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= n16) return;
  int64_t q = j / row16;
  const int64_t c = (j - q * row16) * 16;
  int64_t od = c, os = c;
  for (int d = sh.ndim - 2; d >= 0; --d) {
    const int64_t nq = q / sh.sizes[d];
    const int64_t r = q - nq * sh.sizes[d];
    od += r * sh.s0[d];
    os += r * sh.s1[d];
    q = nq;
  }
  __builtin_nontemporal_store(__builtin_nontemporal_load((const u32x4*)(src + os)), (u32x4*)(dst + od));
}

template <typename S>
__global__ __launch_bounds__(256) void raw_nd(void* dst, const void* src, Shape sh, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    int64_t od, os;
    offsets(sh, i, od, os);
    ((S*)dst)[od] = ((const S*)src)[os];
  }
}

template <typename S>
__global__ __launch_bounds__(256) void fill_nd(void* dst, uint64_t bits, Shape sh, int64_t n) {
  const S v = (S)bits;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    int64_t od, os;
    offsets(sh, i, od, os);
    ((S*)dst)[od] = v;
  }
}

uint64_t elem_size(int code) {
  switch (code) {
    case HRT_F32: return 4;
    case HRT_BF16: return 2;
    case HRT_F16: return 2;
    case HRT_RAW8: return 1;
    case HRT_RAW16: return 2;
    case HRT_RAW32: return 4;
    case HRT_RAW64: return 8;
    default: return 0;
  }
}

uint32_t grid_for(int64_t n, int per_thread) {
  int64_t g = cdiv(n, 256 * (int64_t)per_thread);
  if (g > 16384) g = 16384;
  if (g < 1) g = 1;
  return (uint32_t)g;
}

template <int DC, int SC>
void queue_cast(const hrt_copy_args& a, const Shape& sh, int64_t n, bool contig, hipStream_t s) {
  if (contig)
    hipLaunchKernelGGL((cast_1d<DC, SC>), dim3(grid_for(n, 4)), dim3(256), 0, s, (void*)a.dst, (const void*)a.src, n);
  else
    hipLaunchKernelGGL((cast_nd<DC, SC>), dim3(grid_for(n, 1)), dim3(256), 0, s, (void*)a.dst, (const void*)a.src, sh, n);
}

// Same-type copy with a contiguous innermost dimension of whole 16-byte chunks and 16-byte aligned rows.
bool rows16_ok(const hrt_copy_args& a, const Shape& sh, uint64_t es, int64_t n) {
  if (a.dst_dtype != a.src_dtype || a.ndim < 2) return false;
  const int in = a.ndim - 1;
  if (sh.s0[in] != 1 || sh.s1[in] != 1 || (sh.sizes[in] * (int64_t)es) % 16 || a.dst % 16 || a.src % 16) return false;
  for (int d = 0; d < in; ++d)
    if ((sh.s0[d] * (int64_t)es) % 16 || (sh.s1[d] * (int64_t)es) % 16) return false;
  return cdiv(n * (int64_t)es / 16, 256) < ((int64_t)1 << 31);
}

bool launch_copy(const void* p, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_copy_args*>(p);
  if (a.ndim < 0 || a.ndim > HRT_MAX_DIMS) return ctx.fail("ndim out of range");
  const uint64_t de = elem_size(a.dst_dtype), se = elem_size(a.src_dtype);
  if (!de || !se) return ctx.fail("unknown dtype code");
  const bool dfloat = a.dst_dtype <= HRT_F16, sfloat = a.src_dtype <= HRT_F16;
  if (!(dfloat && sfloat) && a.dst_dtype != a.src_dtype) return ctx.fail("raw copies need equal dtypes");
  Shape sh{};
  sh.ndim = a.ndim;
  int64_t n = 1;
  bool contig = true;
  int64_t expect = 1;
  for (int d = a.ndim - 1; d >= 0; --d) {
    if (a.sizes[d] < 0 || a.dst_strides[d] < 0 || a.src_strides[d] < 0) return ctx.fail("negative size or stride");
    sh.sizes[d] = a.sizes[d];
    sh.s0[d] = a.dst_strides[d];
    sh.s1[d] = a.src_strides[d];
    if (a.sizes[d] != 1 && (a.dst_strides[d] != expect || a.src_strides[d] != expect)) contig = false;
    expect *= a.sizes[d];
    n *= a.sizes[d];
  }
  if (n == 0) return true;
  if (!ctx.check(a.dst, hrt::span_bytes(a.ndim, a.sizes, a.dst_strides, de), "dst") ||
      !ctx.check(a.src, hrt::span_bytes(a.ndim, a.sizes, a.src_strides, se), "src"))
    return false;
  hipStream_t s = ctx.stream;
  if (dfloat && sfloat && a.dst_dtype != a.src_dtype) {
    switch (a.dst_dtype * 3 + a.src_dtype) {
      case HRT_F32 * 3 + HRT_BF16: queue_cast<HRT_F32, HRT_BF16>(a, sh, n, contig, s); break;
      case HRT_F32 * 3 + HRT_F16: queue_cast<HRT_F32, HRT_F16>(a, sh, n, contig, s); break;
      case HRT_BF16 * 3 + HRT_F32: queue_cast<HRT_BF16, HRT_F32>(a, sh, n, contig, s); break;
      case HRT_BF16 * 3 + HRT_F16: queue_cast<HRT_BF16, HRT_F16>(a, sh, n, contig, s); break;
      case HRT_F16 * 3 + HRT_F32: queue_cast<HRT_F16, HRT_F32>(a, sh, n, contig, s); break;
      case HRT_F16 * 3 + HRT_BF16: queue_cast<HRT_F16, HRT_BF16>(a, sh, n, contig, s); break;
      default: return ctx.fail("unsupported cast");
    }
  } else if (contig && (n * de) % 16 == 0 && a.dst % 16 == 0 && a.src % 16 == 0 && (n * de) / 16 < ((int64_t)1 << 39)) {
    const int64_t n16 = (int64_t)(n * de) / 16;
    hipLaunchKernelGGL(ew_copy_vec16, dim3((uint32_t)((n16 + 255) / 256)), dim3(256), 0, s, (u32x4*)a.dst,
                       (const u32x4*)a.src, n16);
  } else if (rows16_ok(a, sh, de, n)) {
    Shape b = sh;  // byte strides; the row is the last dimension
    for (int d = 0; d < a.ndim; ++d) {
      b.s0[d] = sh.s0[d] * (int64_t)de;
      b.s1[d] = sh.s1[d] * (int64_t)de;
    }
    const int64_t row16 = sh.sizes[a.ndim - 1] * (int64_t)de / 16;
    const int64_t n16 = n * (int64_t)de / 16;
    hipLaunchKernelGGL(copy_rows16, dim3((uint32_t)cdiv(n16, 256)), dim3(256), 0, s, (uint8_t*)a.dst, (const uint8_t*)a.src,
                       b, row16, n16);
  } else {
    dim3 g(grid_for(n, 1));
    switch (de) {
      case 1: hipLaunchKernelGGL(raw_nd<uint8_t>, g, dim3(256), 0, s, (void*)a.dst, (const void*)a.src, sh, n); break;
      case 2: hipLaunchKernelGGL(raw_nd<uint16_t>, g, dim3(256), 0, s, (void*)a.dst, (const void*)a.src, sh, n); break;
      case 4: hipLaunchKernelGGL(raw_nd<uint32_t>, g, dim3(256), 0, s, (void*)a.dst, (const void*)a.src, sh, n); break;
      default: hipLaunchKernelGGL(raw_nd<uint64_t>, g, dim3(256), 0, s, (void*)a.dst, (const void*)a.src, sh, n); break;
    }
  }
  return hrt::launch_ok(hipGetLastError(), ctx, "ew_copy");
}
HRT_REGISTER("ew_copy", hrt_copy_args, launch_copy);

bool launch_fill(const void* p, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_fill_args*>(p);
  if (a.ndim < 0 || a.ndim > HRT_MAX_DIMS) return ctx.fail("ndim out of range");
  const uint64_t es = elem_size(a.dtype);
  if (!es) return ctx.fail("unknown dtype code");
  Shape sh{};
  sh.ndim = a.ndim;
  int64_t n = 1;
  for (int d = 0; d < a.ndim; ++d) {
    if (a.sizes[d] < 0 || a.strides[d] < 0) return ctx.fail("negative size or stride");
    sh.sizes[d] = a.sizes[d];
    sh.s0[d] = a.strides[d];
    sh.s1[d] = 0;
    n *= a.sizes[d];
  }
  if (n == 0) return true;
  if (!ctx.check(a.dst, hrt::span_bytes(a.ndim, a.sizes, a.strides, es), "dst")) return false;
  dim3 g(grid_for(n, 1));
  switch (es) {
    case 1: hipLaunchKernelGGL(fill_nd<uint8_t>, g, dim3(256), 0, ctx.stream, (void*)a.dst, a.value_bits, sh, n); break;
    case 2: hipLaunchKernelGGL(fill_nd<uint16_t>, g, dim3(256), 0, ctx.stream, (void*)a.dst, a.value_bits, sh, n); break;
    case 4: hipLaunchKernelGGL(fill_nd<uint32_t>, g, dim3(256), 0, ctx.stream, (void*)a.dst, a.value_bits, sh, n); break;
    default: hipLaunchKernelGGL(fill_nd<uint64_t>, g, dim3(256), 0, ctx.stream, (void*)a.dst, a.value_bits, sh, n); break;
  }
  return hrt::launch_ok(hipGetLastError(), ctx, "ew_fill");
}
HRT_REGISTER("ew_fill", hrt_fill_args, launch_fill);

// ---- cat: all parts in one launch --------------------------------------------------------------------------
// One 16-byte chunk per lane: out row r, byte column cb in [col[0], col[n-1] + row_bytes[n-1]); the part
// holding cb is the last one starting at or before it (selected with constant indices, so the argument
// arrays stay in scalar registers).
__global__ __launch_bounds__(256) void cat_rows16_k(hrt_cat_args a, int64_t span16, int64_t n16) {
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= n16) return;
  const int64_t r = j / span16, cb = a.col[0] + (j - r * span16) * 16;
  uint64_t sp = a.src[0];
  int64_t rb = a.row_bytes[0], c0 = a.col[0];
#pragma unroll
  for (int k = 1; k < HRT_CAT_MAX_PARTS; ++k)
    if (k < a.nparts && a.col[k] <= cb) {
      sp = a.src[k];
      rb = a.row_bytes[k];
      c0 = a.col[k];
    }
  const u32x4 v = __builtin_nontemporal_load((const u32x4*)((const uint8_t*)sp + r * rb + (cb - c0)));
  __builtin_nontemporal_store(v, (u32x4*)((uint8_t*)a.out + r * a.out_row_bytes + cb));
}

bool launch_cat(const void* p, const uint32_t*, hrt::LaunchCtx& ctx) {
  const auto& a = *static_cast<const hrt_cat_args*>(p);
  if (a.nparts < 1 || a.nparts > HRT_CAT_MAX_PARTS || a.outer < 0) return ctx.fail("cat: 1..8 parts, outer >= 0");
  if (a.out % 16 || a.out_row_bytes % 16 || a.out_row_bytes <= 0) return ctx.fail("cat: out rows of 16-byte chunks");
  for (int k = 0; k < a.nparts; ++k) {
    if (a.src[k] % 16 || a.row_bytes[k] <= 0 || a.row_bytes[k] % 16 || a.col[k] % 16 || a.col[k] < 0)
      return ctx.fail("cat: parts of whole 16-byte chunks");
    if (k > 0 && a.col[k] != a.col[k - 1] + a.row_bytes[k - 1]) return ctx.fail("cat: parts must be adjacent");
  }
  const int64_t end = a.col[a.nparts - 1] + a.row_bytes[a.nparts - 1];
  if (end > a.out_row_bytes) return ctx.fail("cat: parts exceed the out row");
  if (!ctx.check(a.out, (uint64_t)(a.outer * a.out_row_bytes), "out")) return false;
  for (int k = 0; k < a.nparts; ++k)
    if (!ctx.check(a.src[k], (uint64_t)(a.outer * a.row_bytes[k]), "src")) return false;
  const int64_t span16 = (end - a.col[0]) / 16, n16 = a.outer * span16;
  if (n16 == 0) return true;
  hipLaunchKernelGGL(cat_rows16_k, dim3((uint32_t)cdiv(n16, 256)), dim3(256), 0, ctx.stream, a, span16, n16);
  return hrt::launch_ok(hipGetLastError(), ctx, "cat_rows16");
}
HRT_REGISTER("cat_rows16", hrt_cat_args, launch_cat);

}  // namespace
}  // namespace hk
