/*
 * Argument blocks of the operator kernels registered in the hrt runtime (see hrt.h).
 *
 * `hrt_dispatch(hrt_kernel_index(name), &args, sizeof(args), 0, 0, 0)` queues kernel `name` with one
 * of the blocks below.  They play the role of the reference's push-constant structs (MmPush
 * `csrc/ops_mm.cpp:19-29`, AttnPush/CoopPush `csrc/ops_attn.cpp:25-42`, SoftmaxPush
 * `csrc/ops_rows.cpp:37-41`, LnPush `csrc/ops_rows.cpp:103-109`, Dq8Push `csrc/ops_quant.cpp:15-19`,
 * EwPush `csrc/ops_ew.cpp:22-28`) with two deliberate differences: sizes, strides and offsets are 64-bit
 * (no 2^32 element limit on a 288 GB device), and each kernel picks its own tiling and grid.
 *
 * All addresses are device addresses inside live hrt blocks; the runtime checks every operand's byte
 * extent against its allocator before launching and rejects out-of-range operands.  Strides are in
 * elements and must be non-negative.  Arithmetic is fp32 for every dtype; bf16 and f16 results are
 * rounded once, to nearest-even (bf16: NaN -> 0x7FC0), as `vkrt/shaders/types.glsl:18-50`.
 */
#ifndef HRT_OPS_H_
#define HRT_OPS_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type codes.  0..2 are the float kinds used in kernel names (f32/bf16/f16, the reference's
 * KIND numbering, vkrt/shaders/types.glsl:1); 3..6 are raw element sizes for same-type copies/fills. */
enum {
  HRT_F32 = 0,
  HRT_BF16 = 1,
  HRT_F16 = 2,
  HRT_RAW8 = 3,
  HRT_RAW16 = 4,
  HRT_RAW32 = 5,
  HRT_RAW64 = 6
};

#define HRT_MAX_DIMS 8

/* "add_f32" — raw-grid smoke kernel, 256 threads per workgroup: c[i] = a[i] + b[i] for i < n.
 * Same argument block and meaning as the reference's runtime smoke kernel (vkrt/tests/basic.rs:53-76). */
typedef struct hrt_add_f32_args {
  uint64_t a, b, c, n;
} hrt_add_f32_args;

/* "ew_copy" — dst[i] = convert(src[i]) over an ndim-dimensional index space (ndim <= 8, sizes shared,
 * separate strides).  Float kinds convert among each other; raw kinds require dst_dtype == src_dtype.
 * Replaces the strided copy/cast `ew_copy` (csrc/ops_ew.cpp:495-506). */
typedef struct hrt_copy_args {
  uint64_t dst, src;
  int32_t ndim, dst_dtype, src_dtype, pad;
  int64_t sizes[HRT_MAX_DIMS];
  int64_t dst_strides[HRT_MAX_DIMS];
  int64_t src_strides[HRT_MAX_DIMS];
} hrt_copy_args;

/* "cat_rows16" — torch.cat of up to HRT_CAT_MAX_PARTS same-dtype contiguous parts in one launch (the
 * reference copies each part with its own kernel: csrc/ops_rows.cpp:272-332).  Tensors are viewed as rows
 * of bytes: part p as [outer, row_bytes[p]], out as [outer, out_row_bytes]; part p fills byte columns
 * [col[p], col[p] + row_bytes[p]) of every out row, the parts in column order and adjacent (col[p + 1] =
 * col[p] + row_bytes[p]).  Pointers, row_bytes, col and out_row_bytes are multiples of 16 bytes and
 * row_bytes[p] > 0.  More parts: one launch per group of HRT_CAT_MAX_PARTS. */
#define HRT_CAT_MAX_PARTS 8
typedef struct hrt_cat_args {
  uint64_t out;
  uint64_t src[HRT_CAT_MAX_PARTS];
  int64_t row_bytes[HRT_CAT_MAX_PARTS];
  int64_t col[HRT_CAT_MAX_PARTS];
  int64_t outer, out_row_bytes;
  int32_t nparts, pad;
} hrt_cat_args;

/* "ew_fill" — dst[i] = value over a strided index space; value_bits holds the element's bit pattern in
 * its low bytes (dtype selects the element size).  Replaces `try_fill` (csrc/ops_ew.cpp:382-392). */
typedef struct hrt_fill_args {
  uint64_t dst, value_bits;
  int32_t ndim, dtype, pad0, pad1;
  int64_t sizes[HRT_MAX_DIMS];
  int64_t strides[HRT_MAX_DIMS];
} hrt_fill_args;

/* "ew_map" — out[i] = f(a[i], b[i], c[i]; s0, s1) over an ndim-dimensional index space (ndim <= 8):
 * every operand has its own element strides (stride 0 = broadcast along that dimension), a, b, c are
 * read as HRT_F32/BF16/F16 (c as HRT_RAW8 bytes for HRT_EW_WHERE), converted to fp32, f is evaluated in
 * fp32 and rounded once to out_dtype.  Operands an op does not read must have address 0.  Additions and
 * products are evaluated in the written order without fused multiply-add (division and square root
 * correctly rounded), so the arithmetic ops equal a float32 evaluation of the same formula bit for bit;
 * the activations are within a few float32 ulps.  Replaces the generated `ew_<op>_<kinds>` kernel family
 * (vkrt/shaders/ew.comp.in:115-257, op table tools/gen_shaders.py:53-120) driven by `ew_prepare` /
 * `ew_run` (csrc/ops_ew.cpp:76-139); the op code is an argument instead of part of the kernel name. */
enum hrt_ew_op {
  /* (a, b) */
  HRT_EW_ADD = 0,      /* a + s0 * b                 add.Tensor (alpha = s0)          ops_ew.cpp:146-190 */
  HRT_EW_SUB = 1,      /* a - s0 * b                 sub.Tensor                                         */
  HRT_EW_MUL = 2,      /* a * b                                                                         */
  HRT_EW_DIV = 3,      /* a / b                                                                         */
  /* (a) with host scalars */
  HRT_EW_ADD_S = 4,    /* a + s0                     add/sub with a scalar, s0 = +-(alpha * value)     */
  HRT_EW_MUL_S = 5,    /* a * s0                                                                        */
  HRT_EW_DIV_S = 6,    /* a / s0                                                                        */
  HRT_EW_AXPB = 7,     /* s1 + s0 * a                scalar on the left of add/sub (ops_ew.cpp:222-229) */
  HRT_EW_RDIV_S = 8,   /* s0 / a                     scalar on the left of div                          */
  HRT_EW_POW_S = 9,    /* pow(a, s0)                 pow.Tensor_Scalar                                  */
  /* (a) unary (ops_ew.cpp:283-334) */
  HRT_EW_NEG = 10,
  HRT_EW_RSQRT = 11,
  HRT_EW_RECIP = 12,
  HRT_EW_EXP = 13,
  HRT_EW_SIN = 14,
  HRT_EW_COS = 15,
  HRT_EW_SQRT = 16,
  HRT_EW_TANH = 17,
  HRT_EW_SIGMOID = 18,
  HRT_EW_RELU = 19,
  HRT_EW_SILU = 20,
  HRT_EW_GELU_ERF = 21,
  HRT_EW_GELU_TANH = 22,
  /* (a = grad, b = input) activation backward (ops_ew.cpp:336-372) */
  HRT_EW_SILU_BWD = 23,
  HRT_EW_GELU_ERF_BWD = 24,
  HRT_EW_GELU_TANH_BWD = 25,
  /* optimizer forms (ops_ew.cpp:394-455) */
  HRT_EW_ADDCMUL = 26, /* a + s0 * b * c                                                                */
  HRT_EW_ADDCDIV = 27, /* a + s0 * b / c                                                                */
  HRT_EW_LERP_S = 28,  /* a + s0 * (b - a), as b - (b - a) * (1 - s0) when |s0| >= 0.5                  */
  /* (a, b, c = bool) */
  HRT_EW_WHERE = 29,   /* c != 0 ? a : b             where.self (ops_ew.cpp:374-392)                    */
  HRT_EW_OP_COUNT = 30
};

typedef struct hrt_ew_args {
  uint64_t out, a, b, c;
  int32_t op, ndim;
  int32_t out_dtype, a_dtype, b_dtype, c_dtype;
  float s0, s1;
  int64_t sizes[HRT_MAX_DIMS];
  int64_t out_strides[HRT_MAX_DIMS];
  int64_t a_strides[HRT_MAX_DIMS];
  int64_t b_strides[HRT_MAX_DIMS];
  int64_t c_strides[HRT_MAX_DIMS];
} hrt_ew_args;

/* "mm_{f32,bf16,f16}" (portable FMA kernel) and "mm_mfma_{bf16,f16}" (gfx950 matrix cores):
 *   c[b, m, n] = alpha * sum_k a[b, m, k] * b[b, k, n] + beta * bias[b, m, n]     (bias only if has_bias)
 * a, b, bias: any non-negative strides (transposed / sliced views are read in place; bias broadcasts
 * with stride 0); c: written with strides c_s*.  fp32 accumulation, one rounding at the store.
 * Same meaning as MmPush (csrc/ops_mm.cpp:19-29) and the epilogue of vkrt/shaders/mm_coop.comp.in:195-208. */
typedef struct hrt_mm_args {
  uint64_t a, b, c, bias;
  int64_t M, N, K, batch;
  int64_t a_sb, a_sm, a_sk;
  int64_t b_sb, b_sk, b_sn;
  int64_t c_sb, c_sm, c_sn;
  int64_t bias_sb, bias_sm, bias_sn;
  float alpha, beta;
  uint32_t has_bias, flags;
} hrt_mm_args;
/* flags bit for "mm_mfma_{bf16,f16}": c is fp32 and receives alpha * acc + beta * bias unrounded (no
 * counterpart in the reference: the split-K partial products of "mm_reduce_*"). */
#define HRT_MM_F32_OUT 1u

/* "mm_reduce_{bf16,f16}" — the second half of a split-K product (no counterpart in the reference, whose
 * small-N / small-M products run on one workgroup per 64 x 64 tile; composes csrc/ops_mm.cpp:61-175):
 *   c[m, n] = round(alpha * sum_{s < splits} ws[s, m, n] + beta * bias[m, n])     (bias only if has_bias)
 * ws: fp32 [splits, M, N] contiguous (the partial products over disjoint K ranges, from "mm_mfma_*" with
 * HRT_MM_F32_OUT); the splits are summed in order s = 0, 1, ..., so the result is deterministic.  c: strides
 * (c_sm, c_sn); bias broadcasts through stride 0 like hrt_mm_args. */
typedef struct hrt_mm_reduce_args {
  uint64_t ws, c, bias;
  int64_t M, N, splits;
  int64_t c_sm, c_sn, bias_sm, bias_sn;
  float alpha, beta;
  uint32_t has_bias, pad;
} hrt_mm_reduce_args;

/* "mm_dq8_{bf16,f16}" — fused int8 weight-only linear (no reference counterpart; composes
 * csrc/ops_quant.cpp:34-59 with csrc/ops_mm.cpp:61-175):
 *   y[m, n] = alpha * sum_k x[m, k] * deq(q)[n, k] + beta * bias[n]
 *   deq(q)[n, k] = round_dtype(float(q[n, k]) * float(scale[n, k / 64]))      (bit-exact dequant value)
 * x: [M, K] with strides (x_sm, x_sk); q: int8 [N, K] contiguous; scale: bf16 [N, nblocks] contiguous,
 * nblocks = ceil(K / 64); bias: [N] (if has_bias); y: [M, N] contiguous, dtype of x.
 * ws (optional, 0 = none): 16-byte aligned workspace of N * K elements of x's dtype.  For large M (the
 * weights would otherwise be converted once per 256-row block of x) the weights are dequantized into it
 * once and the product runs on them; the values are the same either way. */
typedef struct hrt_mm_dq8_args {
  uint64_t x, q, scale, bias, y;
  int64_t M, N, K, nblocks;
  int64_t x_sm, x_sk;
  float alpha, beta;
  uint32_t has_bias, flags;
  uint64_t ws;
} hrt_mm_dq8_args;

/* Fused scaled-dot-product attention, non-causal, no mask, D <= 128 (vkrt/shaders/attn.comp.in:1-14,
 * attn_coop.comp.in:1-9).  q: [B, H, Sq, D], k, v: [B, H, Sk, D] views given by (batch, head, seq)
 * element strides, d contiguous.  Outputs o / o32 / dq / dk / dv are [B, S, H, D]-contiguous (PyTorch
 * returns them permuted to [B, H, S, D], csrc/ops_attn.cpp:159-162; dq / dk / dv may instead follow the
 * inputs' layout, HRT_ATTN_GRAD_LIKE_INPUT); lse and delta are fp32 [B, H, Sq].
 *
 *  "attn_fwd_{dt}":   o = softmax(scale * q k^T) v (rounded to dt), lse = rowwise logsumexp (fp32),
 *                     o32 = the unrounded fp32 o when o32 != 0.
 *  "attn_delta_{dt}": delta[b, h, i] = sum_d O[b, i, h, d] * dout[b, h, i, d], with O read from o
 *                     (fp32 when flags & HRT_ATTN_O_F32, else dt), as attn.comp.in:210-240.
 *  "attn_dkdv_{dt}":  dk = scale * dS^T q, dv = P^T dout     (P = exp(scale * q k^T - lse),
 *  "attn_dq_{dt}":    dq = scale * dS k                        dS = P * (dout v^T - delta))
 * For bf16/f16 the matrix-core kernels round P and dS to dt before the second product, as
 * attn_coop.comp.in:182-183, 235-236, 283-284; the f32 kernels keep everything fp32. */
#define HRT_ATTN_O_F32 1u
/* "attn_dq_{bf16,f16}" with this flag first computes delta (as "attn_delta_{dt}", from o per
 * HRT_ATTN_O_F32) into `delta`, then dQ from it; "attn_dkdv_{dt}" can then run on that delta.  No
 * counterpart in the reference, which always launches the delta pass on its own (csrc/ops_attn.cpp:240-248):
 * it saves a launch and a second read of dO. */
#define HRT_ATTN_DQ_DELTA 2u
/* "attn_dq_{dt}" / "attn_dkdv_{dt}" with this flag write dq, dk, dv in the layout of q, k, v (the element
 * strides q_sb/q_sh/q_ss, k_*, v_* with d contiguous) instead of [B, S, H, D]-contiguous.  No counterpart
 * in the reference: PyTorch's autograd copies a leaf's gradient into the leaf's own layout, so gradients
 * in the input's layout cost nothing there; the caller must give q, k, v non-overlapping dense layouts. */
#define HRT_ATTN_GRAD_LIKE_INPUT 4u
typedef struct hrt_attn_args {
  uint64_t q, k, v;
  uint64_t o, lse, o32;
  uint64_t dout, delta;
  uint64_t dq, dk, dv;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t do_sb, do_sh, do_ss;
  int32_t B, H, Sq, Sk, D;
  float scale;
  uint32_t flags, pad;
} hrt_attn_args;

/* Row softmax over R of a contiguous [outer, R, inner] tensor (vkrt/shaders/softmax.comp.in:27-50):
 *  "softmax_fwd_{dt}": y = exp(x - max) / sum(exp(x - max)); with safe != 0 a row whose entries are all
 *                      -inf gives 0 (_safe_softmax).
 *  "softmax_bwd_{dt}": dx = y * (g - sum(g * y)). */
typedef struct hrt_softmax_args {
  uint64_t x, y, g, dx;
  int64_t outer, R, inner;
  uint32_t safe, pad;
} hrt_softmax_args;

/* layer_norm over the last D elements of contiguous [rows, D] (vkrt/shaders/ln.comp.in:1-84):
 *  "ln_fwd_{dt}":   mean = sum(x)/D, var = sum((x-mean)^2)/D (two-pass), rstd = 1/sqrt(var+eps),
 *                   y = (x-mean)*rstd*w + b   (w, b optional = 0); mean, rstd fp32 [rows].
 *  "ln_bwd_{dt}":   dx = rstd*(gw - mean(gw) - xhat*mean(gw*xhat)), gw = g*w, xhat = (x-mean)*rstd
 *                   (dx optional); when ws != 0 also writes per-chunk partial sums of g*xhat and g to
 *                   ws = fp32 [hrt_ln_chunks(rows, D)][2][D], and when dw or db is also given, queues the
 *                   "ln_wgrad_{dt}" reduction of them right behind (one call for dx, dw and db).  dw / db
 *                   without ws is an error.
 *  "ln_wgrad_{dt}": dw[d] = sum over chunks of ws[c][0][d], db[d] = sum of ws[c][1][d] (each optional). */
typedef struct hrt_ln_args {
  uint64_t x, y, mean, rstd, w, b;
  uint64_t g, dx, dw, db, ws;
  int64_t rows, D;
  float eps;
  uint32_t pad;
} hrt_ln_args;

/* Row chunking of the layer_norm weight-gradient partial sums.  A chunk is one workgroup of the backward
 * (one wavefront per row) and writes 2 D fp32 sums: a third of the bf16 bytes of its rows' x, g and dx at
 * 4 rows, a sixth at 8, a twelfth at 16.  The chunk doubles from 4 rows while it holds at least 8192
 * elements, at least 128 chunks remain and its rows of fp32 (staged in LDS to be added) fit in 128 KiB
 * (short rows keep more, smaller workgroups: [1024, 1024] is faster with 4-row chunks). */
static inline int64_t hrt_ln_rows_per_chunk(int64_t rows, int64_t D) {
  int64_t r = 4;
  while (r < 16 && r * D >= 8192 && rows >= 256 * r && 2 * r * D * 4 <= 131072) r *= 2;
  return r;
}
static inline int64_t hrt_ln_chunks(int64_t rows, int64_t D) {
  int64_t r = hrt_ln_rows_per_chunk(rows, D);
  return (rows + r - 1) / r;
}

/* hrt_ln_bwd_noalloc — "ln_bwd_{dt}" with dw / db (dx, dw, db of layer_norm, as "ln_bwd_{dt}" followed by
 * "ln_wgrad_{dt}" computes them) without any
 * allocation.  No counterpart in the reference: it is for callers that cannot allocate device memory
 * (code recorded into a HIP graph, tight serving loops, harnesses that forbid hipMalloc).  The caller
 * passes inputs and outputs as for "ln_bwd_{dt}" with ws = 0; the per-chunk partial sums of dw / db go to a
 * file-scope device array of HRT_LN_SCRATCH_BYTES that the library holds on each GPU until the process
 * ends.  Its size bounds the problem: hrt_ln_chunks(rows, D) * 2 * D * 4 bytes must fit (rows * D up to
 * 4 Mi elements with 4-row chunks, 8 Mi with 8-row chunks, e.g. [1024, 2048], [1024, 4096] or
 * [2048, 4096]) whenever dw or db is requested; larger calls fail with
 * an error and queue nothing.  dx alone needs no scratch and has no such limit.  Every call writes the
 * partial sums before reading them, so nothing needs clearing; calls on the runtime's one stream run in
 * order, but work that overlaps on one GPU (a recorded graph replayed beside another call) shares the array
 * and races.  dtype: HRT_F32, HRT_BF16 or HRT_F16.  0 = queued, -1 = error (hrt_last_error). */
#define HRT_LN_SCRATCH_BYTES (8u << 20)
int hrt_ln_bwd_noalloc(const hrt_ln_args* args, int32_t dtype);

/* "dq8_{f32,bf16,f16}" — weight-only int8 dequant (vkrt/shaders/dq8.comp.in:39-62, closed form
 * torch_vulkan/__init__.py:203-205): out[r, c] = round_dt(float(q[r, c]) * float(scale[r, c / 64])).
 * q: int8 [rows, cols] contiguous; scale: bf16 [rows, nblocks] contiguous, nblocks = ceil(cols / 64);
 * out: [rows, cols] contiguous.  Bit-exact: the fp32 product is exact, the only rounding is the store. */
typedef struct hrt_dq8_args {
  uint64_t q, scale, out;
  int64_t rows, cols, nblocks;
} hrt_dq8_args;

/* "reduce_sum" — out[k] = (sum over the reduced coordinates r of x[k, r]) / div, accumulated in fp32 and
 * rounded once to out_dtype.  x: an ndim-dimensional strided view (ndim <= 8, non-negative strides) of
 * HRT_F32/BF16/F16; bit d of reduce_mask marks dimension d as summed; out: the kept dimensions, in order,
 * contiguous (what sum/mean with or without keepdim return); div: 1 for sum, the reduced element count
 * for mean.  When the reduced range is split across workgroups the fp32 partial sums go to ws and a
 * second pass adds them in order (deterministic); ws must then hold hrt_reduce_workspace(&args) floats,
 * otherwise it may be 0.  Replaces `try_reduce` / "reduce_{dt}" (csrc/ops_rows.cpp:183-270,
 * vkrt/shaders/reduce.comp.in:1-45), which took 4 kept and 2 reduced dimensions and one workgroup per
 * output. */
typedef struct hrt_reduce_args {
  uint64_t x, out, ws;
  int32_t ndim, x_dtype, out_dtype;
  uint32_t reduce_mask;
  float div;
  uint32_t pad;
  int64_t sizes[HRT_MAX_DIMS];
  int64_t strides[HRT_MAX_DIMS];
} hrt_reduce_args;

/* fp32 elements of workspace "reduce_sum" needs for these arguments (0: none, -1: invalid arguments). */
int64_t hrt_reduce_workspace(const hrt_reduce_args* args);

/* "im2col_{f32,bf16,f16}" / "col2im_{f32,bf16,f16}" — the unfolding behind conv2d (NCHW, stride, zero
 * padding, no dilation) and its adjoint.  im2col: cols[n, (c, kh, kw), (oh, ow)] = x[n, c, oh*SH - PH + kh,
 * ow*SW - PW + kw] (0 outside x).  col2im: x[n, c, h, w] = sum of the cols entries that im2col takes from
 * (n, c, h, w), accumulated in fp32 in a fixed order (a gather: no atomics).  x: [N, C, H, W] contiguous,
 * cols: [N, C*KH*KW, OH*OW] contiguous.  Replaces "im2col_{dt}" / "col2im_{dt}" and Im2colPush
 * (csrc/ops_conv.cpp:31-35, 78-88, 153-162; vkrt/shaders/im2col.comp.in). */
typedef struct hrt_im2col_args {
  uint64_t x, cols;
  int64_t N, C, H, W, OH, OW, KH, KW, SH, SW, PH, PW;
} hrt_im2col_args;

/* "conv3x3_wprep_{bf16,f16}" and "conv3x3_{bf16,f16}" — a direct 3x3 convolution (stride 1, zero padding 1,
 * no dilation, one group) without the column matrix: an implicit GEMM that stages each 16-channel block of
 * the input rows once and applies the nine taps from it.  No counterpart in the reference, whose
 * convolution is im2col + GEMM (csrc/ops_conv.cpp:89-140); the result is the same convolution in fp32
 * accumulation with one rounding (the reduction order differs from im2col + GEMM).
 *  "conv3x3_wprep_{dt}": reorders the weights into wr, hrt_conv3_wr_bytes(O, I) bytes (16-byte aligned):
 *                        for output block b = o / 128 and channel block cb, a tile of 128 rows of 152
 *                        values at byte ((b * I / 16 + cb) * 128 + o % 128) * 304, value 16 t + i of row
 *                        o % 128 = w[o, 16 cb + i, t] for the forward (flip = 0, w: [O, I, 3, 3], O = Co,
 *                        I = C) or w[16 cb + i, o, 8 - t] for the input gradient (flip = 1, w: [I, O, 3, 3]
 *                        read as the flipped transpose, O = C, I = Co); values 144..151 of a row are 0.
 *                        O a multiple of 128, I of 16, w 16-byte aligned.
 *  "conv3x3_{dt}":       y[n, o, h, w] = sum_{i, kh, kw} wr(o, i, 3 kh + kw) * x[n, i, h + kh - 1, w + kw - 1]
 *                        (0 outside x) + bias[o] when has_bias; x: [N, I, H, W], y: [N, O, H, W], both
 *                        contiguous and 16-byte aligned; I a multiple of 16, O of 128, W of 64.  The input
 *                        channels are split over `splits` (>= 1, dividing I / 16) workgroups per output
 *                        tile; splits > 1 needs ws, splits * N * O * H * W fp32 values (16-byte aligned),
 *                        for the partial sums, which a second kernel queued by the same call adds in split
 *                        order.  hrt_conv3_splits gives the split the shim uses.  The forward is
 *                        (x, wprep(w, 0)); the input gradient of y = conv(x, w) is (dy, wprep(w, 1)) with
 *                        I = Co, O = C. */
#define HRT_CONV3_SLAB_BYTES 38912
static inline int64_t hrt_conv3_wr_bytes(int64_t O, int64_t I) { return (O / 128) * (I / 16) * HRT_CONV3_SLAB_BYTES; }
/* Input-channel split of "conv3x3_{dt}": doubles while the grid (N * ceil(H / 2) * W / 64 * O / 128 tiles,
 * times the split) stays under 256 workgroups and every split keeps at least 4 channel blocks. */
static inline int64_t hrt_conv3_splits(int64_t N, int64_t I, int64_t O, int64_t H, int64_t W) {
  const int64_t tiles = N * ((H + 1) / 2) * (W / 64) * (O / 128), nb = I / 16;
  int64_t s = 1;
  while (tiles * s * 2 <= 256 && nb % (2 * s) == 0 && nb / (2 * s) >= 4) s *= 2;
  return s;
}
typedef struct hrt_conv3_wprep_args {
  uint64_t w, wr;
  int64_t O, I;
  uint32_t flip, pad;
} hrt_conv3_wprep_args;
typedef struct hrt_conv3_args {
  uint64_t x, wr, bias, y, ws;
  int64_t N, I, O, H, W;
  uint32_t has_bias, splits;
} hrt_conv3_args;

/* "upsample_nearest_fwd_{dt}" / "upsample_nearest_bwd_{dt}" — nearest-neighbour upsampling of [NC, H, W]
 * by the integer factors OH / H and OW / W (src index = dst index / factor) and its backward, dst [NC, H, W]
 * = the sum of each factor block of src [NC, OH, OW] (fp32, fixed order).  Contiguous.  Replaces "up_fwd" /
 * "up_bwd" and UpPush (csrc/ops_conv.cpp:37-41, 185-221). */
typedef struct hrt_upsample_args {
  uint64_t src, dst;
  int64_t NC, H, W, OH, OW;
} hrt_upsample_args;

/* "gn_fwd_{dt}": y = (x - mean[n, g]) * rstd[n, g] * w[c] + b[c] over x [N, C, HW] contiguous, G groups of
 * C / G channels; mean and rstd = 1 / sqrt(var + eps) (biased variance) are written [N, G] in x's dtype,
 * as PyTorch's CPU kernel returns them; w, b optional (0).  Statistics: fp32 Welford partials over chunks
 * of each group, merged in a fixed order.  ws: fp32 [hrt_gn_workspace(N, C, HW, G)].
 * "gn_bwd_{dt}": from g = dL/dy, x, mean, rstd (x's dtype) and optional w: dx (if nonzero) =
 * rstd*w*g + c2*x + c3 per (n, g) with c2 = (db_g*mean - ds_g)*rstd^3/M, c3 = -c2*mean - db_g*rstd/M,
 * ds_g = sum over the group of w[c]*sum_hw(g*x), db_g = sum of w[c]*sum_hw(g), M = HW*C/G; dw[c] (if
 * nonzero) = sum_n (sum_hw(g*x) - sum_hw(g)*mean)*rstd; db[c] = sum_n sum_hw(g).  ws as for the forward.
 * Replaces "gn_fwd" / "gn_bwd" / "gn_wgrad" and GnPush (csrc/ops_norm.cpp:27-33, 67-142). */
typedef struct hrt_gn_args {
  uint64_t x, y, g, mean, rstd, w, b, dx, dw, db, ws;
  int64_t N, C, HW, G;
  float eps;
  uint32_t pad;
} hrt_gn_args;

/* Workspace of "gn_fwd_*" / "gn_bwd_*": fp32 elements (group-statistics partials, per-channel sums). */
static inline int64_t hrt_gn_chunks(int64_t C, int64_t HW, int64_t G) {
  const int64_t m = (C / G) * HW; /* elements per group */
  int64_t k = (m + 16383) / 16384;
  return k < 1 ? 1 : (k > 256 ? 256 : k);
}
static inline int64_t hrt_gn_workspace(int64_t N, int64_t C, int64_t HW, int64_t G) {
  const int64_t fwd = N * G * hrt_gn_chunks(C, HW, G) * 3, bwd = 2 * N * C + 2 * N * G;
  return fwd > bwd ? fwd : bwd;
}

#ifdef __cplusplus
}
#endif

#endif /* HRT_OPS_H_ */
