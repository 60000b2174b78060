"""numpy restatements of the reference's hot-path algorithms (test infrastructure only; see __init__).

Every function takes and returns numpy arrays.  Floating-point arithmetic is float64 (the reference's
own tests compare against CPU float64); the bit-exact parts (rounding, dequant) reproduce the exact
float32 bit patterns the reference kernels store.
"""

import numpy as np

# ---------------------------------------------------------------------------------------------------------
# Rounding contract — vkrt/shaders/types.glsl:18-50
# ---------------------------------------------------------------------------------------------------------


def round_bf16(x):
    """float32 -> bf16 bit pattern (uint16): round to nearest even, every NaN -> 0x7FC0.
    types.glsl:45-50 (f2bf)."""
    shape = np.shape(x)  # ascontiguousarray makes 0-dim arrays 1-dim
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, 0x7FC0, r)
    return r.astype(np.uint16).reshape(shape)


def bf16_to_f32(bits):
    """bf16 bit pattern -> float32 (exact).  types.glsl:44 (bf2f)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_f16(x):
    """float32 -> IEEE half bit pattern (uint16), round to nearest even including subnormals, overflow
    -> inf, NaN -> quiet NaN with the top payload bits.  types.glsl:18-41 (f2h)."""
    shape = np.shape(x)
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.int64)
    sign = (u >> 16) & 0x8000
    e = (u >> 23) & 0xFF
    m = u & 0x7FFFFF
    out = np.zeros(u.shape, dtype=np.int64)
    # inf / NaN
    special = e == 0xFF
    out = np.where(special, sign | 0x7C00 | np.where(m != 0, 0x200 | (m >> 13), 0), out)
    ne = e - 127 + 15
    over = (~special) & (ne >= 31)
    out = np.where(over, sign | 0x7C00, out)
    # subnormal or zero result
    sub = (~special) & (ne <= 0)
    tiny = sub & (ne < -10)
    out = np.where(tiny, sign, out)
    subn = sub & ~tiny
    mm = m | 0x800000
    shift = np.clip(14 - ne, 1, 63)
    hm = mm >> shift
    rem = mm & ((np.int64(1) << shift) - 1)
    half = np.int64(1) << (shift - 1)
    up = (rem > half) | ((rem == half) & ((hm & 1) != 0))
    out = np.where(subn, sign | (hm + up.astype(np.int64)), out)
    # normal result (a carry out of the mantissa propagates into the exponent, as intended)
    norm = (~special) & (~over) & (~sub)
    hm = m >> 13
    rem = m & 0x1FFF
    h = sign | (ne << 10) | hm
    up = (rem > 0x1000) | ((rem == 0x1000) & ((hm & 1) != 0))
    out = np.where(norm, h + up.astype(np.int64), out)
    return out.astype(np.uint16).reshape(shape)


def f16_to_f32(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def _round_to(x32, kind):
    """Store rounding of a float32 array for kind "f32" / "bf16" / "f16": returns the stored value as
    float32 (and the raw bits for the 16-bit kinds)."""
    if kind == "f32":
        return x32.astype(np.float32), x32.astype(np.float32).view(np.uint32)
    if kind == "bf16":
        b = round_bf16(x32)
        return bf16_to_f32(b), b
    if kind == "f16":
        b = round_f16(x32)
        return f16_to_f32(b), b
    raise ValueError(kind)


# ---------------------------------------------------------------------------------------------------------
# int8 weight-only dequant — vkrt/shaders/dq8.comp.in:39-62, closed form torch_vulkan/__init__.py:203-205
# ---------------------------------------------------------------------------------------------------------


def dequant_int8(q, scale_bits, kind):
    """out[r, c] = round_kind(float32(q[r, c]) * float32(scale[r, c // 64])).

    q: int8 [rows, cols]; scale_bits: uint16 bf16 patterns [rows, ceil(cols / 64)].  The float32 product
    of an 8-bit integer and an 8-bit-significand bf16 is exact, so the only rounding is the store.
    Returns the stored bit patterns (uint32 for f32, uint16 for bf16/f16)."""
    q = np.asarray(q, dtype=np.int8)
    rows, cols = q.shape
    nb = (cols + 63) // 64
    s = bf16_to_f32(np.asarray(scale_bits, dtype=np.uint16).reshape(rows, nb))
    col_block = np.arange(cols) // 64
    prod = q.astype(np.float32) * s[:, col_block]  # exact in float32
    return _round_to(prod, kind)[1]


# ---------------------------------------------------------------------------------------------------------
# GEMM — epilogue vkrt/shaders/mm.comp.in:142-153 / mm_coop.comp.in:195-208, bias broadcast ops_mm.cpp:80-99
# ---------------------------------------------------------------------------------------------------------


def gemm(a, b, bias=None, alpha=1.0, beta=0.0):
    """alpha * (a @ b) + beta * bias in float64; a [.., M, K], b [.., K, N], bias broadcastable to the
    output (it is ignored when beta == 0, as the reference ignores it)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    acc = np.matmul(a, b)
    r = alpha * acc
    if bias is not None and beta != 0.0:
        r = r + beta * np.broadcast_to(np.asarray(bias, dtype=np.float64), r.shape)
    return r


# ---------------------------------------------------------------------------------------------------------
# softmax — vkrt/shaders/softmax.comp.in:27-50
# ---------------------------------------------------------------------------------------------------------


def softmax_fwd(x, dim=-1, safe=False):
    """y = exp(x - max) / sum(exp(x - max)) along dim; safe: rows whose entries are all -inf give 0."""
    x = np.asarray(x, dtype=np.float64)
    m = np.max(x, axis=dim, keepdims=True)
    all_masked = np.isneginf(m)
    with np.errstate(invalid="ignore", divide="ignore"):
        e = np.exp(x - m)
        y = e / np.sum(e, axis=dim, keepdims=True)
    if safe:
        y = np.where(all_masked, 0.0, y)
    return y


def softmax_bwd(y, g, dim=-1):
    """dx = y * (g - sum(g * y)) along dim."""
    y = np.asarray(y, dtype=np.float64)
    g = np.asarray(g, dtype=np.float64)
    return y * (g - np.sum(g * y, axis=dim, keepdims=True))


# ---------------------------------------------------------------------------------------------------------
# layer_norm — vkrt/shaders/ln.comp.in:42-62 (forward), :63-81 (dx), :27-38 (dw, db)
# ---------------------------------------------------------------------------------------------------------


def layer_norm_fwd(x, ndim_norm=1, w=None, b=None, eps=1e-5):
    """Normalise over the trailing ndim_norm dims.  Two-pass variance.  Returns (y, mean, rstd) with the
    statistics shaped like x with the normalised dims set to 1."""
    x = np.asarray(x, dtype=np.float64)
    axes = tuple(range(x.ndim - ndim_norm, x.ndim))
    mean = np.mean(x, axis=axes, keepdims=True)
    var = np.mean((x - mean) ** 2, axis=axes, keepdims=True)
    rstd = 1.0 / np.sqrt(var + eps)
    y = (x - mean) * rstd
    if w is not None:
        y = y * np.asarray(w, dtype=np.float64)
    if b is not None:
        y = y + np.asarray(b, dtype=np.float64)
    return y, mean, rstd


def layer_norm_bwd(g, x, mean, rstd, ndim_norm=1, w=None):
    """dx = rstd * (gw - mean(gw) - xhat * mean(gw * xhat)), gw = g * w; dw = sum_rows g * xhat;
    db = sum_rows g.  Returns (dx, dw, db)."""
    g = np.asarray(g, dtype=np.float64)
    x = np.asarray(x, dtype=np.float64)
    axes = tuple(range(x.ndim - ndim_norm, x.ndim))
    lead = tuple(range(0, x.ndim - ndim_norm))
    xhat = (x - mean) * rstd
    gw = g * np.asarray(w, dtype=np.float64) if w is not None else g
    s1 = np.mean(gw, axis=axes, keepdims=True)
    s2 = np.mean(gw * xhat, axis=axes, keepdims=True)
    dx = rstd * (gw - s1 - xhat * s2)
    dw = np.sum(g * xhat, axis=lead)
    db = np.sum(g, axis=lead)
    return dx, dw, db


# ---------------------------------------------------------------------------------------------------------
# fused attention — forward vkrt/shaders/attn.comp.in:256-313 / attn_coop.comp.in:158-211,
# delta attn.comp.in:210-240 with ops_attn.cpp:240-248, backward attn.comp.in:315-395 / attn_coop.comp.in:213-301
# ---------------------------------------------------------------------------------------------------------


def attention_fwd(q, k, v, scale):
    """q [B,H,Sq,D], k, v [B,H,Sk,D] -> (out [B,H,Sq,D], lse [B,H,Sq]); online-softmax result written as the
    closed form softmax(scale q k^T) v, lse = log sum exp(scale q k^T)."""
    q, k, v = (np.asarray(t, dtype=np.float64) for t in (q, k, v))
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * scale
    m = np.max(s, axis=-1, keepdims=True)
    p = np.exp(s - m)
    l = np.sum(p, axis=-1, keepdims=True)
    out = np.matmul(p / l, v)
    lse = (m + np.log(l))[..., 0]
    return out, lse


def attention_delta(o, dout):
    """delta[b,h,i] = sum_d O[b,h,i,d] * dO[b,h,i,d] (O is the unrounded forward output)."""
    return np.sum(np.asarray(o, dtype=np.float64) * np.asarray(dout, dtype=np.float64), axis=-1)


def attention_bwd(q, k, v, dout, lse, delta, scale, round_pds=None):
    """Flash-attention backward from the saved lse and delta:
        P = exp(scale q k^T - lse), dP = dO v^T, dS = P * (dP - delta),
        dV = P^T dO, dK = scale dS^T q, dQ = scale dS k.
    round_pds: optional function applied to P and dS before the second products (the matrix-core
    kernels feed them to the MFMA in the input dtype, attn_coop.comp.in:235-236, 283-284)."""
    q, k, v, dout = (np.asarray(t, dtype=np.float64) for t in (q, k, v, dout))
    lse = np.asarray(lse, dtype=np.float64)[..., None]
    delta = np.asarray(delta, dtype=np.float64)[..., None]
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * scale
    p = np.exp(s - lse)
    dp = np.matmul(dout, np.swapaxes(v, -1, -2))
    ds = p * (dp - delta)
    if round_pds is not None:
        p, ds = round_pds(p), round_pds(ds)
    dv = np.matmul(np.swapaxes(p, -1, -2), dout)
    dk = np.matmul(np.swapaxes(ds, -1, -2), q) * scale
    dq = np.matmul(ds, k) * scale
    return dq, dk, dv


def rel_l2(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(got - ref) / (np.linalg.norm(ref) + 1e-300))


# ---------------------------------------------------------------------------------------------------------
# Elementwise — vkrt/shaders/ew.comp.in:115-257 (op expressions tools/gen_shaders.py:53-92), adapters
# csrc/ops_ew.cpp:146-455
# ---------------------------------------------------------------------------------------------------------

# Ops whose float32 evaluation the restatement reproduces bit for bit: sums, products, quotients and
# square roots rounded one at a time in the written order (numpy never fuses a multiply-add).  The
# others contain exp / erf / tanh / sin / cos / pow, whose float32 library results differ between
# implementations in the last bits; for them the restatement evaluates the same formula in float64.
EW_EXACT = frozenset({
    "add", "sub", "mul", "div", "add_s", "mul_s", "div_s", "axpb", "rdiv_s", "neg", "rsqrt", "recip", "sqrt",
    "relu", "addcmul", "addcdiv", "lerp_s", "where",
})
EW_POW_EXACT = (2.0, 3.0, 0.5, -0.5, -1.0, -2.0)  # exponents evaluated by products / sqrt / reciprocal

_SQRT_HALF = 0.70710678118654752440
_INV_SQRT_2PI = 0.39894228040143267794
_SQRT_2_OVER_PI = 0.79788456080286535588
_KAPPA = 0.044715


def _erf(x):
    try:
        from scipy.special import erf
    except ImportError:  # pragma: no cover - scipy is part of the image
        import math

        erf = np.vectorize(math.erf, otypes=[np.float64])
    return erf(x)


def _ew_formula(op, x, y, z, s0, s1, f):
    """The formula of `op` with every constant and intermediate in the float type f (np.float32 for the
    exact ops, np.float64 for the rest)."""
    s0, s1 = f(s0), f(s1)
    one, half = f(1.0), f(0.5)
    if op == "add":
        return x + s0 * y
    if op == "sub":
        return x - s0 * y
    if op == "mul":
        return x * y
    if op == "div":
        return x / y
    if op == "add_s":
        return x + s0
    if op == "mul_s":
        return x * s0
    if op == "div_s":
        return x / s0
    if op == "axpb":
        return s1 + s0 * x
    if op == "rdiv_s":
        return s0 / x
    if op == "pow_s":
        e = float(s0)
        if e == 2.0:
            return x * x
        if e == 3.0:
            return x * x * x
        if e == 0.5:
            return np.sqrt(x)
        if e == -0.5:
            return one / np.sqrt(x)
        if e == -1.0:
            return one / x
        if e == -2.0:
            return one / (x * x)
        return np.power(x, s0)
    if op == "neg":
        return -x
    if op == "rsqrt":
        return one / np.sqrt(x)
    if op == "recip":
        return one / x
    if op == "exp":
        return np.exp(x)
    if op == "sin":
        return np.sin(x)
    if op == "cos":
        return np.cos(x)
    if op == "sqrt":
        return np.sqrt(x)
    if op == "tanh":
        return np.tanh(x)
    if op == "sigmoid":
        return one / (one + np.exp(-x))
    if op == "relu":
        return np.where(x < 0, f(0.0), x)
    if op == "silu":
        return x / (one + np.exp(-x))
    if op == "gelu_erf":
        return half * x * (one + _erf(x * f(_SQRT_HALF)))
    if op == "gelu_tanh":
        return half * x * (one + np.tanh(f(_SQRT_2_OVER_PI) * (x + f(_KAPPA) * x * x * x)))
    if op == "silu_bwd":  # x = grad, y = input
        s = one / (one + np.exp(-y))
        return x * s * (one + y * (one - s))
    if op == "gelu_erf_bwd":
        cdf = half * (one + _erf(y * f(_SQRT_HALF)))
        pdf = f(_INV_SQRT_2PI) * np.exp(-half * y * y)
        return x * (cdf + y * pdf)
    if op == "gelu_tanh_bwd":
        y2 = y * y
        t = np.tanh(f(_SQRT_2_OVER_PI) * (y + f(_KAPPA) * y2 * y))
        dright = half * y * (one - t * t) * f(_SQRT_2_OVER_PI) * (one + f(3.0) * f(_KAPPA) * y2)
        return x * (half * (one + t) + dright)
    if op == "addcmul":
        return x + s0 * y * z
    if op == "addcdiv":
        return x + s0 * y / z
    if op == "lerp_s":
        return x + s0 * (y - x) if abs(float(s0)) < 0.5 else y - (y - x) * (one - s0)
    if op == "where":
        return np.where(z != 0, x, y)
    raise ValueError(op)


def ew_map(op, a, b=None, c=None, s0=0.0, s1=0.0, out_kind="f32"):
    """out = f(a, b, c; s0, s1) as the device computes it: inputs (float arrays holding values of their
    storage type, broadcast numpy-style) widened to float32, the formula in float32, one store rounding
    to out_kind.  Ops outside EW_EXACT (and pow_s with another exponent) evaluate the formula in float64
    from the same float32 inputs and round that to float32 first: the correctly rounded result the
    device's float32 evaluation approximates.  Returns (stored value as float32, stored bits)."""
    exact = op in EW_EXACT or (op == "pow_s" and float(s0) in EW_POW_EXACT)
    f = np.float32 if exact else np.float64
    arrs = [np.asarray(t, dtype=np.float32) for t in (a, b, c) if t is not None]
    shape = np.broadcast_shapes(*[t.shape for t in arrs])
    x, y, z = (np.broadcast_to(np.asarray(t, dtype=np.float32), shape).astype(f) if t is not None else None
               for t in (a, b, c))
    with np.errstate(all="ignore"):
        r = _ew_formula(op, x, y, z, s0, s1, f)
        r32 = np.asarray(r, dtype=np.float64).astype(np.float32).reshape(shape)
    return _round_to(r32, out_kind)


# ---------------------------------------------------------------------------------------------------------
# sum / mean — csrc/ops_rows.cpp:183-270, vkrt/shaders/reduce.comp.in:27-44
# ---------------------------------------------------------------------------------------------------------


def reduce_sum(x, dims=None, keepdim=False, mean=False, out_kind="f32"):
    """sum (or mean: the sum divided by the reduced element count) of x over `dims` (every dimension when
    None or empty), accumulated in float64, then one store rounding to out_kind.  The device accumulates in
    float32, which the reduction tolerance covers.  Returns (stored value as float32, stored bits)."""
    x = np.asarray(x, dtype=np.float64)
    axes = tuple(range(x.ndim)) if not dims else tuple(sorted(d % x.ndim for d in dims))
    n = 1
    for d in axes:
        n *= x.shape[d]
    s = np.sum(x, axis=axes, keepdims=keepdim)
    with np.errstate(all="ignore"):
        r = s / n if mean else s
        r32 = np.asarray(r, dtype=np.float64).astype(np.float32)
    return _round_to(r32, out_kind)


# ---------------------------------------------------------------------------------------------------------
# conv2d, nearest upsampling, group_norm — csrc/ops_conv.cpp:60-221, vkrt/shaders/im2col.comp.in,
# upsample.comp.in; csrc/ops_norm.cpp:67-142, vkrt/shaders/gn.comp.in
# ---------------------------------------------------------------------------------------------------------


def _taps(x, KH, KW, stride, padding):
    """(kh, kw, patch) for every kernel tap: patch[n, c, oh, ow] = zero-padded x at (oh*sh + kh, ow*sw + kw)."""
    (sh, sw), (ph, pw) = stride, padding
    N, C, H, W = x.shape
    OH, OW = (H + 2 * ph - KH) // sh + 1, (W + 2 * pw - KW) // sw + 1
    xp = np.pad(x, ((0, 0), (0, 0), (ph, ph), (pw, pw)))
    for kh in range(KH):
        for kw in range(KW):
            yield kh, kw, xp[:, :, kh:kh + sh * (OH - 1) + 1:sh, kw:kw + sw * (OW - 1) + 1:sw]


def conv2d(x, w, b=None, stride=(1, 1), padding=(0, 0)):
    """NCHW cross-correlation in float64: out[n, o, oh, ow] = sum_{c, kh, kw} w[o, c, kh, kw] * x[n, c,
    oh*sh - ph + kh, ow*sw - pw + kw] (0 outside x) + b[o].  ops_conv.cpp:91-97 (im2col + product)."""
    x, w = np.asarray(x, np.float64), np.asarray(w, np.float64)
    out = None
    for kh, kw, patch in _taps(x, w.shape[2], w.shape[3], stride, padding):
        t = np.einsum("nchw,oc->nohw", patch, w[:, :, kh, kw])
        out = t if out is None else out + t
    if b is not None:
        out = out + np.asarray(b, np.float64)[None, :, None, None]
    return out


def conv2d_backward(x, w, gout, stride=(1, 1), padding=(0, 0)):
    """(dx, dw, db) of conv2d for the output gradient gout, float64: dw[o, c, kh, kw] = sum gout * tap,
    dx = the adjoint scatter of every tap, db = gout summed over n, h, w.  ops_conv.cpp:126-178."""
    x, w, gout = (np.asarray(t, np.float64) for t in (x, w, gout))
    (sh, sw), (ph, pw) = stride, padding
    N, C, H, W = x.shape
    KH, KW = w.shape[2], w.shape[3]
    OH, OW = gout.shape[2], gout.shape[3]
    gxp = np.zeros((N, C, H + 2 * ph, W + 2 * pw))
    dw = np.zeros_like(w)
    for kh, kw, patch in _taps(x, KH, KW, stride, padding):
        dw[:, :, kh, kw] = np.einsum("nohw,nchw->oc", gout, patch)
        gxp[:, :, kh:kh + sh * (OH - 1) + 1:sh, kw:kw + sw * (OW - 1) + 1:sw] += np.einsum("nohw,oc->nchw", gout, w[:, :, kh, kw])
    return gxp[:, :, ph:ph + H, pw:pw + W], dw, gout.sum(axis=(0, 2, 3))


def upsample_nearest(x, OH, OW):
    """Nearest upsampling by integer factors: out[..., oh, ow] = x[..., oh // fh, ow // fw].  upsample.comp.in."""
    x = np.asarray(x, np.float64)
    H, W = x.shape[-2:]
    return x[..., np.arange(OH) // (OH // H), :][..., np.arange(OW) // (OW // W)]


def upsample_nearest_backward(g, H, W):
    """Adjoint of upsample_nearest: the sum of each fh x fw block of g."""
    g = np.asarray(g, np.float64)
    *lead, OH, OW = g.shape
    return g.reshape(*lead, H, OH // H, W, OW // W).sum(axis=(-3, -1))


def group_norm_fwd(x, G, w=None, b=None, eps=1e-5):
    """(y, mean, rstd) of group_norm over x [N, C, *], float64: statistics over the C / G channels of each
    group and all spatial positions (biased variance), rstd = 1 / sqrt(var + eps), y = (x - mean) * rstd *
    w[c] + b[c].  ops_norm.cpp:67-95, gn.comp.in."""
    x = np.asarray(x, np.float64)
    N, C = x.shape[:2]
    xg = x.reshape(N, G, -1)
    mean, var = xg.mean(-1), xg.var(-1)
    rstd = 1.0 / np.sqrt(var + eps)
    y = ((xg - mean[..., None]) * rstd[..., None]).reshape(x.shape)
    shape = (1, C) + (1,) * (x.ndim - 2)
    if w is not None:
        y = y * np.asarray(w, np.float64).reshape(shape)
    if b is not None:
        y = y + np.asarray(b, np.float64).reshape(shape)
    return y, mean, rstd


def group_norm_bwd(g, x, mean, rstd, G, w=None):
    """(dx, dw, db) of group_norm, float64, from per-(n, c) sums ds = sum_hw g*x and db = sum_hw g:
    ds_g, db_g = sums over a group's channels weighted by w; dx = rstd*w*g + c2*x + c3 with
    c2 = (db_g*mean - ds_g)*rstd^3/M, c3 = -c2*mean - db_g*rstd/M (M = elements per group);
    dw[c] = sum_n (ds - db*mean)*rstd, db[c] = sum_n db.  ops_norm.cpp:97-142, gn.comp.in."""
    g, x = np.asarray(g, np.float64), np.asarray(x, np.float64)
    mean, rstd = np.asarray(mean, np.float64), np.asarray(rstd, np.float64)
    N, C = x.shape[:2]
    Cg = C // G
    gf, xf = g.reshape(N, C, -1), x.reshape(N, C, -1)
    M = Cg * gf.shape[-1]
    ds, dbs = (gf * xf).sum(-1), gf.sum(-1)
    wv = np.ones(C) if w is None else np.asarray(w, np.float64)
    dsg = (ds * wv).reshape(N, G, Cg).sum(-1)
    dbg = (dbs * wv).reshape(N, G, Cg).sum(-1)
    c2 = (dbg * mean - dsg) * rstd ** 3 / M
    c3 = -c2 * mean - dbg * rstd / M
    rep = lambda t: np.repeat(t, Cg, axis=1)[..., None]  # noqa: E731  [N, G] -> [N, C, 1]
    dx = (rep(rstd) * wv[None, :, None] * gf + rep(c2) * xf + rep(c3)).reshape(x.shape)
    dw = ((ds - dbs * np.repeat(mean, Cg, axis=1)) * np.repeat(rstd, Cg, axis=1)).sum(0)
    return dx, dw, dbs.sum(0)
