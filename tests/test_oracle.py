"""Pins the CPU oracle (oracle/) before it is trusted as the parity reference (CPU only).

Each oracle function is checked against something that does not share its code: the committed golden
fixtures (torch's closed forms, tests/golden/make_golden.py), torch's own float64 kernels and autograd,
the C restatement, and closed forms / invariants chosen so that a plausible mistake (a dropped term, a
wrong sign, a transposed operand) fails.  The last tests plant such mistakes in copies of the oracle and
assert that the pins catch them.
"""

import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import build as oracle_build

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")


def torch_bits(t):
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.view(torch.int16).numpy().view(np.uint16)


@pytest.fixture(scope="module")
def clib():
    oracle_build.build()
    return oracle_build.load()


# ---- rounding ------------------------------------------------------------------------------------------------
def all_bf16_neighbourhood():
    """Every bf16 pattern, plus the exact halfway point and its neighbours above each one."""
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    xs = [hi, hi | 0x8000, hi | 0x7FFF, hi | 0x8001, hi | 0x0001]
    return np.concatenate(xs).view(np.float32)


def test_round_bf16_matches_torch_on_all_patterns_and_halfway_cases():
    x = all_bf16_neighbourhood()
    got = oracle.round_bf16(x)
    ref = torch_bits(torch.from_numpy(x.copy()).to(torch.bfloat16))
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all(got[nan] == 0x7FC0)  # the reference canonicalises every NaN (types.glsl:46)


def test_round_f16_matches_torch_including_subnormals_and_overflow():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        all_bf16_neighbourhood(),
        rng.standard_normal(200000).astype(np.float32) * np.float32(2.0) ** rng.integers(-30, 18, 200000).astype(np.float32),
    ]).astype(np.float32)
    got = oracle.round_f16(x)
    ref = torch_bits(torch.from_numpy(x.copy()).to(torch.float16))
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x3FF) != 0)


def test_rounding_golden_fixture(clib):
    d = np.load(os.path.join(GOLD, "rounding.npz"))
    x = d["x"]
    assert np.array_equal(oracle.round_bf16(x), d["bf16"])
    assert np.array_equal(oracle.round_f16(x), d["f16"])
    out = np.empty(x.shape, np.uint16)
    clib.oracle_round_bf16(x.ctypes.data, out.ctypes.data, x.size)
    assert np.array_equal(out, d["bf16"])
    clib.oracle_round_f16(x.ctypes.data, out.ctypes.data, x.size)
    assert np.array_equal(out, d["f16"])


def test_c_rounding_matches_numpy_rounding(clib):
    x = all_bf16_neighbourhood()
    out = np.empty(x.shape, np.uint16)
    clib.oracle_round_bf16(x.ctypes.data, out.ctypes.data, x.size)
    assert np.array_equal(out, oracle.round_bf16(x))
    clib.oracle_round_f16(x.ctypes.data, out.ctypes.data, x.size)
    assert np.array_equal(out, oracle.round_f16(x))


# ---- dequant -----------------------------------------------------------------------------------------------------
def golden_dq_cases():
    d = np.load(os.path.join(GOLD, "dequant_int8.npz"))
    keys = sorted({k.rsplit("_q", 1)[0] for k in d.files if k.endswith("_q")})
    return d, keys


@pytest.mark.parametrize("kind", ["f32", "bf16", "f16"])
def test_dequant_oracle_matches_golden_fixtures(kind, clib):
    d, keys = golden_dq_cases()
    assert len(keys) >= 9
    for key in keys:
        q, s, ref = d[key + "_q"], d[key + "_scale"], d[key + "_out_" + kind]
        assert np.array_equal(oracle.dequant_int8(q, s, kind), ref), key
        out = np.empty(ref.shape, ref.dtype)
        clib.oracle_dequant_int8(np.ascontiguousarray(q).ctypes.data, np.ascontiguousarray(s).ctypes.data, q.shape[0],
                                 q.shape[1], {"f32": 0, "bf16": 1, "f16": 2}[kind], out.ctypes.data)
        assert np.array_equal(out, ref), key


def test_dequant_product_is_exact_in_float32():
    """The only rounding is the store: int8 x bf16 has at most 16 significant bits."""
    q = np.arange(-128, 128, dtype=np.int8).reshape(4, 64)
    s = oracle.round_bf16(np.random.default_rng(3).uniform(1e-4, 0.02, (4, 1)).astype(np.float32))
    exact = q.astype(np.float64) * oracle.bf16_to_f32(s).astype(np.float64)
    f32 = oracle.dequant_int8(q, s, "f32").view(np.float32)
    assert np.array_equal(f32.astype(np.float64), exact)


def test_dequant_matches_torch_closed_form_on_large_random_case():
    g = torch.Generator().manual_seed(5)
    q = torch.randint(-127, 128, (64, 2048), generator=g, dtype=torch.int8)
    scale = (torch.rand(64, 32, generator=g) * 0.019 + 0.001).to(torch.bfloat16)
    ref = (q.float() * scale.float().repeat_interleave(64, dim=1)).to(torch.bfloat16)
    got = oracle.dequant_int8(q.numpy(), torch_bits(scale), "bf16")
    assert np.array_equal(got, torch_bits(ref))


# ---- GEMM ----------------------------------------------------------------------------------------------------------
def test_gemm_matches_torch_float64_with_bias_broadcast():
    rng = np.random.default_rng(0)
    a, b = rng.standard_normal((3, 7, 5)), rng.standard_normal((3, 5, 9))
    bias = rng.standard_normal((3, 1, 9))
    got = oracle.gemm(a, b, bias, alpha=0.5, beta=2.0)
    ref = torch.baddbmm(torch.from_numpy(bias), torch.from_numpy(a), torch.from_numpy(b), alpha=0.5, beta=2.0).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
    # beta = 0 ignores the bias entirely, even a NaN one (the reference skips it, csrc/ops_mm.cpp:80)
    got0 = oracle.gemm(a, b, np.full((9,), np.nan), alpha=1.0, beta=0.0)
    np.testing.assert_allclose(got0, np.matmul(a, b), rtol=1e-12)


def test_gemm_closed_forms():
    rng = np.random.default_rng(1)
    a = rng.standard_normal((6, 6))
    np.testing.assert_allclose(oracle.gemm(a, np.eye(6)), a)
    np.testing.assert_allclose(oracle.gemm(np.eye(6), a), a)
    # (AB)^T = B^T A^T — a transposed operand would break this
    b = rng.standard_normal((6, 4))
    np.testing.assert_allclose(oracle.gemm(a, b).T, oracle.gemm(b.T, a.T), rtol=1e-12)


# ---- softmax ------------------------------------------------------------------------------------------------------
def test_softmax_matches_torch_and_invariants():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 5, 37)) * 3
    for dim in (0, 1, 2, -1):
        ref = torch.softmax(torch.from_numpy(x), dim).numpy()
        got = oracle.softmax_fwd(x, dim)
        np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-15)
        np.testing.assert_allclose(got.sum(axis=dim), 1.0, rtol=1e-12)
    np.testing.assert_allclose(oracle.softmax_fwd(x + 123.0), oracle.softmax_fwd(x), rtol=1e-9)


def test_safe_softmax_zero_rows_and_masked_entries():
    x = np.random.default_rng(3).standard_normal((4, 33))
    x[1, :] = -np.inf
    x[2, :5] = -np.inf
    got = oracle.softmax_fwd(x, -1, safe=True)
    ref = torch._safe_softmax(torch.from_numpy(x), -1).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=0)
    assert np.all(got[1] == 0.0) and np.all(got[2, :5] == 0.0)
    assert np.all(np.isnan(oracle.softmax_fwd(x, -1, safe=False)[1]))  # plain softmax of an all -inf row is NaN


def test_softmax_backward_matches_autograd():
    rng = np.random.default_rng(4)
    x = torch.from_numpy(rng.standard_normal((5, 4, 37)) * 2).requires_grad_(True)
    g = rng.standard_normal((5, 4, 37))
    y = torch.softmax(x, -1)
    y.backward(torch.from_numpy(g))
    np.testing.assert_allclose(oracle.softmax_bwd(y.detach().numpy(), g, -1), x.grad.numpy(), rtol=1e-10, atol=1e-14)


# ---- layer_norm -----------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("affine", [False, True])
def test_layer_norm_forward_backward_match_torch(affine):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, 96)) * 2
    w = rng.standard_normal(96) if affine else None
    b = rng.standard_normal(96) if affine else None
    g = rng.standard_normal((6, 96))
    xt = torch.from_numpy(x).requires_grad_(True)
    wt = torch.from_numpy(w).requires_grad_(True) if affine else None
    bt = torch.from_numpy(b).requires_grad_(True) if affine else None
    yt = F.layer_norm(xt, (96,), wt, bt, 1e-5)
    yt.backward(torch.from_numpy(g))
    y, mean, rstd = oracle.layer_norm_fwd(x, 1, w, b, 1e-5)
    np.testing.assert_allclose(y, yt.detach().numpy(), rtol=1e-10, atol=1e-12)
    _, tm, trs = torch.native_layer_norm(torch.from_numpy(x), (96,), None, None, 1e-5)
    np.testing.assert_allclose(mean, tm.numpy(), rtol=1e-12)
    np.testing.assert_allclose(rstd, trs.numpy(), rtol=1e-10)
    dx, dw, db = oracle.layer_norm_bwd(g, x, mean, rstd, 1, w)
    np.testing.assert_allclose(dx, xt.grad.numpy(), rtol=1e-9, atol=1e-12)
    if affine:
        np.testing.assert_allclose(dw, wt.grad.numpy(), rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(db, bt.grad.numpy(), rtol=1e-12, atol=1e-12)


def test_layer_norm_moments_and_multi_dim():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((4, 3, 5)) * 3 + 7
    y, mean, rstd = oracle.layer_norm_fwd(x, 2, None, None, 0.0)
    np.testing.assert_allclose(y.mean(axis=(1, 2)), 0.0, atol=1e-12)
    np.testing.assert_allclose(y.var(axis=(1, 2)), 1.0, rtol=1e-10)
    assert mean.shape == (4, 1, 1) and rstd.shape == (4, 1, 1)
    b = rng.standard_normal((3, 5))
    yb, _, _ = oracle.layer_norm_fwd(x, 2, None, b, 0.0)
    np.testing.assert_allclose(yb.mean(axis=0), (y + b).mean(axis=0), atol=1e-12)


# ---- attention ------------------------------------------------------------------------------------------------------
def torch_sdpa_with_grads(q, k, v, g, scale):
    qt, kt, vt = (torch.from_numpy(t).requires_grad_(True) for t in (q, k, v))
    with torch.nn.attention.sdpa_kernel(torch.nn.attention.SDPBackend.MATH):
        o = F.scaled_dot_product_attention(qt, kt, vt, scale=scale)
    o.backward(torch.from_numpy(g))
    return o.detach().numpy(), qt.grad.numpy(), kt.grad.numpy(), vt.grad.numpy()


@pytest.mark.parametrize("shape", [(1, 2, 40, 50, 64), (2, 3, 33, 17, 40), (1, 1, 5, 77, 20)])
def test_attention_matches_torch_math_sdpa_and_autograd(shape):
    B, H, Sq, Sk, D = shape
    rng = np.random.default_rng(7)
    q, k, v = rng.uniform(-1, 1, (B, H, Sq, D)), rng.uniform(-1, 1, (B, H, Sk, D)), rng.uniform(-1, 1, (B, H, Sk, D))
    g = rng.uniform(-1, 1, (B, H, Sq, D))
    scale = 1 / np.sqrt(D)
    ro, rq, rk, rv = torch_sdpa_with_grads(q, k, v, g, scale)
    out, lse = oracle.attention_fwd(q, k, v, scale)
    np.testing.assert_allclose(out, ro, rtol=1e-10, atol=1e-12)
    s = np.einsum("bhqd,bhkd->bhqk", q, k) * scale
    np.testing.assert_allclose(lse, np.log(np.exp(s).sum(-1)), rtol=1e-12)
    delta = oracle.attention_delta(out, g)
    dq, dk, dv = oracle.attention_bwd(q, k, v, g, lse, delta, scale)
    np.testing.assert_allclose(dq, rq, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dk, rk, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dv, rv, rtol=1e-9, atol=1e-11)


def test_attention_special_cases():
    rng = np.random.default_rng(8)
    q, v = rng.standard_normal((1, 2, 9, 16)), rng.standard_normal((1, 2, 1, 16))
    k = rng.standard_normal((1, 2, 1, 16))
    out, lse = oracle.attention_fwd(q, k, v, 0.25)
    np.testing.assert_allclose(out, np.broadcast_to(v, out.shape))  # Sk = 1: every row is v
    k2 = np.broadcast_to(rng.standard_normal((1, 2, 1, 16)), (1, 2, 7, 16))
    v2 = rng.standard_normal((1, 2, 7, 16))
    out2, lse2 = oracle.attention_fwd(q, k2, v2, 0.25)
    np.testing.assert_allclose(out2, np.broadcast_to(v2.mean(axis=2, keepdims=True), out2.shape), rtol=1e-12)
    np.testing.assert_allclose(lse2, np.einsum("bhqd,bhd->bhq", q, k2[:, :, 0]) * 0.25 + np.log(7), rtol=1e-12)
    z = np.zeros((1, 2, 9, 16))
    dq, dk, dv = oracle.attention_bwd(q, k2, v2, z, lse2, oracle.attention_delta(out2, z), 0.25)
    assert not dq.any() and not dk.any() and not dv.any()


# ---- the pins catch planted mistakes -----------------------------------------------------------------------------------
def test_planted_attention_sign_error_is_caught():
    rng = np.random.default_rng(9)
    B, H, Sq, Sk, D = 1, 2, 12, 10, 8
    q, k, v = rng.uniform(-1, 1, (B, H, Sq, D)), rng.uniform(-1, 1, (B, H, Sk, D)), rng.uniform(-1, 1, (B, H, Sk, D))
    g = rng.uniform(-1, 1, (B, H, Sq, D))
    _, rq, rk, _ = torch_sdpa_with_grads(q, k, v, g, 0.3)
    out, lse = oracle.attention_fwd(q, k, v, 0.3)
    # mistake 1: delta with the wrong sign; mistake 2: dK from dS instead of dS^T (transposed operand)
    bad_delta = -oracle.attention_delta(out, g)
    dq_bad, _, _ = oracle.attention_bwd(q, k, v, g, lse, bad_delta, 0.3)
    assert not np.allclose(dq_bad, rq, rtol=1e-6)
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * 0.3
    p = np.exp(s - lse[..., None])
    ds = p * (np.matmul(g, np.swapaxes(v, -1, -2)) - oracle.attention_delta(out, g)[..., None])
    dk_bad = np.matmul(ds[..., :Sk, :Sk], q[..., :Sk, :]) * 0.3  # wrong orientation
    assert not np.allclose(dk_bad, rk, rtol=1e-6)


def test_planted_layer_norm_dropped_term_is_caught():
    rng = np.random.default_rng(10)
    x, g = rng.standard_normal((3, 16)), rng.standard_normal((3, 16))
    xt = torch.from_numpy(x).requires_grad_(True)
    F.layer_norm(xt, (16,), None, None, 1e-5).backward(torch.from_numpy(g))
    _, mean, rstd = oracle.layer_norm_fwd(x, 1, None, None, 1e-5)
    xhat = (x - mean) * rstd
    dx_bad = rstd * (g - g.mean(-1, keepdims=True))  # dropped the xhat * mean(g * xhat) term
    assert not np.allclose(dx_bad, xt.grad.numpy(), rtol=1e-6)
    assert np.allclose(oracle.layer_norm_bwd(g, x, mean, rstd)[0], xt.grad.numpy(), rtol=1e-9, atol=1e-12)
    assert xhat.shape == x.shape


def test_planted_rounding_truncation_is_caught():
    x = all_bf16_neighbourhood()
    truncated = (x.view(np.uint32) >> 16).astype(np.uint16)  # round-toward-zero instead of RNE
    ref = torch_bits(torch.from_numpy(x.copy()).to(torch.bfloat16))
    nan = np.isnan(x)
    assert not np.array_equal(truncated[~nan], ref[~nan])


# ---- elementwise (oracle.ew_map) -------------------------------------------------------------------------------
# The reference's own checks compare each op with CPU PyTorch at these tolerances (tests/test_ops_ew.py:17)
EW_TOL = {torch.float32: (1e-5, 1e-6), torch.bfloat16: (2e-2, 1e-3), torch.float16: (4e-3, 1e-4)}
EW_KIND = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}
_gelu_bwd = torch.ops.aten.gelu_backward
# op -> (torch CPU form, input range (lo, hi) of every operand, scalars s0, s1, tolerance scale)
EW_CASES = {
    "add": (lambda x, y, z, s0, s1: torch.add(x, y, alpha=s0), (-3, 3), 2.0, 0.0, 1.0),
    "sub": (lambda x, y, z, s0, s1: torch.sub(x, y, alpha=s0), (-3, 3), 0.5, 0.0, 1.0),
    "mul": (lambda x, y, z, s0, s1: torch.mul(x, y), (-3, 3), 0.0, 0.0, 1.0),
    "div": (lambda x, y, z, s0, s1: torch.div(x, y), (0.5, 3), 0.0, 0.0, 1.0),
    "add_s": (lambda x, y, z, s0, s1: torch.add(x, s0), (-3, 3), 2.5, 0.0, 1.0),
    "mul_s": (lambda x, y, z, s0, s1: torch.mul(x, s0), (-3, 3), 0.999, 0.0, 1.0),
    "div_s": (lambda x, y, z, s0, s1: torch.div(x, s0), (-3, 3), 3.0, 0.0, 1.0),
    "axpb": (lambda x, y, z, s0, s1: torch.add(s1, x, alpha=s0), (-3, 3), 2.0, 2.0, 2.0),
    "rdiv_s": (lambda x, y, z, s0, s1: torch.div(torch.full_like(x, s0), x), (0.5, 3), 2.0, 0.0, 1.0),
    "pow_s": (lambda x, y, z, s0, s1: torch.pow(x, s0), (0.3, 3), 2.5, 0.0, 4.0),
    "neg": (lambda x, y, z, s0, s1: torch.neg(x), (-3, 3), 0.0, 0.0, 1.0),
    "rsqrt": (lambda x, y, z, s0, s1: torch.rsqrt(x), (0.1, 5), 0.0, 0.0, 1.0),
    "recip": (lambda x, y, z, s0, s1: torch.reciprocal(x), (0.2, 5), 0.0, 0.0, 1.0),
    "exp": (lambda x, y, z, s0, s1: torch.exp(x), (-4, 4), 0.0, 0.0, 2.0),
    "sin": (lambda x, y, z, s0, s1: torch.sin(x), (-8, 8), 0.0, 0.0, 1.0),
    "cos": (lambda x, y, z, s0, s1: torch.cos(x), (-8, 8), 0.0, 0.0, 1.0),
    "sqrt": (lambda x, y, z, s0, s1: torch.sqrt(x), (0.0, 6), 0.0, 0.0, 1.0),
    "tanh": (lambda x, y, z, s0, s1: torch.tanh(x), (-4, 4), 0.0, 0.0, 1.0),
    "sigmoid": (lambda x, y, z, s0, s1: torch.sigmoid(x), (-6, 6), 0.0, 0.0, 1.0),
    "relu": (lambda x, y, z, s0, s1: torch.relu(x), (-3, 3), 0.0, 0.0, 1.0),
    "silu": (lambda x, y, z, s0, s1: F.silu(x), (-6, 6), 0.0, 0.0, 1.0),
    "gelu_erf": (lambda x, y, z, s0, s1: F.gelu(x), (-6, 6), 0.0, 0.0, 2.0),
    "gelu_tanh": (lambda x, y, z, s0, s1: F.gelu(x, approximate="tanh"), (-6, 6), 0.0, 0.0, 2.0),
    "silu_bwd": (lambda x, y, z, s0, s1: torch.ops.aten.silu_backward(x, y), (-5, 5), 0.0, 0.0, 3.0),
    "gelu_erf_bwd": (lambda x, y, z, s0, s1: _gelu_bwd(x, y, approximate="none"), (-5, 5), 0.0, 0.0, 3.0),
    "gelu_tanh_bwd": (lambda x, y, z, s0, s1: _gelu_bwd(x, y, approximate="tanh"), (-5, 5), 0.0, 0.0, 3.0),
    "addcmul": (lambda x, y, z, s0, s1: torch.addcmul(x, y, z, value=s0), (0.5, 3), 0.3, 0.0, 2.0),
    "addcdiv": (lambda x, y, z, s0, s1: torch.addcdiv(x, y, z, value=s0), (0.5, 3), -0.7, 0.0, 2.0),
    "lerp_s": (lambda x, y, z, s0, s1: torch.lerp(x, y, s0), (-3, 3), 0.75, 0.0, 2.0),
    "where": (lambda x, y, z, s0, s1: torch.where(z != 0, x, y), (-3, 3), 0.0, 0.0, 1.0),
}
EW_ARITY = {"add": 2, "sub": 2, "mul": 2, "div": 2, "silu_bwd": 2, "gelu_erf_bwd": 2, "gelu_tanh_bwd": 2,
            "lerp_s": 2, "addcmul": 3, "addcdiv": 3, "where": 3}


def ew_inputs(op, dtype, shape=(37, 53), seed=0):
    lo, hi = EW_CASES[op][1]
    g = torch.Generator().manual_seed(seed)
    ts = [(torch.rand(shape, generator=g) * (hi - lo) + lo).to(dtype) for _ in range(EW_ARITY.get(op, 1))]
    if op == "where":
        ts[2] = (torch.rand(shape, generator=g) > 0.5).to(dtype)
    while len(ts) < 3:
        ts.append(None)
    return ts


def ew_oracle(op, ts, s0, s1, dtype):
    arr = [None if t is None else t.float().numpy() for t in ts]
    return oracle.ew_map(op, *arr, s0=s0, s1=s1, out_kind=EW_KIND[dtype])


@pytest.mark.parametrize("dtype", list(EW_KIND))
@pytest.mark.parametrize("op", list(EW_CASES))
def test_ew_oracle_matches_torch_cpu(op, dtype):
    """Every op against CPU PyTorch, the reference tests' own oracle, at their tolerances."""
    fn, _, s0, s1, scale = EW_CASES[op]
    ts = ew_inputs(op, dtype)
    ref = fn(*ts, s0, s1).float().numpy()
    got, _ = ew_oracle(op, ts, s0, s1, dtype)
    rtol, atol = EW_TOL[dtype]
    np.testing.assert_allclose(got, ref, rtol=rtol * scale, atol=atol * scale)


# The CPU kernels round these ops once from a float32 evaluation in the same order, so the restatement must
# give PyTorch's bits exactly (add/sub with alpha 1, where fused and separate multiply-add agree).  Not
# in the list: sqrt and rsqrt, whose CPU float32 kernels are not correctly rounded in the last bit.
EW_BIT_EXACT = ["mul", "div", "add_s", "neg", "recip", "relu", "where"]


@pytest.mark.parametrize("dtype", list(EW_KIND))
@pytest.mark.parametrize("op", ["add", "sub"] + EW_BIT_EXACT)
def test_ew_oracle_bits_equal_torch_where_rounding_is_fixed(op, dtype):
    fn, _, s0, s1, _ = EW_CASES[op]
    if op in ("add", "sub"):
        s0 = 1.0
    ts = ew_inputs(op, dtype, seed=7)
    ref = fn(*ts, s0, s1).contiguous()
    _, got = ew_oracle(op, ts, s0, s1, dtype)
    np.testing.assert_array_equal(got, torch_bits(ref))


def _fd_error(fwd, bwd, x):
    """max |bwd(g=1, x) - central difference of fwd| in float64."""
    h = 1e-5
    one = np.ones_like(x)
    num = (fwd(x + h) - fwd(x - h)) / (2 * h)
    return float(np.max(np.abs(bwd(one, x) - num)))


def _f64(op):
    from oracle.ops import _ew_formula

    return lambda *a: _ew_formula(op, *(list(a) + [None] * (3 - len(a))), 0.0, 0.0, np.float64)


@pytest.mark.parametrize("act", ["silu", "gelu_erf", "gelu_tanh"])
def test_ew_oracle_backward_is_the_derivative(act):
    """silu_bwd / gelu_*_bwd equal the finite-difference derivative of the forward formulas."""
    x = np.linspace(-7, 7, 2001)
    assert _fd_error(_f64(act), _f64(act + "_bwd"), x) < 1e-7


def test_planted_gelu_backward_dropped_factor_is_caught():
    """A tanh-GELU backward without the 3 of d/dx x^3 fails the derivative pin."""
    from oracle.ops import _SQRT_2_OVER_PI, _KAPPA

    def planted(g, y):
        t = np.tanh(_SQRT_2_OVER_PI * (y + _KAPPA * y ** 3))
        return g * (0.5 * (1 + t) + 0.5 * y * (1 - t * t) * _SQRT_2_OVER_PI * (1 + _KAPPA * y * y))

    x = np.linspace(-7, 7, 2001)
    assert _fd_error(_f64("gelu_tanh"), planted, x) > 1e-3


def test_ew_oracle_identities():
    g = np.random.default_rng(3)
    a = g.uniform(-3, 3, 1000).astype(np.float32)
    b = g.uniform(-3, 3, 1000).astype(np.float32)
    # lerp's two-sided form returns its end points exactly
    assert np.array_equal(oracle.ew_map("lerp_s", a, b, s0=0.0)[0], a)
    assert np.array_equal(oracle.ew_map("lerp_s", a, b, s0=1.0)[0], b)
    m = (g.uniform(size=1000) > 0.5).astype(np.float32)
    assert np.array_equal(oracle.ew_map("where", a, b, m)[0], np.where(m != 0, a, b))
    assert np.array_equal(oracle.ew_map("addcmul", a, b, b, s0=0.0)[0], a)
    assert np.array_equal(oracle.ew_map("pow_s", a, s0=2.0)[1], oracle.ew_map("mul", a, a)[1])
    assert np.array_equal(oracle.ew_map("sub", a, a, s0=1.0)[0], np.zeros_like(a))
    assert np.array_equal(oracle.ew_map("relu", a)[0], np.maximum(a, 0))
    # silu = x * sigmoid(x); the tanh GELU stays within 5e-4 of the erf GELU (its published accuracy)
    s = oracle.ew_map("sigmoid", a)[0].astype(np.float64)
    np.testing.assert_allclose(oracle.ew_map("silu", a)[0], a * s, rtol=1e-6, atol=1e-7)
    assert np.max(np.abs(oracle.ew_map("gelu_tanh", a)[0] - oracle.ew_map("gelu_erf", a)[0])) < 5e-4
    # broadcasting and the bf16 store rounding
    r, bits = oracle.ew_map("add", a.reshape(10, 100), b[:100], s0=1.0, out_kind="bf16")
    assert r.shape == (10, 100) and np.array_equal(bits, oracle.round_bf16(a.reshape(10, 100) + b[:100]))


def test_ew_oracle_large_argument_sin_cos():
    """RoPE-like arguments up to ~1500 (the reference's range-reduction case)."""
    x = torch.arange(0, 4000, dtype=torch.float32) * 0.37
    for op, fn in (("sin", torch.sin), ("cos", torch.cos)):
        np.testing.assert_allclose(oracle.ew_map(op, x.numpy())[0], fn(x).numpy(), rtol=4e-4, atol=4e-5)


# ---- sum / mean (oracle.reduce_sum) ------------------------------------------------------------------------------
@pytest.mark.parametrize("dims", [None, (0,), (-1,), (1, 2), (0, 3), (0, 1, 2, 3)])
@pytest.mark.parametrize("keepdim", [False, True])
@pytest.mark.parametrize("mean", [False, True])
def test_reduce_oracle_matches_torch(dims, keepdim, mean):
    x = torch.randn(3, 5, 4, 6, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    fn = torch.mean if mean else torch.sum
    ref = fn(x) if dims is None else fn(x, dim=dims, keepdim=keepdim)
    got, _ = oracle.reduce_sum(x.numpy(), dims, keepdim and dims is not None, mean)
    assert got.shape == tuple(ref.shape)
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-6, atol=1e-6)


def test_reduce_oracle_closed_forms():
    n = 1 << 12
    a = np.arange(n, dtype=np.float64).reshape(64, 64)
    assert oracle.reduce_sum(a)[0] == n * (n - 1) / 2
    assert oracle.reduce_sum(a, mean=True)[0] == (n - 1) / 2
    np.testing.assert_array_equal(oracle.reduce_sum(a, (0,))[0], 64 * np.arange(64) + 64 * 63 * 64 / 2)
    np.testing.assert_array_equal(oracle.reduce_sum(a, (1,), keepdim=True)[0][:, 0], 64 * 64 * np.arange(64) + 63 * 64 / 2)
    e = np.zeros((3, 0))
    assert np.array_equal(oracle.reduce_sum(e, (1,))[0], np.zeros(3))
    assert np.all(np.isnan(oracle.reduce_sum(e, (1,), mean=True)[0]))
    # bf16 store rounding of the float64 result
    r, b = oracle.reduce_sum(np.full((3, 7), 1.0 / 3.0), (1,), out_kind="bf16")
    assert np.array_equal(b, oracle.round_bf16(np.full(3, 7.0 / 3.0, dtype=np.float32)))


# ---- conv2d / nearest upsampling / group_norm --------------------------------------------------------------
CONV_CASES = [(1, 8, 16, 16, 16, 3, 1, 1), (1, 8, 16, 16, 16, 3, 2, 1), (2, 6, 10, 12, 5, 1, 1, 0), (2, 3, 9, 11, 4, 3, 1, 1),
              (1, 5, 13, 7, 6, 3, 2, 0), (1, 4, 9, 9, 3, (3, 5), (2, 1), (1, 2))]


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv2d_oracle_matches_torch_and_autograd(case):
    N, C, H, W, Co, k, s, p = case
    k, s, p = (v if isinstance(v, tuple) else (v, v) for v in (k, s, p))
    g = torch.Generator().manual_seed(3)
    x = torch.randn(N, C, H, W, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(Co, C, *k, generator=g, dtype=torch.float64, requires_grad=True)
    b = torch.randn(Co, generator=g, dtype=torch.float64, requires_grad=True)
    y = F.conv2d(x, w, b, stride=s, padding=p)
    go = torch.randn(y.shape, generator=g, dtype=torch.float64)
    y.backward(go)
    np.testing.assert_allclose(oracle.conv2d(x.detach().numpy(), w.detach().numpy(), b.detach().numpy(), s, p), y.detach().numpy(),
                               rtol=1e-12, atol=1e-12)
    dx, dw, db = oracle.conv2d_backward(x.detach().numpy(), w.detach().numpy(), go.numpy(), s, p)
    for got, ref in ((dx, x.grad), (dw, w.grad), (db, b.grad)):
        np.testing.assert_allclose(got, ref.numpy(), rtol=1e-11, atol=1e-11)


def test_conv2d_oracle_closed_forms():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 3, 7, 8))
    delta = np.zeros((3, 3, 3, 3))
    for c in range(3):
        delta[c, c, 1, 1] = 1.0
    np.testing.assert_array_equal(oracle.conv2d(x, delta, None, (1, 1), (1, 1)), x)  # identity kernel
    w = rng.standard_normal((4, 3, 3, 3))
    y = oracle.conv2d(x, w, None, (2, 2), (1, 1))
    g = rng.standard_normal(y.shape)
    dx, _, _ = oracle.conv2d_backward(x, w, g, (2, 2), (1, 1))
    assert abs((y * g).sum() - (x * dx).sum()) < 1e-9  # the backward is the adjoint


def test_upsample_oracle_matches_torch():
    gen = torch.Generator().manual_seed(11)
    x = torch.randn(2, 3, 5, 7, dtype=torch.float64, generator=gen).requires_grad_(True)
    y = F.interpolate(x, scale_factor=(2, 3), mode="nearest")
    g = torch.randn(y.shape, dtype=torch.float64, generator=gen)
    y.backward(g)
    np.testing.assert_array_equal(oracle.upsample_nearest(x.detach().numpy(), 10, 21), y.detach().numpy())
    dx = oracle.upsample_nearest_backward(g.numpy(), 5, 7)
    # The 2x3 source blocks summed in a fixed order (a closed form independent of both implementations);
    # torch sums in another order, so terms that nearly cancel need an absolute tolerance.
    blocks = g.numpy().reshape(2, 3, 5, 2, 7, 3).sum(axis=(3, 5))
    np.testing.assert_allclose(dx, blocks, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(dx, x.grad.numpy(), rtol=1e-13, atol=1e-13)
    assert np.array_equal(oracle.upsample_nearest_backward(np.ones((1, 1, 4, 6)), 2, 3), np.full((1, 1, 2, 3), 4.0))


@pytest.mark.parametrize("affine", [False, True])
@pytest.mark.parametrize("shape,G", [((2, 8, 5, 5), 4), ((1, 6, 3, 7), 3), ((3, 4, 9), 2), ((1, 32, 4, 4), 32)])
def test_group_norm_oracle_matches_torch_and_autograd(affine, shape, G):
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(shape, generator=g, dtype=torch.float64) * 2 + 0.5).requires_grad_(True)
    C = shape[1]
    w = (torch.randn(C, generator=g, dtype=torch.float64)).requires_grad_(True) if affine else None
    b = (torch.randn(C, generator=g, dtype=torch.float64)).requires_grad_(True) if affine else None
    y = F.group_norm(x, G, w, b, 1e-5)
    go = torch.randn(shape, generator=g, dtype=torch.float64)
    y.backward(go)
    wn = None if w is None else w.detach().numpy()
    yo, mean, rstd = oracle.group_norm_fwd(x.detach().numpy(), G, wn, None if b is None else b.detach().numpy(), 1e-5)
    np.testing.assert_allclose(yo, y.detach().numpy(), rtol=1e-10, atol=1e-10)
    dx, dw, db = oracle.group_norm_bwd(go.numpy(), x.detach().numpy(), mean, rstd, G, wn)
    np.testing.assert_allclose(dx, x.grad.numpy(), rtol=1e-9, atol=1e-9)
    if affine:
        np.testing.assert_allclose(dw, w.grad.numpy(), rtol=1e-9, atol=1e-9)
        np.testing.assert_allclose(db, b.grad.numpy(), rtol=1e-9, atol=1e-9)
    # each group of the plain output has mean 0 and variance 1 - eps-correction
    y0, _, _ = oracle.group_norm_fwd(x.detach().numpy(), G)
    yg = y0.reshape(shape[0], G, -1)
    np.testing.assert_allclose(yg.mean(-1), 0.0, atol=1e-12)
    assert np.all(np.abs(yg.var(-1) - 1.0) < 1e-3)


def test_planted_group_norm_dropped_term_is_caught():
    """A group_norm backward without its c3 term fails the autograd pin."""
    x = torch.randn(2, 4, 6, dtype=torch.float64, requires_grad=True)
    y = F.group_norm(x, 2, None, None, 1e-5)
    go = torch.randn(y.shape, dtype=torch.float64)
    y.backward(go)
    _, mean, rstd = oracle.group_norm_fwd(x.detach().numpy(), 2)
    dx, _, _ = oracle.group_norm_bwd(go.numpy(), x.detach().numpy(), mean, rstd, 2)
    gf = go.numpy().reshape(2, 4, -1)
    dsg = (gf * x.detach().numpy().reshape(2, 4, -1)).sum(-1).reshape(2, 2, 2).sum(-1)
    dbg = gf.sum(-1).reshape(2, 2, 2).sum(-1)
    c3 = -((dbg * mean - dsg) * rstd ** 3 / 12) * mean - dbg * rstd / 12
    planted = dx - np.repeat(np.repeat(c3, 2, axis=1)[..., None], 6, axis=2).reshape(dx.shape)
    assert np.abs(dx - x.grad.numpy()).max() < 1e-10 and np.abs(planted - x.grad.numpy()).max() > 1e-3
