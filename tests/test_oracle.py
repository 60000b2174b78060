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
