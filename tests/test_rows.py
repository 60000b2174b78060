"""softmax / layer_norm on the GPU vs the float64 oracle (reference tests/test_rows.py:1-230, softmax and
layer_norm parts), with the reference tolerance rule max|err| <= TOL * max(|ref|, 1) * mult, plus the
BASELINE shapes: softmax fp32 [16384, 1024] and layer_norm bf16 [1024, 2048], forward and backward."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from vkutil import f64, max_abs_close, randn

pytestmark = pytest.mark.gpu

import torch_vulkan  # noqa: E402

dev = torch.device("vk")
DTYPES = [torch.float32, torch.bfloat16, torch.float16]
TOL = {torch.float32: 3e-5, torch.bfloat16: 1.2e-2, torch.float16: 2.5e-3}


def no_fallback(*names):
    fb = torch_vulkan.fallback_counts()
    assert not {n: fb[n] for n in names if n in fb}, fb


# ---- softmax ----------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("shape,dim", [((7, 33), -1), ((3, 5, 4), 1), ((3, 5, 4), 0), ((2, 1000), 1), ((4, 5000), -1),
                                       ((5, 1), -1), ((2, 3, 4, 5), 2), ((3, 4096), -1), ((2, 2048), -1), ((6, 8), -1)])
def test_softmax_forward(dt, shape, dim):
    x = randn(shape, dt, scale=3.0)
    out = torch.softmax(x.to(dev), dim)
    assert out.dtype == dt
    max_abs_close(out, oracle.softmax_fwd(f64(x), dim), TOL[dt])
    no_fallback("aten::_softmax")
    assert torch_vulkan.kernel_counts().get("aten::_softmax", 0) == 1


def test_softmax_masked_entries_and_large_values():
    x = randn((4, 40), torch.float32, scale=50.0)
    x[:, 5:12] = float("-inf")
    out = torch.softmax(x.to(dev), -1)
    max_abs_close(out, oracle.softmax_fwd(f64(x), -1), TOL[torch.float32])
    assert torch.all(out.cpu()[:, 5:12] == 0)


def test_softmax_non_contiguous_input():
    x = randn((6, 8, 9), torch.float32)
    xd = x.to(dev).transpose(0, 2)
    max_abs_close(torch.softmax(xd, -1), oracle.softmax_fwd(f64(x.transpose(0, 2)), -1), TOL[torch.float32])


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(5, 4, 37), (3, 1024), (2, 6000)])
def test_softmax_backward(dt, shape):
    x = randn(shape, dt, scale=2.0)
    g = randn(shape, dt, seed=3)
    xd = x.to(dev).requires_grad_(True)
    y = torch.softmax(xd, -1)
    y.backward(g.to(dev))
    # oracle backward from the device's own (rounded) forward output, as the reference kernel computes it
    ref = oracle.softmax_bwd(f64(y), f64(g), -1)
    max_abs_close(xd.grad, ref, TOL[dt], mult=2.0)
    no_fallback("aten::_softmax_backward_data")


def test_softmax_backward_over_inner_dim():
    x = randn((3, 7, 5), torch.float32)
    g = randn((3, 7, 5), torch.float32, seed=4)
    xd = x.to(dev).requires_grad_(True)
    y = torch.softmax(xd, 1)
    y.backward(g.to(dev))
    max_abs_close(xd.grad, oracle.softmax_bwd(f64(y), f64(g), 1), TOL[torch.float32], mult=2.0)


def test_softmax_half_to_float_and_safe_softmax():
    x = randn((4, 33), torch.bfloat16, scale=3.0)
    out = torch.softmax(x.to(dev), -1, dtype=torch.float32)
    assert out.dtype == torch.float32
    max_abs_close(out, oracle.softmax_fwd(f64(x), -1), 1e-6)
    y = randn((4, 33), torch.float32)
    y[1, :] = float("-inf")
    y[2, :5] = float("-inf")
    o = torch._safe_softmax(y.to(dev), -1)
    ref = oracle.softmax_fwd(f64(y), -1, safe=True)
    max_abs_close(o, ref, 1e-6)
    assert torch.equal(o.cpu()[1], torch.zeros(33))
    no_fallback("aten::_safe_softmax")


def test_softmax_baseline_shape_fp32_16384x1024():
    x = randn((16384, 1024), torch.float32, seed=4, scale=2.0)
    out = torch.softmax(x.to(dev), -1)
    ref = oracle.softmax_fwd(f64(x), -1)
    max_abs_close(out, ref, 3e-5)
    assert oracle.rel_l2(f64(out), ref) <= 1e-5
    g = randn((16384, 1024), torch.float32, seed=5)
    dx = torch.ops.aten._softmax_backward_data(g.to(dev), out, -1, torch.float32)
    refb = oracle.softmax_bwd(f64(out), f64(g), -1)
    assert oracle.rel_l2(f64(dx), refb) <= 1e-5


# ---- layer_norm -------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("rows,D", [(3, 7), (5, 256), (4, 1000), (2, 2048), (1, 1), (3, 5000), (9, 4096)])
@pytest.mark.parametrize("affine", [False, True])
def test_layer_norm_forward(dt, rows, D, affine):
    x = randn((rows, D), dt, scale=2.0)
    w = randn((D,), dt, 1) if affine else None
    b = randn((D,), dt, 2) if affine else None
    out = F.layer_norm(x.to(dev), (D,), None if w is None else w.to(dev), None if b is None else b.to(dev), 1e-5)
    ref, _, _ = oracle.layer_norm_fwd(f64(x), 1, None if w is None else f64(w), None if b is None else f64(b), 1e-5)
    max_abs_close(out, ref, TOL[dt], mult=2.0)
    no_fallback("aten::native_layer_norm")


def test_layer_norm_multi_dim_and_5d():
    x = randn((1, 1, 8, 8, 128), torch.bfloat16, scale=2.0)
    out = F.layer_norm(x.to(dev), (128,), eps=1e-6)
    max_abs_close(out, oracle.layer_norm_fwd(f64(x), 1, None, None, 1e-6)[0], TOL[torch.bfloat16], mult=2.0)
    y = randn((4, 3, 5), torch.float32)
    max_abs_close(F.layer_norm(y.to(dev), (3, 5)), oracle.layer_norm_fwd(f64(y), 2)[0], TOL[torch.float32])
    no_fallback("aten::native_layer_norm")


def test_layer_norm_stats_are_fp32_with_reference_shape():
    x = randn((4, 64), torch.bfloat16).to(dev)
    out, mean, rstd = torch.native_layer_norm(x, (64,), None, None, 1e-5)
    assert mean.dtype == torch.float32 and rstd.dtype == torch.float32 and out.dtype == torch.bfloat16
    assert mean.shape == (4, 1)
    _, rm, rr = oracle.layer_norm_fwd(f64(x), 1, None, None, 1e-5)
    assert np.allclose(f64(mean), rm, rtol=1e-6, atol=1e-6) and np.allclose(f64(rstd), rr, rtol=1e-5)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("affine", [False, True])
@pytest.mark.parametrize("rows,D", [(6, 96), (10, 2048), (5, 5000), (1030, 2048)])
def test_layer_norm_backward(dt, affine, rows, D):
    x = randn((rows, D), dt, scale=2.0)
    w = randn((D,), dt, 1) if affine else None
    b = randn((D,), dt, 2) if affine else None
    g = randn((rows, D), dt, 3)
    xd = x.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True) if affine else None
    bd = b.to(dev).requires_grad_(True) if affine else None
    F.layer_norm(xd, (D,), wd, bd, 1e-5).backward(g.to(dev))
    _, mean, rstd = oracle.layer_norm_fwd(f64(x), 1, None, None, 1e-5)
    dx, dw, db = oracle.layer_norm_bwd(f64(g), f64(x), mean, rstd, 1, None if w is None else f64(w))
    max_abs_close(xd.grad, dx, TOL[dt], mult=4.0)
    if affine:
        max_abs_close(wd.grad, dw, TOL[dt], mult=4.0)
        max_abs_close(bd.grad, db, TOL[dt], mult=4.0)
    no_fallback("aten::native_layer_norm_backward")


def test_layer_norm_baseline_shape_bf16_1024x2048():
    x = randn((1024, 2048), torch.bfloat16, seed=1)
    w = randn((2048,), torch.bfloat16, seed=2)
    b = randn((2048,), torch.bfloat16, seed=3)
    g = randn((1024, 2048), torch.bfloat16, seed=4)
    xd, wd, bd = (t.to(dev).requires_grad_(True) for t in (x, w, b))
    y = F.layer_norm(xd, (2048,), wd, bd, 1e-5)
    ref, mean, rstd = oracle.layer_norm_fwd(f64(x), 1, f64(w), f64(b), 1e-5)
    assert oracle.rel_l2(f64(y), ref) <= 1e-2
    y.backward(g.to(dev))
    dx, dw, db = oracle.layer_norm_bwd(f64(g), f64(x), mean, rstd, 1, f64(w))
    assert oracle.rel_l2(f64(xd.grad), dx) <= 1e-2
    assert oracle.rel_l2(f64(wd.grad), dw) <= 1e-2
    assert oracle.rel_l2(f64(bd.grad), db) <= 1e-2


def _ln_bwd_args(x, g, w, mean, rstd, dx, dw, db, ws):
    from torch_vulkan import abi
    a = abi.LnArgs()
    a.x, a.g, a.mean, a.rstd = x.data_ptr(), g.data_ptr(), mean.data_ptr(), rstd.data_ptr()
    a.w = w.data_ptr() if w is not None else 0
    a.dx = dx.data_ptr() if dx is not None else 0
    a.dw = dw.data_ptr() if dw is not None else 0
    a.db = db.data_ptr() if db is not None else 0
    a.ws, a.rows, a.D, a.eps = ws, x.shape[0], x.shape[1], 1e-5
    return a


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,D,affine", [(1024, 2048, True), (1021, 2048, True), (37, 512, False), (13, 1000, True),
                                           (2, 4096, True), (300, 200, True), (2100, 2048, True), (4096, 2048, False),
                                           (1500, 4096, True), (1024, 1024, True)])
def test_layer_norm_backward_one_call_matches_two(dt, rows, D, affine):
    """"ln_bwd" given dw / db also reduces the partial sums (one call for dx, dw, db, as the shim queues it);
    it must give the bits of "ln_bwd" followed by "ln_wgrad", on ragged row counts, rows off the full-chunk
    path and without affine parameters, with chunks of 4, 8 and 16 rows (8 from 1024 rows, 16 from 2048 when
    16 rows of D floats fit 128 KiB: (2100, 2048) and (4096, 2048); (1500, 4096) stays at 8, (1024, 1024)
    at 4), and two calls in a row on different inputs must each see their own partial sums."""
    from torch_vulkan import abi
    rt = abi.Runtime()
    kind = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[dt]
    chunks = abi.ln_chunks(rows, D)
    outs = []
    for seed in (5, 6):
        gen = torch.Generator().manual_seed(seed * 1000 + rows)
        x = (torch.randn(rows, D, generator=gen) * 1.5 + 0.2).to(dt).to(dev)
        g = torch.randn(rows, D, generator=gen).to(dt).to(dev)
        w = torch.randn(D, generator=gen).to(dt).to(dev) if affine else None
        b = torch.randn(D, generator=gen).to(dt).to(dev) if affine else None
        _, mean, rstd = torch.native_layer_norm(x, [D], w, b, 1e-5)
        mean, rstd = mean.contiguous(), rstd.contiguous()
        res = {}
        for mode in ("one", "two"):
            dx = torch.empty_like(x)
            dw = torch.empty(D, dtype=dt, device=dev)
            db = torch.empty(D, dtype=dt, device=dev)
            ws = torch.empty(chunks * 2 * D, dtype=torch.float32, device=dev)
            if mode == "one":
                rt.dispatch(f"ln_bwd_{kind}", _ln_bwd_args(x, g, w, mean, rstd, dx, dw, db, ws.data_ptr()))
            else:
                rt.dispatch(f"ln_bwd_{kind}", _ln_bwd_args(x, g, w, mean, rstd, dx, None, None, ws.data_ptr()))
                rt.dispatch(f"ln_wgrad_{kind}", _ln_bwd_args(x, g, w, mean, rstd, None, dw, db, ws.data_ptr()))
            res[mode] = [t.cpu() for t in (dx, dw, db)]
        for a_, b_ in zip(res["one"], res["two"]):
            assert torch.equal(a_.view(torch.int16 if a_.element_size() == 2 else torch.int32),
                               b_.view(torch.int16 if b_.element_size() == 2 else torch.int32))
        # and against float64: dw = sum(g * xhat), db = sum(g)
        xh = (f64(x) - f64(mean).reshape(-1, 1)) * f64(rstd).reshape(-1, 1)
        gd = f64(g)
        tol = 1e-5 if dt == torch.float32 else 1e-2
        assert oracle.rel_l2(f64(res["one"][1]), (gd * xh).sum(0)) <= tol
        assert oracle.rel_l2(f64(res["one"][2]), gd.sum(0)) <= tol
        outs.append(res["one"])
    assert not torch.equal(outs[0][1], outs[1][1])  # the two calls saw different inputs
