"""softmax / layer_norm on the GPU against the float64 oracle.

The reference's tests/test_rows.py (its softmax and layer_norm parts) fixes the behaviours (softmax over any
dimension, masked and large inputs, views, half inputs with a float32 result, its backward; layer_norm with
and without affine parameters, over trailing dimensions, float32 statistics, its backward) and the
tolerance: the largest error at most 3e-5 / 1.2e-2 / 2.5e-3 (float32 / bfloat16 / float16) times
max(1, largest |reference|), widened per case.  Here the cases are tables run forward and backward
together, plus _safe_softmax, the BASELINE shapes (softmax fp32 [16384, 1024], layer_norm bf16
[1024, 2048]) and the layer_norm backward's chunked weight-gradient sums."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from vkutil import f64, max_abs_close, randn

pytestmark = pytest.mark.gpu

import torch_vulkan  # noqa: E402

dev = torch.device("vk")
FLOATS = [torch.float32, torch.bfloat16, torch.float16]
ROW_TOL = {torch.float32: 3e-5, torch.bfloat16: 1.2e-2, torch.float16: 2.5e-3}


def assert_on_device(*names):
    fb = torch_vulkan.fallback_counts()
    hit = {n: fb[n] for n in names if n in fb}
    assert not hit, f"ran on the CPU: {hit}"


# ---- softmax ----------------------------------------------------------------------------------------------------
# (shape, dim): last and inner dimensions, a length-1 axis, rows of 1000 / 2048 / 4096 / 5000 elements
SOFTMAX = [((7, 33), -1), ((3, 5, 4), 1), ((3, 5, 4), 0), ((2, 1000), 1), ((4, 5000), -1), ((5, 1), -1),
           ((2, 3, 4, 5), 2), ((3, 4096), -1), ((2, 2048), -1), ((6, 8), -1), ((3, 7, 5), 1), ((5, 4, 37), -1)]


@pytest.mark.parametrize("shape,dim", SOFTMAX, ids=str)
@pytest.mark.parametrize("dt", FLOATS)
def test_softmax_and_its_gradient(dt, shape, dim):
    x, gy = randn(shape, dt, 0, 3.0), randn(shape, dt, 3)
    xd = x.to(dev).requires_grad_(True)
    y = torch.softmax(xd, dim)
    assert y.dtype == dt
    max_abs_close(y, oracle.softmax_fwd(f64(x), dim), ROW_TOL[dt])
    assert torch_vulkan.kernel_counts().get("aten::_softmax", 0) == 1
    (gx,) = torch.autograd.grad(y, xd, gy.to(dev))
    # the backward from the device's own (rounded) forward output, as the kernel computes it
    max_abs_close(gx, oracle.softmax_bwd(f64(y), f64(gy), dim), ROW_TOL[dt], mult=2.0)
    assert_on_device("aten::_softmax", "aten::_softmax_backward_data")


def test_softmax_of_masked_large_and_strided_inputs():
    x = randn((4, 40), torch.float32, 0, 50.0)  # large logits: the row maximum is subtracted first
    x[:, 5:12] = float("-inf")
    y = torch.softmax(x.to(dev), -1)
    max_abs_close(y, oracle.softmax_fwd(f64(x), -1), ROW_TOL[torch.float32])
    assert torch.all(y.cpu()[:, 5:12] == 0)
    z = randn((6, 8, 9), torch.float32, 1)
    max_abs_close(torch.softmax(z.to(dev).permute(2, 1, 0), -1), oracle.softmax_fwd(f64(z.permute(2, 1, 0)), -1),
                  ROW_TOL[torch.float32])


def test_softmax_half_to_float_and_safe_softmax():
    x = randn((4, 33), torch.bfloat16, 2, 3.0)
    y = torch.softmax(x.to(dev), -1, dtype=torch.float32)
    assert y.dtype == torch.float32
    max_abs_close(y, oracle.softmax_fwd(f64(x), -1), 1e-6)
    z = randn((4, 33), torch.float32, 3)
    z[1, :] = float("-inf")  # a fully masked row: zeros instead of NaN
    z[2, :5] = float("-inf")
    s = torch._safe_softmax(z.to(dev), -1)
    max_abs_close(s, oracle.softmax_fwd(f64(z), -1, safe=True), 1e-6)
    assert torch.equal(s.cpu()[1], torch.zeros(33))
    assert_on_device("aten::_safe_softmax")


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
def ln_operands(rows, D, dt, affine, seed=0):
    x = randn((rows, D), dt, seed, 2.0)
    w = randn((D,), dt, seed + 1) if affine else None
    b = randn((D,), dt, seed + 2) if affine else None
    return x, w, b


def dev_or_none(t, grad=False):
    return None if t is None else t.to(dev).requires_grad_(grad)


def f64_or_none(t):
    return None if t is None else f64(t)


@pytest.mark.parametrize("affine", [False, True])
@pytest.mark.parametrize("rows,D", [(3, 7), (5, 256), (4, 1000), (2, 2048), (1, 1), (3, 5000), (9, 4096)])
@pytest.mark.parametrize("dt", FLOATS)
def test_layer_norm_forward(dt, rows, D, affine):
    x, w, b = ln_operands(rows, D, dt, affine)
    y = F.layer_norm(x.to(dev), (D,), dev_or_none(w), dev_or_none(b), 1e-5)
    want, _, _ = oracle.layer_norm_fwd(f64(x), 1, f64_or_none(w), f64_or_none(b), 1e-5)
    max_abs_close(y, want, ROW_TOL[dt], mult=2.0)
    assert_on_device("aten::native_layer_norm")


def test_layer_norm_over_trailing_dimensions_of_higher_rank_inputs():
    x = randn((1, 1, 8, 8, 128), torch.bfloat16, 4, 2.0)  # the DiT's [B, T, H, W, D] tokens, no affine
    max_abs_close(F.layer_norm(x.to(dev), (128,), eps=1e-6), oracle.layer_norm_fwd(f64(x), 1, None, None, 1e-6)[0],
                  ROW_TOL[torch.bfloat16], mult=2.0)
    z = randn((4, 3, 5), torch.float32, 5)  # normalized over the last two dimensions
    max_abs_close(F.layer_norm(z.to(dev), (3, 5)), oracle.layer_norm_fwd(f64(z), 2)[0], ROW_TOL[torch.float32])
    assert_on_device("aten::native_layer_norm")


def test_layer_norm_statistics_are_float32_rows():
    x = randn((4, 64), torch.bfloat16, 6)
    y, mean, rstd = torch.native_layer_norm(x.to(dev), (64,), None, None, 1e-5)
    assert (y.dtype, mean.dtype, rstd.dtype) == (torch.bfloat16, torch.float32, torch.float32)
    assert mean.shape == rstd.shape == (4, 1)
    _, rm, rr = oracle.layer_norm_fwd(f64(x), 1, None, None, 1e-5)
    assert np.allclose(f64(mean), rm, rtol=1e-6, atol=1e-6) and np.allclose(f64(rstd), rr, rtol=1e-5)


@pytest.mark.parametrize("rows,D", [(6, 96), (10, 2048), (5, 5000), (1030, 2048)])
@pytest.mark.parametrize("affine", [False, True])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_layer_norm_gradients(dt, affine, rows, D):
    x, w, b = ln_operands(rows, D, dt, affine, seed=7)
    gy = randn((rows, D), dt, 10)
    xd, wd, bd = x.to(dev).requires_grad_(True), dev_or_none(w, True), dev_or_none(b, True)
    y = F.layer_norm(xd, (D,), wd, bd, 1e-5)
    inputs = [xd] + ([wd, bd] if affine else [])
    got = torch.autograd.grad(y, inputs, gy.to(dev))
    _, mean, rstd = oracle.layer_norm_fwd(f64(x), 1, None, None, 1e-5)
    want = oracle.layer_norm_bwd(f64(gy), f64(x), mean, rstd, 1, f64_or_none(w))
    for g, r in zip(got, want):
        max_abs_close(g, r, ROW_TOL[dt], mult=4.0)
    assert_on_device("aten::native_layer_norm_backward")


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
