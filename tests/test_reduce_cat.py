"""sum / mean (kernel "reduce_sum") and cat on the vk device.

Mirrors the reference's tests/test_rows.py:136-196 (its tolerance rule :15, :30-35: max error <= TOL x
max(|ref|, 1) x mult against float64), and compares every reduction with oracle.reduce_sum as well.  On
top: the three kernel layouts (columns with 16-byte loads, rows, generic strided), split reductions with
their in-order second pass (run-to-run identical bits), empty, 0-dim and 8-dimensional inputs, an output
dtype, the DiT bias gradient at full size, and cat with mixed float dtypes, integer parts and views.
"""

import math

import numpy as np
import pytest
import torch

import oracle
from vkutil import bits

pytestmark = pytest.mark.gpu

import torch_vulkan  # noqa: E402
from torch_vulkan import abi  # noqa: E402

dev = torch.device("vk")
DTYPES = [torch.float32, torch.bfloat16, torch.float16]
TOL = {torch.float32: 3e-5, torch.bfloat16: 1.2e-2, torch.float16: 2.5e-3}
KIND = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}


@pytest.fixture(autouse=True)
def _reset():
    torch_vulkan.reset_fallback_counts()
    yield


def rnd(shape, dtype=torch.float32, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def close(out, ref64, dtype, mult=1.0):
    o, r = out.cpu().double(), torch.as_tensor(ref64).double()
    assert o.shape == r.shape, (o.shape, r.shape)
    scale = max(r.abs().max().item(), 1.0) if r.numel() else 1.0
    err = (o - r).abs().max().item() if r.numel() else 0.0
    assert err <= TOL[dtype] * scale * mult, f"max err {err} (scale {scale})"


def check(out, x, dims, keepdim, mean, mult=1.0):
    """Against the oracle (float64 sum, one rounding) with the reference's tolerance rule."""
    ref, _ = oracle.reduce_sum(x.detach().cpu().double().numpy(), dims, keepdim, mean, KIND[out.dtype])
    close(out, ref, out.dtype, mult)


def no_fallback(*names):
    fb = torch_vulkan.fallback_counts()
    assert not {n: fb[n] for n in names if n in fb}, fb


# ---- the reference's cases ---------------------------------------------------------------------------------
@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("dim", [None, -1, 0, 1, (0, 1), (1, 2), (0, 2), (0, 1, 2), (0, 3)])
@pytest.mark.parametrize("keepdim", [False, True])
@pytest.mark.parametrize("fn", ["sum", "mean"])
def test_reduce_dims(dt, dim, keepdim, fn):
    x = rnd((3, 5, 4, 6), dt)
    kwargs = {} if dim is None else {"dim": dim, "keepdim": keepdim}
    out = getattr(torch, fn)(x.to(dev), **kwargs)
    ref = getattr(torch, fn)(x.double(), **kwargs)
    assert out.dtype == dt and out.device.type == "vk"
    close(out, ref, dt, mult=1.5)
    dims = None if dim is None else ((dim,) if isinstance(dim, int) else dim)
    check(out, x, dims, keepdim and dim is not None, fn == "mean", mult=1.5)
    no_fallback("aten::" + fn)


def test_reduce_non_contiguous_and_large():
    x = rnd((40, 50, 30))
    xd = x.to(dev)
    close(xd.transpose(0, 2).sum(1), x.transpose(0, 2).double().sum(1), torch.float32, mult=3.0)
    close(xd[5:30, ::2, 3:20].mean((0, 2)), x[5:30, ::2, 3:20].double().mean((0, 2)), torch.float32, mult=3.0)
    big = rnd((1 << 22,), seed=7)
    close(big.to(dev).sum(), big.double().sum().reshape(()), torch.float32, mult=50.0)
    no_fallback("aten::sum", "aten::mean")


def test_mean_backward_and_sum_backward():
    x = rnd((4, 7))
    xd = x.to(dev).requires_grad_(True)
    (xd.mean(-1) * torch.arange(4, dtype=torch.float32, device=dev)).sum().backward()
    xc = x.clone().requires_grad_(True)
    (xc.mean(-1) * torch.arange(4, dtype=torch.float32)).sum().backward()
    assert torch.allclose(xd.grad.cpu(), xc.grad, atol=1e-6)


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("dim", [0, 1, -1])
def test_cat(dt, dim):
    parts = [rnd((3, 4, 5), dt, seed=i) for i in range(3)]
    if dim == 1:
        parts[1] = rnd((3, 2, 5), dt, seed=9)
    elif dim in (-1, 2):
        parts[1] = rnd((3, 4, 1), dt, seed=9)
    else:
        parts[1] = rnd((2, 4, 5), dt, seed=9)
    out = torch.cat([p.to(dev) for p in parts], dim)
    assert torch.equal(out.cpu(), torch.cat(parts, dim))
    no_fallback("aten::cat")


def test_cat_legacy_empty_and_noncontiguous_and_backward():
    a, b = rnd((4, 3)), rnd((4, 3), seed=1)
    out = torch.cat([a.to(dev).t(), torch.empty(0, device=dev), b.to(dev).t()], 0)
    assert torch.equal(out.cpu(), torch.cat([a.t(), b.t()], 0))
    ad = a.to(dev).requires_grad_(True)
    bd = b.to(dev).requires_grad_(True)
    (torch.cat([ad, bd], 1) * torch.arange(6, dtype=torch.float32, device=dev)).sum().backward()
    ac, bc = a.clone().requires_grad_(True), b.clone().requires_grad_(True)
    (torch.cat([ac, bc], 1) * torch.arange(6, dtype=torch.float32)).sum().backward()
    assert torch.equal(ad.grad.cpu(), ac.grad) and torch.equal(bd.grad.cpu(), bc.grad)


# ---- layouts, splits and edge cases --------------------------------------------------------------------
@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("shape,dims", [
    ((1024, 8192), (0,)),          # columns, 16-byte loads, split over rows (bias gradient)
    ((37, 1000), (0,)),            # columns, one output per lane (width not a multiple of the vector)
    ((5, 70000), (1,)),            # rows, split reduced range
    ((4096, 2048), (1,)),          # rows, one workgroup per row
    ((1 << 20,), None),            # full sum, split
    ((64, 3, 128), (0, 2)),        # kept middle dimension: generic strided walk
    ((8, 16, 32), (0, 1)),         # columns with two reduced dimensions
])
def test_reduce_layouts(dt, shape, dims):
    x = rnd(shape, dt, seed=len(shape) + shape[0])
    xd = x.to(dev)
    for mean in (False, True):
        fn = torch.mean if mean else torch.sum
        out = fn(xd) if dims is None else fn(xd, dim=dims)
        check(out, x, dims, False, mean, mult=3.0)
        out2 = fn(xd) if dims is None else fn(xd, dim=dims)
        assert np.array_equal(bits(out), bits(out2)), "two runs differ"
    no_fallback("aten::sum", "aten::mean")


def test_reduce_transposed_and_strided_views():
    x = rnd((256, 96, 40), seed=3)
    xd = x.to(dev)
    for view, vref in ((xd.permute(2, 0, 1), x.permute(2, 0, 1)), (xd[:, ::3, 5:], x[:, ::3, 5:]),
                       (xd.transpose(0, 1)[::2], x.transpose(0, 1)[::2])):
        for dims in ((0,), (1,), (2,), (0, 2), (1, 2)):
            check(view.sum(dims), vref, dims, False, False, mult=3.0)
            check(view.mean(dims, keepdim=True), vref, dims, True, True, mult=3.0)


def test_reduce_output_dtype_and_edge_cases():
    x = rnd((33, 65), torch.bfloat16, seed=4)
    out = torch.sum(x.to(dev), dim=1, dtype=torch.float32)
    assert out.dtype == torch.float32
    check(out, x, (1,), False, False)
    e = torch.empty(3, 0, device=dev)
    assert torch.equal(e.sum(1).cpu(), torch.zeros(3))
    assert torch.isnan(e.mean(1).cpu()).all()
    assert e.sum(0).shape == (0,)
    s = torch.tensor(2.5, device=dev)
    assert s.sum().item() == 2.5 and s.mean().item() == 2.5
    y = rnd((2, 1, 3, 1, 2, 1, 2, 3), seed=5)
    for dims in ((1, 3, 5), (0, 2, 4, 6, 7), (1,), None):
        out = y.to(dev).sum() if dims is None else y.to(dev).sum(dims)
        check(out, y, dims, False, False)
    no_fallback("aten::sum", "aten::mean")


def test_dit_bias_gradient_full_size():
    """grad_output.sum(0) of the DiT MLP up-projection (M = 1024 tokens, 8192 features, bf16) through
    autograd of a Linear with bias."""
    x = rnd((1024, 2048), torch.bfloat16, seed=6)
    w = rnd((8192, 2048), torch.bfloat16, seed=7, scale=0.02)
    b = rnd((8192,), torch.bfloat16, seed=8, scale=0.02)
    g = rnd((1024, 8192), torch.bfloat16, seed=9)
    bd = b.to(dev).requires_grad_(True)
    y = torch.nn.functional.linear(x.to(dev), w.to(dev), bd)
    y.backward(g.to(dev))
    check(bd.grad, g, (0,), False, False, mult=2.0)
    assert torch_vulkan.kernel_counts().get("aten::sum.dim_IntList", 0) >= 1
    no_fallback("aten::sum")


def test_cat_mixed_dtypes_ints_and_views():
    a, b = rnd((4, 6), torch.bfloat16), rnd((4, 2), torch.float32, seed=1)
    out = torch.cat([a.to(dev), b.to(dev)], 1)
    ref = torch.cat([a, b], 1)
    assert out.dtype == ref.dtype and torch.equal(out.cpu(), ref)
    i, j = torch.arange(12, dtype=torch.int64).reshape(3, 4), torch.arange(8, dtype=torch.int64).reshape(2, 4)
    assert torch.equal(torch.cat([i.to(dev), j.to(dev)], 0).cpu(), torch.cat([i, j], 0))
    m = torch.tensor([[True, False], [False, True]])
    assert torch.equal(torch.cat([m.to(dev), m.to(dev)], 1).cpu(), torch.cat([m, m], 1))
    x = rnd((8, 10, 12), seed=2)
    xd = x.to(dev)
    out = torch.cat([xd[:, ::2], xd[:, 1:4].transpose(1, 2).transpose(1, 2), xd[:, :1]], 1)
    assert torch.equal(out.cpu(), torch.cat([x[:, ::2], x[:, 1:4], x[:, :1]], 1))
    no_fallback("aten::cat")


# ---- cat in one launch ("cat_rows16": same-dtype contiguous parts, rows of whole 16-byte chunks) -------------
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.int64])
@pytest.mark.parametrize("shapes,dim", [
    ([(64, 256), (64, 128), (64, 8)], 1),
    ([(4, 16, 32)] * 3, 0),
    ([(2, 8, 16), (2, 0, 16), (2, 24, 16)], 1),  # the empty part is skipped
    ([(16, 64)] * 11, 1),                         # two launches: 8 parts, then 3
    ([(1024, 2048)] * 3, 1),                      # the benchmark shape
])
def test_cat_one_launch(dt, shapes, dim):
    parts = [(torch.arange(math.prod(sh), dtype=torch.int64) * 3 + 1000 * i).reshape(sh).to(dt) for i, sh in enumerate(shapes)]
    out = torch.cat([p.to(dev) for p in parts], dim)
    assert torch.equal(out.cpu(), torch.cat(parts, dim))
    no_fallback("aten::cat")


def test_cat_rows16_c_abi_and_checks():
    """The kernel through the C ABI: parts land at their byte columns; non-adjacent parts are rejected."""
    rt = abi.Runtime()
    a, b = rnd((32, 24), seed=1), rnd((32, 40), seed=2)
    ad, bd = a.to(dev), b.to(dev)
    out = torch.zeros(32, 64, device=dev)
    A = abi.CatArgs()
    A.out, A.outer, A.out_row_bytes, A.nparts = out.data_ptr(), 32, 64 * 4, 2
    A.src[0], A.src[1] = ad.data_ptr(), bd.data_ptr()
    A.row_bytes[0], A.row_bytes[1] = 24 * 4, 40 * 4
    A.col[0], A.col[1] = 0, 24 * 4
    rt.dispatch("cat_rows16", A)
    rt.synchronize()
    assert torch.equal(out.cpu(), torch.cat([a, b], 1))
    A.col[1] = 32 * 4
    with pytest.raises(RuntimeError, match="adjacent"):
        rt.dispatch("cat_rows16", A)
    rt.synchronize()
