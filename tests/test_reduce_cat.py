"""sum / mean (kernel "reduce_sum") and cat on the vk device.

The reference's tests/test_rows.py:136-196 fixes the behaviours (reductions over every combination of
dimensions with and without keepdim, views, a long vector, the backward of mean and sum; cat along each
dimension, with empty parts, views and its backward) and the tolerance: the largest error at most
3e-5 / 1.2e-2 / 2.5e-3 (float32 / bfloat16 / float16) times max(1, largest |reference|), widened per case.
Here every reduction is also compared with oracle.reduce_sum; on top come the three kernel layouts
(columns with 16-byte loads, rows, generic strided), split reductions with their in-order second pass
(run-to-run identical bits), empty, 0-dim and 8-dimensional inputs, an output dtype, the DiT bias gradient
at full size, and cat with mixed float dtypes, integer parts and views.
"""

import itertools
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
FLOATS = [torch.float32, torch.bfloat16, torch.float16]
SUM_TOL = {torch.float32: 3e-5, torch.bfloat16: 1.2e-2, torch.float16: 2.5e-3}
KIND = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}


def gauss(shape, dtype=torch.float32, seed=0, scale=1.0):
    """Seeded standard-normal values times scale, rounded to dtype."""
    return torch.empty(shape).normal_(0.0, scale, generator=torch.Generator().manual_seed(seed)).to(dtype)


def assert_sum_close(out, want64, dtype, widen=1.0):
    """Largest error within SUM_TOL[dtype] x max(1, largest |want|) x widen."""
    o, w = out.cpu().double(), torch.as_tensor(want64).double()
    assert o.shape == w.shape, (o.shape, w.shape)
    if w.numel() == 0:
        return
    bound = SUM_TOL[dtype] * max(w.abs().max().item(), 1.0) * widen
    err = (o - w).abs().max().item()
    assert err <= bound, f"largest error {err} > {bound}"


def check(out, x, dims, keepdim, mean, widen=1.0):
    """Against the oracle (float64 sum, one rounding)."""
    ref, _ = oracle.reduce_sum(x.detach().cpu().double().numpy(), dims, keepdim, mean, KIND[out.dtype])
    assert_sum_close(out, ref, out.dtype, widen)


def assert_on_device(*names):
    fb = torch_vulkan.fallback_counts()
    hit = {n: fb[n] for n in names if n in fb}
    assert not hit, f"ran on the CPU: {hit}"


# every reduced-dimension set of a rank-4 tensor: none (a full reduction), each single dimension (also
# negative), pairs and triples
DIM_SETS = [None, 0, 1, 2, 3, -1, -3] + [c for r in (2, 3) for c in itertools.combinations(range(4), r)]


@pytest.mark.parametrize("fn", ["sum", "mean"])
@pytest.mark.parametrize("dims", DIM_SETS, ids=str)
@pytest.mark.parametrize("dt", FLOATS)
def test_reduce_over_dimension_sets(dt, dims, fn):
    x = gauss((3, 5, 4, 6), dt, seed=3)
    for keepdim in (False, True):
        kw = {} if dims is None else {"dim": dims, "keepdim": keepdim}
        out = getattr(torch, fn)(x.to(dev), **kw)
        assert out.dtype == dt and out.device.type == "vk"
        assert_sum_close(out, getattr(torch, fn)(x.double(), **kw), dt, widen=1.5)
        ds = None if dims is None else ((dims,) if isinstance(dims, int) else dims)
        check(out, x, ds, keepdim and dims is not None, fn == "mean", widen=1.5)
    assert_on_device("aten::" + fn)


def test_reductions_of_views_and_of_a_long_vector():
    x = gauss((40, 50, 30), seed=4)
    xd = x.to(dev)
    for view in (lambda t: t.permute(2, 0, 1).sum(1), lambda t: t[5:30, ::2, 3:20].mean((0, 2)),
                 lambda t: t.transpose(0, 1)[::3].sum((1, 2))):
        assert_sum_close(view(xd), view(x.double()), torch.float32, widen=3.0)
    v = gauss((1 << 22,), seed=7)
    assert_sum_close(v.to(dev).sum(), v.double().sum().reshape(()), torch.float32, widen=50.0)
    assert_on_device("aten::sum", "aten::mean")


def test_gradients_of_sum_and_mean():
    x = gauss((4, 7), seed=5)
    wt = gauss((16,), seed=6)  # output-gradient values, as many as the largest output needs
    for red in (lambda t: t.mean(-1), lambda t: t.sum(0), lambda t: t.sum()):
        xd = x.to(dev).requires_grad_(True)
        xc = x.clone().requires_grad_(True)
        yd, yc = red(xd), red(xc)
        gd = wt[: yd.numel()].reshape(yd.shape)
        (got,) = torch.autograd.grad(yd, xd, gd.to(dev))
        (want,) = torch.autograd.grad(yc, xc, gd)
        assert torch.allclose(got.cpu(), want, atol=1e-6)


@pytest.mark.parametrize("dim", [0, 1, 2, -1])
@pytest.mark.parametrize("dt", FLOATS)
def test_cat_along_each_dimension(dt, dim):
    """Three parts, the middle one of a different length along the joined dimension."""
    base = [3, 4, 5]
    sizes = []
    for i, n in enumerate((2, 1, 3)):
        s = list(base)
        s[dim] = n if i == 1 else s[dim]
        sizes.append(s)
    parts = [gauss(s, dt, seed=10 + i) for i, s in enumerate(sizes)]
    out = torch.cat([p.to(dev) for p in parts], dim)
    assert torch.equal(out.cpu(), torch.cat(parts, dim))
    assert_on_device("aten::cat")


def test_cat_of_views_and_empty_parts_and_its_gradient():
    a, b = gauss((4, 3), seed=1), gauss((4, 3), seed=2)
    out = torch.cat([a.to(dev).t(), torch.empty(0, device=dev), b.to(dev).t()], 0)  # legacy 1-d empty part
    assert torch.equal(out.cpu(), torch.cat([a.t(), b.t()], 0))
    gy = gauss((4, 6), seed=3)
    ad, bd = a.to(dev).requires_grad_(True), b.to(dev).requires_grad_(True)
    ga, gb = torch.autograd.grad(torch.cat([ad, bd], 1), (ad, bd), gy.to(dev))
    assert torch.equal(ga.cpu(), gy[:, :3]) and torch.equal(gb.cpu(), gy[:, 3:])


# ---- layouts, splits and edge cases --------------------------------------------------------------------
@pytest.mark.parametrize("dt", FLOATS)
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
    x = gauss(shape, dt, seed=len(shape) + shape[0])
    xd = x.to(dev)
    for mean in (False, True):
        fn = torch.mean if mean else torch.sum
        out = fn(xd) if dims is None else fn(xd, dim=dims)
        check(out, x, dims, False, mean, widen=3.0)
        out2 = fn(xd) if dims is None else fn(xd, dim=dims)
        assert np.array_equal(bits(out), bits(out2)), "two runs differ"
    assert_on_device("aten::sum", "aten::mean")


def test_reduce_transposed_and_strided_views():
    x = gauss((256, 96, 40), seed=3)
    xd = x.to(dev)
    for view, vref in ((xd.permute(2, 0, 1), x.permute(2, 0, 1)), (xd[:, ::3, 5:], x[:, ::3, 5:]),
                       (xd.transpose(0, 1)[::2], x.transpose(0, 1)[::2])):
        for dims in ((0,), (1,), (2,), (0, 2), (1, 2)):
            check(view.sum(dims), vref, dims, False, False, widen=3.0)
            check(view.mean(dims, keepdim=True), vref, dims, True, True, widen=3.0)


def test_reduce_output_dtype_and_edge_cases():
    x = gauss((33, 65), torch.bfloat16, seed=4)
    out = torch.sum(x.to(dev), dim=1, dtype=torch.float32)
    assert out.dtype == torch.float32
    check(out, x, (1,), False, False)
    e = torch.empty(3, 0, device=dev)
    assert torch.equal(e.sum(1).cpu(), torch.zeros(3))
    assert torch.isnan(e.mean(1).cpu()).all()
    assert e.sum(0).shape == (0,)
    s = torch.tensor(2.5, device=dev)
    assert s.sum().item() == 2.5 and s.mean().item() == 2.5
    y = gauss((2, 1, 3, 1, 2, 1, 2, 3), seed=5)
    for dims in ((1, 3, 5), (0, 2, 4, 6, 7), (1,), None):
        out = y.to(dev).sum() if dims is None else y.to(dev).sum(dims)
        check(out, y, dims, False, False)
    assert_on_device("aten::sum", "aten::mean")


def test_dit_bias_gradient_full_size():
    """grad_output.sum(0) of the DiT MLP up-projection (M = 1024 tokens, 8192 features, bf16) through
    autograd of a Linear with bias."""
    x = gauss((1024, 2048), torch.bfloat16, seed=6)
    w = gauss((8192, 2048), torch.bfloat16, seed=7, scale=0.02)
    b = gauss((8192,), torch.bfloat16, seed=8, scale=0.02)
    g = gauss((1024, 8192), torch.bfloat16, seed=9)
    bd = b.to(dev).requires_grad_(True)
    y = torch.nn.functional.linear(x.to(dev), w.to(dev), bd)
    y.backward(g.to(dev))
    check(bd.grad, g, (0,), False, False, widen=2.0)
    assert torch_vulkan.kernel_counts().get("aten::sum.dim_IntList", 0) >= 1
    assert_on_device("aten::sum")


def test_cat_mixed_dtypes_ints_and_views():
    a, b = gauss((4, 6), torch.bfloat16), gauss((4, 2), torch.float32, seed=1)
    out = torch.cat([a.to(dev), b.to(dev)], 1)
    ref = torch.cat([a, b], 1)
    assert out.dtype == ref.dtype and torch.equal(out.cpu(), ref)
    i, j = torch.arange(12, dtype=torch.int64).reshape(3, 4), torch.arange(8, dtype=torch.int64).reshape(2, 4)
    assert torch.equal(torch.cat([i.to(dev), j.to(dev)], 0).cpu(), torch.cat([i, j], 0))
    m = torch.tensor([[True, False], [False, True]])
    assert torch.equal(torch.cat([m.to(dev), m.to(dev)], 1).cpu(), torch.cat([m, m], 1))
    x = gauss((8, 10, 12), seed=2)
    xd = x.to(dev)
    out = torch.cat([xd[:, ::2], xd[:, 1:4].transpose(1, 2).transpose(1, 2), xd[:, :1]], 1)
    assert torch.equal(out.cpu(), torch.cat([x[:, ::2], x[:, 1:4], x[:, :1]], 1))
    assert_on_device("aten::cat")


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
    assert_on_device("aten::cat")


def test_cat_rows16_c_abi_and_checks():
    """The kernel through the C ABI: parts land at their byte columns; non-adjacent parts are rejected."""
    rt = abi.Runtime()
    a, b = gauss((32, 24), seed=1), gauss((32, 40), seed=2)
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
