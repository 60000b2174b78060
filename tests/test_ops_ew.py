"""Elementwise ops on the vk device (kernel "ew_map") against the oracle and CPU PyTorch.

Mirrors the reference's tests/test_ops_ew.py: every case checks the values against CPU PyTorch at the
reference's tolerances (:17), that a GPU kernel ran and that nothing fell back to the CPU.  On top of
that each result is compared with oracle.ew_map: bit for bit for the ops whose float32 evaluation the
oracle restates exactly (oracle.EW_EXACT), within one unit in the last place of the output type
(float32: the reference tolerance) for the transcendental ones.  The later tests cover the device
layouts (16-byte vector path with a ragged tail, row broadcasts, misaligned views, 8-dimensional
spaces), the C-ABI's argument checks, and full-size DiT activations.
"""

import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from vkutil import bits

pytestmark = pytest.mark.gpu

import torch_vulkan  # noqa: E402
from torch_vulkan import abi  # noqa: E402

dev = torch.device("vk")
DTYPES = [torch.float32, torch.bfloat16, torch.float16]
TOL = {torch.float32: (1e-5, 1e-6), torch.bfloat16: (2e-2, 1e-3), torch.float16: (4e-3, 1e-4)}
KIND = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}
ULP = {torch.float32: 2.0 ** -23, torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}  # largest relative spacing


@pytest.fixture(autouse=True)
def _reset():
    torch_vulkan.reset_fallback_counts()  # clears the kernel counts too
    yield


def rnd(shape, dtype=torch.float32, lo=-3.0, hi=3.0, seed=0):
    """tests/test_ops_ew.py:30-32 of the reference."""
    g = torch.Generator().manual_seed(seed)
    return (torch.rand(shape, generator=g) * (hi - lo) + lo).to(dtype)


def close(gpu, cpu, dtype=None, scale=1.0):
    dtype = dtype or cpu.dtype
    rtol, atol = TOL[dtype]
    g, c = gpu.cpu().float(), cpu.float()
    assert g.shape == c.shape, (g.shape, c.shape)
    assert torch.allclose(g, c, rtol=rtol * scale, atol=atol * scale), f"max diff {(g - c).abs().max().item()}"


def no_fallback(*names):
    fb = torch_vulkan.fallback_counts()
    bad = {n: fb[n] for n in names if n in fb}
    assert not bad, f"CPU fallback: {bad}"


def ran_on_gpu(name):
    assert torch_vulkan.kernel_counts().get(name, 0) >= 1, (name, torch_vulkan.kernel_counts())


def np32(t):
    return None if t is None else t.detach().cpu().float().numpy()


def check_oracle(out, op, a, b=None, c=None, s0=0.0, s1=0.0, scale=1.0):
    """out (a vk tensor) against oracle.ew_map on the same inputs: equal bits for the exactly restated ops,
    else NaN where the oracle has NaN, equal infinities, and finite values within one unit in the last
    place of out's type plus the reference's float32 tolerance (times `scale`, as the reference scales it
    per op)."""
    ref, ref_bits = oracle.ew_map(op, np32(a), np32(b), np32(c), s0=s0, s1=s1, out_kind=KIND[out.dtype])
    if op in oracle.EW_EXACT or (op == "pow_s" and float(np.float32(s0)) in (2.0, 3.0, 0.5, -0.5, -1.0, -2.0)):
        # equal bits, except that any NaN matches any NaN (IEEE leaves the sign and payload of a NaN
        # created by an invalid operation open: x86 makes -NaN where the GPU makes +NaN)
        got = bits(out)
        gnan = np.isnan(out.detach().cpu().float().numpy())
        rnan = np.isnan(ref)
        assert np.array_equal(gnan, rnan), f"{op}: NaN positions differ"
        diff = (got != ref_bits) & ~rnan
        if diff.any():
            i = np.flatnonzero(diff.ravel())
            raise AssertionError(f"{op}: {i.size} elements differ from the oracle, first at {i[:4]}")
        return
    got = out.detach().cpu().float().numpy().astype(np.float64)
    r = ref.astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(r)), f"{op}: NaN positions differ"
    inf = np.isinf(r) | np.isinf(got)
    assert np.array_equal(got[inf], r[inf]), f"{op}: infinities differ"
    fin = ~(np.isnan(r) | inf)
    rtol, atol = TOL[torch.float32]
    lim = np.abs(r[fin]) * (ULP[out.dtype] + rtol * scale) + atol * scale
    err = np.abs(got[fin] - r[fin])
    assert np.all(err <= lim), f"{op}: max excess {(err - lim).max()}"


# ---- binary ops (reference tests/test_ops_ew.py:51-121) ---------------------------------------------------
OPS = {
    "add": (torch.add, "aten::add.Tensor"),
    "sub": (torch.sub, "aten::sub.Tensor"),
    "mul": (torch.mul, "aten::mul.Tensor"),
    "div": (torch.div, "aten::div.Tensor"),
}
PAIRS = [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
         (torch.float32, torch.bfloat16), (torch.bfloat16, torch.float32), (torch.bfloat16, torch.float16)]


@pytest.mark.parametrize("op", list(OPS))
@pytest.mark.parametrize("da,db", PAIRS)
def test_binary_same_shape_and_promotion(op, da, db):
    fn, name = OPS[op]
    a, b = rnd((5, 7), da, seed=1), rnd((5, 7), db, 0.5, 3.0, seed=2)
    ref = fn(a, b)
    out = fn(a.to(dev), b.to(dev))
    assert out.dtype == ref.dtype and out.device.type == "vk"
    close(out, ref)
    check_oracle(out, op, a, b, s0=1.0)
    ran_on_gpu(name)
    no_fallback(name.split(".")[0])


@pytest.mark.parametrize("op", list(OPS))
def test_binary_broadcast_and_noncontiguous(op):
    fn, name = OPS[op]
    for sa, sb in [((3, 1, 5), (1, 4, 1)), ((4, 5), (5,)), ((2, 3, 4, 5), (4, 1)), ((1,), (6, 7))]:
        a, b = rnd(sa, seed=3), rnd(sb, lo=0.5, hi=3.0, seed=4)
        out = fn(a.to(dev), b.to(dev))
        close(out, fn(a, b))
        check_oracle(out, op, a, b, s0=1.0)
    a, b = rnd((6, 8)), rnd((8, 6), lo=0.5, hi=3.0)
    out = fn(a.to(dev), b.to(dev).t())  # transposed view
    close(out, fn(a, b.t()))
    check_oracle(out, op, a, b.t(), s0=1.0)
    x = rnd((4, 10), lo=0.5, hi=3.0)
    close(fn(x.to(dev)[:, 2:7], x.to(dev)[:, 3:8]), fn(x[:, 2:7], x[:, 3:8]))  # offset slices
    ran_on_gpu(name)
    no_fallback(name.split(".")[0])


@pytest.mark.parametrize("op", list(OPS))
@pytest.mark.parametrize("dt", DTYPES)
def test_binary_with_host_scalar(op, dt):
    fn, name = OPS[op]
    x = rnd((6, 5), dt, lo=0.5, hi=3.0)
    for s in (2.5, 3):
        out = fn(x.to(dev), s)
        assert out.dtype == dt
        close(out, fn(x, s))
        sop = {"add": "add_s", "sub": "add_s", "mul": "mul_s", "div": "div_s"}[op]
        check_oracle(out, sop, x, s0=(-s if op == "sub" else s))
    if op in ("add", "mul"):
        close(fn(2.5, x.to(dev)), fn(2.5, x))  # scalar on the left
    ran_on_gpu(name)
    no_fallback(name.split(".")[0])


def test_alpha_and_zero_dim_vk_tensor():
    a, b = rnd((9,)), rnd((9,))
    out = torch.add(a.to(dev), b.to(dev), alpha=2.0)
    close(out, torch.add(a, b, alpha=2.0))
    check_oracle(out, "add", a, b, s0=2.0)
    out = torch.sub(a.to(dev), b.to(dev), alpha=0.5)
    close(out, torch.sub(a, b, alpha=0.5))
    check_oracle(out, "sub", a, b, s0=0.5)
    s = torch.tensor(1.5)
    close(a.to(dev) * s.to(dev), a * s)  # 0-dim vk tensor
    no_fallback("aten::add", "aten::sub", "aten::mul")


def test_zero_dim_f32_vk_tensor_rounds_to_the_bf16_result_type():
    """bf16 tensor + 0-dim f32 tensor computes in bf16 with the 0-dim value rounded to bf16, as on the CPU."""
    x = rnd((64,), torch.bfloat16, seed=11)
    s = torch.tensor(1.001)  # 1.001 is not a bf16 value; rounded it is 1.0
    out = x.to(dev) + s.to(dev)
    ref = x + s
    assert out.dtype == ref.dtype == torch.bfloat16
    assert not torch.equal(ref, (x.float() + 1.001).to(torch.bfloat16))  # the rounding matters here
    assert torch.equal(out.cpu(), ref)
    no_fallback("aten::add")


@pytest.mark.parametrize("op", ["add_", "sub_", "mul_", "div_"])
def test_inplace_on_strided_view_only_touches_the_view(op):
    x = rnd((6, 8), lo=0.5, hi=3.0)
    y = rnd((6, 4), lo=0.5, hi=3.0, seed=5)
    xd = x.to(dev)
    getattr(xd[:, 2:6], op)(y.to(dev))
    getattr(x[:, 2:6], op)(y)
    close(xd, x)
    getattr(xd, op)(2.0)
    getattr(x, op)(2.0)
    close(xd, x)
    no_fallback("aten::" + op.rstrip("_"))


def test_inplace_partial_overlap_is_rejected_like_the_cpu():
    x = rnd((16,)).to(dev)
    with pytest.raises(RuntimeError, match="overlap|single memory location"):
        x[1:].add_(x[:-1])


def test_inplace_mixed_dtype_rounds_into_self():
    """bf16.add_(f32 tensor): computed in f32, stored rounded to bf16."""
    a, b = rnd((33, 17), torch.bfloat16, seed=1), rnd((33, 17), torch.float32, seed=2)
    ad = a.to(dev)
    ad.add_(b.to(dev), alpha=0.5)
    ref = a.clone().add_(b, alpha=0.5)
    assert ad.dtype == torch.bfloat16
    close(ad, ref)
    got = bits(ad)
    _, want = oracle.ew_map("add", np32(a), np32(b), s0=0.5, out_kind="bf16")
    assert np.array_equal(got, want)


# ---- unary ops (reference :124-155) -----------------------------------------------------------------------
UNARY = {
    "neg": (torch.neg, -3, 3, "neg"), "rsqrt": (torch.rsqrt, 0.1, 5, "rsqrt"),
    "reciprocal": (torch.reciprocal, 0.2, 5, "recip"), "exp": (torch.exp, -4, 4, "exp"),
    "sqrt": (torch.sqrt, 0.0, 6, "sqrt"), "tanh": (torch.tanh, -4, 4, "tanh"),
    "sigmoid": (torch.sigmoid, -6, 6, "sigmoid"), "relu": (torch.relu, -3, 3, "relu"), "silu": (F.silu, -6, 6, "silu"),
    "gelu": (F.gelu, -6, 6, "gelu_erf"), "gelu_tanh": (lambda x: F.gelu(x, approximate="tanh"), -6, 6, "gelu_tanh"),
    "sin": (torch.sin, -8, 8, "sin"), "cos": (torch.cos, -8, 8, "cos"),
}


@pytest.mark.parametrize("name", list(UNARY))
@pytest.mark.parametrize("dt", DTYPES)
def test_unary(name, dt):
    fn, lo, hi, op = UNARY[name]
    x = rnd((4, 33), dt, lo, hi)
    out = fn(x.to(dev))
    close(out, fn(x), scale=2.0 if name in ("exp", "gelu", "gelu_tanh") else 1.0)
    check_oracle(out, op, x)
    no_fallback("aten::" + name.replace("_tanh", ""))


INPLACE = {"relu": torch.relu_, "silu": lambda t: F.silu(t, inplace=True), "sigmoid": torch.sigmoid_,
           "tanh": torch.tanh_, "exp": torch.exp_, "neg": torch.neg_, "sqrt": torch.sqrt_, "rsqrt": torch.rsqrt_,
           "reciprocal": torch.reciprocal_, "gelu": lambda t: torch._C._nn.gelu_(t)}


@pytest.mark.parametrize("name", list(INPLACE))
def test_inplace_unary_on_a_view(name):
    x = rnd((6, 16), torch.bfloat16, 0.2, 4.0, seed=4)
    xd = x.to(dev)
    INPLACE[name](xd[:, 4:12])
    INPLACE[name](x[:, 4:12])
    assert torch.equal(xd.cpu()[:, :4], x[:, :4]) and torch.equal(xd.cpu()[:, 12:], x[:, 12:])
    close(xd, x, scale=2.0)
    no_fallback("aten::" + name + "_")
    ran_on_gpu("aten::" + name + "_")


def test_sin_cos_with_large_arguments():
    """RoPE-like position x frequency arguments (reference :158-163)."""
    x = torch.arange(0, 4000, dtype=torch.float32).reshape(40, 100) * 0.37
    for fn, op in ((torch.sin, "sin"), (torch.cos, "cos")):
        out = fn(x.to(dev))
        close(out, fn(x), scale=40.0)
        check_oracle(out, op, x)
    no_fallback("aten::sin", "aten::cos")


@pytest.mark.parametrize("e", [2, 3, 0.5, -1, 2.5, 1.0, 0.0, -2, -0.5])
def test_pow_scalar(e):
    x = rnd((5, 6), lo=0.3, hi=3.0)
    out = torch.pow(x.to(dev), e)
    close(out, torch.pow(x, e), scale=4.0)
    check_oracle(out, "pow_s", x, s0=float(e))
    no_fallback("aten::pow")


def test_pow_negative_base_integer_exponent():
    x = rnd((50,), lo=-3.0, hi=3.0)
    for e in (2, 3, 4, -3):
        out = torch.pow(x.to(dev), e)
        close(out, torch.pow(x, e), scale=4.0)
        check_oracle(out, "pow_s", x, s0=float(e))


# ---- activation backward (reference :182-196) -------------------------------------------------------------
@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("act", ["silu", "gelu", "gelu_tanh"])
def test_activation_backward(act, dt):
    fn = {"silu": F.silu, "gelu": F.gelu, "gelu_tanh": lambda x: F.gelu(x, approximate="tanh")}[act]
    x = rnd((6, 17), dt, -5, 5)
    xc = x.clone().requires_grad_(True)
    xg = x.to(dev).requires_grad_(True)
    gout = rnd((6, 17), dt, seed=9)
    fn(xc).backward(gout)
    fn(xg).backward(gout.to(dev))
    close(xg.grad, xc.grad, scale=3.0)
    check_oracle(xg.grad, {"silu": "silu_bwd", "gelu": "gelu_erf_bwd", "gelu_tanh": "gelu_tanh_bwd"}[act], gout, x,
                 scale=3.0)
    no_fallback("aten::silu_backward", "aten::gelu_backward")
    ran_on_gpu("aten::silu_backward" if act == "silu" else "aten::gelu_backward")


# ---- where / fill (reference :200-220) --------------------------------------------------------------------
@pytest.mark.parametrize("dt", DTYPES)
def test_where_with_broadcast(dt):
    a, b = rnd((4, 6), dt, seed=1), rnd((1, 6), dt, seed=2)
    cond = rnd((4, 1), seed=3) > 0
    out = torch.where(cond.to(dev), a.to(dev), b.to(dev))
    assert torch.equal(out.cpu(), torch.where(cond, a, b))
    no_fallback("aten::where")
    ran_on_gpu("aten::where.self")


def test_where_mixed_dtypes_promote():
    a, b = rnd((8, 16), torch.bfloat16, seed=1), rnd((8, 16), torch.float32, seed=2)
    cond = rnd((8, 16), seed=3) > 0
    out = torch.where(cond.to(dev), a.to(dev), b.to(dev))
    ref = torch.where(cond, a, b)
    assert out.dtype == ref.dtype and torch.equal(out.cpu(), ref)
    no_fallback("aten::where")


@pytest.mark.parametrize("dt", DTYPES)
def test_fill_and_zero_on_view(dt):
    x = rnd((5, 8), dt)
    xd = x.to(dev)
    xd[1:4, 2:6].fill_(1.25)
    x[1:4, 2:6].fill_(1.25)
    close(xd, x)
    xd[:, ::2].zero_()
    x[:, ::2].zero_()
    close(xd, x)
    no_fallback("aten::fill_", "aten::zero_")


# ---- training loop (reference :235-260) -------------------------------------------------------------------
def test_mlp_training_matches_cpu_and_uses_gpu_kernels():
    def run(device):
        torch.manual_seed(0)
        m = torch.nn.Sequential(torch.nn.Linear(16, 32), torch.nn.SiLU(), torch.nn.Linear(32, 32), torch.nn.GELU(),
                                torch.nn.Linear(32, 4)).to(device)
        x = torch.randn(64, 16).to(device)
        y = torch.randn(64, 4).to(device)
        opt = torch.optim.SGD(m.parameters(), lr=0.05)
        ls = []
        for _ in range(15):
            opt.zero_grad()
            loss = F.mse_loss(m(x), y)
            loss.backward()
            opt.step()
            ls.append(loss.item())
        return ls

    cpu = run("cpu")
    torch_vulkan.reset_fallback_counts()
    gpu = run(dev)
    assert max(abs(a - b) for a, b in zip(cpu, gpu)) < 1e-4, (cpu, gpu)
    kc, fb = torch_vulkan.kernel_counts(), torch_vulkan.fallback_counts()
    assert kc.get("aten::silu_backward") and kc.get("aten::gelu_backward"), kc
    for n in ("aten::silu", "aten::gelu", "aten::add", "aten::mul", "aten::sub"):
        assert n not in fb, (n, fb)


# ---- scalar on the left (reference :268-282) --------------------------------------------------------------
@pytest.mark.parametrize("dt", DTYPES)
def test_scalar_on_the_left_stays_on_device_and_uses_gpu_kernels(dt):
    x = rnd((5, 7), dt, lo=0.5, hi=3.0)
    xd = x.to(dev)
    cases = {
        "1 - x": (lambda t: 1 - t), "2 / x": (lambda t: 2 / t), "0.5 + x": (lambda t: 0.5 + t), "3 * x": (lambda t: 3 * t),
        "sub alpha": (lambda t: torch.sub(2.0, t, alpha=3)), "add alpha": (lambda t: torch.add(2.0, t, alpha=2)),
        "div scalar tensor": (lambda t: torch.div(torch.tensor(2.0), t)),
    }
    for name, fn in cases.items():
        out = fn(xd)
        assert out.device.type == "vk", f"{name}: output on {out.device}"
        close(out, fn(x), dt, scale=2.0)
    check_oracle(torch.sub(2.0, xd, alpha=3), "axpb", x, s0=-3.0, s1=2.0)
    check_oracle(torch.div(torch.tensor(2.0), xd), "rdiv_s", x, s0=2.0)
    no_fallback("aten::sub", "aten::add", "aten::div", "aten::mul")


# ---- optimizer forms (reference :295-310) -----------------------------------------------------------------
@pytest.mark.parametrize("dt", DTYPES)
def test_addcmul_addcdiv_lerp(dt):
    a, b, c = rnd((6, 9), dt, seed=1), rnd((6, 9), dt, seed=2), rnd((6, 9), dt, 0.5, 3.0, seed=3)
    ad = a.to(dev)
    out = torch.addcmul(ad, b.to(dev), c.to(dev), value=0.3)
    close(out, torch.addcmul(a, b, c, value=0.3), dt, scale=2.0)
    check_oracle(out, "addcmul", a, b, c, s0=0.3)
    out = torch.addcdiv(ad, b.to(dev), c.to(dev), value=-0.7)
    close(out, torch.addcdiv(a, b, c, value=-0.7), dt, scale=2.0)
    check_oracle(out, "addcdiv", a, b, c, s0=-0.7)
    for w in (0.1, 0.75):
        out = torch.lerp(ad, b.to(dev), w)
        close(out, torch.lerp(a, b, w), dt, scale=2.0)
        check_oracle(out, "lerp_s", a, b, s0=w)
    x, xd = a.clone(), a.to(dev)
    xd.addcmul_(b.to(dev), c.to(dev), value=0.3)
    x.addcmul_(b, c, value=0.3)
    xd.addcdiv_(b.to(dev), c.to(dev), value=2.0)
    x.addcdiv_(b, c, value=2.0)
    xd.lerp_(b.to(dev), 0.25)
    x.lerp_(b, 0.25)
    close(xd, x, dt, scale=4.0)
    no_fallback("aten::addcmul", "aten::addcdiv", "aten::lerp")


@pytest.mark.parametrize("dt", DTYPES)
def test_scalar_overloads_do_not_promote_dtype(dt):
    x = rnd((5, 5), dt, lo=0.5, hi=3.0)
    xd = x.to(dev)
    for name, fn in {"mul_": lambda t: t.mul_(0.999), "add_": lambda t: t.add_(0.5, alpha=2), "sub_": lambda t: t.sub_(1.5),
                     "div_": lambda t: t.div_(3.0)}.items():
        a, b = x.clone(), xd.clone()
        fn(a)
        fn(b)
        assert b.dtype == dt, name
        close(b, a, dt, scale=2.0)
    for fn in (lambda t: torch.mul(t, 2.5), lambda t: torch.add(t, 1.5, alpha=2), lambda t: torch.sub(t, 0.5),
               lambda t: torch.div(t, 4.0)):
        out = fn(xd)
        assert out.dtype == dt
        close(out, fn(x), dt, scale=2.0)
    no_fallback("aten::mul", "aten::add", "aten::sub", "aten::div")


# ---- device layouts: vector path, ragged tails, row broadcasts, alignment, rank 8 -------------------------
@pytest.mark.parametrize("n", [1, 7, 8, 9, 4095, 1000003])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_flat_lengths_and_ragged_tail(n, dt):
    a, b = rnd((n,), dt, seed=n), rnd((n,), torch.float32, 0.5, 3.0, seed=n + 1)
    out = torch.div(a.to(dev), b.to(dev))  # mixed types: the general vector kernel
    check_oracle(out, "div", a, b)
    out = F.gelu(a.to(dev))  # one type, contiguous: the flat kernel
    check_oracle(out, "gelu_erf", a)
    c = b.to(dt)
    out = torch.mul(a.to(dev), c.to(dev))
    check_oracle(out, "mul", a, c)
    m = a > 0
    out = torch.where(m.to(dev), a.to(dev), c.to(dev))
    check_oracle(out, "where", a, c, m.float())
    out = torch.addcdiv(a.to(dev), c.to(dev), c.to(dev) + 1.0, value=0.5)
    check_oracle(out, "addcdiv", a, c, c.to(dev) + 1.0, s0=0.5)


@pytest.mark.parametrize("rows,cols", [(64, 1024), (33, 40), (7, 12)])
def test_bias_row_and_column_broadcasts(rows, cols):
    """[M, N] + [N] (the vector kernel with a stride-0 leading index when N % 8 == 0) and [M, N] * [M, 1]."""
    x = rnd((rows, cols), torch.bfloat16, seed=1)
    bias = rnd((cols,), torch.bfloat16, seed=2)
    sc = rnd((rows, 1), torch.float32, 0.5, 2.0, seed=3)
    out = x.to(dev) + bias.to(dev)
    check_oracle(out, "add", x, bias, s0=1.0)
    out = x.to(dev) * sc.to(dev)
    check_oracle(out, "mul", x, sc)
    out = torch.where((x > 0).to(dev), x.to(dev), bias.to(dev))
    check_oracle(out, "where", x, bias, (x > 0).float())
    no_fallback("aten::add", "aten::mul", "aten::where")


def test_misaligned_views_take_the_element_path():
    x = rnd((1, 4099), torch.bfloat16, seed=5)
    xd = x.to(dev)
    for off in (1, 3, 8):
        out = F.silu(xd[:, off:])
        check_oracle(out, "silu", x[:, off:])
        out = xd[:, off:] * xd[:, :4099 - off]
        check_oracle(out, "mul", x[:, off:], x[:, :4099 - off])


def test_eight_dimensional_broadcast_and_permuted_views():
    a = rnd((2, 3, 2, 3, 2, 3, 2, 5), seed=1)
    b = rnd((3, 1, 3, 1, 3, 1, 5), lo=0.5, hi=2.0, seed=2)
    out = torch.div(a.to(dev), b.to(dev))
    close(out, a / b)
    check_oracle(out, "div", a, b)
    p = a.permute(7, 5, 3, 1, 0, 2, 4, 6)
    out = torch.sigmoid(a.to(dev).permute(7, 5, 3, 1, 0, 2, 4, 6))
    check_oracle(out, "sigmoid", p)
    no_fallback("aten::div", "aten::sigmoid")


def test_empty_and_one_element_tensors():
    e = torch.empty(0, 5, device=dev)
    assert (e + e).shape == (0, 5) and F.gelu(e).shape == (0, 5)
    one = rnd((1,), seed=3)
    check_oracle(torch.exp(one.to(dev)), "exp", one)
    s = torch.tensor(0.75)
    out = torch.sigmoid(s.to(dev))
    assert out.dim() == 0
    check_oracle(out, "sigmoid", s)


def test_special_values():
    """NaN, infinities, signed zeros and subnormals against the oracle (PyTorch's CPU GELU returns NaN at
    +inf, where the formula and the oracle give +inf; finite entries are also checked against the CPU)."""
    x = torch.tensor([float("nan"), float("inf"), -float("inf"), 0.0, -0.0, 1e-40, -3.0, 100.0, -100.0, 20.0])
    for dt in DTYPES:
        xd = x.to(dt)
        for fn, op in ((torch.relu, "relu"), (torch.neg, "neg"), (torch.exp, "exp"), (torch.sigmoid, "sigmoid"),
                       (torch.tanh, "tanh"), (F.silu, "silu"), (F.gelu, "gelu_erf"),
                       (lambda t: F.gelu(t, approximate="tanh"), "gelu_tanh"), (torch.sqrt, "sqrt")):
            out = fn(xd.to(dev))
            check_oracle(out, op, xd)
            got, ref = out.cpu().float(), fn(xd).float()
            m = torch.isfinite(ref) & torch.isfinite(xd.float())
            assert torch.allclose(got[m], ref[m], rtol=TOL[dt][0], atol=TOL[dt][1]), (op, dt, got, ref)


@pytest.mark.parametrize("op,fn,bwd", [("silu", F.silu, "silu_bwd"), ("gelu_erf", F.gelu, "gelu_erf_bwd"),
                                       ("gelu_tanh", lambda t: F.gelu(t, approximate="tanh"), "gelu_tanh_bwd")])
def test_dit_mlp_activation_full_size(op, fn, bwd):
    """The DiT MLP hidden activation at the BASELINE DiT shape (M = 1024 tokens, 8192 features, bf16),
    forward and backward, against the oracle element by element."""
    x = rnd((1024, 8192), torch.bfloat16, -6, 6, seed=21)
    g = rnd((1024, 8192), torch.bfloat16, seed=22)
    xd = x.to(dev).requires_grad_(True)
    y = fn(xd)
    y.backward(g.to(dev))
    check_oracle(y, op, x)
    check_oracle(xd.grad, bwd, g, x, scale=3.0)


def test_adamw_step_on_device_matches_cpu():
    """torch.optim.AdamW (for-loop form) on bf16 parameters: mul_/lerp_/addcmul_/addcdiv_/sqrt/div on vk."""
    def run(device):
        torch.manual_seed(0)
        p = [torch.nn.Parameter(torch.randn(64, 48).to(torch.float32).to(device)) for _ in range(2)]
        opt = torch.optim.AdamW(p, lr=1e-2, weight_decay=0.1, foreach=False)
        for step in range(3):
            for i, q in enumerate(p):
                q.grad = (torch.randn(64, 48, generator=torch.Generator().manual_seed(10 * step + i))).to(device)
            opt.step()
        return [q.detach().cpu() for q in p]

    cpu, gpu = run("cpu"), run(dev)
    for a, b in zip(cpu, gpu):
        assert torch.allclose(a, b, rtol=1e-5, atol=1e-6), (a - b).abs().max()
    fb = torch_vulkan.fallback_counts()
    for n in ("aten::mul", "aten::lerp", "aten::addcmul", "aten::addcdiv", "aten::div", "aten::sqrt", "aten::add"):
        assert n not in fb, (n, fb)


# ---- the C ABI directly ----------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def rt():
    return abi.Runtime()


def _ew(op, out, a, b=None, c=None, s0=0.0, s1=0.0, sizes=None, strides=None):
    A = abi.EwArgs()
    A.op = abi.EW_OPS[op]
    sizes = list(out.shape) if sizes is None else sizes
    A.ndim = len(sizes)
    dtc = {torch.float32: abi.F32, torch.bfloat16: abi.BF16, torch.float16: abi.F16, torch.bool: abi.RAW8}
    for name, t in (("out", out), ("a", a), ("b", b), ("c", c)):
        if t is None:
            continue
        setattr(A, name, t.data_ptr())
        setattr(A, name + "_dtype", dtc[t.dtype])
        st = list(t.stride()) if strides is None or name not in strides else strides[name]
        arr = getattr(A, name + "_strides")
        for i, s in enumerate(st):
            arr[i] = s
    for i, s in enumerate(sizes):
        A.sizes[i] = s
    A.s0, A.s1 = s0, s1
    return A


def test_c_abi_map_with_explicit_strides(rt):
    """out[i, j] = a[j, i] + 2 * b[i] through hrt_dispatch: a transposed operand and a broadcast column."""
    a = rnd((24, 16), seed=1)
    b = rnd((16,), seed=2)
    ad, bd = a.to(dev), b.to(dev)
    out = torch.empty(16, 24, device=dev)
    A = _ew("add", out, ad, bd, s0=2.0, strides={"a": [1, 16], "b": [1, 0]})
    rt.dispatch("ew_map", A)
    rt.synchronize()
    _, want = oracle.ew_map("add", a.t().numpy(), b.numpy()[:, None], s0=2.0)
    assert np.array_equal(bits(out), want)


@pytest.mark.parametrize("case", ["op", "unused", "stride0_out", "negative", "where_c", "out_of_block"])
def test_c_abi_rejects_bad_arguments(rt, case):
    x = torch.zeros(64, device=dev)
    y = torch.zeros(64, device=dev)
    A = _ew("add", y, x, x, s0=1.0)
    if case == "op":
        A.op = 99
    elif case == "unused":
        A = _ew("exp", y, x)
        A.b = x.data_ptr()
    elif case == "stride0_out":
        A.out_strides[0] = 0
    elif case == "negative":
        A.a_strides[0] = -1
    elif case == "where_c":
        A = _ew("where", y, x, x, x)
    elif case == "out_of_block":
        A.sizes[0] = 1 << 30
    with pytest.raises(RuntimeError, match="ew_map"):
        rt.dispatch("ew_map", A)
    rt.synchronize()
    assert torch.count_nonzero(y.cpu()) == 0
