"""Elementwise ops on the vk device (kernel "ew_map") against the oracle and CPU PyTorch.

The reference's tests/test_ops_ew.py fixes what this device must do for its elementwise operators: binary
ops with promotion, broadcasting, views and host scalars on either side, the unary activations and their
backward, where / fill, in-place forms, the optimizer updates, and a small training loop that stays on the
device.  These tests cover the same behaviours as tables of cases: each result against CPU PyTorch at the
reference's tolerances per dtype (float32 1e-5 / 1e-6, bfloat16 2e-2 / 1e-3, float16 4e-3 / 1e-4, widened
per op where the reference widens it), against oracle.ew_map (bit for bit for the ops whose float32
evaluation the oracle restates exactly, oracle.EW_EXACT; within one unit in the last place of the output
type for the transcendental ones), and that a GPU kernel ran with nothing falling back to the CPU.  The
later tests cover the device layouts (16-byte vector path with a ragged tail, row broadcasts, misaligned
views, 8-dimensional spaces), the C-ABI's argument checks, and full-size DiT activations.
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
FLOATS = [torch.float32, torch.bfloat16, torch.float16]
# (rtol, atol) per result dtype for comparisons with CPU PyTorch
TOL = {torch.float32: (1e-5, 1e-6), torch.bfloat16: (2e-2, 1e-3), torch.float16: (4e-3, 1e-4)}
KIND = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}
ULP = {torch.float32: 2.0 ** -23, torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}  # largest relative spacing


def uni(shape, dtype=torch.float32, lo=-3.0, hi=3.0, seed=0):
    """Seeded uniform values in [lo, hi), rounded to dtype."""
    return torch.empty(shape).uniform_(lo, hi, generator=torch.Generator().manual_seed(seed)).to(dtype)


def assert_cpu_close(got, want, dtype=None, widen=1.0, magnitude=None, what=""):
    """A vk result against the CPU's: same shape, within TOL[dtype] (the CPU result's dtype by default)
    scaled by `widen`, relative to |want| or, where the result can cancel (a - b with a ~ b), to the given
    `magnitude` of the terms."""
    rtol, atol = TOL[dtype or want.dtype]
    g, w = got.cpu().float(), want.float()
    assert g.shape == w.shape, (what, g.shape, w.shape)
    err = (g - w).abs()
    size = w.abs() if magnitude is None else torch.maximum(w.abs(), magnitude.float())
    lim = atol * widen + rtol * widen * size
    assert bool((err <= lim).all()), f"{what}: worst excess {(err - lim).max().item()} (max diff {err.max().item()})"


def no_cpu_fallback(*names):
    fb = torch_vulkan.fallback_counts()
    hit = {n: fb[n] for n in names if n in fb}
    assert not hit, f"ran on the CPU: {hit}"


def kernel_ran(name):
    assert torch_vulkan.kernel_counts().get(name, 0) >= 1, (name, torch_vulkan.kernel_counts())


def np32(t):
    return None if t is None else t.detach().cpu().float().numpy()


def check_oracle(out, op, a, b=None, c=None, s0=0.0, s1=0.0, scale=1.0):
    """out (a vk tensor) against oracle.ew_map on the same inputs: equal bits for the exactly restated ops,
    else NaN where the oracle has NaN, equal infinities, and finite values within one unit in the last
    place of out's type plus the float32 tolerance (times `scale`, widened per op as for the CPU)."""
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


# ---- binary ops: dtype pairs x operand layouts ----------------------------------------------------------
# name -> (torch function, the shim's kernel-count key, oracle op)
BINARY = {"add": (torch.add, "aten::add.Tensor", "add"), "sub": (torch.sub, "aten::sub.Tensor", "sub"),
          "mul": (torch.mul, "aten::mul.Tensor", "mul"), "div": (torch.div, "aten::div.Tensor", "div")}
# How the two operands are built: (shape of a, shape of b, view applied to the device and CPU operands).
# b stays in [0.5, 3) so division is well conditioned.
LAYOUTS = {
    "same shape": ((5, 7), (5, 7), lambda a, b: (a, b)),
    "outer broadcast": ((3, 1, 5), (1, 4, 1), lambda a, b: (a, b)),
    "row vector": ((4, 5), (5,), lambda a, b: (a, b)),
    "trailing column": ((2, 3, 4, 5), (4, 1), lambda a, b: (a, b)),
    "one element": ((1,), (6, 7), lambda a, b: (a, b)),
    "transposed b": ((6, 8), (8, 6), lambda a, b: (a, b.t())),
    "overlapping slices": ((4, 10), (4, 10), lambda a, b: (b[:, 2:7], b[:, 3:8])),
}
DTYPE_PAIRS = [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
               (torch.float32, torch.bfloat16), (torch.bfloat16, torch.float32), (torch.bfloat16, torch.float16)]


@pytest.mark.parametrize("layout", list(LAYOUTS))
@pytest.mark.parametrize("op", list(BINARY))
def test_binary_layouts(op, layout):
    fn, key, oop = BINARY[op]
    sa, sb, view = LAYOUTS[layout]
    a, b = uni(sa, seed=len(layout)), uni(sb, lo=0.5, hi=3.0, seed=len(layout) + 1)
    ga, gb = view(a.to(dev), b.to(dev))
    ca, cb = view(a, b)
    out = fn(ga, gb)
    assert out.device.type == "vk"
    assert_cpu_close(out, fn(ca, cb))
    check_oracle(out, oop, ca, cb, s0=1.0)
    kernel_ran(key)
    no_cpu_fallback(key.split(".")[0])


@pytest.mark.parametrize("da,db", DTYPE_PAIRS)
@pytest.mark.parametrize("op", list(BINARY))
def test_binary_dtype_promotion(op, da, db):
    fn, key, oop = BINARY[op]
    a, b = uni((5, 7), da, seed=1), uni((5, 7), db, 0.5, 3.0, seed=2)
    want = fn(a, b)
    out = fn(a.to(dev), b.to(dev))
    assert out.dtype == want.dtype
    assert_cpu_close(out, want)
    check_oracle(out, oop, a, b, s0=1.0)
    no_cpu_fallback(key.split(".")[0])


# Scalar forms, each as (device expression, CPU expression, oracle op and scalars or None).  Results keep the
# tensor's dtype (a Python scalar does not promote it), also in place.
def _scalar_cases(x):
    two = torch.tensor(2.0)
    return {
        "x + 2.5": (lambda t: t + 2.5, ("add_s", 2.5)),
        "x - 3": (lambda t: t - 3, ("add_s", -3.0)),
        "x * 2.5": (lambda t: t * 2.5, ("mul_s", 2.5)),
        "x / 3": (lambda t: t / 3, ("div_s", 3.0)),
        "2.5 + x": (lambda t: 2.5 + t, None),
        "3 * x": (lambda t: 3 * t, None),
        "1 - x": (lambda t: 1 - t, None),
        "2 / x": (lambda t: 2 / t, None),
        "sub(2, x, alpha=3)": (lambda t: torch.sub(2.0, t, alpha=3), ("axpb", -3.0, 2.0)),
        "add(2, x, alpha=2)": (lambda t: torch.add(2.0, t, alpha=2), None),
        "div(0-dim 2, x)": (lambda t: torch.div(two.to(t.device), t), ("rdiv_s", 2.0)),
        "add(x, 1.5, alpha=2)": (lambda t: torch.add(t, 1.5, alpha=2), None),
        "x.mul_(0.999)": (lambda t: t.clone().mul_(0.999), None),
        "x.add_(0.5, alpha=2)": (lambda t: t.clone().add_(0.5, alpha=2), None),
        "x.sub_(1.5)": (lambda t: t.clone().sub_(1.5), None),
        "x.div_(3)": (lambda t: t.clone().div_(3.0), None),
    }


@pytest.mark.parametrize("dt", FLOATS)
def test_scalar_operands_on_either_side(dt):
    x = uni((6, 5), dt, lo=0.5, hi=3.0, seed=7)
    xd = x.to(dev)
    for name, (fn, orc) in _scalar_cases(x).items():
        out = fn(xd)
        assert out.device.type == "vk" and out.dtype == dt, (name, out.device, out.dtype)
        # terms up to 3 |x| + 2 (the scalars below): a difference of two can cancel
        assert_cpu_close(out, fn(x), dt, widen=2.0, magnitude=3 * x.float().abs() + 2, what=name)
        if orc is not None:
            check_oracle(out, orc[0], x, s0=orc[1], s1=orc[2] if len(orc) > 2 else 0.0)
    no_cpu_fallback("aten::add", "aten::sub", "aten::mul", "aten::div")


def test_alpha_and_zero_dim_device_operands():
    a, b = uni((9,), seed=1), uni((9,), seed=2)
    for fn, op, alpha in ((torch.add, "add", 2.0), (torch.sub, "sub", 0.5)):
        out = fn(a.to(dev), b.to(dev), alpha=alpha)
        assert_cpu_close(out, fn(a, b, alpha=alpha))
        check_oracle(out, op, a, b, s0=alpha)
    s = torch.tensor(1.5)
    assert_cpu_close(a.to(dev) * s.to(dev), a * s)  # a 0-dim vk operand
    no_cpu_fallback("aten::add", "aten::sub", "aten::mul")


def test_zero_dim_f32_vk_tensor_rounds_to_the_bf16_result_type():
    """bf16 tensor + 0-dim f32 tensor computes in bf16 with the 0-dim value rounded to bf16, as on the CPU."""
    x = uni((64,), torch.bfloat16, seed=11)
    s = torch.tensor(1.001)  # 1.001 is not a bf16 value; rounded it is 1.0
    out = x.to(dev) + s.to(dev)
    ref = x + s
    assert out.dtype == ref.dtype == torch.bfloat16
    assert not torch.equal(ref, (x.float() + 1.001).to(torch.bfloat16))  # the rounding matters here
    assert torch.equal(out.cpu(), ref)
    no_cpu_fallback("aten::add")


# ---- in-place forms ----------------------------------------------------------------------------------------
@pytest.mark.parametrize("op", ["add_", "sub_", "mul_", "div_"])
def test_inplace_binary_writes_only_its_view(op):
    base = uni((6, 8), lo=0.5, hi=3.0, seed=12)
    other = uni((6, 4), lo=0.5, hi=3.0, seed=13)
    gpu, cpu = base.to(dev), base.clone()
    for target_g, target_c, arg_g, arg_c in ((gpu[:, 2:6], cpu[:, 2:6], other.to(dev), other), (gpu, cpu, 2.0, 2.0)):
        getattr(target_g, op)(arg_g)
        getattr(target_c, op)(arg_c)
        assert_cpu_close(gpu, cpu)  # the columns outside the view are compared too
    no_cpu_fallback("aten::" + op.rstrip("_"))


def test_inplace_partial_overlap_is_rejected_like_the_cpu():
    x = uni((16,)).to(dev)
    with pytest.raises(RuntimeError, match="overlap|single memory location"):
        x[1:].add_(x[:-1])


def test_inplace_mixed_dtype_rounds_into_self():
    """bf16.add_(f32 tensor): computed in f32, stored rounded to bf16."""
    a, b = uni((33, 17), torch.bfloat16, seed=1), uni((33, 17), torch.float32, seed=2)
    ad = a.to(dev)
    ad.add_(b.to(dev), alpha=0.5)
    ref = a.clone().add_(b, alpha=0.5)
    assert ad.dtype == torch.bfloat16
    assert_cpu_close(ad, ref)
    got = bits(ad)
    _, want = oracle.ew_map("add", np32(a), np32(b), s0=0.5, out_kind="bf16")
    assert np.array_equal(got, want)


# ---- unary ops ----------------------------------------------------------------------------------------------
# name -> (function, input range, oracle op, tolerance widening against the CPU, in-place form or None)
UNARY = {
    "neg": (torch.neg, (-3, 3), "neg", 1.0, torch.neg_),
    "rsqrt": (torch.rsqrt, (0.1, 5), "rsqrt", 1.0, torch.rsqrt_),
    "reciprocal": (torch.reciprocal, (0.2, 5), "recip", 1.0, torch.reciprocal_),
    "exp": (torch.exp, (-4, 4), "exp", 2.0, torch.exp_),
    "sqrt": (torch.sqrt, (0.0, 6), "sqrt", 1.0, torch.sqrt_),
    "tanh": (torch.tanh, (-4, 4), "tanh", 1.0, torch.tanh_),
    "sigmoid": (torch.sigmoid, (-6, 6), "sigmoid", 1.0, torch.sigmoid_),
    "relu": (torch.relu, (-3, 3), "relu", 1.0, torch.relu_),
    "silu": (F.silu, (-6, 6), "silu", 1.0, lambda t: F.silu(t, inplace=True)),
    "gelu": (F.gelu, (-6, 6), "gelu_erf", 2.0, lambda t: torch._C._nn.gelu_(t)),
    "gelu_tanh": (lambda t: F.gelu(t, approximate="tanh"), (-6, 6), "gelu_tanh", 2.0, None),
    "sin": (torch.sin, (-8, 8), "sin", 1.0, None),
    "cos": (torch.cos, (-8, 8), "cos", 1.0, None),
}


@pytest.mark.parametrize("dt", FLOATS)
@pytest.mark.parametrize("name", list(UNARY))
def test_unary(name, dt):
    fn, (lo, hi), op, widen, _ = UNARY[name]
    x = uni((4, 33), dt, lo, hi, seed=list(UNARY).index(name))
    out = fn(x.to(dev))
    assert_cpu_close(out, fn(x), widen=widen)
    check_oracle(out, op, x)
    no_cpu_fallback("aten::" + name.replace("_tanh", ""))


@pytest.mark.parametrize("name", [n for n, v in UNARY.items() if v[4] is not None])
def test_inplace_unary_writes_only_its_view(name):
    inplace = UNARY[name][4]
    x = uni((6, 16), torch.bfloat16, 0.2, 4.0, seed=4)
    xd = x.to(dev)
    inplace(xd[:, 4:12])
    inplace(x[:, 4:12])
    got = xd.cpu()
    assert torch.equal(got[:, :4], x[:, :4]) and torch.equal(got[:, 12:], x[:, 12:])
    assert_cpu_close(xd, x, widen=2.0)
    no_cpu_fallback("aten::" + name + "_")
    kernel_ran("aten::" + name + "_")


def test_sin_cos_of_rotary_angles():
    """Arguments up to ~1500 rad, as rotary position embeddings produce (position x frequency)."""
    pos = torch.arange(1500, dtype=torch.float32)[:, None]
    x = pos * 10000.0 ** (-torch.arange(0, 64, 2, dtype=torch.float32) / 64)  # [1500, 32], up to 1499 rad
    for fn, op in ((torch.sin, "sin"), (torch.cos, "cos")):
        out = fn(x.to(dev))
        assert_cpu_close(out, fn(x), widen=40.0)
        check_oracle(out, op, x)
    no_cpu_fallback("aten::sin", "aten::cos")


@pytest.mark.parametrize("e", [2, 3, 0.5, -1, 2.5, 1.0, 0.0, -2, -0.5, 4, -3])
def test_pow_scalar_exponents(e):
    """Positive bases for every exponent; negative bases too where the exponent is an integer."""
    lo = -3.0 if float(e).is_integer() else 0.3
    x = uni((5, 10), lo=lo, hi=3.0, seed=int(e * 10) % 97)
    out = torch.pow(x.to(dev), e)
    assert_cpu_close(out, torch.pow(x, e), widen=4.0)
    check_oracle(out, "pow_s", x, s0=float(e))
    no_cpu_fallback("aten::pow")


# ---- activation gradients --------------------------------------------------------------------------------
ACT = {"silu": (F.silu, "silu_bwd", "aten::silu_backward"),
       "gelu": (F.gelu, "gelu_erf_bwd", "aten::gelu_backward"),
       "gelu_tanh": (lambda t: F.gelu(t, approximate="tanh"), "gelu_tanh_bwd", "aten::gelu_backward")}


@pytest.mark.parametrize("dt", FLOATS)
@pytest.mark.parametrize("act", list(ACT))
def test_activation_gradients(act, dt):
    fn, oop, key = ACT[act]
    x = uni((6, 17), dt, -5, 5, seed=31)
    gy = uni((6, 17), dt, seed=32)
    xc = x.clone().requires_grad_(True)
    (want,) = torch.autograd.grad(fn(xc), xc, gy)
    xg = x.to(dev).requires_grad_(True)
    (got,) = torch.autograd.grad(fn(xg), xg, gy.to(dev))
    assert_cpu_close(got, want, widen=3.0)
    check_oracle(got, oop, gy, x, scale=3.0)
    kernel_ran(key)
    no_cpu_fallback("aten::silu_backward", "aten::gelu_backward")


# ---- where / fill ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dt", FLOATS)
def test_where_selects_across_broadcasts_and_promotes(dt):
    cond = uni((4, 1), seed=3) > 0
    a, b = uni((4, 6), dt, seed=1), uni((1, 6), dt, seed=2)
    out = torch.where(cond.to(dev), a.to(dev), b.to(dev))
    assert torch.equal(out.cpu(), torch.where(cond, a, b))
    kernel_ran("aten::where.self")
    other = torch.float32 if dt != torch.float32 else torch.bfloat16  # mixed operand dtypes promote
    c2 = uni((8, 16), seed=5) > 0
    p, q = uni((8, 16), dt, seed=6), uni((8, 16), other, seed=7)
    out = torch.where(c2.to(dev), p.to(dev), q.to(dev))
    want = torch.where(c2, p, q)
    assert out.dtype == want.dtype and torch.equal(out.cpu(), want)
    no_cpu_fallback("aten::where")


@pytest.mark.parametrize("dt", FLOATS)
def test_fill_and_zero_write_only_their_views(dt):
    x = uni((5, 8), dt, seed=8)
    xd = x.to(dev)
    for edit in (lambda t: t[1:4, 2:6].fill_(1.25), lambda t: t[:, ::2].zero_(), lambda t: t.t()[3].fill_(-2.0)):
        edit(xd)
        edit(x)
        assert torch.equal(xd.cpu(), x)
    no_cpu_fallback("aten::fill_", "aten::zero_")


# ---- a training loop and the optimizer updates ---------------------------------------------------------
def test_small_network_trains_like_on_the_cpu():
    """Eight SGD-with-momentum steps of a two-hidden-layer network (SiLU, tanh-GELU) on a fixed regression
    batch: the parameters after training match the CPU's, and the activations and their gradients ran as
    vk kernels."""
    def train(device):
        g = torch.Generator().manual_seed(5)
        dims = [12, 24, 24, 3]
        ws = [torch.randn(o, i, generator=g) * i ** -0.5 for i, o in zip(dims[:-1], dims[1:])]
        bs = [torch.randn(o, generator=g) * 0.1 for o in dims[1:]]
        params = [t.to(device).requires_grad_(True) for t in ws + bs]
        x = torch.randn(48, dims[0], generator=g).to(device)
        y = torch.randn(48, dims[-1], generator=g).to(device)
        opt = torch.optim.SGD(params, lr=0.03, momentum=0.9)
        acts = [F.silu, lambda t: F.gelu(t, approximate="tanh"), lambda t: t]
        for _ in range(8):
            h = x
            for w, b, act in zip(params[:3], params[3:], acts):
                h = act(h @ w.t() + b)
            loss = ((h - y) ** 2).mean()
            opt.zero_grad()
            loss.backward()
            opt.step()
        return [p.detach().cpu() for p in params]

    cpu = train("cpu")
    torch_vulkan.reset_fallback_counts()
    gpu = train(dev)
    for a, b in zip(cpu, gpu):
        assert torch.allclose(a, b, rtol=1e-4, atol=1e-5), (a - b).abs().max()
    kernel_ran("aten::silu_backward")
    kernel_ran("aten::gelu_backward")
    no_cpu_fallback("aten::silu", "aten::gelu", "aten::add", "aten::mul", "aten::sub")


@pytest.mark.parametrize("dt", FLOATS)
def test_optimizer_update_forms(dt):
    """addcmul, addcdiv and lerp (the Adam-family updates), out of place against the oracle and chained in
    place."""
    p, m, v = uni((6, 9), dt, seed=1), uni((6, 9), dt, seed=2), uni((6, 9), dt, 0.5, 3.0, seed=3)
    pd, md, vd = p.to(dev), m.to(dev), v.to(dev)
    cases = [(lambda a, b, c: torch.addcmul(a, b, c, value=0.3), ("addcmul", p, m, v, 0.3)),
             (lambda a, b, c: torch.addcdiv(a, b, c, value=-0.7), ("addcdiv", p, m, v, -0.7)),
             (lambda a, b, c: torch.lerp(a, b, 0.1), ("lerp_s", p, m, None, 0.1)),
             (lambda a, b, c: torch.lerp(a, b, 0.75), ("lerp_s", p, m, None, 0.75))]
    for fn, (op, a, b, c, s) in cases:
        out = fn(pd, md, vd)
        assert_cpu_close(out, fn(p, m, v), dt, widen=2.0)
        check_oracle(out, op, a, b, c, s0=s)
    chained_g, chained_c = pd.clone(), p.clone()
    for t, b, c in ((chained_g, md, vd), (chained_c, m, v)):
        t.addcmul_(b, c, value=0.3).addcdiv_(b, c, value=2.0).lerp_(b, 0.25)
    assert_cpu_close(chained_g, chained_c, dt, widen=4.0)
    no_cpu_fallback("aten::addcmul", "aten::addcdiv", "aten::lerp")


# ---- device layouts: vector path, ragged tails, row broadcasts, alignment, rank 8 -------------------------
@pytest.mark.parametrize("n", [1, 7, 8, 9, 4095, 1000003])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_flat_lengths_and_ragged_tail(n, dt):
    a, b = uni((n,), dt, seed=n), uni((n,), torch.float32, 0.5, 3.0, seed=n + 1)
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
    x = uni((rows, cols), torch.bfloat16, seed=1)
    bias = uni((cols,), torch.bfloat16, seed=2)
    sc = uni((rows, 1), torch.float32, 0.5, 2.0, seed=3)
    out = x.to(dev) + bias.to(dev)
    check_oracle(out, "add", x, bias, s0=1.0)
    out = x.to(dev) * sc.to(dev)
    check_oracle(out, "mul", x, sc)
    out = torch.where((x > 0).to(dev), x.to(dev), bias.to(dev))
    check_oracle(out, "where", x, bias, (x > 0).float())
    no_cpu_fallback("aten::add", "aten::mul", "aten::where")


def test_misaligned_views_take_the_element_path():
    x = uni((1, 4099), torch.bfloat16, seed=5)
    xd = x.to(dev)
    for off in (1, 3, 8):
        out = F.silu(xd[:, off:])
        check_oracle(out, "silu", x[:, off:])
        out = xd[:, off:] * xd[:, :4099 - off]
        check_oracle(out, "mul", x[:, off:], x[:, :4099 - off])


def test_eight_dimensional_broadcast_and_permuted_views():
    a = uni((2, 3, 2, 3, 2, 3, 2, 5), seed=1)
    b = uni((3, 1, 3, 1, 3, 1, 5), lo=0.5, hi=2.0, seed=2)
    out = torch.div(a.to(dev), b.to(dev))
    assert_cpu_close(out, a / b)
    check_oracle(out, "div", a, b)
    p = a.permute(7, 5, 3, 1, 0, 2, 4, 6)
    out = torch.sigmoid(a.to(dev).permute(7, 5, 3, 1, 0, 2, 4, 6))
    check_oracle(out, "sigmoid", p)
    no_cpu_fallback("aten::div", "aten::sigmoid")


def test_empty_and_one_element_tensors():
    e = torch.empty(0, 5, device=dev)
    assert (e + e).shape == (0, 5) and F.gelu(e).shape == (0, 5)
    one = uni((1,), seed=3)
    check_oracle(torch.exp(one.to(dev)), "exp", one)
    s = torch.tensor(0.75)
    out = torch.sigmoid(s.to(dev))
    assert out.dim() == 0
    check_oracle(out, "sigmoid", s)


def test_special_values():
    """NaN, infinities, signed zeros and subnormals against the oracle (PyTorch's CPU GELU returns NaN at
    +inf, where the formula and the oracle give +inf; finite entries are also checked against the CPU)."""
    x = torch.tensor([float("nan"), float("inf"), -float("inf"), 0.0, -0.0, 1e-40, -3.0, 100.0, -100.0, 20.0])
    for dt in FLOATS:
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
    x = uni((1024, 8192), torch.bfloat16, -6, 6, seed=21)
    g = uni((1024, 8192), torch.bfloat16, seed=22)
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
    a = uni((24, 16), seed=1)
    b = uni((16,), seed=2)
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
