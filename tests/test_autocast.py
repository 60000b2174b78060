"""torch.autocast(device_type="vk") with the policy the shim registers (the reference's
csrc/shim.cpp:376-394, exercised by its tests/probe_m1.py:143-156): products and attention run in the
autocast dtype, layer_norm and softmax in fp32, and enabled=False leaves dtypes alone.  Values against
float64 CPU references of the same (cast) inputs."""

import pytest
import torch
import torch.nn.functional as F

import oracle
from vkutil import f64, randn

pytestmark = pytest.mark.gpu

import torch_vulkan  # noqa: E402

dev = torch.device("vk")


def test_linear_and_matmul_run_in_bf16():
    lin = torch.nn.Linear(64, 48).to(dev)
    x = randn((8, 64), torch.float32, 1).to(dev)
    with torch.autocast(device_type="vk", dtype=torch.bfloat16):
        y = lin(x)
        z = torch.mm(x, x.t())
    assert y.dtype == torch.bfloat16 and z.dtype == torch.bfloat16
    xb, wb, bb = (t.detach().to(torch.bfloat16).cpu() for t in (x, lin.weight, lin.bias))
    ref = oracle.gemm(f64(xb), f64(wb).T, f64(bb), 1.0, 1.0)
    assert oracle.rel_l2(f64(y), ref) <= 1e-2
    assert oracle.rel_l2(f64(z), f64(xb) @ f64(xb).T) <= 1e-2
    kc = torch_vulkan.kernel_counts()
    assert kc.get("aten::addmm", 0) >= 1 and kc.get("aten::mm", 0) >= 1, kc


def test_attention_in_bf16_norms_and_softmax_in_fp32():
    q, k, v = (randn((1, 2, 64, 64), torch.float32, s).to(dev) for s in (2, 3, 4))
    xl = randn((16, 96), torch.bfloat16, 5).to(dev)
    w, b = torch.ones(96, device=dev), torch.zeros(96, device=dev)
    with torch.autocast(device_type="vk", dtype=torch.bfloat16):
        o = F.scaled_dot_product_attention(q, k, v)
        ln = F.layer_norm(xl, (96,), w, b)
        sm = torch.softmax(xl, dim=-1)
    assert o.dtype == torch.bfloat16 and ln.dtype == torch.float32 and sm.dtype == torch.float32
    qa, ka, va = (f64(t.to(torch.bfloat16)) for t in (q, k, v))
    ref, _ = oracle.attention_fwd(qa, ka, va, 64 ** -0.5)
    assert oracle.rel_l2(f64(o), ref) <= 1e-2
    x64 = f64(xl)
    mu, var = x64.mean(-1, keepdims=True), x64.var(-1, keepdims=True)
    assert oracle.rel_l2(f64(ln), (x64 - mu) / (var + 1e-5) ** 0.5) <= 1e-5
    e = (x64 - x64.max(-1, keepdims=True)).__array__()
    import numpy as np
    ref_sm = np.exp(e) / np.exp(e).sum(-1, keepdims=True)
    assert oracle.rel_l2(f64(sm), ref_sm) <= 1e-5
    assert torch_vulkan.kernel_counts().get("aten::_scaled_dot_product_fused_attention_overrideable", 0) >= 1


def test_disabled_autocast_keeps_dtypes():
    x = randn((4, 4), torch.float32, 6).to(dev)
    with torch.autocast(device_type="vk", dtype=torch.bfloat16, enabled=False):
        y = torch.mm(x, x) * 2
    assert y.dtype == torch.float32
    assert oracle.rel_l2(f64(y), 2 * f64(x) @ f64(x)) <= 1e-5


def test_autocast_backward_gives_fp32_gradients_of_fp32_leaves():
    lin = torch.nn.Linear(32, 16).to(dev)
    x = randn((8, 32), torch.float32, 7).to(dev).requires_grad_(True)
    with torch.autocast(device_type="vk", dtype=torch.bfloat16):
        loss = lin(x).float().pow(2).sum()
    loss.backward()
    assert x.grad.dtype == torch.float32 and lin.weight.grad.dtype == torch.float32
    assert torch.isfinite(x.grad.cpu()).all() and torch.isfinite(lin.weight.grad.cpu()).all()
