"""DiT-block linear stack with rank-16 LoRA, bf16 forward + backward through torch autograd on the vk device
(M = 1024 tokens; QKV 2048->6144, out-proj 2048->2048, MLP 2048->8192->2048, addmm with
bias; LoRA A ~N(0, 0.02), B zero-initialised then ~N(0, 0.01); weights ~N(0, 0.02); frozen base weights,
trainable LoRA factors and input).  Every product runs through the vk mm / addmm registrations (the
reference's csrc/ops_mm.cpp:61-175 path, as sd-scripts LoRA training drives it); the oracle recomputes the
layer in float64 from the same bf16 inputs, with h = x A^T rounded to bf16 as the device stores it.
Tolerance: bf16 rel-L2 <= 1e-2."""

import numpy as np
import pytest
import torch

import oracle
from vkutil import f64, randn

pytestmark = pytest.mark.gpu

import torch_vulkan  # noqa: E402,F401

dev = torch.device("vk")
bf = torch.bfloat16
RANK = 16
LAYERS = [("qkv", 2048, 6144), ("out_proj", 2048, 2048), ("mlp_up", 2048, 8192), ("mlp_down", 8192, 2048)]


def rb(x):
    """Round a float64 array to bf16 values (as float64), like a bf16 store on the device."""
    return oracle.bf16_to_f32(oracle.round_bf16(x.astype(np.float32))).astype(np.float64)


def rel(got, ref):
    return oracle.rel_l2(f64(got), ref)


@pytest.mark.parametrize("name,fin,fout", LAYERS)
def test_linear_with_lora_forward_backward(name, fin, fout):
    M = 1024
    seed = fin + fout
    x = randn((M, fin), bf, seed)
    W = randn((fout, fin), bf, seed + 1, 0.02)
    b = randn((fout,), bf, seed + 2, 0.02)
    A = randn((RANK, fin), bf, seed + 3, 0.02)
    B = randn((fout, RANK), bf, seed + 4, 0.01)
    g = randn((M, fout), bf, seed + 5)

    xd = x.to(dev).requires_grad_(True)
    Ad = A.to(dev).requires_grad_(True)
    Bd = B.to(dev).requires_grad_(True)
    h = torch.nn.functional.linear(xd, Ad)
    y = torch.nn.functional.linear(xd, W.to(dev), b.to(dev)) + torch.nn.functional.linear(h, Bd)
    y.backward(g.to(dev))

    x64, W64, b64, A64, B64, g64 = (f64(t) for t in (x, W, b, A, B, g))
    h64 = rb(x64 @ A64.T)
    y_ref = rb(oracle.gemm(x64, W64.T, b64, 1.0, 1.0)) + rb(h64 @ B64.T)  # every row of y and dx is checked
    assert rel(y, y_ref) <= 1e-2

    dh = rb(g64 @ B64)                 # dL/dh
    dB_ref = g64.T @ h64               # [fout, 16]
    dA_ref = dh.T @ x64                # [16, fin]
    dx_ref = g64 @ W64 + dh @ A64
    assert rel(Bd.grad, dB_ref) <= 1e-2
    assert rel(Ad.grad, dA_ref) <= 1e-2
    assert rel(xd.grad, dx_ref) <= 1e-2
    assert "aten::mm" not in torch_vulkan.fallback_counts()


def test_first_pass_with_zero_lora_b():
    """BASELINE config 4's first pass: B is zero-initialised, so the LoRA branch adds exactly 0 (the output
    equals the base linear bit for bit) and dA = (g B)^T x is exactly 0, while dB = g^T h is not."""
    M, fin, fout = 1024, 2048, 2048
    x = randn((M, fin), bf, 61)
    W = randn((fout, fin), bf, 62, 0.02)
    b = randn((fout,), bf, 63, 0.02)
    A = randn((RANK, fin), bf, 64, 0.02)
    g = randn((M, fout), bf, 65)
    xd = x.to(dev)
    Ad = A.to(dev).requires_grad_(True)
    Bd = torch.zeros((fout, RANK), dtype=bf, device=dev).requires_grad_(True)
    h = torch.nn.functional.linear(xd, Ad)
    base = torch.nn.functional.linear(xd, W.to(dev), b.to(dev))
    y = base + torch.nn.functional.linear(h, Bd)
    y.backward(g.to(dev))
    assert torch.equal(y.detach().cpu(), base.cpu())
    assert not Ad.grad.cpu().any()
    x64, A64, g64 = f64(x), f64(A), f64(g)
    assert rel(Bd.grad, g64.T @ rb(x64 @ A64.T)) <= 1e-2
