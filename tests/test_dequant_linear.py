"""Fused int8 weight-only linear (dequant inside the GEMM) vs the oracle: y = x @ deq(q, scale)^T + bias,
with deq bit-identical to dequant_int8 (int8 [8192, 2048], per-output-channel scales,
M = 1024 / 4096 activations ~N(0, 1)).  GEMM tolerance of the reference (tests/test_mm.py:31-38)."""

import numpy as np
import pytest
import torch

import oracle
from vkutil import bits, f64, randn

pytestmark = pytest.mark.gpu

import torch_vulkan  # noqa: E402

dev = torch.device("vk")


def weights(N, K, seed, per_channel=True):
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    nb = (K + 63) // 64
    if per_channel:  # per-output-channel scale, expressed as nb identical block scales per row
        s = (torch.rand(N, 1, generator=g) * 0.019 + 0.001).to(torch.bfloat16).expand(N, nb).contiguous()
    else:
        s = (torch.rand(N, nb, generator=g) * 0.02 + 1e-4).to(torch.bfloat16)
    return q, s


def deq64(q, s, kind="bf16"):
    b = oracle.dequant_int8(q.numpy(), bits(s), kind)
    return oracle.bf16_to_f32(b).astype(np.float64) if kind == "bf16" else oracle.f16_to_f32(b).astype(np.float64)


def check(out, ref, K):
    o = f64(out)
    scale = max(float(np.abs(ref).max()), 1.0)
    assert float(np.abs(o - ref).max()) <= 1.2e-2 * scale * (1 + 0.01 * K ** 0.5)
    assert oracle.rel_l2(o, ref) <= 1e-2


@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (37, 200, 320), (256, 512, 2048), (1024, 8192, 2048)])
@pytest.mark.parametrize("bias", [False, True])
def test_dequant_linear_matches_oracle(M, N, K, bias):
    q, s = weights(N, K, M + N + K, per_channel=(M != 37))
    x = randn((M, K), torch.bfloat16, 3)
    b = randn((N,), torch.bfloat16, 4) if bias else None
    y = torch_vulkan.dequant_int8_linear(x.to(dev), q.to(dev), s.to(dev), None if b is None else b.to(dev))
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    ref = oracle.gemm(f64(x), deq64(q, s).T, None if b is None else f64(b), 1.0, 1.0 if bias else 0.0)
    check(y, ref, K)
    assert torch_vulkan.kernel_counts().get("torch_vulkan::dequant_int8_linear", 0) == 1


def test_dequant_linear_equals_dequant_then_mm():
    """Same values as the unfused path (dequant_int8 then x @ W^T through the matrix-core GEMM)."""
    q, s = weights(512, 1024, 9)
    x = randn((300, 1024), torch.bfloat16, 5)
    fused = torch_vulkan.dequant_int8_linear(x.to(dev), q.to(dev), s.to(dev))
    w = torch_vulkan.dequant_int8(q.to(dev), s.to(dev), torch.bfloat16)
    unfused = torch.mm(x.to(dev), w.t())
    assert oracle.rel_l2(f64(fused), f64(unfused)) < 1e-3


@pytest.mark.parametrize("M,N,K,per_channel,xt,bias", [(1024, 1024, 1088, False, False, True),
                                                       (1024, 8192, 2048, True, False, False),
                                                       (512, 1024, 512, False, True, True),
                                                       (2048, 8192, 1024, True, False, True)])
def test_fast_path_bit_identical_to_dequant_then_mm(M, N, K, per_channel, xt, bias):
    """Tile-aligned shapes take the direct-to-LDS GEMM with the dequant done in LDS (or, from M = 2048, a
    dequant pass into a workspace followed by the GEMM); the unfused dequant_int8 + mm accumulates every
    output element in the same order on the same dequantized weights, so the outputs must be bit-identical
    (per-block scales, 17 K steps, x given transposed, the workspace path)."""
    q, s = weights(N, K, 31 + K, per_channel)
    x = randn((K, M) if xt else (M, K), torch.bfloat16, 8)
    X = x.to(dev).t() if xt else x.to(dev)
    b = randn((N,), torch.bfloat16, 9).to(dev) if bias else None
    fused = torch_vulkan.dequant_int8_linear(X, q.to(dev), s.to(dev), b)
    w = torch_vulkan.dequant_int8(q.to(dev), s.to(dev), torch.bfloat16)
    unfused = torch.addmm(b, X, w.t()) if bias else torch.mm(X, w.t())
    assert torch.equal(fused.cpu(), unfused.cpu())
    rows = slice(0, 64)
    ref = oracle.gemm(f64(x.t() if xt else x)[rows], deq64(q, s).T, f64(b) if bias else None, 1.0, 1.0 if bias else 0.0)
    check(fused[rows], ref, K)


def test_dequant_linear_3d_input_and_f16():
    q, s = weights(128, 256, 11)
    x = randn((2, 5, 256), torch.float16, 6)
    y = torch_vulkan.dequant_int8_linear(x.to(dev), q.to(dev), s.to(dev))
    assert y.shape == (2, 5, 128) and y.dtype == torch.float16
    ref = oracle.gemm(f64(x).reshape(10, 256), deq64(q, s, "f16").T)
    o = f64(y).reshape(10, 128)
    assert oracle.rel_l2(o, ref) <= 4e-3


@pytest.mark.parametrize("M", [4096])
def test_baseline_m4096(M):
    q, s = weights(8192, 2048, 21)
    x = randn((M, 2048), torch.bfloat16, 7)
    y = torch_vulkan.dequant_int8_linear(x.to(dev), q.to(dev), s.to(dev))
    ref = oracle.gemm(f64(x), deq64(q, s).T)  # all 4096 rows (a float64 GEMM of ~2 s)
    check(y, ref, 2048)
    assert oracle.rel_l2(f64(y), ref) <= 1e-2
