"""A DiT block with LoRA through the PyTorch operator API on the vk device, forward and backward, against
the same block in float64 on the CPU.  The reference checks this end to end with a scaled-down Anima from
sd-scripts (tests/anima_on_vk.py:25-102: head_dim 128, AdaLN modulation, LoRA); sd-scripts is not in this
image, so the block is written out: AdaLN shift / scale / gate from a conditioning vector, LayerNorm without
affine parameters, fused attention at head_dim 128 ([B, T, H, D] projections viewed as [B, H, T, D]), a tanh-GELU
MLP, and rank-16 LoRA on the four linears (frozen base weights).  Tolerance: rel-L2 <= 1e-2 for the output
and <= 2e-2 for the gradients: every intermediate is stored in bf16 (2^-9 relative), through two norms,
attention and eight products."""

import pytest
import torch
import torch.nn.functional as F

import oracle
from vkutil import f64

pytestmark = pytest.mark.gpu

import torch_vulkan  # noqa: E402

dev = torch.device("vk")
C, HEADS, T, RANK = 512, 4, 256, 16


def make_params(seed=0):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s, sc=0.02: (torch.randn(*s, generator=g) * sc).to(torch.bfloat16)  # noqa: E731
    P = {"ada_w": r(6 * C, C), "ada_b": r(6 * C)}
    for name, fin, fout in (("qkv", C, 3 * C), ("proj", C, C), ("fc1", C, 4 * C), ("fc2", 4 * C, C)):
        P[name + "_w"], P[name + "_b"] = r(fout, fin), r(fout)
        P[name + "_A"], P[name + "_B"] = r(RANK, fin), r(fout, RANK, sc=0.01)
    return P


def lora_linear(x, P, name):
    return F.linear(x, P[name + "_w"], P[name + "_b"]) + F.linear(F.linear(x, P[name + "_A"]), P[name + "_B"])


def block(x, c, P):
    """x [B, T, C], c [B, C]"""
    B = x.shape[0]
    shift1, scale1, gate1, shift2, scale2, gate2 = F.linear(F.silu(c), P["ada_w"], P["ada_b"]).unsqueeze(1).chunk(6, dim=-1)
    h = F.layer_norm(x, (C,), eps=1e-6) * (1 + scale1) + shift1
    q, k, v = lora_linear(h, P, "qkv").view(B, T, 3, HEADS, C // HEADS).unbind(2)
    a = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
    x = x + gate1 * lora_linear(a.transpose(1, 2).reshape(B, T, C), P, "proj")
    h = F.layer_norm(x, (C,), eps=1e-6) * (1 + scale2) + shift2
    return x + gate2 * lora_linear(F.gelu(lora_linear(h, P, "fc1"), approximate="tanh"), P, "fc2")


def run(P, x, c, g, device, dtype):
    Q = {k: v.to(device=device, dtype=dtype).requires_grad_(k.endswith(("_A", "_B"))) for k, v in P.items()}
    xd = x.to(device=device, dtype=dtype).requires_grad_(True)
    y = block(xd, c.to(device=device, dtype=dtype), Q)
    y.backward(g.to(device=device, dtype=dtype))
    grads = {k: v.grad for k, v in Q.items() if v.grad is not None}
    grads["x"] = xd.grad
    return y.detach(), grads


def test_dit_block_forward_backward_matches_float64():
    P = make_params()
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(1, T, C, generator=gen).to(torch.bfloat16)
    c = torch.randn(1, C, generator=gen).to(torch.bfloat16)
    g = torch.randn(1, T, C, generator=gen).to(torch.bfloat16)
    y, grads = run(P, x, c, g, dev, torch.bfloat16)
    y64, grads64 = run(P, x, c, g, "cpu", torch.float64)
    e = oracle.rel_l2(f64(y), y64.numpy())
    print("block output rel-L2", e)
    assert e <= 1e-2
    assert set(grads) == set(grads64) and len(grads) == 9  # x and the A, B factors of the four linears
    for k in grads:
        e = oracle.rel_l2(f64(grads[k]), grads64[k].numpy())
        print(f"grad {k} rel-L2 {e:.2e}")
        assert e <= 2e-2, (k, e)
    kc, fb = torch_vulkan.kernel_counts(), torch_vulkan.fallback_counts()
    for op in ("aten::_scaled_dot_product_fused_attention_overrideable",
               "aten::_scaled_dot_product_fused_attention_overrideable_backward", "aten::native_layer_norm",
               "aten::native_layer_norm_backward", "aten::addmm", "aten::mm"):
        assert kc.get(op, 0) >= 1, (op, kc)
    hot = ("mm", "addmm", "bmm", "_softmax", "native_layer_norm", "scaled_dot_product", "gelu", "silu")
    assert not [n for n in fb if any(h in n for h in hot)], fb
