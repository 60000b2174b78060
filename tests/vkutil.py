"""Shared helpers of the GPU parity tests: seeded inputs (the reference tests' generators), conversion to
the oracle's numpy float64, and the reference's tolerance rules."""

import numpy as np
import torch


def randn(shape, dtype, seed=0, scale=1.0):
    """tests/test_mm.py:26-28 and tests/test_rows.py:24-26 of the reference."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def uniform(shape, dtype=torch.float32, seed=0, scale=1.0):
    """tests/test_fused_attention.py:43-45 of the reference: uniform[-1, 1) * scale."""
    g = torch.Generator().manual_seed(seed)
    return ((torch.rand(shape, generator=g) * 2 - 1) * scale).to(dtype)


def f64(t):
    """Exact float64 numpy copy of a (rounded) CPU or vk tensor."""
    return t.detach().cpu().double().numpy()


def bits(t):
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.view(torch.int16).numpy().view(np.uint16)


def max_abs_close(out, ref64, tol, mult=1.0):
    """Reference rule (tests/test_rows.py:29-34): max|out - ref| <= tol * max(|ref|max, 1) * mult."""
    o = f64(out)
    assert o.shape == ref64.shape, (o.shape, ref64.shape)
    scale = max(float(np.abs(ref64).max()) if ref64.size else 0.0, 1.0)
    err = float(np.abs(o - ref64).max()) if o.size else 0.0
    assert err <= tol * scale * mult, f"max err {err} > {tol * scale * mult} (scale {scale})"


def rel_l2(got, ref64):
    g = f64(got) if isinstance(got, torch.Tensor) else np.asarray(got, dtype=np.float64)
    return float(np.linalg.norm(g - ref64) / (np.linalg.norm(ref64) + 1e-300))
