"""Writes the committed golden fixtures of tests/golden/ (run: python tests/golden/make_golden.py).

The reference keeps no stored vectors: its tests regenerate inputs from torch.Generator seeds
(tests/test_dequant_int8.py:24-29) and compare against its pure-PyTorch closed form
(torch_vulkan/__init__.py:203-205) or against torch's own `.to()` rounding.  These fixtures freeze such
inputs and the closed-form outputs computed with torch's CPU kernels (not with oracle/), so that the
oracle is checked against an independent implementation and against torch-version drift of the
random generators.

  dequant_int8.npz  per case: q (int8), scale (bf16 bits), out_{f32,bf16,f16} (bit patterns)
  rounding.npz      x (float32 specials, halfway cases, subnormals) and torch's bf16 / f16 bit patterns
"""

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def make_dq(rows, cols, seed):
    """The inputs the reference's tests/test_dequant_int8.py:24-29 draws for a shape and seed (the same
    generator calls in the same order, so the same values)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-127, 128, (rows, cols), generator=g, dtype=torch.int8)
    nb = (cols + 63) // 64
    scale = (torch.rand(rows, nb, generator=g) * 0.02 + 1e-4).to(torch.bfloat16)
    return q, scale


def closed_form(q, scale, dt):
    """The closed form of torch_vulkan/__init__.py:203-205 (one float32 product per element, rounded once to
    dt), executed by torch's CPU kernels: the row is padded to whole 64-element blocks, each block times its
    scale."""
    rows, cols = q.shape
    nb = scale.shape[1]
    blocks = torch.zeros(rows, nb * 64)
    blocks[:, :cols] = q.float()
    prod = blocks.view(rows, nb, 64) * scale.float().unsqueeze(-1)
    return prod.view(rows, nb * 64)[:, :cols].to(dt)


def bits(t):
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.view(torch.int16).numpy().view(np.uint16)


def dequant_fixtures():
    cases = {}
    shapes = [(1, 64), (1, 36), (3, 100), (2, 63), (7, 65), (4, 1), (1, 1), (33, 130), (3, 640)]
    for rows, cols in shapes:
        q, scale = make_dq(rows, cols, seed=rows * 1000 + cols)
        key = f"r{rows}_c{cols}"
        cases[key + "_q"] = q.numpy()
        cases[key + "_scale"] = bits(scale)
        for name, dt in (("f32", torch.float32), ("bf16", torch.bfloat16), ("f16", torch.float16)):
            cases[key + "_out_" + name] = bits(closed_form(q, scale, dt))
    # extreme values and a zero scale (reference tests/test_dequant_int8.py:51-55)
    q = torch.tensor([[-128, -127, 0, 1, 127] * 13], dtype=torch.int8)
    scale = torch.tensor([[0.5, 0.0]], dtype=torch.bfloat16)
    cases["extreme_q"] = q.numpy()
    cases["extreme_scale"] = bits(scale)
    for name, dt in (("f32", torch.float32), ("bf16", torch.bfloat16), ("f16", torch.float16)):
        cases["extreme_out_" + name] = bits(closed_form(q, scale, dt))
    np.savez_compressed(os.path.join(HERE, "dequant_int8.npz"), **cases)


def rounding_fixtures():
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65520.0, 65519.99, 1e-8, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 3.4e38, -3.4e38,
            float("inf"), float("-inf"), 1.0 / 3.0, 1e-40, -1e-45]
    x = np.array(vals, dtype=np.float32)
    # bf16 halfway cases: low 16 bits exactly 0x8000 with even / odd kept part, and neighbours
    base = np.array([0x3F800000, 0x3F810000, 0x40490000, 0x00010000, 0x7F7F0000], dtype=np.uint32)
    half = np.concatenate([base | 0x8000, base | 0x7FFF, base | 0x8001]).view(np.float32)
    # f16 halfway cases in the normal and subnormal ranges
    f16h = np.array([1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 2.0 ** -15 + 2.0 ** -25, 2.0 ** -20 * 1.5, 2.0 ** -24 * 0.5,
                     2.0 ** -24 * 1.5, 2048.0 + 1.0, 2048.0 + 3.0], dtype=np.float32)
    rng = np.random.default_rng(7)
    rand = np.concatenate([rng.standard_normal(2000).astype(np.float32) * 10.0 ** rng.integers(-8, 6, 2000)]).astype(np.float32)
    x = np.concatenate([x, half, f16h, rand]).astype(np.float32)
    t = torch.from_numpy(x.copy())
    np.savez_compressed(os.path.join(HERE, "rounding.npz"), x=x, bf16=bits(t.to(torch.bfloat16)), f16=bits(t.to(torch.float16)))


if __name__ == "__main__":
    dequant_fixtures()
    rounding_fixtures()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
