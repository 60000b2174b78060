"""Weight-only int8 dequant on the GPU vs the oracle, bit-exact (reference tests/test_dequant_int8.py:1-121):
13 reference shapes x 3 output dtypes, the BASELINE [8192, 2048] shape, -128 / zero scale, non-contiguous
and offset views, the golden fixtures, and int8 tensor transfers/views/module moves."""

import os

import numpy as np
import pytest
import torch

import oracle
from vkutil import bits

pytestmark = pytest.mark.gpu

import torch_vulkan  # noqa: E402

dev = torch.device("vk")
OUT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "dequant_int8.npz")


def make(rows, cols, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-127, 128, (rows, cols), generator=g, dtype=torch.int8)
    nb = (cols + 63) // 64
    scale = (torch.rand(rows, nb, generator=g) * 0.02 + 1e-4).to(torch.bfloat16)
    return q, scale


def expect(q, scale, kind):
    return oracle.dequant_int8(q.contiguous().numpy(), bits(scale), kind)


@pytest.mark.parametrize("kind", list(OUT))
@pytest.mark.parametrize(
    "rows,cols",
    [(1, 64), (1, 36), (3, 100), (5, 4608), (2, 63), (7, 65), (4, 1), (1, 1), (320, 2880), (1280, 5120), (2048, 8192),
     (640, 1280), (33, 130), (8192, 2048)],
)
def test_dequant_matches_oracle_bitwise(kind, rows, cols):
    q, scale = make(rows, cols, seed=rows * 1000 + cols)
    ve = torch_vulkan.validation_errors()
    out = torch_vulkan.dequant_int8(q.to(dev), scale.to(dev), OUT[kind])
    assert out.device.type == "vk" and out.dtype == OUT[kind] and out.shape == (rows, cols)
    assert np.array_equal(bits(out), expect(q, scale, kind)), f"{kind} {rows}x{cols}"
    assert torch_vulkan.fallback_counts() == {}, torch_vulkan.fallback_counts()
    assert torch_vulkan.kernel_counts().get("torch_vulkan::dequant_int8", 0) >= 1
    assert torch_vulkan.validation_errors() == ve


@pytest.mark.parametrize("kind", list(OUT))
def test_dequant_golden_fixtures(kind):
    d = np.load(GOLD)
    keys = sorted({k.rsplit("_q", 1)[0] for k in d.files if k.endswith("_q")})
    for key in keys:
        q = torch.from_numpy(d[key + "_q"].copy())
        s = torch.from_numpy(d[key + "_scale"].view(np.int16).copy()).view(torch.bfloat16)
        out = torch_vulkan.dequant_int8(q.to(dev), s.to(dev), OUT[kind])
        assert np.array_equal(bits(out), d[key + "_out_" + kind]), key


def test_dequant_extreme_values_and_zero_scale():
    q = torch.tensor([[-128, -127, 0, 1, 127] * 13], dtype=torch.int8)
    scale = torch.tensor([[0.5, 0.0]], dtype=torch.bfloat16)
    for kind, dt in OUT.items():
        assert np.array_equal(bits(torch_vulkan.dequant_int8(q.to(dev), scale.to(dev), dt)), expect(q, scale, kind))


@pytest.mark.parametrize("cols", [2048, 64, 1040])
def test_dequant_nonfinite_subnormal_and_overflowing_scales(cols):
    """Scales of +-inf, NaN, bf16 subnormals and values whose product with an int8 overflows to inf, each
    on its own 64-column block: the bf16 output rounds every non-NaN product to nearest even (subnormals
    included, never flushed), gives 0x7FC0 for every NaN (0 * inf, NaN * q) and keeps +-inf; f16 / f32 as
    the oracle.  2048 columns take the row-per-wavefront path of the 16-bit kernel, 64 and 1040 the
    per-lane one."""
    rows, nb = 6, (cols + 63) // 64
    g = torch.Generator().manual_seed(cols)
    q = torch.randint(-128, 128, (rows, cols), generator=g, dtype=torch.int8)
    q[:, ::7] = 0  # zero times inf is NaN
    special = np.array([0x7F80, 0xFF80, 0x7FC1, 0xFFC0, 0x0001, 0x8003, 0x007F, 0x7F7F, 0xFF7F, 0x0080, 0x3F80],
                       dtype=np.uint16)
    sb = special[np.arange(rows * nb) % len(special)].reshape(rows, nb)
    scale = torch.from_numpy(sb.view(np.int16).copy()).view(torch.bfloat16)
    for kind, dt in OUT.items():
        out = torch_vulkan.dequant_int8(q.to(dev), scale.to(dev), dt)
        with np.errstate(invalid="ignore", over="ignore"):  # 0 * inf and the overflowing products
            ref = oracle.dequant_int8(q.numpy(), sb, kind)
        assert np.array_equal(bits(out), ref), f"{kind} {cols}"


def test_dequant_noncontiguous_inputs_are_made_contiguous():
    q, scale = make(8, 200, 3)
    sub = q.to(dev)[:, :128]
    sc = scale[:, :2]
    out = torch_vulkan.dequant_int8(sub, sc.to(dev), torch.bfloat16)
    assert np.array_equal(bits(out), expect(q[:, :128], sc, "bf16"))


def test_dequant_view_with_storage_offset():
    q, scale = make(9, 64, 5)
    out = torch_vulkan.dequant_int8(q.to(dev)[1:8], scale[1:8].contiguous().to(dev), torch.float32)
    assert np.array_equal(bits(out), expect(q[1:8], scale[1:8], "f32"))
    odd = torch.arange(3 * 64 + 1, dtype=torch.int64).to(torch.int8)[1:].view(3, 64)  # starts one byte in
    sc = (torch.rand(3, 1) + 0.1).to(torch.bfloat16)
    got = torch_vulkan.dequant_int8(odd.to(dev), sc.to(dev), torch.bfloat16)
    assert np.array_equal(bits(got), expect(odd, sc, "bf16"))
    dodd = torch.arange(3 * 64 + 1, dtype=torch.int64).to(torch.int8).to(dev)[1:].view(3, 64)  # device view, offset 1
    got2 = torch_vulkan.dequant_int8(dodd, sc.to(dev), torch.float16)
    assert np.array_equal(bits(got2), expect(odd, sc, "f16"))


def test_int8_tensor_roundtrip_and_views():
    q = torch.randint(-128, 128, (5, 100), dtype=torch.int8)
    qd = q.to(dev)
    assert qd.dtype == torch.int8 and qd.device.type == "vk"
    assert torch.equal(qd.cpu(), q)
    assert torch.equal(qd.clone().cpu(), q)
    assert torch.equal(qd.view(10, 50).cpu(), q.view(10, 50))
    assert torch.equal(qd.reshape(-1).cpu(), q.reshape(-1))
    assert torch.equal(qd[2].cpu(), q[2])
    assert torch.equal(qd[1:4, 10:50].cpu(), q[1:4, 10:50])
    assert torch.equal(qd[:, 10:50].contiguous().cpu(), q[:, 10:50])
    assert torch.equal(qd.t().contiguous().cpu(), q.t().contiguous())
    assert torch.equal(torch.empty_like(q, device=dev).copy_(q).cpu(), q)
    assert qd.to(dev) is qd


def test_int8_buffers_move_with_module():
    m = torch.nn.Module()
    q = torch.randint(-128, 128, (4, 128), dtype=torch.int8)
    scale = (torch.rand(4, 2) + 0.1).to(torch.bfloat16)
    m.register_buffer("q", q.clone())
    m.register_buffer("scale", scale.clone())
    m.to(dev)
    assert m.q.device.type == "vk" and m.scale.device.type == "vk"
    assert np.array_equal(bits(torch_vulkan.dequant_int8(m.q, m.scale, torch.bfloat16)), expect(q, scale, "bf16"))
    m.to("cpu")
    assert m.q.device.type == "cpu" and torch.equal(m.q, q) and torch.equal(m.scale, scale)


def test_int8_pinned_host_to_device_like_block_swap():
    q = torch.randint(-128, 128, (16, 256), dtype=torch.int8)
    host = q.pin_memory()
    buf = torch.empty_like(q, device=dev)
    buf.copy_(host, non_blocking=True)
    assert torch.equal(buf.cpu(), q)
