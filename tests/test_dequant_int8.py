"""Weight-only int8 dequant on the GPU against the oracle, bit for bit.

The reference's tests/test_dequant_int8.py fixes the behaviours: bit-exact results for every output dtype
over shapes with partial 64-column blocks, extreme int8 values and a zero scale, non-contiguous and offset
inputs, and int8 tensors that transfer, view and move with modules like any other.  Here: a shape table
up to the BASELINE [8192, 2048], the committed golden fixtures (the reference tests' own inputs and
closed-form outputs), all 256 int8 values under special scales, non-finite and subnormal scales, windows and
unaligned views, and the int8 operations block swapping uses."""

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


def int8_weights(rows, cols, seed=0):
    """int8 weights over the full range (-128 included) and one bf16 scale per 64-column block, spread
    log-uniformly over [1e-4, 2e-2]."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-128, 128, (rows, cols), generator=g, dtype=torch.int8)
    nb = -(-cols // 64)
    scale = torch.exp(torch.empty(rows, nb).uniform_(np.log(1e-4), np.log(2e-2), generator=g)).to(torch.bfloat16)
    return q, scale


def expect(q, scale, kind):
    return oracle.dequant_int8(q.contiguous().numpy(), bits(scale.contiguous()), kind)


# (rows, cols): one element, partial / whole / several 64-column blocks, ragged last blocks, the reference's
# larger weight shapes, and the BASELINE [8192, 2048]
DQ_SHAPES = [(1, 1), (1, 40), (1, 64), (2, 63), (3, 65), (4, 130), (6, 1), (5, 4608), (33, 100), (300, 2880),
             (640, 1280), (1024, 5120), (2048, 8192), (8192, 2048)]


@pytest.mark.parametrize("rows,cols", DQ_SHAPES)
@pytest.mark.parametrize("kind", list(OUT))
def test_dequant_bits_match_the_oracle(kind, rows, cols):
    q, scale = int8_weights(rows, cols, seed=7 * rows + cols)
    ve = torch_vulkan.validation_errors()
    out = torch_vulkan.dequant_int8(q.to(dev), scale.to(dev), OUT[kind])
    assert out.device.type == "vk" and out.dtype == OUT[kind] and tuple(out.shape) == (rows, cols)
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


def test_every_int8_value_against_zero_negative_and_tiny_scales():
    """All 256 int8 values in each 64-column block, under scales 0.5, 0, -3 and the smallest normal bf16."""
    q = torch.arange(-128, 128, dtype=torch.int16).to(torch.int8).repeat(2, 1)  # [2, 256]: 4 blocks a row
    sbits = np.array([[0x3F00, 0x0000, 0xC040, 0x0080], [0x8000, 0x3F80, 0x0080, 0xBF00]], dtype=np.uint16)
    scale = torch.from_numpy(sbits.view(np.int16).copy()).view(torch.bfloat16)
    for kind, dt in OUT.items():
        assert np.array_equal(bits(torch_vulkan.dequant_int8(q.to(dev), scale.to(dev), dt)), expect(q, scale, kind)), kind


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


def test_dequant_of_windows_and_unaligned_views():
    """A column window (not contiguous), a row window (a storage offset) and int8 data starting one byte
    past an allocation's start, on the host and on the device side."""
    q, scale = int8_weights(9, 200, 3)
    qd = q.to(dev)
    cases = [(qd[:, :128], q[:, :128], scale[:, :2], "bf16"), (qd[1:8, :64], q[1:8, :64], scale[1:8, :1], "f32")]
    flat = torch.randint(-128, 128, (3 * 64 + 1,), generator=torch.Generator().manual_seed(4), dtype=torch.int8)
    sc = int8_weights(3, 64, 5)[1]
    cases += [(flat[1:].view(3, 64).to(dev), flat[1:].view(3, 64), sc, "bf16"),
              (flat.to(dev)[1:].view(3, 64), flat[1:].view(3, 64), sc, "f16")]
    for qv, qh, s_, kind in cases:
        out = torch_vulkan.dequant_int8(qv, s_.to(dev), OUT[kind])
        assert np.array_equal(bits(out), expect(qh, s_, kind)), (tuple(qv.shape), kind)


# ---- int8 tensors on the device: the operations weight storage and block swapping use ----------------------
INT8_VIEWS = {
    "whole": lambda t: t, "clone": lambda t: t.clone(), "view": lambda t: t.view(10, 50),
    "flatten": lambda t: t.reshape(-1), "row": lambda t: t[2], "window": lambda t: t[1:4, 10:50],
    "window made contiguous": lambda t: t[:, 10:50].contiguous(), "transposed copy": lambda t: t.t().contiguous(),
}


@pytest.mark.parametrize("name", list(INT8_VIEWS))
def test_int8_tensor_views_read_back(name):
    q = torch.randint(-128, 128, (5, 100), generator=torch.Generator().manual_seed(6), dtype=torch.int8)
    qd = q.to(dev)
    assert qd.dtype == torch.int8 and qd.device.type == "vk" and qd.to(dev) is qd
    assert torch.equal(INT8_VIEWS[name](qd).cpu(), INT8_VIEWS[name](q))


def test_int8_weights_travel_with_their_module_and_parameters():
    q, scale = int8_weights(4, 128, 8)
    m = torch.nn.Module()
    m.register_buffer("q", q.clone())
    m.register_buffer("scale", scale.clone())
    m.frozen = torch.nn.Parameter(q[:, :64].clone(), requires_grad=False)
    m.to(dev)
    assert {t.device.type for t in (m.q, m.scale, m.frozen)} == {"vk"}
    assert np.array_equal(bits(torch_vulkan.dequant_int8(m.q, m.scale, torch.bfloat16)), expect(q, scale, "bf16"))
    m.to("cpu")
    assert torch.equal(m.q, q) and torch.equal(m.scale, scale) and torch.equal(m.frozen.data, q[:, :64])


def test_int8_upload_from_pinned_host_memory():
    """Block swapping's transfer: a pinned host original copied into a device buffer without blocking."""
    q = torch.randint(-128, 128, (16, 256), generator=torch.Generator().manual_seed(9), dtype=torch.int8)
    buf = torch.empty(q.shape, dtype=torch.int8, device=dev)
    buf.copy_(q.pin_memory(), non_blocking=True)
    assert torch.equal(buf.cpu(), q)
