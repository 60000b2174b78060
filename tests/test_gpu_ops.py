"""Transfers, views and device copies across the vk boundary.  The reference's tests/test_gpu_ops.py:27-89
fix what its device must do here (round trips of every dtype, host <-> device copies with dtype conversion
and broadcast, non-contiguous sources and destinations, storage offsets, device-side copies and casts, empty
tensors, a large transfer whose memory is released, resize_); these tests check the same behaviours as a
matrix of dtypes x layouts x directions, every result bit for bit against the same operation on the CPU."""

import pytest
import torch

pytestmark = pytest.mark.gpu

import torch_vulkan  # noqa: E402

dev = torch.device("vk")
DTYPES = [torch.float32, torch.float16, torch.bfloat16, torch.int64, torch.int32, torch.int8, torch.uint8, torch.bool]


def sample(dtype, shape, seed):
    """Deterministic values of `dtype` with both signs (where the dtype has them), zeros and, for floats,
    values that do not fit the narrower float types."""
    g = torch.Generator().manual_seed(seed)
    if dtype == torch.bool:
        return torch.rand(shape, generator=g) < 0.5
    if dtype.is_floating_point:
        return ((torch.randn(shape, generator=g) * 3.0).exp() * torch.randn(shape, generator=g).sign()).to(dtype)
    lo, hi = (0, 256) if dtype == torch.uint8 else (-128, 128) if dtype == torch.int8 else (-1000, 1000)
    return torch.randint(lo, hi, shape, generator=g, dtype=torch.int64).to(dtype)


def same_bits(got, ref):
    """Equal shape, dtype and bits (so -0.0, NaN payloads and rounding all count)."""
    assert got.shape == ref.shape and got.dtype == ref.dtype, (got.shape, ref.shape, got.dtype, ref.dtype)
    got, ref = got.contiguous(), ref.contiguous()
    if got.dtype.is_floating_point:
        as_int = {8: torch.int64, 4: torch.int32, 2: torch.int16}[got.element_size()]
        got, ref = got.view(as_int), ref.view(as_int)
    assert torch.equal(got, ref)


# How a [6, 10] tensor is viewed before it crosses the boundary: contiguous, transposed, a strided window,
# a flat window at a storage offset, a broadcast row.
LAYOUTS = {
    "contiguous": lambda t: t,
    "transposed": lambda t: t.t(),
    "strided window": lambda t: t[1::2, 2::3],
    "storage offset": lambda t: t.reshape(-1)[7:41],
    "broadcast row": lambda t: t[2:3].expand(4, 10),
}


def test_runs_on_an_mi355x():
    assert "gfx950" in torch_vulkan.device_name()


@pytest.mark.parametrize("layout", list(LAYOUTS))
@pytest.mark.parametrize("dtype", DTYPES)
def test_views_cross_the_boundary_both_ways(dtype, layout):
    host = sample(dtype, (6, 10), seed=DTYPES.index(dtype))
    view = LAYOUTS[layout](host)
    same_bits(view.to(dev).cpu(), view)                   # host view -> device -> host
    same_bits(LAYOUTS[layout](host.to(dev)).cpu(), view)  # the same view taken on the device, read back
    same_bits(LAYOUTS[layout](host.to(dev)).clone().cpu(), view)  # device -> device copy of the view


@pytest.mark.parametrize("src,dst", [(torch.float32, torch.float32), (torch.float32, torch.bfloat16),
                                     (torch.float16, torch.float32), (torch.int64, torch.float32),
                                     (torch.float32, torch.int32), (torch.uint8, torch.int64)])
def test_copy_into_a_device_tensor_converts_and_broadcasts(src, dst):
    row = sample(src, (5,), seed=11)
    ref = torch.zeros(3, 5, dtype=dst).copy_(row)
    got = torch.zeros(3, 5, dtype=dst, device=dev)
    got.copy_(row)                   # host row, broadcast over the device rows, converted on the way
    same_bits(got.cpu(), ref)
    got2 = torch.zeros(3, 5, dtype=dst, device=dev)
    got2.copy_(row.to(dev))          # the same from a device row
    same_bits(got2.cpu(), ref)
    same_bits(row.to(dev).to(dst).cpu(), row.to(dst))  # a device-side cast


def test_writes_through_device_views_land_where_the_cpu_puts_them():
    host = sample(torch.float32, (8, 12), seed=3)
    ref, d = host.clone(), host.to(dev)
    ops = [
        lambda t: t[2:5].fill_(-1.5),                                       # rows at a storage offset
        lambda t: t[:, 3].copy_(torch.arange(8, dtype=torch.float32)),      # a strided column, host source
        lambda t: t.t()[1:4].copy_(sample(torch.float32, (3, 8), seed=4)),  # transposed destination
        lambda t: t.reshape(-1)[50:70].copy_(torch.linspace(0, 1, 20)),     # flat window
    ]
    for op in ops:
        op(ref)
        op(d)
        same_bits(d.cpu(), ref)


def test_device_copies_casts_and_fills_run_on_the_device():
    x = torch.randn(8, 8)
    a = x.to(dev)
    torch_vulkan.reset_fallback_counts()
    assert torch.equal(a.clone().cpu(), x)
    assert torch.equal(a.t().contiguous().cpu(), x.t().contiguous())
    assert torch.equal(a.to(torch.float16).cpu(), x.to(torch.float16))
    assert torch.equal(a.to(torch.bfloat16).cpu(), x.to(torch.bfloat16))
    assert torch.equal(a.to(torch.bfloat16).to(torch.float16).cpu(), x.to(torch.bfloat16).to(torch.float16))
    z = torch.zeros(5, 7, device=dev, dtype=torch.bfloat16)
    assert torch.equal(z.cpu(), torch.zeros(5, 7, dtype=torch.bfloat16))
    f = torch.full((3, 3), 2.5, device=dev)
    assert torch.equal(f.cpu(), torch.full((3, 3), 2.5))
    assert torch_vulkan.fallback_counts() == {}, torch_vulkan.fallback_counts()


def test_bf16_cast_rounds_to_nearest_even_like_torch():
    x = torch.randn(1 << 16) * torch.logspace(-30, 30, 1 << 16)
    x[:5] = torch.tensor([float("nan"), float("inf"), -float("inf"), 0.0, -0.0])
    got = x.to(dev).to(torch.bfloat16).cpu()
    ref = x.to(torch.bfloat16)
    assert torch.equal(got[5:].view(torch.int16), ref[5:].view(torch.int16))
    assert torch.isnan(got[0])
    got16 = x.to(dev).to(torch.float16).cpu()
    assert torch.equal(got16[5:].view(torch.int16), x.to(torch.float16)[5:].view(torch.int16))


def test_empty_tensors_pass_through_transfers_views_and_ops():
    for shape in [(0,), (0, 3), (4, 0, 2)]:
        e = torch.empty(shape, device=dev)
        assert e.cpu().shape == shape and e.numel() == 0
        assert (e + e).shape == shape and e.to(torch.bfloat16).shape == shape
        assert torch.zeros(shape).to(dev).clone().cpu().shape == shape
    assert torch.empty(5, 0, device=dev).t().contiguous().shape == (0, 5)


def test_a_256_mib_transfer_round_trips_and_its_memory_is_released():
    base = torch_vulkan.live_bytes()
    host = sample(torch.float32, (64 << 20,), seed=9)  # 256 MiB
    d = host.to(dev)
    assert torch_vulkan.live_bytes() >= base + host.numel() * 4
    same_bits(d.cpu(), host)
    same_bits(d[-1000:].cpu(), host[-1000:])  # the far end of the block, through a view
    del d
    assert torch_vulkan.live_bytes() == base


def test_resize_keeps_the_data_it_had():
    host = sample(torch.float32, (10,), seed=5)
    d = host.to(dev)
    d.resize_(25)    # grows: the first ten values stay
    same_bits(d.cpu()[:10], host)
    d.resize_(4)     # shrinks to a prefix
    same_bits(d.cpu(), host[:4])
    d.resize_(3, 2)  # a new shape over the same storage
    same_bits(d.cpu().reshape(-1)[:4], host[:4])


def test_memory_api():
    info = torch.vk.memory_info()
    assert info["heap"] > 200 << 30 and 0 < info["budget"] <= info["heap"]
    torch_vulkan.reset_peak_live_bytes()
    base = torch_vulkan.live_bytes()
    t = torch.empty(1 << 20, device=dev)
    assert torch_vulkan.peak_live_bytes() >= base + (4 << 20)
    del t
    assert torch_vulkan.reserved_bytes() >= torch_vulkan.live_bytes()


def test_stats_dictionary_matches_the_reference_keys():
    """torch_vulkan._C.stats() (the reference's pybind name, csrc/shim.cpp:455-468) and torch_vulkan.stats()
    return the same keys, and after a device product the dispatch count is positive."""
    a = torch.randn(64, 64, device=dev)
    (a @ a).cpu()
    c, p = torch_vulkan._C.stats(), torch_vulkan.stats()
    assert set(c) == set(p) == {"dispatch_s", "dispatch_n", "transfer_s", "transfer_n", "pipeline_create_s",
                                "upload_MB", "download_MB", "gpu_wait_s", "fallback_s"}
    assert c["dispatch_n"] >= 1 and c["download_MB"] > 0
