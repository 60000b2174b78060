"""Transfers, views and device copies of the vk boundary (reference tests/test_gpu_ops.py:27-89): dtype
round trips, host<->device conversion and broadcast, non-contiguous sources and destinations, storage
offsets, device-side casts/fills, empty tensors, large transfers with memory release, resize_."""

import pytest
import torch

pytestmark = pytest.mark.gpu

import torch_vulkan  # noqa: E402

dev = torch.device("vk")


def test_runs_on_an_mi355x():
    assert "gfx950" in torch_vulkan.device_name()


def test_roundtrip_dtypes():
    for dt in (torch.float32, torch.float16, torch.bfloat16, torch.int64, torch.uint8, torch.bool, torch.int8, torch.int32):
        x = (torch.rand(7, 5) * 10).to(dt)
        assert torch.equal(x.to(dev).cpu(), x), dt


def test_cpu_to_vk_with_dtype_conversion_and_broadcast():
    x = torch.arange(6, dtype=torch.float32)
    assert torch.equal(x.to(dev).to(torch.int32).cpu(), x.to(torch.int32))
    dst = torch.zeros(3, 4, device=dev)
    dst.copy_(torch.tensor([1.0, 2.0, 3.0, 4.0]))
    assert torch.equal(dst.cpu(), torch.tensor([1.0, 2.0, 3.0, 4.0]).expand(3, 4))


def test_noncontiguous_source_and_destination():
    x = torch.randn(4, 6)
    assert torch.equal(x.t().to(dev).cpu(), x.t())
    v = x.to(dev).t()
    assert torch.equal(v.cpu(), x.t())
    d = torch.zeros(4, 6, device=dev)
    d.t().copy_(torch.arange(24, dtype=torch.float32).reshape(6, 4))
    assert torch.equal(d.cpu(), torch.arange(24, dtype=torch.float32).reshape(6, 4).t())


def test_view_with_storage_offset_reads_and_writes():
    x = torch.arange(100, dtype=torch.float32)
    d = x.to(dev)
    assert torch.equal(d[10:20].cpu(), x[10:20])
    d[10:20] = -1.0
    ref = x.clone()
    ref[10:20] = -1.0
    assert torch.equal(d.cpu(), ref)


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


def test_empty_tensors_do_not_crash():
    e = torch.empty(0, 3, device=dev)
    assert e.cpu().shape == (0, 3)
    assert (e + e).shape == (0, 3)


def test_large_tensor_roundtrip_and_memory_is_released():
    before = torch_vulkan.live_bytes()
    x = torch.randn(64 << 20)
    d = x.to(dev)
    assert torch_vulkan.live_bytes() - before >= x.numel() * 4
    assert torch.equal(d.cpu(), x)
    del d
    assert torch_vulkan.live_bytes() == before


def test_resize_keeps_existing_data():
    d = torch.arange(10, dtype=torch.float32).to(dev)
    d.resize_(20)
    assert torch.equal(d.cpu()[:10], torch.arange(10, dtype=torch.float32))


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
