"""Memory API and the block-swap transfer path on the vk device.

The reference's tests/test_memory_api.py (the torch.vk memory functions sd-scripts' --vram_budget_mb uses)
and tests/test_block_swap_vk.py (frozen block weights kept on the host and streamed through a ring of
device buffers must give the resident run's loss and LoRA gradients exactly; that test needs sd-scripts'
offloader, absent here, so the same loop is written out below with torch.utils.checkpoint).  Added: pinned
host memory from the runtime, asynchronous uploads that overlap kernels (ordering against earlier readers
of the destination and later users of it), immediate frees of in-flight sources, asynchronous downloads.
"""

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint

pytestmark = pytest.mark.gpu

import torch_vulkan  # noqa: E402

DEV = torch.device("vk")


# ---- memory API (the functions the reference's tests/test_memory_api.py requires of torch.vk) -------------
@pytest.mark.parametrize("name", ["memory_info", "set_memory_limit", "peak_live_bytes", "reset_peak_live_bytes",
                                  "empty_pinned", "synchronize", "empty_cache"])
def test_device_module_function(name):
    assert callable(getattr(torch.vk, name, None)), name


def test_memory_info_is_consistent():
    info = torch.vk.memory_info()
    assert set(info) >= {"budget", "usage", "heap"}
    assert 0 <= info["usage"] < info["budget"] <= info["heap"]
    before = torch.vk.memory_info()["usage"]
    blk = torch.empty(64 << 20, dtype=torch.uint8, device=DEV)  # 64 MiB more in use
    assert torch.vk.memory_info()["usage"] >= before
    del blk


def test_memory_limit_caps_allocations_until_lifted():
    cap_mb = 96
    torch.vk.set_memory_limit(cap_mb)
    try:
        torch.vk.reset_peak_live_bytes()
        small = torch.ones(4096, device=DEV)  # well inside the cap
        assert torch.vk.peak_live_bytes() >= small.numel() * 4
        with pytest.raises(RuntimeError):
            torch.empty((cap_mb + 32) << 20, dtype=torch.uint8, device=DEV)
    finally:
        torch.vk.set_memory_limit(0)
    big = torch.empty((cap_mb + 32) << 20, dtype=torch.uint8, device=DEV)  # allowed again
    del big


# ---- pinned memory and asynchronous transfers ---------------------------------------------------------------
def test_pinned_host_memory():
    h = torch_vulkan.empty_pinned((1000, 3), torch.bfloat16)
    assert h.device.type == "cpu" and torch_vulkan.is_pinned(h) and tuple(h.shape) == (1000, 3)
    with pytest.warns(DeprecationWarning):  # PyTorch's own query reaches the same runtime check
        assert h.is_pinned(device="vk")
    assert not torch_vulkan.is_pinned(torch.zeros(8))
    p = torch_vulkan.pin_memory(torch.arange(10.0))
    assert torch_vulkan.is_pinned(p) and torch.equal(p, torch.arange(10.0))
    assert torch_vulkan.pin_memory(p) is p


def test_async_upload_then_kernel_reads_the_new_data():
    n = 1 << 20
    d = torch.empty(n, device=DEV)
    for i in range(20):
        h = torch_vulkan.empty_pinned((n,))
        h.fill_(float(i))
        d.copy_(h, non_blocking=True)
        del h  # freed while the copy may still be in flight
        s = d.sum().item()  # the reduction waits for the upload into d
        assert s == float(i) * n, (i, s)


def test_ring_buffer_reuse_orders_uploads_after_earlier_readers():
    """Each step overwrites the same device slot; the kernel of step i must see step i's data, and the
    upload of step i + 1 must not overwrite the slot before that kernel has read it."""
    n, steps = 1 << 22, 12
    hosts = [torch_vulkan.empty_pinned((n,)) for _ in range(steps)]
    for i, h in enumerate(hosts):
        h.copy_(torch.full((n,), float(i + 1)))
    slot = torch.empty(n, device=DEV)
    outs = []
    for i in range(steps):
        slot.copy_(hosts[i], non_blocking=True)
        outs.append(slot * 2.0)  # a kernel reading the slot, queued right behind the upload
    torch_vulkan.synchronize()
    for i, o in enumerate(outs):
        v = o.cpu()
        assert torch.all(v == 2.0 * (i + 1)), (i, v.min().item(), v.max().item())


def test_async_uploads_to_many_buffers_and_async_download():
    n, k = 1 << 18, 32
    src = [torch_vulkan.pin_memory(torch.randn(n, generator=torch.Generator().manual_seed(i))) for i in range(k)]
    dev = [torch.empty(n, device=DEV) for _ in range(k)]
    for d, s in zip(dev, src):
        d.copy_(s, non_blocking=True)
    back = [torch_vulkan.empty_pinned((n,)) for _ in range(k)]
    for b, d in zip(back, dev):
        b.copy_(d, non_blocking=True)
    torch_vulkan.synchronize()
    for b, s in zip(back, src):
        assert torch.equal(b, s)
    # non-pinned or mismatched copies take the synchronous path and stay correct
    pageable = torch.randn(n)
    dev[0].copy_(pageable, non_blocking=True)
    assert torch.equal(dev[0].cpu(), pageable)


def test_graph_recording_rejects_async_uploads():
    from torch_vulkan import abi

    rt = abi.Runtime()
    h = torch_vulkan.empty_pinned((256,))
    d = torch.empty(256, device=DEV)
    rt.check(rt.lib.hrt_graph_begin(), "hrt_graph_begin")
    try:
        assert rt.lib.hrt_upload_async(d.data_ptr(), h.data_ptr(), 1024) == -1
        assert "graph" in rt.last_error()
    finally:
        gid = rt.lib.hrt_graph_end()
    rt.graph_destroy(gid)
    assert rt.lib.hrt_upload_async(d.data_ptr(), torch.zeros(256).data_ptr(), 1024) == -1  # pageable source
    assert "pinned" in rt.last_error()


# ---- block swap -------------------------------------------------------------------------------------------------
# The reference's tests/test_block_swap_vk.py requires that frozen block weights kept on the host and streamed
# through a ring of device buffers give the resident run's loss and adapter gradients exactly.  Its loop
# needs sd-scripts' offloader (absent here); the same pattern is written out: a stack of residual MLP blocks
# whose frozen weights are fetched into ring slots inside activation-checkpointed segments (so the backward
# fetches them again), with trainable low-rank adapters beside the first projection of each block.
WIDTH, DEPTH, ADAPTER_RANK = 64, 6, 4


def frozen_blocks():
    g = torch.Generator().manual_seed(11)
    return [{"up": (torch.randn(3 * WIDTH, WIDTH, generator=g) * WIDTH ** -0.5).to(torch.bfloat16),
             "up_bias": (torch.randn(3 * WIDTH, generator=g) * 0.02).to(torch.bfloat16),
             "down": (torch.randn(WIDTH, 3 * WIDTH, generator=g) * (3 * WIDTH) ** -0.5).to(torch.bfloat16)}
            for _ in range(DEPTH)]


def adapters():
    g = torch.Generator().manual_seed(12)
    return [(nn.Parameter((torch.randn(ADAPTER_RANK, WIDTH, generator=g) * 0.1).to(torch.bfloat16).to(DEV)),
             nn.Parameter((torch.randn(3 * WIDTH, ADAPTER_RANK, generator=g) * 0.1).to(torch.bfloat16).to(DEV)))
            for _ in range(DEPTH)]


def mlp_block(x, w, ad):
    down_a, up_b = ad
    h = F.linear(x, w["up"], w["up_bias"]) + F.linear(F.linear(x, down_a), up_b)
    return x + F.linear(F.silu(h), w["down"])


def train_steps(swap, ring=2, steps=2, non_blocking=True):
    """Per step: a fresh input through the stack, loss = mean square, backward; returns (loss, adapter
    gradients) per step."""
    blocks, ads = frozen_blocks(), adapters()
    if swap:
        host = [{k: torch_vulkan.pin_memory(v) for k, v in b.items()} for b in blocks]
        slots = [{k: torch.empty(v.shape, dtype=v.dtype, device=DEV) for k, v in blocks[0].items()} for _ in range(ring)]
    else:
        on_device = [{k: v.to(DEV) for k, v in b.items()} for b in blocks]
    results = []
    for step in range(steps):
        x = torch.randn(3, 8, WIDTH, generator=torch.Generator().manual_seed(50 + step)).to(torch.bfloat16).to(DEV)
        x.requires_grad_(True)
        for p in (p for ad in ads for p in ad):
            p.grad = None
        for i in range(DEPTH):
            if swap:
                def segment(t, i=i):  # block i's weights into slot i % ring, again when recomputed
                    slot = slots[i % ring]
                    for k, dst in slot.items():
                        dst.copy_(host[i][k], non_blocking=non_blocking)
                    return mlp_block(t, slot, ads[i])
            else:
                def segment(t, i=i):
                    return mlp_block(t, on_device[i], ads[i])
            x = checkpoint(segment, x, use_reentrant=False)
        loss = x.float().square().mean()
        loss.backward()
        results.append((loss.item(), [p.grad.detach().float().cpu() for ad in ads for p in ad]))
    return results


@pytest.fixture(scope="module")
def resident():
    return train_steps(swap=False)


@pytest.mark.parametrize("ring,non_blocking", [(2, True), (3, True), (2, False)])
def test_block_swap_matches_resident(resident, ring, non_blocking):
    swapped = train_steps(swap=True, ring=ring, non_blocking=non_blocking)
    for (loss_r, grads_r), (loss_s, grads_s) in zip(resident, swapped):
        assert loss_s == loss_r
        assert all(torch.equal(a, b) for a, b in zip(grads_r, grads_s))


def test_swapped_weights_leave_the_device():
    torch_vulkan.synchronize()
    torch_vulkan.empty_cache()
    base = torch_vulkan.live_bytes()
    blocks = frozen_blocks()
    on_device = [{k: v.to(DEV) for k, v in b.items()} for b in blocks]
    torch_vulkan.synchronize()
    all_resident = torch_vulkan.live_bytes() - base
    del on_device
    ring = [{k: torch.empty(v.shape, dtype=v.dtype, device=DEV) for k, v in blocks[0].items()} for _ in range(2)]
    ring_only = torch_vulkan.live_bytes() - base
    per_block = sum(v.numel() * v.element_size() for v in blocks[0].values())
    assert all_resident - ring_only >= (DEPTH - 2) * per_block
    del ring
