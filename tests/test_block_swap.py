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


# ---- memory API (reference tests/test_memory_api.py:11-30) ------------------------------------------------
def test_device_module_exposes_memory_api():
    for name in ("memory_info", "set_memory_limit", "peak_live_bytes", "reset_peak_live_bytes", "empty_pinned"):
        assert hasattr(torch.vk, name), name
    info = torch.vk.memory_info()
    assert info["budget"] > 0 and info["heap"] >= info["budget"] > info["usage"] >= 0


def test_memory_limit_is_enforced_through_device_module():
    torch.vk.set_memory_limit(64)
    try:
        torch.vk.reset_peak_live_bytes()
        x = torch.zeros(1024, device="vk")
        assert torch.vk.peak_live_bytes() >= x.numel() * 4
        with pytest.raises(RuntimeError):
            torch.empty(256 << 20, dtype=torch.uint8, device="vk")  # over the 64 MiB cap
    finally:
        torch.vk.set_memory_limit(0)


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


# ---- block swap (reference tests/test_block_swap_vk.py:23-124, loop written out) -----------------------------
D, N_BLOCKS, RANK = 64, 6, 4


class Lora(nn.Module):
    def __init__(self):
        super().__init__()
        self.a = nn.Parameter(torch.randn(D, RANK, dtype=torch.bfloat16) * 0.1)
        self.b = nn.Parameter(torch.randn(RANK, D, dtype=torch.bfloat16) * 0.1)


def make_weights():
    torch.manual_seed(0)
    loras = [Lora() for _ in range(N_BLOCKS)]
    blocks = []
    for _ in range(N_BLOCKS):
        blocks.append({"w1": (torch.randn(4 * D, D) * D ** -0.5).to(torch.bfloat16),
                       "w2": (torch.randn(D, 4 * D) * (4 * D) ** -0.5).to(torch.bfloat16),
                       "g": torch.ones(D, dtype=torch.bfloat16), "beta": torch.zeros(D, dtype=torch.bfloat16)})
    return loras, blocks


def block_fn(x, w, lo):
    h = F.linear(F.gelu(F.linear(F.layer_norm(x, (D,), w["g"], w["beta"]), w["w1"])), w["w2"])
    return x + h + (x @ lo.a) @ lo.b


def run(swap, ring=2, steps=2, non_blocking=True):
    loras, blocks = make_weights()
    for lo in loras:
        lo.to(DEV)
    if swap:
        host = [{k: torch_vulkan.pin_memory(v) for k, v in b.items()} for b in blocks]
        slots = [{k: torch.empty_like(v, device=DEV) for k, v in blocks[0].items()} for _ in range(ring)]
    else:
        resident = [{k: v.to(DEV) for k, v in b.items()} for b in blocks]
    out = []
    for step in range(steps):
        torch.manual_seed(100 + step)
        x = torch.randn(2, 16, D).to(torch.bfloat16).to(DEV).requires_grad_(True)
        for lo in loras:
            for p in lo.parameters():
                p.grad = None
        for i in range(N_BLOCKS):
            if swap:
                def fn(x, i=i):  # fetches block i's weights into its ring slot (again when recomputed)
                    s = slots[i % ring]
                    for k in s:
                        s[k].copy_(host[i][k], non_blocking=non_blocking)
                    return block_fn(x, s, loras[i])
            else:
                def fn(x, i=i):
                    return block_fn(x, resident[i], loras[i])
            x = checkpoint(fn, x, use_reentrant=False)
        loss = x.float().pow(2).mean()
        loss.backward()
        out.append((loss.item(), [p.grad.detach().float().cpu() for lo in loras for p in lo.parameters()]))
    return out


@pytest.fixture(scope="module")
def resident():
    return run(swap=False)


@pytest.mark.parametrize("ring,non_blocking", [(2, True), (3, True), (2, False)])
def test_block_swap_matches_resident(resident, ring, non_blocking):
    got = run(swap=True, ring=ring, non_blocking=non_blocking)
    for (loss_r, grads_r), (loss_g, grads_g) in zip(resident, got):
        assert loss_g == loss_r
        for gr, gg in zip(grads_r, grads_g):
            assert torch.equal(gr, gg)


def test_swapped_weights_leave_the_device():
    torch_vulkan.synchronize()
    torch_vulkan.empty_cache()
    base = torch_vulkan.live_bytes()
    loras, blocks = make_weights()
    resident = [{k: v.to(DEV) for k, v in b.items()} for b in blocks]
    torch_vulkan.synchronize()
    live_resident = torch_vulkan.live_bytes() - base
    del resident
    ring = [{k: torch.empty_like(v, device=DEV) for k, v in blocks[0].items()} for _ in range(2)]
    live_swapped = torch_vulkan.live_bytes() - base
    block_bytes = 2 * (D * 4 * D) * 2
    assert live_resident - live_swapped >= (N_BLOCKS - 2) * block_bytes
    del ring
