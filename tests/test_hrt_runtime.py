"""The hrt C ABI on the GPU, called directly through ctypes (no torch): the reference runtime's own test
list (vkrt/tests/basic.rs:14-182) — round trips, offsets, large transfers, the raw smoke kernel, rejection
of out-of-range / unknown addresses and double frees, the device limit, many small allocations,
coalescing and dedicated blocks — plus the argument-size and grid checks of hrt_dispatch."""

import ctypes
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "torch-vulkan_amd", "torch_vulkan", "libhrt.so")


@pytest.fixture(scope="module")
def hrt():
    lib = ctypes.CDLL(LIB)
    u64, u32, vp, sz = ctypes.c_uint64, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_size_t
    lib.hrt_alloc.restype = u64
    lib.hrt_alloc.argtypes = [u64]
    lib.hrt_free.argtypes = [u64]
    lib.hrt_upload.argtypes = [u64, vp, u64]
    lib.hrt_download.argtypes = [vp, u64, u64]
    lib.hrt_copy_d2d.argtypes = [u64, u64, u64]
    lib.hrt_kernel_index.argtypes = [ctypes.c_char_p]
    lib.hrt_dispatch.argtypes = [u32, vp, u32, u32, u32, u32]
    lib.hrt_max_alloc.restype = u64
    lib.hrt_reserved_bytes.restype = u64
    lib.hrt_live_bytes.restype = u64
    lib.hrt_slab_count.restype = sz
    lib.hrt_empty_cache.restype = sz
    lib.hrt_validation_errors.restype = sz
    lib.hrt_last_error.restype = sz
    lib.hrt_last_error.argtypes = [ctypes.c_char_p, sz]
    lib.hrt_device_name.restype = sz
    lib.hrt_device_name.argtypes = [ctypes.c_char_p, sz]
    lib.hrt_memory_info.argtypes = [ctypes.POINTER(u64)]
    assert lib.hrt_init() == 0, err(lib)
    return lib


def err(lib):
    b = ctypes.create_string_buffer(1024)
    lib.hrt_last_error(b, 1024)
    return b.value.decode()


def test_device_is_an_mi355x(hrt):
    b = ctypes.create_string_buffer(256)
    hrt.hrt_device_name(b, 256)
    print("device:", b.value.decode())
    assert b"gfx950" in b.value
    info = (ctypes.c_uint64 * 3)()
    assert hrt.hrt_memory_info(info) == 0
    assert info[2] > 200 << 30 and info[0] <= info[2]


def test_upload_download_roundtrip_offsets_and_d2d(hrt):
    n = 1000
    src = (np.arange(n, dtype=np.float32) * 0.5)
    a, b = hrt.hrt_alloc(n * 4), hrt.hrt_alloc(n * 4)
    assert a and b and a % 512 == 0
    assert hrt.hrt_upload(a, src.ctypes.data, n * 4) == 0
    assert hrt.hrt_copy_d2d(b, a, n * 4) == 0
    out = np.zeros(n, np.float32)
    assert hrt.hrt_download(out.ctypes.data, b, n * 4) == 0
    assert np.array_equal(out, src)
    part = np.zeros(100, np.float32)
    assert hrt.hrt_download(part.ctypes.data, b + 400, 400) == 0
    assert np.array_equal(part, src[100:200])
    assert hrt.hrt_free(a) == 0 and hrt.hrt_free(b) == 0


def test_large_transfer(hrt):
    n = (40 << 20) // 4
    src = (np.arange(n) % 1000).astype(np.float32)
    a = hrt.hrt_alloc(n * 4)
    assert hrt.hrt_upload(a, src.ctypes.data, n * 4) == 0
    out = np.zeros(n, np.float32)
    assert hrt.hrt_download(out.ctypes.data, a, n * 4) == 0
    assert np.array_equal(out, src)
    assert hrt.hrt_free(a) == 0


def test_add_f32_raw_kernel(hrt):
    n = 100003
    x = np.sin(np.arange(n, dtype=np.float32))
    y = np.cos(np.arange(n, dtype=np.float32) * 0.3)
    da, db, dc = (hrt.hrt_alloc(n * 4) for _ in range(3))
    hrt.hrt_upload(da, x.ctypes.data, n * 4)
    hrt.hrt_upload(db, y.ctypes.data, n * 4)
    k = hrt.hrt_kernel_index(b"add_f32")
    assert k >= 0
    args = np.array([da, db, dc, n], dtype=np.uint64)
    groups = (n + 255) // 256
    assert hrt.hrt_dispatch(k, args.ctypes.data, 32, groups, 1, 1) == 0, err(hrt)
    out = np.zeros(n, np.float32)
    hrt.hrt_download(out.ctypes.data, dc, n * 4)
    assert np.array_equal(out, x + y)
    # argument-size and grid checks
    assert hrt.hrt_dispatch(k, args.ctypes.data, 24, groups, 1, 1) == -1 and "argument block" in err(hrt)
    assert hrt.hrt_dispatch(k, args.ctypes.data, 32, 0, 1, 1) == -1
    kd = hrt.hrt_kernel_index(b"dq8_bf16")
    blob = np.zeros(6, np.uint64)
    assert hrt.hrt_dispatch(kd, blob.ctypes.data, 48, 4, 1, 1) == -1 and "own grid" in err(hrt)
    for p in (da, db, dc):
        hrt.hrt_free(p)


def test_out_of_range_operands_are_rejected_before_launch(hrt):
    a = hrt.hrt_alloc(64)
    buf = np.zeros(128, np.uint8)
    before = hrt.hrt_validation_errors()
    assert hrt.hrt_download(buf.ctypes.data, a, 128) == -1 and "out-of-range" in err(hrt)
    assert hrt.hrt_download(buf.ctypes.data, 0x1234, 4) == -1
    # a kernel whose operand extends past its block is refused by the launcher's extent check
    q = hrt.hrt_alloc(64)
    out = hrt.hrt_alloc(64)
    sc = hrt.hrt_alloc(2)
    kd = hrt.hrt_kernel_index(b"dq8_bf16")
    args = np.array([q, sc, out, 1, 64, 1], dtype=np.int64)  # out needs 128 bytes, the block holds 64
    assert hrt.hrt_dispatch(kd, args.ctypes.data, 48, 0, 0, 0) == -1 and "out" in err(hrt)
    assert hrt.hrt_validation_errors() >= before + 2
    assert hrt.hrt_free(0x1234) == -1
    for p in (a, q, out, sc):
        assert hrt.hrt_free(p) == 0
    assert hrt.hrt_free(a) == -1


def test_dispatch_batch_queues_in_order_and_stops_at_a_rejected_launch(hrt):
    """hrt_dispatch_batch: every launch as hrt_dispatch; the first rejected one stops the batch with
    -(index + 1) and the launches before it stay queued."""
    u32, vp = ctypes.c_uint32, ctypes.c_void_p
    hrt.hrt_dispatch_batch.argtypes = [ctypes.POINTER(u32), ctypes.POINTER(vp), ctypes.POINTER(u32), u32]
    q = hrt.hrt_alloc(64)
    sc = hrt.hrt_alloc(2)
    outs = [hrt.hrt_alloc(128) for _ in range(2)]
    small = hrt.hrt_alloc(64)
    qv = np.arange(-32, 32, dtype=np.int8)
    assert hrt.hrt_upload(q, qv.ctypes.data, 64) == 0
    one = np.array([0x3F80], dtype=np.uint16)  # bf16 1.0
    assert hrt.hrt_upload(sc, one.ctypes.data, 2) == 0
    kd = hrt.hrt_kernel_index(b"dq8_bf16")
    blocks = [np.array([q, sc, o, 1, 64, 1], dtype=np.int64) for o in outs + [small]]
    ids = (u32 * 3)(kd, kd, kd)
    ptrs = (vp * 3)(*[b.ctypes.data for b in blocks])
    lens = (u32 * 3)(48, 48, 48)
    assert hrt.hrt_dispatch_batch(ids, ptrs, lens, 2) == 0, err(hrt)
    assert hrt.hrt_synchronize() == 0
    for o in outs:
        got = np.zeros(64, np.uint16)
        assert hrt.hrt_download(got.ctypes.data, o, 128) == 0
        f = (got.astype(np.uint32) << 16).view(np.float32)
        assert np.array_equal(f, qv.astype(np.float32))
    # third block writes 128 bytes into a 64-byte block: rejected, batch stops at index 2
    zero = np.zeros(64, np.uint16)
    assert hrt.hrt_upload(outs[0], zero.ctypes.data, 128) == 0
    ids2 = (u32 * 3)(kd, kd, kd)
    ptrs2 = (vp * 3)(blocks[0].ctypes.data, blocks[2].ctypes.data, blocks[1].ctypes.data)
    assert hrt.hrt_dispatch_batch(ids2, ptrs2, lens, 3) == -2 and "out" in err(hrt)
    assert hrt.hrt_synchronize() == 0
    got = np.zeros(64, np.uint16)
    assert hrt.hrt_download(got.ctypes.data, outs[0], 128) == 0
    assert np.array_equal((got.astype(np.uint32) << 16).view(np.float32), qv.astype(np.float32))
    for p in [q, sc, small] + outs:
        assert hrt.hrt_free(p) == 0


def test_allocation_above_device_limit_fails(hrt):
    assert hrt.hrt_alloc(hrt.hrt_max_alloc() + 1) == 0


def test_many_small_allocations_and_coalescing(hrt):
    before = hrt.hrt_slab_count()
    addrs = [hrt.hrt_alloc(1000 + (i % 7) * 100) for i in range(20000)]
    assert all(addrs) and len(set(addrs)) == len(addrs)
    assert hrt.hrt_slab_count() - before < 20
    for p in addrs:
        assert hrt.hrt_free(p) == 0
    a, b, c = (hrt.hrt_alloc(4096) for _ in range(3))
    da, dc = np.full(4096, 0xAA, np.uint8), np.full(4096, 0xCC, np.uint8)
    hrt.hrt_upload(a, da.ctypes.data, 4096)
    hrt.hrt_upload(c, dc.ctypes.data, 4096)
    hrt.hrt_free(b)
    big = hrt.hrt_alloc(8192)
    bd = np.full(8192, 0x55, np.uint8)
    hrt.hrt_upload(big, bd.ctypes.data, 8192)
    ra, rc = np.zeros(4096, np.uint8), np.zeros(4096, np.uint8)
    hrt.hrt_download(ra.ctypes.data, a, 4096)
    hrt.hrt_download(rc.ctypes.data, c, 4096)
    assert np.array_equal(ra, da) and np.array_equal(rc, dc)
    for p in (a, c, big):
        hrt.hrt_free(p)
    allb = hrt.hrt_alloc(3 * 4096 + 8192)
    assert allb
    hrt.hrt_free(allb)


def test_dedicated_blocks_and_empty_cache(hrt):
    big = hrt.hrt_alloc(300 << 20)
    assert big
    reserved = hrt.hrt_reserved_bytes()
    assert reserved >= 300 << 20
    hrt.hrt_free(big)
    assert hrt.hrt_reserved_bytes() < reserved  # a dedicated block goes straight back to the driver
    # regular blocks: allocate until a fresh slab appears (other tests of this process may hold slabs),
    # free them, and the slabs they created come back through empty_cache
    hrt.hrt_empty_cache()
    before = hrt.hrt_slab_count()
    blocks = []
    while hrt.hrt_slab_count() == before and len(blocks) < 16:
        blocks.append(hrt.hrt_alloc(200 << 20))
    new_slabs = hrt.hrt_slab_count() - before
    assert new_slabs >= 1 and all(blocks)
    for p in blocks:
        assert hrt.hrt_free(p) == 0
    assert hrt.hrt_empty_cache() >= new_slabs
    assert hrt.hrt_slab_count() <= before
    assert hrt.hrt_synchronize() == 0
