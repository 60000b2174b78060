"""The allocation-free layer_norm backward (hrt_ln_bwd_noalloc, include/hrt_ops.h) through the C ABI,
against the allocating entry point it varies: "ln_bwd_{dt}" + "ln_wgrad_{dt}" with a workspace the caller
allocated.  Both run the same kernels, so dx, dw and db must agree bit for bit (the bar for index work;
the layer_norm numerics themselves are checked against the oracle in test_rows.py).  Two calls in a row,
the second smaller, show that the scratch array's leftover contents from the first call do not leak in."""

import numpy as np
import pytest
import torch

import torch_vulkan  # noqa: F401  (registers the vk device)
from torch_vulkan import abi

pytestmark = pytest.mark.gpu
DEV = torch.device("vk")
CODE = {torch.float32: abi.F32, torch.bfloat16: abi.BF16, torch.float16: abi.F16}
KIND = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}


def _bits(t):
    t = t.detach().cpu().contiguous()
    return t.view(torch.int32 if t.dtype == torch.float32 else torch.int16).numpy()


def _case(rows, D, dtype, seed, affine=True):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(rows, D, generator=g) * 2 + 0.3).to(dtype).to(DEV)
    gy = torch.randn(rows, D, generator=g).to(dtype).to(DEV)
    w = torch.randn(D, generator=g).to(dtype).to(DEV) if affine else None
    b = torch.randn(D, generator=g).to(dtype).to(DEV) if affine else None
    _, mean, rstd = torch.native_layer_norm(x, [D], w, b, 1e-5)
    return x, gy, w, mean.contiguous(), rstd.contiguous()


def _args(x, gy, w, mean, rstd, dx, dw, db, ws=0):
    a = abi.LnArgs()
    a.x, a.g, a.mean, a.rstd = x.data_ptr(), gy.data_ptr(), mean.data_ptr(), rstd.data_ptr()
    a.w = w.data_ptr() if w is not None else 0
    a.dx = dx.data_ptr() if dx is not None else 0
    a.dw = dw.data_ptr() if dw is not None else 0
    a.db = db.data_ptr() if db is not None else 0
    a.ws, a.rows, a.D, a.eps = ws, x.shape[0], x.shape[1], 1e-5
    return a


def _allocating(rt, dtype, x, gy, w, mean, rstd):
    rows, D = x.shape
    dx, dw, db = torch.empty_like(x), torch.empty(D, dtype=dtype, device=DEV), torch.empty(D, dtype=dtype, device=DEV)
    ws = torch.empty(abi.ln_chunks(rows, D) * 2 * D, dtype=torch.float32, device=DEV)
    a = _args(x, gy, w, mean, rstd, dx, dw, db, ws.data_ptr())
    rt.dispatch(f"ln_bwd_{KIND[dtype]}", a)
    rt.dispatch(f"ln_wgrad_{KIND[dtype]}", a)
    return dx, dw, db


def _noalloc(rt, dtype, x, gy, w, mean, rstd):
    rows, D = x.shape
    dx, dw, db = torch.empty_like(x), torch.empty(D, dtype=dtype, device=DEV), torch.empty(D, dtype=dtype, device=DEV)
    rt.ln_bwd_noalloc(_args(x, gy, w, mean, rstd, dx, dw, db), CODE[dtype])
    return dx, dw, db


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_noalloc_matches_the_allocating_entry_point_twice(dtype):
    rt = abi.Runtime()
    # first the benchmark shape (4 MiB of partial sums), then a smaller ragged one on the same scratch array
    for rows, D, seed in ((1024, 2048, 1), (37, 200, 2)):
        print(f"case rows={rows} D={D} dtype={dtype}", flush=True)
        t = _case(rows, D, dtype, seed)
        want = _allocating(rt, dtype, *t)
        rt.synchronize()
        live, reserved = rt.lib.hrt_live_bytes(), rt.lib.hrt_reserved_bytes()
        outs = torch.empty(rows, t[0].shape[1], dtype=dtype, device=DEV), *(torch.empty(D, dtype=dtype, device=DEV) for _ in range(2))
        live_outs = rt.lib.hrt_live_bytes()
        rt.ln_bwd_noalloc(_args(*t, *outs), CODE[dtype])
        assert rt.lib.hrt_live_bytes() == live_outs and rt.lib.hrt_reserved_bytes() == reserved  # nothing allocated
        got = outs
        rt.synchronize()
        assert live_outs >= live
        for n, a, b in zip(("dx", "dw", "db"), got, want):
            assert np.array_equal(_bits(a), _bits(b)), (n, rows, D)


def test_noalloc_without_affine_and_dx_only():
    rt = abi.Runtime()
    x, gy, _, mean, rstd = _case(64, 512, torch.bfloat16, 3, affine=False)
    want = _allocating(rt, torch.bfloat16, x, gy, None, mean, rstd)
    dx = torch.empty_like(x)
    rt.ln_bwd_noalloc(_args(x, gy, None, mean, rstd, dx, None, None), abi.BF16)  # dx only: no scratch use
    got = _noalloc(rt, torch.bfloat16, x, gy, None, mean, rstd)
    rt.synchronize()
    assert np.array_equal(_bits(dx), _bits(want[0]))
    for a, b in zip(got, want):
        assert np.array_equal(_bits(a), _bits(b))


def test_noalloc_rejects_what_it_cannot_serve():
    rt = abi.Runtime()
    rows, D = 4096, 4096  # 512 chunks of 8 rows x 32 KiB = 16 MiB of partial sums > the 8 MiB array
    assert abi.ln_chunks(rows, D) * 2 * D * 4 > abi.LN_SCRATCH_BYTES
    x = torch.zeros(rows, D, dtype=torch.bfloat16, device=DEV)
    stats = torch.zeros(rows, dtype=torch.float32, device=DEV)
    dw = torch.empty(D, dtype=torch.bfloat16, device=DEV)
    a = _args(x, x, None, stats, stats, None, dw, None)
    with pytest.raises(RuntimeError, match="scratch array holds"):
        rt.ln_bwd_noalloc(a, abi.BF16)
    a.ws = dw.data_ptr()
    with pytest.raises(RuntimeError, match="ws must be 0"):
        rt.ln_bwd_noalloc(a, abi.BF16)
    a.ws = 0
    with pytest.raises(RuntimeError, match="dtype"):
        rt.ln_bwd_noalloc(a, 7)
    rt.synchronize()
