"""mm / bmm / addmm / baddbmm on the GPU against the float64 oracle.

The reference's tests/test_mm.py fixes the behaviours (odd shapes, transposed and sliced operands read in
place, bias broadcast with alpha / beta, batched products, nn.Linear autograd, the matrix-core and FMA
kernels agreeing) and the tolerance: the largest error at most tol x max(1, largest |reference|) x
(1 + sqrt(K) / 100) with tol = 2e-5 (float32), 1.2e-2 (bfloat16), 2e-3 (float16).  These tests build each
operand through one helper (row-major, or stored transposed and read through its .t() view) and add the
device's own tile paths (direct-to-LDS tiles of every size, split K, narrow and short-K products) and the
BASELINE shapes (1024^3 + bias, 1024x2048x8192)."""

import os

import numpy as np
import pytest
import torch

import oracle
from vkutil import f64, randn

pytestmark = pytest.mark.gpu

import torch_vulkan  # noqa: E402

dev = torch.device("vk")
FLOATS = [torch.float32, torch.bfloat16, torch.float16]
GEMM_TOL = {torch.float32: 2e-5, torch.bfloat16: 1.2e-2, torch.float16: 2e-3}


def assert_gemm_close(out, want64, dt, k):
    """out (a vk tensor) against the float64 product: largest error within GEMM_TOL[dt] x max(1, largest
    |want|) x (1 + sqrt(k) / 100)."""
    got = f64(out)
    assert got.shape == want64.shape, (got.shape, want64.shape)
    bound = GEMM_TOL[dt] * max(1.0, float(np.abs(want64).max()) if want64.size else 0.0) * (1.0 + np.sqrt(k) / 100.0)
    err = float(np.abs(got - want64).max()) if got.size else 0.0
    assert err <= bound, f"largest error {err} > {bound}"


def assert_on_device(*names):
    fb = torch_vulkan.fallback_counts()
    hit = {n: fb[n] for n in names if n in fb}
    assert not hit, f"ran on the CPU: {hit}"


def stored(rows, cols, dt, seed, transposed=False, scale=1.0):
    """A logical [rows, cols] operand as (CPU values, device tensor): row-major, or with `transposed` stored
    as [cols, rows] and handed over as its .t() view, which the kernels read in place."""
    if transposed:
        host = randn((cols, rows), dt, seed, scale)
        return host.t(), host.to(dev).t()
    host = randn((rows, cols), dt, seed, scale)
    return host, host.to(dev)


# (M, K, N): single elements, primes around the tile sizes, long K with few outputs, one row, tall and thin
PRODUCT_SHAPES = [(1, 1, 1), (3, 7, 2), (64, 32, 64), (63, 31, 65), (127, 255, 129), (40, 1500, 24),
                  (9, 3000, 5), (256, 256, 256), (520, 72, 300), (1, 2048, 24), (2048, 16, 1024)]


@pytest.mark.parametrize("m,k,n", PRODUCT_SHAPES)
@pytest.mark.parametrize("dt", FLOATS)
def test_product_shapes(dt, m, k, n):
    a, A = stored(m, k, dt, 1)
    b, B = stored(k, n, dt, 2)
    out = torch.mm(A, B)
    assert out.dtype == dt and tuple(out.shape) == (m, n)
    assert_gemm_close(out, oracle.gemm(f64(a), f64(b)), dt, k)
    assert torch_vulkan.kernel_counts().get("aten::mm") == 1  # one product, one kernel
    assert_on_device("aten::mm")


@pytest.mark.parametrize("lb", ["row-major", "transposed", "window"])
@pytest.mark.parametrize("la", ["row-major", "transposed", "window"])
@pytest.mark.parametrize("dt", FLOATS)
def test_operand_layouts_are_read_in_place(dt, la, lb):
    """Row-major, transposed and windowed (a sub-block of a larger tensor, at a storage offset) operands:
    no copy kernel runs before the product."""
    m, k, n = 70, 45, 90

    def make(rows, cols, seed, layout):
        if layout == "window":
            host = randn((rows + 6, cols + 9), dt, seed)
            return host[4:4 + rows, 5:5 + cols], host.to(dev)[4:4 + rows, 5:5 + cols]
        return stored(rows, cols, dt, seed, layout == "transposed")

    a, A = make(m, k, 3, la)
    b, B = make(k, n, 4, lb)
    torch_vulkan.reset_fallback_counts()
    assert_gemm_close(torch.mm(A, B), oracle.gemm(f64(a), f64(b)), dt, k)
    kc = torch_vulkan.kernel_counts()
    assert kc.get("aten::copy_", 0) == 0 and "aten::clone" not in torch_vulkan.fallback_counts(), kc
    assert_on_device("aten::mm")


@pytest.mark.parametrize("m,k,n", [(96, 80, 70), (256, 512, 384), (200, 136, 264)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_matrix_core_layouts_with_scaled_bias(dt, ta, tb, m, k, n):
    a, A = stored(m, k, dt, 3, ta)
    b, B = stored(k, n, dt, 4, tb)
    assert_gemm_close(torch.mm(A, B), oracle.gemm(f64(a), f64(b)), dt, k)
    bias = randn((n,), dt, 5)
    out = torch.addmm(bias.to(dev), A, B, alpha=0.5, beta=2.0)
    assert_gemm_close(out, oracle.gemm(f64(a), f64(b), f64(bias), 0.5, 2.0), dt, k)


@pytest.mark.parametrize("dt", FLOATS)
def test_batched_products(dt):
    """bmm with a plain and a column-major right operand, and baddbmm with a bias broadcast over rows."""
    a, b = randn((5, 37, 29), dt, 1), randn((5, 29, 41), dt, 2)
    want = oracle.gemm(f64(a), f64(b))
    bd_colmajor = b.to(dev).mT.contiguous().mT  # same values, strides (29 * 41, 1, 29)
    for B in (b.to(dev), bd_colmajor):
        assert_gemm_close(torch.bmm(a.to(dev), B), want, dt, 29)
    p, q, bias = randn((3, 10, 8), dt, 6), randn((3, 8, 12), dt, 7), randn((3, 1, 12), dt, 8)
    out = torch.baddbmm(bias.to(dev), p.to(dev), q.to(dev), alpha=0.5, beta=1.5)
    assert_gemm_close(out, oracle.gemm(f64(p), f64(q), f64(bias), 0.5, 1.5), dt, 8)
    assert_on_device("aten::bmm", "aten::baddbmm")


@pytest.mark.parametrize("bias_shape", [(), (40,), (1, 40), (30, 1), (30, 40)])
@pytest.mark.parametrize("dt", FLOATS)
def test_addmm_bias_shapes_and_scales(dt, bias_shape):
    a, b, bias = randn((30, 20), dt, 1), randn((20, 40), dt, 2), randn(bias_shape, dt, 3)
    for alpha, beta in [(1.0, 1.0), (0.5, 2.0), (2.0, 0.0), (-1.0, 0.25)]:
        out = torch.addmm(bias.to(dev), a.to(dev), b.to(dev), alpha=alpha, beta=beta)
        want = np.broadcast_to(oracle.gemm(f64(a), f64(b), f64(bias), alpha, beta), (30, 40))
        assert_gemm_close(out, want, dt, 20)
    assert_on_device("aten::addmm")


def test_mismatched_dtypes_raise_and_empty_reductions_give_zeros():
    with pytest.raises(RuntimeError):
        torch.mm(randn((4, 5), torch.float32).to(dev), randn((5, 6), torch.bfloat16).to(dev))
    for dt in (torch.float32, torch.bfloat16):
        z = torch.mm(torch.zeros(3, 0, dtype=dt, device=dev), torch.zeros(0, 4, dtype=dt, device=dev))
        assert torch.equal(z.cpu(), torch.zeros(3, 4, dtype=dt))
    assert torch.mm(torch.zeros(0, 5, device=dev), torch.zeros(5, 2, device=dev)).shape == (0, 2)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_linear_layer_gradients(dt):
    """F.linear on [2, 10, 48] tokens with a [32, 48] weight and bias: output, input, weight and bias
    gradients against float64."""
    x, w, bias, gy = randn((2, 10, 48), dt, 5), randn((32, 48), dt, 6, 0.15), randn((32,), dt, 7), randn((2, 10, 32), dt, 8)
    xd, wd, bd = (t.to(dev).requires_grad_(True) for t in (x, w, bias))
    y = torch.nn.functional.linear(xd, wd, bd)
    gx, gw, gb = torch.autograd.grad(y, (xd, wd, bd), gy.to(dev))
    x2, g2 = f64(x).reshape(20, 48), f64(gy).reshape(20, 32)
    assert_gemm_close(y, oracle.gemm(x2, f64(w).T, f64(bias), 1.0, 1.0).reshape(2, 10, 32), dt, 48)
    assert_gemm_close(gx, oracle.gemm(g2, f64(w)).reshape(2, 10, 48), dt, 32)
    assert_gemm_close(gw, oracle.gemm(g2.T, x2), dt, 20)
    assert np.allclose(f64(gb), g2.sum(0), rtol=GEMM_TOL[dt], atol=GEMM_TOL[dt] * 5)
    assert_on_device("aten::mm", "aten::addmm")


def test_matrix_core_and_fma_kernels_agree():
    """The same batched bf16 product with the matrix-core kernels on and off (the FMA path)."""
    a, b = randn((4, 70, 90), torch.bfloat16, 1), randn((4, 90, 50), torch.bfloat16, 2)
    results = {}
    for mfma in (True, False):
        torch_vulkan.set_coop_enabled(mfma)
        try:
            results[mfma] = torch.bmm(a.to(dev), b.to(dev)).cpu().float()
        finally:
            torch_vulkan.set_coop_enabled(True)
    want = oracle.gemm(f64(a), f64(b))
    for r in results.values():
        assert_gemm_close(r, want, torch.bfloat16, 90)
    assert torch.allclose(results[True], results[False], rtol=1.5e-2, atol=3e-2)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("m,k,n", [(1024, 192, 6144), (10240, 64, 640)])
def test_tile_aligned_fast_path_layouts_and_bias(dt, ta, tb, m, k, n):
    """Problems that fill the GPU with 128x256 (first shape) or 256x128 (second) tiles take the
    direct-to-LDS kernel; every operand layout, bias broadcast over rows, alpha and beta."""
    a, A = stored(m, k, dt, 13, ta)
    b, B = stored(k, n, dt, 14, tb)
    bias = randn((n,), dt, 15)
    out = torch.addmm(bias.to(dev), A, B, alpha=0.5, beta=2.0)
    ref = oracle.gemm(f64(a), f64(b), f64(bias), 0.5, 2.0)
    assert_gemm_close(out, ref, dt, k)
    assert oracle.rel_l2(f64(out), ref) <= (1e-2 if dt == torch.bfloat16 else 2e-3)


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("m,k,n", [(1024, 128, 1024), (512, 1088, 1024)])
def test_small_tile_fast_path_layouts_and_bias(ta, tb, m, k, n):
    """Tile-aligned problems too small for 128 x 256 tiles take the 64 x 64-tile direct-to-LDS kernel (the
    second shape has a K step count that is not a multiple of the three-buffer ring)."""
    dt = torch.bfloat16
    a, A = stored(m, k, dt, 23, ta)
    b, B = stored(k, n, dt, 24, tb)
    bias = randn((n,), dt, 25)
    out = torch.addmm(bias.to(dev), A, B, alpha=1.5, beta=0.5)
    ref = oracle.gemm(f64(a), f64(b), f64(bias), 1.5, 0.5)
    assert_gemm_close(out, ref, dt, k)
    assert oracle.rel_l2(f64(out), ref) <= 1e-2


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("m,k,n", [(4096, 192, 4096), (2048, 320, 8192)])
def test_large_tile_fast_path_layouts_and_bias(ta, tb, m, k, n):
    """Problems with at least 256 tiles of 256 x 256 take the 256 x 256-tile kernel with a two-buffer ring (odd
    K step counts: the loop's last step runs alone)."""
    dt = torch.bfloat16
    a, A = stored(m, k, dt, 33, ta)
    b, B = stored(k, n, dt, 34, tb)
    bias = randn((n,), dt, 35)
    out = torch.addmm(bias.to(dev), A, B, alpha=1.5, beta=0.5)
    ref = oracle.gemm(f64(a), f64(b), f64(bias), 1.5, 0.5)
    assert_gemm_close(out, ref, dt, k)
    assert oracle.rel_l2(f64(out), ref) <= 1e-2


# rank-16 LoRA factors of the DiT stack: (M, K, N) with the layouts autograd produces for
# h = x A^T, y = h B^T, dB = g^T h, dh = g B, dA = dh^T x, dx = dh A (ta / tb: operand given transposed)
SKINNY = [
    (1024, 2048, 16, False, True), (1024, 8192, 16, False, True),   # x A^T
    (1024, 16, 6144, False, True),                                   # h B^T (K = 16: no split)
    (6144, 1024, 16, True, False), (2048, 1024, 16, True, False),    # g^T h
    (1024, 8192, 16, False, False), (1024, 2048, 16, False, False),  # g B
    (16, 1024, 2048, True, False), (16, 1024, 8192, True, False),    # dh^T x
    (1024, 16, 2048, False, False),                                  # dh A
    (512, 4096, 512, False, False),                                  # 64 tiles, not one wide: no split
]


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,k,n,ta,tb", SKINNY)
def test_skinny_products_split_k(m, k, n, ta, tb, dt):
    """Products one 64-wide tile across split K over fp32 partials and a second, in-order reduction kernel;
    checked against the oracle (with addmm's bias, alpha and beta) and for run-to-run identity."""
    a, A = stored(m, k, dt, 41, ta)
    b, B = stored(k, n, dt, 42, tb)
    bias = randn((n,), dt, 43)
    out = torch.addmm(bias.to(dev), A, B, alpha=0.75, beta=1.25)
    ref = oracle.gemm(f64(a), f64(b), f64(bias), 0.75, 1.25)
    assert_gemm_close(out, ref, dt, k)
    assert oracle.rel_l2(f64(out), ref) <= 1e-2
    out2 = torch.addmm(bias.to(dev), A, B, alpha=0.75, beta=1.25)
    assert torch.equal(out.cpu(), out2.cpu())
    plain = torch.mm(A, B)
    assert oracle.rel_l2(f64(plain), oracle.gemm(f64(a), f64(b), None, 1.0, 0.0)) <= 1e-2


def test_tile_aligned_fast_path_batched_and_full_bias():
    bt, m, k, n = 2, 1024, 128, 6144
    a, b = randn((bt, m, k), torch.bfloat16, 16), randn((bt, k, n), torch.bfloat16, 17)
    bias = randn((bt, m, n), torch.bfloat16, 18)
    out = torch.baddbmm(bias.to(dev), a.to(dev), b.to(dev), alpha=1.5, beta=-1.0)
    ref = np.stack([oracle.gemm(f64(a[i]), f64(b[i]), f64(bias[i]), 1.5, -1.0) for i in range(bt)])
    assert_gemm_close(out, ref, torch.bfloat16, k)


def test_baseline_addmm_1024_cubed_with_bias():
    a, b, bias = randn((1024, 1024), torch.bfloat16, 1), randn((1024, 1024), torch.bfloat16, 2), randn((1024,), torch.bfloat16, 3)
    out = torch.addmm(bias.to(dev), a.to(dev), b.to(dev))
    ref = oracle.gemm(f64(a), f64(b), f64(bias), 1.0, 1.0)
    assert_gemm_close(out, ref, torch.bfloat16, 1024)
    assert oracle.rel_l2(f64(out), ref) <= 1e-2


@pytest.mark.parametrize("layout", ["nn", "linear"])
def test_baseline_gemm_1024x2048x8192(layout):
    M, K, N = 1024, 2048, 8192
    a = randn((M, K), torch.bfloat16, 1)
    if layout == "nn":
        b = randn((K, N), torch.bfloat16, 2)
        out = torch.mm(a.to(dev), b.to(dev))
        ref = oracle.gemm(f64(a), f64(b))
    else:  # F.linear: x @ W^T with W [N, K] read through its transpose view
        w = randn((N, K), torch.bfloat16, 2)
        out = torch.mm(a.to(dev), w.to(dev).t())
        ref = oracle.gemm(f64(a), f64(w).T)
    assert oracle.rel_l2(f64(out), ref) <= 1e-2
    assert_gemm_close(out, ref, torch.bfloat16, K)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False)])
@pytest.mark.parametrize("m,k,n", [(1024, 8192, 2048), (1024, 6144, 2048), (512, 6144, 2048), (1024, 2048, 2048)])
def test_wide_split_k_on_large_tiles(m, k, n, ta, tb, dt):
    """Products whose 128 x 256 tiles alone give fewer than 192 workgroups (the DiT stack's 1024 x 2048
    outputs) split K over the fast kernel's large tiles with fp32 partials (HRT_MM_F32_OUT) and the ordered
    mm_reduce: against the oracle with bias, alpha and beta, and bit-identical run to run."""
    a, A = stored(m, k, dt, 51, ta)
    b, B = stored(k, n, dt, 52, tb)
    bias = randn((n,), dt, 53)
    out = torch.addmm(bias.to(dev), A, B, alpha=0.5, beta=1.5)
    ref = oracle.gemm(f64(a), f64(b), f64(bias), 0.5, 1.5)
    assert_gemm_close(out, ref, dt, k)
    assert oracle.rel_l2(f64(out), ref) <= (1e-2 if dt == torch.bfloat16 else 4e-3)
    again = torch.addmm(bias.to(dev), A, B, alpha=0.5, beta=1.5)
    assert torch.equal(out.cpu(), again.cpu())
    assert_on_device("aten::addmm")


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("k", [2, 4, 8, 16, 32])
@pytest.mark.parametrize("m,n", [(1024, 2048), (37, 520), (5, 8), (300, 6144)])
@pytest.mark.parametrize("wlayout", ["nk", "kn"])
def test_short_k_products(dt, k, m, n, wlayout):
    """K <= 32 (a low-rank adapter's up-projection: y = h B^T with B [N, r], dx = dh A with A [r, K]) runs
    on the output-bound kernel: both layouts of the small factor, plain, with a row-broadcast bias, and
    accumulating into the output (y += h B^T), against float64."""
    h = randn((m, k), dt, m + k)
    if wlayout == "nk":  # B [N, K] read as its transposed view: k-contiguous
        w_store = randn((n, k), dt, n + 1, 0.1)
        w = w_store.t()
    else:                # A [K, N]: n-contiguous rows
        w_store = randn((k, n), dt, n + 2, 0.1)
        w = w_store
    bias = randn((n,), dt, n + 3)
    acc0 = randn((m, n), dt, n + 4)
    hd, wd = h.to(dev), w_store.to(dev)
    wd = wd.t() if wlayout == "nk" else wd
    ref = f64(h) @ f64(w)
    assert_gemm_close(hd @ wd, ref, dt, k)
    assert_gemm_close(torch.addmm(bias.to(dev), hd, wd, beta=0.5, alpha=2.0), 0.5 * f64(bias)[None, :] + 2.0 * ref, dt, k)
    assert_gemm_close(torch.addmm(acc0.to(dev), hd, wd), f64(acc0) + ref, dt, k)  # a full [M, N] bias
    assert_on_device("aten::mm", "aten::addmm")
    # accumulating in place (the bias is the output itself), through the C ABI
    from torch_vulkan import abi
    y = acc0.to(dev)
    a = abi.MmArgs()
    a.a, a.b, a.c, a.bias = hd.data_ptr(), wd.data_ptr(), y.data_ptr(), y.data_ptr()
    a.M, a.N, a.K, a.batch = m, n, k, 1
    a.a_sm, a.a_sk, a.b_sk, a.b_sn, a.c_sm, a.c_sn = hd.stride(0), hd.stride(1), wd.stride(0), wd.stride(1), n, 1
    a.bias_sm, a.bias_sn, a.has_bias, a.alpha, a.beta = n, 1, 1, 1.0, 1.0
    abi.Runtime().dispatch("mm_mfma_" + ("bf16" if dt == torch.bfloat16 else "f16"), a)
    assert_gemm_close(y, f64(acc0) + ref, dt, k)
    if m == 1024 and k == 16:
        assert torch.equal((hd @ wd).cpu(), (hd @ wd).cpu())  # deterministic


NARROW = [(1024, 16, 2048), (37, 3, 40), (2048, 16, 1024), (520, 1, 4096), (64, 12, 104), (136, 16, 4104),
          (1024, 16, 8192), (6144, 16, 1024), (72, 8, 3000)]


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("p,r,q", NARROW)
@pytest.mark.parametrize("form", ["x_At", "g_B", "gt_h", "dht_x", "A_xt"])
def test_narrow_output_products(dt, p, r, q, form):
    """An output side of at most 16 (a rank-r adapter: h = x A^T, dh = g B, dB = g^T h, dA = dh^T x, and
    A x^T) runs as one launch that splits the reduction over the wavefronts of a workgroup (and, for long
    reductions over few rows, over K slices added by a second kernel): every operand layout of those
    products, ragged P, R and Q (Q not a multiple of the 32-wide step, P not of the 16-row tile), addmm's
    bias x alpha/beta, accumulation in place through the C ABI, and run-to-run identity, against float64."""
    if form == "x_At":     # X [P, Q] q-contiguous, Y = A^T read along q
        x, w = randn((p, q), dt, 51), randn((r, q), dt, 52, 0.1)
        mk = lambda X, W: (X, W.mT)
    elif form == "g_B":    # Y [Q, R] r-contiguous
        x, w = randn((p, q), dt, 53), randn((q, r), dt, 54, 0.1)
        mk = lambda X, W: (X, W)
    elif form == "gt_h":   # X = g^T p-contiguous
        x, w = randn((q, p), dt, 55), randn((q, r), dt, 56, 0.1)
        mk = lambda X, W: (X.mT, W)
    elif form == "dht_x":  # output [R, P]: M = R
        w, x = randn((q, r), dt, 57, 0.1), randn((q, p), dt, 58)
        mk = lambda X, W: (W.mT, X)
    else:                  # A x^T: output [R, P], both operands k-contiguous
        w, x = randn((r, q), dt, 59, 0.1), randn((p, q), dt, 60)
        mk = lambda X, W: (W, X.mT)
    A64, B64 = mk(f64(x), f64(w))
    ref = A64 @ B64
    A, B = mk(x.to(dev), w.to(dev))
    m, n = ref.shape
    torch_vulkan.reset_fallback_counts()
    out = A @ B
    assert_gemm_close(out, ref, dt, q)
    bias = randn((n,), dt, 61)
    assert_gemm_close(torch.addmm(bias.to(dev), A, B, alpha=0.75, beta=1.25), 1.25 * f64(bias)[None, :] + 0.75 * ref, dt, q)
    assert_on_device("aten::mm", "aten::addmm")
    assert torch.equal(out.cpu(), (A @ B).cpu())
    from torch_vulkan import abi
    acc0 = randn((m, n), dt, 62)
    y = acc0.to(dev)
    a = abi.MmArgs()
    a.a, a.b, a.c, a.bias = A.data_ptr(), B.data_ptr(), y.data_ptr(), y.data_ptr()
    a.M, a.N, a.K, a.batch = m, n, q, 1
    a.a_sm, a.a_sk, a.b_sk, a.b_sn, a.c_sm, a.c_sn = A.stride(0), A.stride(1), B.stride(0), B.stride(1), n, 1
    a.bias_sm, a.bias_sn, a.has_bias, a.alpha, a.beta = n, 1, 1, 1.0, 1.0
    abi.Runtime().dispatch("mm_mfma_" + ("bf16" if dt == torch.bfloat16 else "f16"), a)
    assert_gemm_close(y, f64(acc0) + ref, dt, q)


@pytest.mark.parametrize("splits", [1, 2, 3, 4, 7])
@pytest.mark.parametrize("bias_kind", [None, "row", "full"])
def test_split_k_reduction_paths_agree(splits, bias_kind):
    """mm_reduce's vector path (8 outputs of a row per thread, C rows contiguous) and its general path (any
    output strides) add the slices in the same order: bit-identical bf16 results, checked against float64."""
    from torch_vulkan import abi
    M, N = 96, 136
    g = torch.Generator().manual_seed(splits)
    ws = torch.randn((splits, M, N), generator=g).to(dev)
    bias = None if bias_kind is None else randn((N,) if bias_kind == "row" else (M, N), torch.bfloat16, 70 + splits).to(dev)
    c_vec = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    c_gen_store = torch.empty((M, 2 * N), dtype=torch.bfloat16, device=dev)
    c_gen = c_gen_store[:, ::2]  # column stride 2: the general path
    for c in (c_vec, c_gen):
        r = abi.MmReduceArgs()
        r.ws, r.c = ws.data_ptr(), c.data_ptr()
        r.M, r.N, r.splits, r.c_sm, r.c_sn = M, N, splits, c.stride(0), c.stride(1)
        r.alpha, r.beta = 0.5, 1.5
        if bias is not None:
            r.bias, r.has_bias = bias.data_ptr(), 1
            r.bias_sm, r.bias_sn = (0, 1) if bias.dim() == 1 else (bias.stride(0), 1)
        abi.Runtime().dispatch("mm_reduce_bf16", r)
    assert torch.equal(c_vec.cpu(), c_gen.cpu())
    ref = 0.5 * ws.double().cpu().sum(0).numpy()
    if bias is not None:
        ref = ref + 1.5 * f64(bias)
    assert_gemm_close(c_vec, ref, torch.bfloat16, splits)


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [True, False])
@pytest.mark.parametrize("m,k,n", [(1024, 256, 6144), (2048, 128, 3072)])
def test_tiles_128x192(m, k, n, ta, tb):
    """Products whose N is a multiple of 192 and whose 128 x 192 tiles fill the GPU's rounds better than
    128 x 256 ones (a DiT block's QKV projection x W^T, N = 6144) take the 128 x 192 tile kernel when B is laid
    out along K (tb: B given as the transposed view of an [N, K] weight), either A layout; B laid out along N
    keeps the 128 x 256 tiles.  Against the oracle, with addmm's bias."""
    a, A = stored(m, k, torch.bfloat16, 81, ta)
    b, B = stored(k, n, torch.bfloat16, 82, tb, 0.1)
    bias = randn((n,), torch.bfloat16, 83)
    out = torch.addmm(bias.to(dev), A, B, alpha=0.5, beta=1.0)
    ref = oracle.gemm(f64(a), f64(b), f64(bias), 0.5, 1.0)
    assert_gemm_close(out, ref, torch.bfloat16, k)
    assert torch.equal(out.cpu(), torch.addmm(bias.to(dev), A, B, alpha=0.5, beta=1.0).cpu())


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [True, False])
@pytest.mark.parametrize("m,k,n", [(2048, 256, 2048), (1024, 192, 4096)])
def test_tiles_64x128(m, k, n, ta, tb, dt):
    """Products with too few 128 x 256 / 256 x 128 tiles to fill the GPU but several hundred 64 x 128 ones
    (2048^2 outputs) take the 64 x 128 tile kernel (four wavefronts of 32 x 64), every A and B layout, both
    16-bit types; against the oracle, with addmm's bias, and run to run bit-identical."""
    a, A = stored(m, k, dt, 91, ta)
    b, B = stored(k, n, dt, 92, tb, 0.1)
    bias = randn((n,), dt, 93)
    out = torch.addmm(bias.to(dev), A, B, alpha=0.5, beta=1.0)
    ref = oracle.gemm(f64(a), f64(b), f64(bias), 0.5, 1.0)
    assert_gemm_close(out, ref, dt, k)
    assert torch.equal(out.cpu(), torch.addmm(bias.to(dev), A, B, alpha=0.5, beta=1.0).cpu())


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [True, False])
@pytest.mark.parametrize("m,k,n", [(1024, 4096, 1024), (512, 4160, 1024), (256, 4288, 2048)])
def test_tiles_64x64_long_k_four_buffer_ring(m, k, n, ta, tb, dt):
    """Long reductions on 64 x 64 tiles (K >= 4096, at most 512 workgroups) copy three steps ahead through
    four LDS buffers; 64, 65 and 67 K steps, so the ring's last block is whole, or leaves 1 or 3 steps.
    Every layout, both 16-bit types, against the oracle, run to run bit-identical."""
    a, A = stored(m, k, dt, 94, ta)
    b, B = stored(k, n, dt, 95, tb, 0.1)
    bias = randn((n,), dt, 96)
    out = torch.addmm(bias.to(dev), A, B, alpha=0.5, beta=1.0)
    ref = oracle.gemm(f64(a), f64(b), f64(bias), 0.5, 1.0)
    assert_gemm_close(out, ref, dt, k)
    assert torch.equal(out.cpu(), torch.addmm(bias.to(dev), A, B, alpha=0.5, beta=1.0).cpu())


VERIFY_PROBE = """
import torch, torch_vulkan
g = torch.Generator().manual_seed(7)
for (m, k, n) in [(256, 512, 384), (1024, 1024, 1024), (64, 4096, 16)]:
    a = torch.randn((m, k), generator=g).to(torch.bfloat16)
    b = torch.randn((k, n), generator=g).to(torch.bfloat16)
    c = (a.to("vk") @ b.to("vk")).cpu().float()
    ref = a.float() @ b.float()
    err = ((c - ref).norm() / ref.norm()).item()
    assert err < 1e-2, (m, k, n, err)
print("PRODUCTS_OK")
"""


def test_verify_mm_cross_check_runs_silently_on_correct_products():
    """VKT_VERIFY_MM=1 (the reference's debug aid, csrc/ops_mm.cpp:148-172) recomputes every matrix-core
    product with the FMA kernel and reports calls whose results differ beyond a few ulp.  The variable is
    read once per process, so the products run in a child process: square, wide and narrow (split-K on the
    narrow-output kernel) bf16 products all pass the check without a report and match the CPU product."""
    import subprocess
    import sys

    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, VKT_VERIFY_MM="1")
    env["PYTHONPATH"] = os.pathsep.join([repo, os.path.join(repo, "torch-vulkan_amd"), env.get("PYTHONPATH", "")])
    r = subprocess.run([sys.executable, "-c", VERIFY_PROBE], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0 and "PRODUCTS_OK" in r.stdout, r.stderr[-800:]
    assert "VERIFY-MM" not in r.stderr, r.stderr[-800:]
