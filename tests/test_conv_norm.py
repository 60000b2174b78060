"""conv2d (forward, input/weight/bias gradients), nearest upsampling and group_norm on the vk device.

The reference's tests/test_conv.py and tests/test_group_norm.py fix the behaviours and the tolerances:
convolution and upsampling results within a relative L2 error of 2e-5 / 2e-2 / 4e-3 (float32 / bfloat16 /
float16) of the exact result, group_norm within a largest error of 5e-5 / 2.5e-2 / 4e-3 times
max(1, largest |reference|).  Here every result is checked against the oracle (float64 restatements):
convolutions as a table of named geometries (frozen weights and full gradients), the direct 3x3 kernel and
its C-ABI entry points, upsampling by integer factors, group_norm forward / backward / statistics up to
262144 elements per group, a VAE-decoder sized chain, and the kernels' argument checks.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

pytestmark = pytest.mark.gpu

import torch_vulkan  # noqa: E402
from torch_vulkan import abi  # noqa: E402

dev = torch.device("vk")
FLOATS = [torch.float32, torch.bfloat16, torch.float16]
REL_L2 = {torch.float32: 2e-5, torch.bfloat16: 2e-2, torch.float16: 4e-3}
GN_TOL = {torch.float32: 5e-5, torch.bfloat16: 2.5e-2, torch.float16: 4e-3}
CONV_KERNELS = ("aten::convolution_overrideable", "aten::convolution_backward_overrideable")


def sym(shape, dtype=torch.float32, seed=0, amp=1.0):
    """Seeded values uniform in [-amp, amp), rounded to dtype."""
    return torch.empty(shape).uniform_(-amp, amp, generator=torch.Generator().manual_seed(seed)).to(dtype)


def f64(t):
    return t.detach().cpu().double().numpy()


def assert_rel_l2(got, want, dt, what=""):
    g, w = f64(got), np.asarray(want, dtype=np.float64)
    assert g.shape == w.shape, (what, g.shape, w.shape)
    err = np.linalg.norm(g - w) / max(np.linalg.norm(w), 1e-12)
    assert err < REL_L2[dt], f"{what}: relative L2 error {err:.3g}"


def assert_gn_close(out, ref, dt, what="", mult=1.0):
    o, r = f64(out), np.asarray(ref, dtype=np.float64)
    assert o.shape == r.shape, (what, o.shape, r.shape)
    bound = GN_TOL[dt] * max(float(np.abs(r).max()), 1.0) * mult
    err = float(np.abs(o - r).max())
    assert err <= bound, f"{what}: largest error {err} > {bound}"


def assert_on_device(*names):
    fb = torch_vulkan.fallback_counts()
    hit = {n: fb[n] for n in names if n in fb}
    assert not hit, f"ran on the CPU: {hit}"


# ---- conv2d -------------------------------------------------------------------------------------------------
# name -> (N, C, H, W, Co, kernel (kh, kw), stride, padding)
CONV = {
    "3x3 same": (1, 8, 16, 16, 16, (3, 3), (1, 1), (1, 1)),
    "3x3 stride 2": (1, 8, 16, 16, 16, (3, 3), (2, 2), (1, 1)),
    "1x1 batched": (2, 6, 10, 12, 5, (1, 1), (1, 1), (0, 0)),
    "3x3 three channels": (2, 3, 9, 11, 4, (3, 3), (1, 1), (1, 1)),
    "3x3 stride 2 unpadded": (1, 5, 13, 7, 6, (3, 3), (2, 2), (0, 0)),
    "3x3 64 channels": (1, 64, 32, 32, 64, (3, 3), (1, 1), (1, 1)),
    "1x1 widening": (1, 16, 8, 8, 32, (1, 1), (1, 1), (0, 0)),
    "3x5 mixed stride": (2, 5, 17, 12, 7, (3, 5), (2, 1), (1, 2)),
}


def conv_case(name, dt, seed):
    """Input, weight, bias and an output gradient for a CONV geometry."""
    N, C, H, W, Co, (kh, kw), (sh, sw), (ph, pw) = CONV[name]
    x = sym((N, C, H, W), dt, seed)
    w = sym((Co, C, kh, kw), dt, seed + 1, amp=0.3)
    b = sym((Co,), dt, seed + 2)
    oh, ow = (H + 2 * ph - kh) // sh + 1, (W + 2 * pw - kw) // sw + 1
    gy = sym((N, Co, oh, ow), dt, seed + 3)
    return x, w, b, gy, (sh, sw), (ph, pw)


@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("name", list(CONV))
@pytest.mark.parametrize("dt", FLOATS)
def test_conv_with_frozen_weights(dt, name, bias):
    """Forward and the input gradient only (weights frozen, as in adapter training)."""
    x, w, b, gy, st, pad = conv_case(name, dt, 10)
    xd = x.to(dev).requires_grad_(True)
    y = F.conv2d(xd, w.to(dev), b.to(dev) if bias else None, stride=st, padding=pad)
    (gx,) = torch.autograd.grad(y, xd, gy.to(dev))
    assert_rel_l2(y, oracle.conv2d(f64(x), f64(w), f64(b) if bias else None, st, pad), dt, "y")
    assert_rel_l2(gx, oracle.conv2d_backward(f64(x), f64(w), f64(gy), st, pad)[0], dt, "dx")
    assert torch_vulkan.kernel_counts().get("aten::convolution_overrideable", 0) >= 1
    assert_on_device(*CONV_KERNELS)


@pytest.mark.parametrize("name", list(CONV))
@pytest.mark.parametrize("dt", FLOATS)
def test_conv_gradients_of_every_operand(dt, name):
    x, w, b, gy, st, pad = conv_case(name, dt, 20)
    ops = [t.to(dev).requires_grad_(True) for t in (x, w, b)]
    y = F.conv2d(*ops, stride=st, padding=pad)
    got = torch.autograd.grad(y, ops, gy.to(dev))
    want = oracle.conv2d_backward(f64(x), f64(w), f64(gy), st, pad)
    for g, r, what in zip(got, want, ("dx", "dw", "db")):
        assert_rel_l2(g, r, dt, what)
    assert_on_device(*CONV_KERNELS)


def test_conv_forms_the_kernels_do_not_take_still_match_the_cpu():
    """Grouped and dilated convolutions leave the device kernels and come back on the device."""
    x = sym((2, 6, 9, 9), seed=31)
    for w, kw in ((sym((6, 3, 3, 3), seed=32), dict(padding=1, groups=2)),
                  (sym((5, 6, 3, 3), seed=33), dict(padding=2, dilation=2)),
                  (sym((6, 1, 3, 3), seed=34), dict(padding=1, groups=6))):
        out = F.conv2d(x.to(dev), w.to(dev), None, **kw)
        assert out.device.type == "vk"
        assert_rel_l2(out, F.conv2d(x, w, None, **kw).numpy(), torch.float32, str(kw))


def test_conv_reads_a_non_contiguous_input():
    x, w, _, _, st, pad = conv_case("3x5 mixed stride", torch.float32, 40)
    xv = x.to(dev).mT.contiguous().mT  # same values, column-major spatial strides
    assert not xv.is_contiguous()
    out = F.conv2d(xv, w.to(dev), None, stride=st, padding=pad)
    assert_rel_l2(out, oracle.conv2d(f64(x), f64(w), None, st, pad), torch.float32, "strided input")


DIRECT = [  # (N, C, H, W, Co): shapes of the direct 3x3 kernel (stride 1, pad 1, C % 16, Co % 128, W % 64)
    (1, 16, 1, 64, 128),
    (2, 32, 3, 128, 256),
    (1, 48, 5, 64, 128),
    (1, 128, 16, 64, 128),
    (1, 512, 64, 64, 512),
]


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", DIRECT)
@pytest.mark.parametrize("bias", [True, False])
def test_conv3x3_direct_forward_and_input_grad(dt, case, bias):
    """3x3 / stride 1 / padding 1 convolutions that the direct kernel (conv3x3: an implicit GEMM over staged
    input rows, no column matrix) takes: forward with and without bias, and the input gradient (the same
    kernel on the output gradient with the flipped, transposed kernel when C % 128 == 0), against the oracle;
    1- and 3-row images exercise the zero rows above and below, 128-pixel rows two segments per row."""
    N, C, H, W, Co = case
    before = torch_vulkan.kernel_counts().get("torch_vulkan::conv3x3", 0)
    x = sym((N, C, H, W), dt, 11)
    w = sym((Co, C, 3, 3), dt, 12, amp=0.3)
    b = sym((Co,), dt, 13) if bias else None
    r = sym((N, Co, H, W), torch.float32, 14)
    ref = oracle.conv2d(f64(x), f64(w), f64(b) if bias else None, (1, 1), (1, 1))
    xd = x.to(dev).requires_grad_(True)
    out = F.conv2d(xd, w.to(dev), b.to(dev) if bias else None, padding=1)
    assert_rel_l2(out, ref, dt, "forward")
    runs = 1
    if C * H * W <= 128 * 16 * 64:  # the oracle's backward is slow at the full size
        gref, _, _ = oracle.conv2d_backward(f64(x), f64(w), f64(r.to(dt)), (1, 1), (1, 1))
        (out * r.to(dt).to(dev)).sum().backward()
        assert_rel_l2(xd.grad, gref, dt, "grad_input")
        runs += C % 128 == 0  # the input gradient takes the direct kernel when C is a multiple of 128
    assert_on_device("aten::convolution_overrideable", "aten::convolution_backward_overrideable")
    assert torch_vulkan.kernel_counts().get("torch_vulkan::conv3x3", 0) - before == runs


def test_conv3x3_im2col_switch(monkeypatch):
    """VKT_CONV_IM2COL=1 keeps the unfolding + GEMM for a shape the direct kernel takes: same convolution
    (to bf16 tolerance against the oracle), and the direct kernel's counter does not move."""
    x = sym((1, 32, 4, 64), torch.bfloat16, 31)
    w = sym((128, 32, 3, 3), torch.bfloat16, 32, amp=0.3)
    ref = oracle.conv2d(f64(x), f64(w), None, (1, 1), (1, 1))
    monkeypatch.setenv("VKT_CONV_IM2COL", "1")
    before = torch_vulkan.kernel_counts().get("torch_vulkan::conv3x3", 0)
    assert_rel_l2(F.conv2d(x.to(dev), w.to(dev), None, padding=1), ref, torch.bfloat16, "unfolded")
    assert torch_vulkan.kernel_counts().get("torch_vulkan::conv3x3", 0) == before


def test_conv3x3_weight_view_at_odd_offset():
    """A contiguous weight view at an odd element offset (a weight inside a flat parameter buffer) is not
    16-byte aligned: the convolution takes the unfolding + GEMM path instead of the direct kernel, with no
    error and the oracle's result, forward and input gradient."""
    x = sym((1, 128, 4, 64), torch.bfloat16, 41)
    w = sym((128, 128, 3, 3), torch.bfloat16, 42, amp=0.3)
    r = sym((1, 128, 4, 64), torch.bfloat16, 43)
    flat = torch.zeros(1 + w.numel(), dtype=torch.bfloat16, device=dev)
    flat[1:] = w.reshape(-1).to(dev)
    wv = flat[1:].view(128, 128, 3, 3)  # contiguous, 2 bytes past a 16-byte boundary
    assert wv.is_contiguous() and wv.data_ptr() % 16 != 0
    before = torch_vulkan.kernel_counts().get("torch_vulkan::conv3x3", 0)
    xd = x.to(dev).requires_grad_(True)
    out = F.conv2d(xd, wv, None, padding=1)
    assert_rel_l2(out, oracle.conv2d(f64(x), f64(w), None, (1, 1), (1, 1)), torch.bfloat16, "forward")
    (out * r.to(dev)).sum().backward()
    gref, _, _ = oracle.conv2d_backward(f64(x), f64(w), f64(r), (1, 1), (1, 1))
    assert_rel_l2(xd.grad, gref, torch.bfloat16, "grad_input")
    assert torch_vulkan.kernel_counts().get("torch_vulkan::conv3x3", 0) == before
    assert_on_device("aten::convolution_overrideable", "aten::convolution_backward_overrideable")


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("flip", [0, 1])
@pytest.mark.parametrize("splits", [1, 2])
def test_conv3x3_c_abi(dt, flip, splits):
    """The two entry points called directly: conv3x3_wprep reorders [O, I, 3, 3] (flip 0) or reads
    [I, O, 3, 3] as its flipped transpose (flip 1), and conv3x3 then gives the convolution (flip 0) or the
    input gradient of the convolution with w (flip 1), against the oracle, with the input channels in one
    piece or split in two (fp32 partial sums added by the same call); an odd row count leaves the last
    workgroup's second output row outside the image.  The argument checks reject channel counts the kernel
    does not take and splits that do not divide the channel blocks."""
    N, H, W, c_small, c_big = 2, 3, 128, 32, 128
    name = "bf16" if dt == torch.bfloat16 else "f16"
    rt = abi.Runtime()
    if flip == 0:  # x [N, 32, H, W], w [128, 32, 3, 3] -> y [N, 128, H, W]
        xin = sym((N, c_small, H, W), dt, 21)
        w = sym((c_big, c_small, 3, 3), dt, 22, amp=0.3)
        ref = oracle.conv2d(f64(xin), f64(w), None, (1, 1), (1, 1))
        I, O = c_small, c_big
    else:  # the input gradient of conv(x [N, 128, H, W], w [32, 128, 3, 3]): dy [N, 32, H, W] -> dx [N, 128, H, W]
        xin = sym((N, c_small, H, W), dt, 23)
        w = sym((c_small, c_big, 3, 3), dt, 24, amp=0.3)
        ref, _, _ = oracle.conv2d_backward(np.zeros((N, c_big, H, W)), f64(w), f64(xin), (1, 1), (1, 1))
        I, O = c_small, c_big
    xd, wd = xin.to(dev), w.to(dev)
    wr = torch.empty(abi.conv3_wr_bytes(O, I) // 2, dtype=dt, device=dev)
    y = torch.empty((N, O, H, W), dtype=dt, device=dev)
    ws = torch.empty(splits * N * O * H * W, dtype=torch.float32, device=dev)
    P = abi.Conv3WprepArgs()
    P.w, P.wr, P.O, P.I, P.flip = wd.data_ptr(), wr.data_ptr(), O, I, flip
    rt.dispatch("conv3x3_wprep_" + name, P)
    A = abi.Conv3Args()
    A.x, A.wr, A.y, A.N, A.I, A.O, A.H, A.W = xd.data_ptr(), wr.data_ptr(), y.data_ptr(), N, I, O, H, W
    A.ws, A.splits = (ws.data_ptr() if splits > 1 else 0), splits
    rt.dispatch("conv3x3_" + name, A)
    assert_rel_l2(y, ref, dt, f"conv3x3 flip {flip} splits {splits}")
    bad = abi.Conv3Args.from_buffer_copy(A)
    bad.O = 64  # not a multiple of 128
    with pytest.raises(RuntimeError):
        rt.dispatch("conv3x3_" + name, bad)
    bad = abi.Conv3Args.from_buffer_copy(A)
    bad.splits = 3  # does not divide I / 16 = 2
    with pytest.raises(RuntimeError):
        rt.dispatch("conv3x3_" + name, bad)


# ---- nearest upsampling --------------------------------------------------------------------------------------
@pytest.mark.parametrize("shape,factor", [((1, 4, 8, 8), 2), ((2, 3, 5, 7), (2, 3)), ((1, 2, 4, 6), 1),
                                          ((1, 2, 4, 8), (3, 2)), ((1, 3, 3, 8), 3), ((2, 8, 16, 32), 2)])
@pytest.mark.parametrize("dt", FLOATS)
def test_nearest_upsampling_by_integer_factors(dt, shape, factor):
    fh, fw = (factor, factor) if isinstance(factor, int) else factor
    x = sym(shape, dt, 1)
    xd = x.to(dev).requires_grad_(True)
    y = F.interpolate(xd, scale_factor=factor, mode="nearest")
    want = torch.from_numpy(oracle.upsample_nearest(f64(x), shape[2] * fh, shape[3] * fw)).to(dt)
    assert torch.equal(y.cpu(), want)  # a copy of input elements: exact
    gy = sym(tuple(y.shape), dt, 2)
    (gx,) = torch.autograd.grad(y, xd, gy.to(dev))
    assert_rel_l2(gx, oracle.upsample_nearest_backward(f64(gy), shape[2], shape[3]), dt, "dx")
    assert_on_device("aten::upsample_nearest2d", "aten::upsample_nearest2d_backward")


def test_nearest_upsampling_to_a_non_multiple_size_matches_the_cpu():
    x = sym((1, 2, 5, 5), seed=3)
    for size in ((8, 8), (7, 11)):
        assert torch.equal(F.interpolate(x.to(dev), size=size, mode="nearest").cpu(), F.interpolate(x, size=size, mode="nearest"))


# ---- group_norm ------------------------------------------------------------------------------------------------
SHAPES = [((2, 8, 5, 5), 4), ((1, 6, 3, 7), 3), ((3, 4, 9), 2), ((2, 32, 16, 16), 32), ((1, 64, 8, 8), 32),
          ((2, 12, 1, 1), 4),
          # the reference's shapes (tests/test_group_norm.py:17-24): SD-scale channel counts
          ((1, 320, 64, 64), 32), ((1, 1280, 8, 8), 32), ((1, 2560, 16, 16), 32), ((2, 64, 8, 8), 4), ((2, 96, 5, 7), 3),
          ((2, 32, 1, 1), 32)]


@pytest.mark.parametrize("dt", FLOATS)
@pytest.mark.parametrize("affine", [True, False])
@pytest.mark.parametrize("eps", [1e-5, 1e-6])
@pytest.mark.parametrize("shape,G", SHAPES)
def test_group_norm_forward(dt, affine, eps, shape, G):
    x = sym(shape, dt, 1, 3.0)
    C = shape[1]
    w = sym((C,), dt, 2) if affine else None
    b = sym((C,), dt, 3) if affine else None
    out = F.group_norm(x.to(dev), G, w.to(dev) if affine else None, b.to(dev) if affine else None, eps)
    assert out.dtype == dt
    y, _, _ = oracle.group_norm_fwd(f64(x), G, f64(w) if affine else None, f64(b) if affine else None, eps)
    assert_gn_close(out, y, dt, "y")
    assert_on_device("aten::native_group_norm")


@pytest.mark.parametrize("dt", FLOATS)
def test_group_norm_mean_rstd_dtype_and_shape_match_cpu(dt):
    x = sym((2, 8, 4, 4), dt, 5)
    gpu = torch.native_group_norm(x.to(dev), None, None, 2, 8, 16, 4, 1e-5)
    cpu = torch.native_group_norm(x, None, None, 2, 8, 16, 4, 1e-5)
    for c, g in zip(cpu, gpu):
        assert c.dtype == g.dtype and c.shape == g.shape
    _, mean, rstd = oracle.group_norm_fwd(f64(x), 4, eps=1e-5)
    assert_gn_close(gpu[1], mean, dt, "mean")
    assert_gn_close(gpu[2], rstd, dt, "rstd")


@pytest.mark.parametrize("dt", FLOATS)
@pytest.mark.parametrize("affine", [True, False])
@pytest.mark.parametrize("shape,G", SHAPES)
def test_group_norm_backward(dt, affine, shape, G):
    x = sym(shape, dt, 6, 2.0)
    C = shape[1]
    w = sym((C,), dt, 7) if affine else None
    b = sym((C,), dt, 8) if affine else None
    g = sym(shape, dt, 9)
    xd = x.to(dev).requires_grad_(True)
    params = [t.to(dev).requires_grad_(True) for t in (w, b)] if affine else [None, None]
    out = F.group_norm(xd, G, params[0], params[1], 1e-5)
    out.backward(g.to(dev))
    _, mean, rstd = oracle.group_norm_fwd(f64(x), G, eps=1e-5)
    dx, dw, db = oracle.group_norm_bwd(f64(g), f64(x), mean, rstd, G, f64(w) if affine else None)
    assert_gn_close(xd.grad, dx, dt, "dx", mult=2.0)
    if affine:
        assert params[0].grad.dtype == dt and params[1].grad.dtype == dt
        assert_gn_close(params[0].grad, dw, dt, "dw", mult=8.0)
        assert_gn_close(params[1].grad, db, dt, "db", mult=8.0)
    assert_on_device("aten::native_group_norm", "aten::native_group_norm_backward")


def test_group_norm_non_contiguous_input_and_weight_dtype():
    x = sym((2, 16, 8, 12), torch.float32, 11)
    w, b = sym((16,), seed=12), sym((16,), seed=13)
    out = F.group_norm(x.to(dev)[:, :, :, ::2], 8, w.to(dev), b.to(dev), 1e-5)
    y, _, _ = oracle.group_norm_fwd(f64(x[:, :, :, ::2]), 8, f64(w), f64(b), 1e-5)
    assert_gn_close(out, y, torch.float32)
    xb = x.to(torch.bfloat16)
    out = F.group_norm(xb.to(dev), 8, w.to(dev), b.to(dev), 1e-5)  # fp32 affine parameters on bf16 input
    y, _, _ = oracle.group_norm_fwd(f64(xb), 8, f64(w.to(torch.bfloat16)), f64(b.to(torch.bfloat16)), 1e-5)
    assert_gn_close(out, y, torch.bfloat16)


@pytest.mark.parametrize("HW,G", [(512 * 512, 32), (128 * 128, 8)])
def test_group_norm_chunked_statistics(HW, G):
    """Groups of 262144 and 32768 elements with a large mean offset: chunked, shifted fp32 statistics."""
    C = 64
    x = (sym((1, C, HW), torch.float32, 14) + 20.0)
    out, mean, rstd = torch.native_group_norm(x.to(dev), None, None, 1, C, HW, G, 1e-6)
    y, m, r = oracle.group_norm_fwd(f64(x), G, eps=1e-6)
    assert_gn_close(mean, m, torch.float32, "mean")
    assert_gn_close(rstd, r, torch.float32, "rstd", mult=4.0)
    assert_gn_close(out, y, torch.float32, "y", mult=4.0)


@pytest.mark.parametrize("shape", [(2, 512, 80, 80), (2, 256, 128, 127)])
def test_group_norm_large_apply_blocks_with_ragged_tail(shape):
    """Groups of 102400 / 130048 elements in >= 256 apply blocks of 16384: the last block of each group
    is partial (vector and scalar loads), with bf16 affine parameters."""
    G, dt = 32, torch.bfloat16
    x = sym(shape, dt, 15)
    w, b = sym((shape[1],), dt, 16), sym((shape[1],), dt, 17)
    out = F.group_norm(x.to(dev), G, w.to(dev), b.to(dev), 1e-6)
    y, _, _ = oracle.group_norm_fwd(f64(x), G, f64(w), f64(b), 1e-6)
    assert_gn_close(out, y, dt)


def test_vae_decoder_block_chain():
    """conv3x3 -> group_norm -> silu -> upsample x2 -> conv3x3 in bf16 at 64x64, forward and backward."""
    dt = torch.bfloat16
    x = sym((1, 128, 64, 64), dt, 20)
    w1, w2 = sym((128, 128, 3, 3), dt, 21, 0.05), sym((64, 128, 3, 3), dt, 22, 0.05)
    gw, gb = sym((128,), dt, 23), sym((128,), dt, 24)
    xd = x.to(dev).requires_grad_(True)
    h = F.conv2d(xd, w1.to(dev), None, padding=1)
    h = F.silu(F.group_norm(h, 32, gw.to(dev), gb.to(dev), 1e-6))
    h = F.interpolate(h, scale_factor=2, mode="nearest")
    y = F.conv2d(h, w2.to(dev), None, padding=1)
    g = sym(y.shape, dt, 25)
    y.backward(g.to(dev))
    # reference: the same chain in float64 torch from the same bf16 inputs
    xc = torch.from_numpy(f64(x)).requires_grad_(True)
    hc = F.conv2d(xc, torch.from_numpy(f64(w1)), None, padding=1)
    hc = F.silu(F.group_norm(hc, 32, torch.from_numpy(f64(gw)), torch.from_numpy(f64(gb)), 1e-6))
    hc = F.interpolate(hc, scale_factor=2, mode="nearest")
    yc = F.conv2d(hc, torch.from_numpy(f64(w2)), None, padding=1)
    yc.backward(torch.from_numpy(f64(g)))
    assert_rel_l2(y, yc.detach().numpy(), dt, "y")
    assert_rel_l2(xd.grad, xc.grad.numpy(), dt, "dx")
    assert_on_device("aten::convolution_overrideable", "aten::convolution_backward_overrideable", "aten::native_group_norm",
                "aten::native_group_norm_backward", "aten::upsample_nearest2d", "aten::upsample_nearest2d_backward")


# ---- argument checks through the C ABI ----------------------------------------------------------------------
def test_c_abi_rejects_inconsistent_shapes():
    rt = abi.Runtime()
    x = torch.zeros(1, 2, 8, 8, device=dev)
    cols = torch.zeros(1, 18, 64, device=dev)
    a = abi.Im2colArgs()
    a.x, a.cols, a.N, a.C, a.H, a.W, a.OH, a.OW, a.KH, a.KW, a.SH, a.SW, a.PH, a.PW = (
        x.data_ptr(), cols.data_ptr(), 1, 2, 8, 8, 8, 8, 3, 3, 1, 1, 1, 1)
    rt.dispatch("im2col_f32", a)  # consistent: accepted
    a.OH = 9
    with pytest.raises(RuntimeError, match="OH/OW"):
        rt.dispatch("im2col_f32", a)
    u = abi.UpsampleArgs()
    u.src, u.dst, u.NC, u.H, u.W, u.OH, u.OW = x.data_ptr(), cols.data_ptr(), 2, 8, 8, 12, 8
    with pytest.raises(RuntimeError, match="integer factors"):
        rt.dispatch("upsample_nearest_fwd_f32", u)
    gn = abi.GnArgs()
    gn.x, gn.N, gn.C, gn.HW, gn.G = x.data_ptr(), 1, 2, 64, 3
    with pytest.raises(RuntimeError, match="G dividing C"):
        rt.dispatch("gn_fwd_f32", gn)
    rt.synchronize()
