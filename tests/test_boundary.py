"""CPU checks of the boundary (no GPU needed): the C-ABI library loads and exports every symbol that
include/*.h declares, the shim registers the reference's operator surface on PrivateUse1, the kernel
registry knows every kernel name the shim asks for, and the slab allocator passes its host test."""

import ctypes
import os
import re
import subprocess

import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "torch-vulkan_amd")
LIBHRT = os.path.join(PKG, "torch_vulkan", "libhrt.so")


def declared_functions():
    names = []
    for h in ("hrt.h", "hrt_ops.h"):
        text = open(os.path.join(REPO, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"static inline[^{]*\{[^}]*\}", "", text)  # header-only helpers are not exported
        names += re.findall(r"\b(hrt_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_libhrt_exports_every_declared_symbol():
    assert os.path.exists(LIBHRT), "libhrt.so is not built (python torch-vulkan_amd/build.py)"
    lib = ctypes.CDLL(LIBHRT)
    names = declared_functions()
    assert len(names) >= 27, names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_runtime_reports_errors_without_a_device():
    """Without hrt_init (and without a GPU here) every call fails cleanly with a message."""
    lib = ctypes.CDLL(LIBHRT)
    lib.hrt_alloc.restype = ctypes.c_uint64
    lib.hrt_alloc.argtypes = [ctypes.c_uint64]
    lib.hrt_last_error.restype = ctypes.c_size_t
    lib.hrt_last_error.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
    lib.hrt_kernel_index.argtypes = [ctypes.c_char_p]
    if torch.cuda.is_available():
        pytest.skip("a GPU is present; the uninitialised-runtime path is only checked on CPU hosts")
    assert lib.hrt_alloc(1024) == 0
    buf = ctypes.create_string_buffer(256)
    lib.hrt_last_error(buf, 256)
    assert b"hrt_init" in buf.value
    # the kernel table is static: names resolve without a device
    assert lib.hrt_kernel_index(b"dq8_bf16") >= 0
    assert lib.hrt_kernel_index(b"no_such_kernel") == -1


KERNELS = (
    ["add_f32", "ew_copy", "ew_fill", "ew_map", "reduce_sum", "cat_rows16"]
    + [f"{op}_{k}" for op in ("im2col", "col2im", "upsample_nearest_fwd", "upsample_nearest_bwd", "gn_fwd", "gn_bwd")
       for k in ("f32", "bf16", "f16")]
    + [f"dq8_{k}" for k in ("f32", "bf16", "f16")]
    + [f"mm_{k}" for k in ("f32", "bf16", "f16")]
    + [f"mm_mfma_{k}" for k in ("bf16", "f16")]
    + [f"softmax_{d}_{k}" for d in ("fwd", "bwd") for k in ("f32", "bf16", "f16")]
    + [f"ln_{d}_{k}" for d in ("fwd", "bwd", "wgrad") for k in ("f32", "bf16", "f16")]
    + [f"attn_{op}_fma_{k}" for op in ("fwd", "dkdv", "dq") for k in ("f32", "bf16", "f16")]
    + [f"attn_{op}_mfma_{k}" for op in ("fwd", "dkdv", "dq") for k in ("bf16", "f16")]
    + [f"attn_delta_{k}" for k in ("f32", "bf16", "f16")]
    + [f"mm_dq8_{k}" for k in ("bf16", "f16")]
    + [f"mm_reduce_{k}" for k in ("bf16", "f16")]
    + [f"conv3x3_{k}" for k in ("bf16", "f16")] + [f"conv3x3_wprep_{k}" for k in ("bf16", "f16")]
)


@pytest.mark.parametrize("name", KERNELS)
def test_kernel_registry_has(name):
    lib = ctypes.CDLL(LIBHRT)
    lib.hrt_kernel_index.argtypes = [ctypes.c_char_p]
    assert lib.hrt_kernel_index(name.encode()) >= 0, name


def test_shim_registers_the_reference_operator_surface():
    import torch_vulkan  # noqa: F401  (loads the shim; no device needed)

    ops = [
        "aten::mm", "aten::bmm", "aten::addmm", "aten::baddbmm",
        "aten::_scaled_dot_product_fused_attention_overrideable",
        "aten::_scaled_dot_product_fused_attention_overrideable_backward",
        "aten::_softmax", "aten::_safe_softmax", "aten::_softmax_backward_data",
        "aten::native_layer_norm", "aten::native_layer_norm_backward",
        "aten::empty.memory_format", "aten::empty_strided", "aten::_copy_from", "aten::_copy_from_and_resize",
        "aten::view", "aten::as_strided", "aten::_reshape_alias", "aten::resize_", "aten::fill_.Scalar", "aten::zero_",
    ] + [  # elementwise (csrc/ops_ew.cpp:510-550)
        f"aten::{n}" for n in (
            "add.Tensor", "add_.Tensor", "sub.Tensor", "sub_.Tensor", "mul.Tensor", "mul_.Tensor", "div.Tensor",
            "div_.Tensor", "neg", "rsqrt", "reciprocal", "exp", "sin", "cos", "sqrt", "tanh", "sigmoid", "relu",
            "silu", "pow.Tensor_Scalar", "gelu", "silu_backward", "gelu_backward", "where.self", "addcmul_",
            "addcdiv_", "addcmul", "addcdiv", "lerp_.Scalar", "lerp.Scalar", "add.Scalar", "add_.Scalar",
            "sub.Scalar", "sub_.Scalar", "mul.Scalar", "mul_.Scalar", "div.Scalar", "div_.Scalar",
            "sum.dim_IntList", "mean.dim", "sum", "mean", "cat",  # + csrc/ops_rows.cpp:342-346
            "convolution_overrideable", "convolution_backward_overrideable", "upsample_nearest2d",
            "upsample_nearest2d_backward", "native_group_norm", "native_group_norm_backward")  # ops_conv/ops_norm
    ]
    missing = [o for o in ops if not torch._C._dispatch_has_kernel_for_dispatch_key(o, "PrivateUse1")]
    assert not missing, missing
    assert torch._C._get_privateuse1_backend_name() == "vk"
    assert hasattr(torch, "vk") and torch.vk.device_count() == 1


# The reference's pybind surface (csrc/shim.cpp:418-493, its m.def names in order).
REFERENCE_PYBIND = (
    "init", "dequant_int8", "device_name", "max_alloc", "live_bytes", "memory_info", "peak_live_bytes",
    "reset_peak_live_bytes", "set_memory_limit", "synchronize", "empty_cache", "reserved_bytes", "live_blocks",
    "slab_count", "validation_errors", "fallback_counts", "kernel_counts", "stats", "fallback_time_by_op",
    "profile", "coop_caps", "set_coop_enabled", "set_fused_attention", "set_coop_range", "reset_coop_calls",
    "coop_calls", "reset_counts",
)


def test_shim_module_has_the_reference_pybind_names():
    """Every function the reference's extension module defines exists in this one (code that calls
    torch_vulkan._C.<name> directly keeps working), and _C.stats() has the reference's keys (no device needed:
    the runtime's counters read zero)."""
    import torch_vulkan

    missing = [n for n in REFERENCE_PYBIND if not hasattr(torch_vulkan._C, n)]
    assert not missing, missing
    keys = {"dispatch_s", "dispatch_n", "transfer_s", "transfer_n", "pipeline_create_s", "upload_MB", "download_MB",
            "gpu_wait_s", "fallback_s"}
    try:
        st = torch_vulkan._C.stats()
    except RuntimeError as e:  # no device in this container: the runtime cannot initialise
        assert "vk" in str(e) or "device" in str(e).lower() or "hip" in str(e).lower(), e
    else:
        assert set(st) == keys, sorted(st)


def test_slab_allocator_host(tmp_path):
    """Compiles tests/cpu/allocator_test.cpp against the runtime's allocator with ASan/UBSan (host code)."""
    exe = tmp_path / "alloc_test"
    src = os.path.join(REPO, "tests", "cpu", "allocator_test.cpp")
    inc = os.path.join(PKG, "csrc", "hrt")
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-I", inc, src, "-o", str(exe)],
                   check=True)
    r = subprocess.run([str(exe)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0 and "ALL OK" in r.stdout, r.stdout


def test_python_abi_structs_match_the_c_headers(tmp_path):
    """torch_vulkan/abi.py mirrors include/hrt_ops.h: same size and field offsets for every argument block."""
    from torch_vulkan import abi

    structs = {
        "hrt_add_f32_args": abi.AddF32Args, "hrt_copy_args": abi.CopyArgs, "hrt_fill_args": abi.FillArgs, "hrt_ew_args": abi.EwArgs, "hrt_reduce_args": abi.ReduceArgs,
        "hrt_cat_args": abi.CatArgs,
        "hrt_im2col_args": abi.Im2colArgs, "hrt_conv3_wprep_args": abi.Conv3WprepArgs, "hrt_conv3_args": abi.Conv3Args, "hrt_upsample_args": abi.UpsampleArgs, "hrt_gn_args": abi.GnArgs,
        "hrt_mm_args": abi.MmArgs, "hrt_mm_dq8_args": abi.MmDq8Args, "hrt_mm_reduce_args": abi.MmReduceArgs,
        "hrt_attn_args": abi.AttnArgs,
        "hrt_softmax_args": abi.SoftmaxArgs, "hrt_ln_args": abi.LnArgs, "hrt_dq8_args": abi.Dq8Args,
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "hrt_ops.h"', "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'  printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    ln_shapes = [(1, 1), (5, 7), (1023, 2048), (1024, 2048), (1024, 4096), (1024, 8192), (2048, 2048), (4096, 2048),
                 (4096, 4096), (100000, 64), (3, 5000)]
    for rows, D in ln_shapes:
        lines.append(f'  printf("ln_chunks {rows}x{D} %lld\\n", (long long)hrt_ln_chunks({rows}, {D}));')
    lines.append("  return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(REPO, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], stdout=subprocess.PIPE, text=True, check=True).stdout.split("\n")
    got = {tuple(l.split()[:2]): int(l.split()[2]) for l in out if l.strip()}
    for cname, py in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for fname, _ in py._fields_:
            assert got[(cname, fname)] == getattr(py, fname).offset, (cname, fname)
    for rows, D in ln_shapes:  # the Python mirror of the chunking rule computes what the header does
        assert got[("ln_chunks", f"{rows}x{D}")] == abi.ln_chunks(rows, D), (rows, D)
    assert abi.ln_chunks(1024, 2048) == 128 and abi.ln_chunks(4096, 2048) == 256 and abi.ln_chunks(5, 7) == 2


def test_conv3_sizes_and_splits_match_the_c_header(tmp_path):
    """abi.conv3_wr_bytes / abi.conv3_splits compute what hrt_conv3_wr_bytes / hrt_conv3_splits do, over
    image sizes and channel counts around the split rule's thresholds (256 workgroups, 4 channel blocks)."""
    from torch_vulkan import abi

    cases = [(n, i, o, h, w) for n in (1, 2, 3) for i in (16, 64, 128, 512) for o in (128, 512) for h in (1, 5, 16, 64)
             for w in (64, 128)]
    lines = ['#include <stdio.h>', '#include "hrt_ops.h"', "int main(void) {"]
    for n, i, o, h, w in cases:
        lines.append(f'  printf("%lld %lld\\n", (long long)hrt_conv3_wr_bytes({o}, {i}), '
                     f'(long long)hrt_conv3_splits({n}, {i}, {o}, {h}, {w}));')
    lines.append("  return 0; }")
    src = tmp_path / "conv3.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "conv3"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(REPO, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], stdout=subprocess.PIPE, text=True, check=True).stdout.split("\n")
    got = [tuple(map(int, l.split())) for l in out if l.strip()]
    assert got == [(abi.conv3_wr_bytes(o, i), abi.conv3_splits(n, i, o, h, w)) for n, i, o, h, w in cases]
    assert abi.conv3_splits(1, 512, 512, 64, 64) == 2 and abi.conv3_splits(1, 128, 128, 16, 64) == 2


def test_python_ew_op_codes_match_the_c_header(tmp_path):
    """abi.EW_OPS names the hrt_ew_op codes of include/hrt_ops.h in order."""
    from torch_vulkan import abi

    enum = {n: "HRT_EW_" + n.upper() for n in abi.EW_OPS}
    lines = ['#include <stdio.h>', '#include "hrt_ops.h"', "int main(void) {"]
    lines += [f'  printf("{n} %d\\n", (int){c});' for n, c in enum.items()]
    lines += ['  printf("count %d\\n", (int)HRT_EW_OP_COUNT);', "  return 0; }"]
    src = tmp_path / "ew_ops.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "ew_ops"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(REPO, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], stdout=subprocess.PIPE, text=True, check=True).stdout.split()
    got = dict(zip(out[::2], map(int, out[1::2])))
    assert got.pop("count") == len(abi.EW_OPS)
    assert got == abi.EW_OPS


def test_reduce_workspace_plan_on_the_host():
    """hrt_reduce_workspace is a pure host function: the fp32 partial-sum workspace "reduce_sum" needs."""
    from torch_vulkan import abi

    lib = ctypes.CDLL(LIBHRT)
    lib.hrt_reduce_workspace.restype = ctypes.c_int64
    lib.hrt_reduce_workspace.argtypes = [ctypes.c_void_p]

    def ws(sizes, strides, mask, dt=abi.BF16, x=1 << 20):
        a = abi.ReduceArgs()
        a.x, a.ndim, a.x_dtype, a.out_dtype, a.reduce_mask, a.div = x, len(sizes), dt, dt, mask, 1.0
        for i, (s, t) in enumerate(zip(sizes, strides)):
            a.sizes[i], a.strides[i] = s, t
        return lib.hrt_reduce_workspace(ctypes.byref(a))

    assert ws([4096, 2048], [2048, 1], 0b10) == 0              # one workgroup per row: no split
    n = ws([1024, 8192], [8192, 1], 0b01)                       # bias gradient: split over rows
    assert n > 0 and n % 8192 == 0 and n // 8192 <= 1024
    assert ws([1 << 20], [1], 0b1) > 0                          # full sum: split, one output
    assert ws([3, 0], [0, 1], 0b10) == 0                        # empty sums
    assert ws([5], [1], 0b10) == -1                             # reduce_mask beyond ndim
    assert ws([5], [-1], 0b1) == -1                             # negative stride
    assert ws([5], [1], 0b1, dt=abi.RAW8) == -1                 # not a float type


def test_group_norm_workspace_formula_matches_the_header(tmp_path):
    from torch_vulkan import abi

    cases = [(1, 64, 262144, 32), (2, 8, 25, 4), (3, 2560, 256, 32), (1, 6, 1, 3)]
    lines = ['#include <stdio.h>', '#include "hrt_ops.h"', "int main(void) {"]
    lines += [f'  printf("%lld\\n", (long long)hrt_gn_workspace({n}, {c}, {hw}, {g}));' for n, c, hw, g in cases]
    lines += ["  return 0; }"]
    src = tmp_path / "gn.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "gn"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(REPO, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], stdout=subprocess.PIPE, text=True, check=True).stdout.split()]
    assert got == [abi.gn_workspace(*c) for c in cases]
