"""ctypes binding of the hrt C ABI (include/hrt.h, include/hrt_ops.h).

This is the Python counterpart of what a maintainer of the reference would bind to the runtime's C ABI
(csrc/vkrt.h:6-32): the same entry points, the argument blocks of the operator kernels as
ctypes.Structure mirrors of the C structs, and a `dispatch` helper that raises with the runtime's
last-error message.  bench.py drives the kernels through it; the PyTorch shim (torch_vulkan_C) calls the
same library from C++.
"""

import ctypes
import os

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libhrt.so")
MAX_DIMS = 8
F32, BF16, F16, RAW8, RAW16, RAW32, RAW64 = range(7)
ATTN_O_F32 = 1
MM_F32_OUT = 1  # hrt_mm_args.flags: fp32 output (split-K partials)
ATTN_DQ_DELTA = 2
ATTN_GRAD_LIKE_INPUT = 4  # hrt_attn_args.flags: dq, dk, dv in the layout of q, k, v

u64, i64, i32, u32, f32 = ctypes.c_uint64, ctypes.c_int64, ctypes.c_int32, ctypes.c_uint32, ctypes.c_float


class AddF32Args(ctypes.Structure):
    _fields_ = [("a", u64), ("b", u64), ("c", u64), ("n", u64)]


class CopyArgs(ctypes.Structure):
    _fields_ = [("dst", u64), ("src", u64), ("ndim", i32), ("dst_dtype", i32), ("src_dtype", i32), ("pad", i32),
                ("sizes", i64 * MAX_DIMS), ("dst_strides", i64 * MAX_DIMS), ("src_strides", i64 * MAX_DIMS)]


class FillArgs(ctypes.Structure):
    _fields_ = [("dst", u64), ("value_bits", u64), ("ndim", i32), ("dtype", i32), ("pad0", i32), ("pad1", i32),
                ("sizes", i64 * MAX_DIMS), ("strides", i64 * MAX_DIMS)]


class EwArgs(ctypes.Structure):
    _fields_ = [("out", u64), ("a", u64), ("b", u64), ("c", u64), ("op", i32), ("ndim", i32), ("out_dtype", i32),
                ("a_dtype", i32), ("b_dtype", i32), ("c_dtype", i32), ("s0", f32), ("s1", f32),
                ("sizes", i64 * MAX_DIMS), ("out_strides", i64 * MAX_DIMS), ("a_strides", i64 * MAX_DIMS),
                ("b_strides", i64 * MAX_DIMS), ("c_strides", i64 * MAX_DIMS)]


# hrt_ew_op codes (include/hrt_ops.h), by the oracle's op names
EW_OPS = {n: i for i, n in enumerate((
    "add", "sub", "mul", "div", "add_s", "mul_s", "div_s", "axpb", "rdiv_s", "pow_s", "neg", "rsqrt", "recip", "exp",
    "sin", "cos", "sqrt", "tanh", "sigmoid", "relu", "silu", "gelu_erf", "gelu_tanh", "silu_bwd", "gelu_erf_bwd",
    "gelu_tanh_bwd", "addcmul", "addcdiv", "lerp_s", "where"))}


class ReduceArgs(ctypes.Structure):
    _fields_ = [("x", u64), ("out", u64), ("ws", u64), ("ndim", i32), ("x_dtype", i32), ("out_dtype", i32),
                ("reduce_mask", u32), ("div", f32), ("pad", u32), ("sizes", i64 * MAX_DIMS), ("strides", i64 * MAX_DIMS)]


CAT_MAX_PARTS = 8


class CatArgs(ctypes.Structure):
    _fields_ = [("out", u64), ("src", u64 * CAT_MAX_PARTS), ("row_bytes", i64 * CAT_MAX_PARTS), ("col", i64 * CAT_MAX_PARTS),
                ("outer", i64), ("out_row_bytes", i64), ("nparts", i32), ("pad", i32)]


class Im2colArgs(ctypes.Structure):
    _fields_ = [("x", u64), ("cols", u64)] + [(n, i64) for n in ("N", "C", "H", "W", "OH", "OW", "KH", "KW", "SH", "SW", "PH", "PW")]


class Conv3WprepArgs(ctypes.Structure):
    _fields_ = [("w", u64), ("wr", u64), ("O", i64), ("I", i64), ("flip", u32), ("pad", u32)]


class Conv3Args(ctypes.Structure):
    _fields_ = [("x", u64), ("wr", u64), ("bias", u64), ("y", u64), ("ws", u64), ("N", i64), ("I", i64), ("O", i64),
                ("H", i64), ("W", i64), ("has_bias", u32), ("splits", u32)]


CONV3_SLAB_BYTES = 38912  # HRT_CONV3_SLAB_BYTES


def conv3_wr_bytes(O, I):
    """hrt_conv3_wr_bytes: bytes of the reordered 3x3 weights of "conv3x3_wprep_*"."""
    return (O // 128) * (I // 16) * CONV3_SLAB_BYTES


def conv3_splits(N, I, O, H, W):
    """hrt_conv3_splits: the input-channel split of "conv3x3_*" the shim uses."""
    tiles, nb, s = N * ((H + 1) // 2) * (W // 64) * (O // 128), I // 16, 1
    while tiles * s * 2 <= 256 and nb % (2 * s) == 0 and nb // (2 * s) >= 4:
        s *= 2
    return s


class UpsampleArgs(ctypes.Structure):
    _fields_ = [("src", u64), ("dst", u64), ("NC", i64), ("H", i64), ("W", i64), ("OH", i64), ("OW", i64)]


class GnArgs(ctypes.Structure):
    _fields_ = [(n, u64) for n in ("x", "y", "g", "mean", "rstd", "w", "b", "dx", "dw", "db", "ws")] + [
        ("N", i64), ("C", i64), ("HW", i64), ("G", i64), ("eps", f32), ("pad", u32)]


def gn_workspace(N, C, HW, G):
    """hrt_gn_workspace (include/hrt_ops.h): fp32 elements of the group_norm workspace."""
    m = (C // G) * HW
    chunks = min(max((m + 16383) // 16384, 1), 256)
    return max(N * G * chunks * 3, 2 * N * C + 2 * N * G)


class MmArgs(ctypes.Structure):
    _fields_ = [("a", u64), ("b", u64), ("c", u64), ("bias", u64), ("M", i64), ("N", i64), ("K", i64), ("batch", i64),
                ("a_sb", i64), ("a_sm", i64), ("a_sk", i64), ("b_sb", i64), ("b_sk", i64), ("b_sn", i64),
                ("c_sb", i64), ("c_sm", i64), ("c_sn", i64), ("bias_sb", i64), ("bias_sm", i64), ("bias_sn", i64),
                ("alpha", f32), ("beta", f32), ("has_bias", u32), ("flags", u32)]


class MmReduceArgs(ctypes.Structure):
    _fields_ = [("ws", u64), ("c", u64), ("bias", u64), ("M", i64), ("N", i64), ("splits", i64), ("c_sm", i64),
                ("c_sn", i64), ("bias_sm", i64), ("bias_sn", i64), ("alpha", f32), ("beta", f32), ("has_bias", u32),
                ("pad", u32)]


class MmDq8Args(ctypes.Structure):
    _fields_ = [("x", u64), ("q", u64), ("scale", u64), ("bias", u64), ("y", u64), ("M", i64), ("N", i64), ("K", i64),
                ("nblocks", i64), ("x_sm", i64), ("x_sk", i64), ("alpha", f32), ("beta", f32), ("has_bias", u32),
                ("flags", u32), ("ws", u64)]


class AttnArgs(ctypes.Structure):
    _fields_ = [("q", u64), ("k", u64), ("v", u64), ("o", u64), ("lse", u64), ("o32", u64), ("dout", u64), ("delta", u64),
                ("dq", u64), ("dk", u64), ("dv", u64),
                ("q_sb", i64), ("q_sh", i64), ("q_ss", i64), ("k_sb", i64), ("k_sh", i64), ("k_ss", i64),
                ("v_sb", i64), ("v_sh", i64), ("v_ss", i64), ("do_sb", i64), ("do_sh", i64), ("do_ss", i64),
                ("B", i32), ("H", i32), ("Sq", i32), ("Sk", i32), ("D", i32), ("scale", f32), ("flags", u32), ("pad", u32)]


class SoftmaxArgs(ctypes.Structure):
    _fields_ = [("x", u64), ("y", u64), ("g", u64), ("dx", u64), ("outer", i64), ("R", i64), ("inner", i64), ("safe", u32),
                ("pad", u32)]


class LnArgs(ctypes.Structure):
    _fields_ = [("x", u64), ("y", u64), ("mean", u64), ("rstd", u64), ("w", u64), ("b", u64), ("g", u64), ("dx", u64),
                ("dw", u64), ("db", u64), ("ws", u64), ("rows", i64), ("D", i64), ("eps", f32), ("pad", u32)]


class Dq8Args(ctypes.Structure):
    _fields_ = [("q", u64), ("scale", u64), ("out", u64), ("rows", i64), ("cols", i64), ("nblocks", i64)]


def ln_rows_per_chunk(rows, D):
    """hrt_ln_rows_per_chunk (include/hrt_ops.h): rows of one layer_norm weight-gradient chunk."""
    r = 4
    while r < 16 and r * D >= 8192 and rows >= 256 * r and 2 * r * D * 4 <= 131072:
        r *= 2
    return r


def ln_chunks(rows, D):
    """hrt_ln_chunks (include/hrt_ops.h): partial-sum rows of the layer_norm weight gradient."""
    r = ln_rows_per_chunk(rows, D)
    return (rows + r - 1) // r


LN_SCRATCH_BYTES = 8 << 20  # HRT_LN_SCRATCH_BYTES (include/hrt_ops.h)


class Runtime:
    """The hrt library with typed entry points; one per process (the runtime is a process singleton)."""

    def __init__(self, path=_LIB_PATH):
        lib = ctypes.CDLL(path)
        sz, vp, cp = ctypes.c_size_t, ctypes.c_void_p, ctypes.c_char_p
        sig = {
            "hrt_init": (ctypes.c_int, []),
            "hrt_last_error": (sz, [cp, sz]),
            "hrt_device_name": (sz, [cp, sz]),
            "hrt_max_alloc": (u64, []),
            "hrt_live_bytes": (u64, []),
            "hrt_memory_info": (i32, [ctypes.POINTER(u64)]),
            "hrt_peak_live_bytes": (u64, []),
            "hrt_reset_peak_live_bytes": (None, []),
            "hrt_set_memory_limit": (None, [u64]),
            "hrt_alloc": (u64, [u64]),
            "hrt_free": (ctypes.c_int, [u64]),
            "hrt_upload": (ctypes.c_int, [u64, vp, u64]),
            "hrt_download": (ctypes.c_int, [vp, u64, u64]),
            "hrt_copy_d2d": (ctypes.c_int, [u64, u64, u64]),
            "hrt_host_alloc": (u64, [u64]),
            "hrt_host_free": (ctypes.c_int, [u64]),
            "hrt_host_is_pinned": (ctypes.c_int, [vp]),
            "hrt_upload_async": (ctypes.c_int, [u64, vp, u64]),
            "hrt_download_async": (ctypes.c_int, [vp, u64, u64]),
            "hrt_kernel_index": (ctypes.c_int, [cp]),
            "hrt_dispatch": (ctypes.c_int, [u32, vp, u32, u32, u32, u32]),
            "hrt_dispatch_batch": (ctypes.c_int, [ctypes.POINTER(u32), ctypes.POINTER(vp), ctypes.POINTER(u32), u32]),
            "hrt_synchronize": (ctypes.c_int, []),
            "hrt_empty_cache": (sz, []),
            "hrt_reserved_bytes": (u64, []),
            "hrt_live_blocks": (sz, []),
            "hrt_slab_count": (sz, []),
            "hrt_validation_errors": (sz, []),
            "hrt_stat": (u64, [u32]),
            "hrt_profile_dump": (sz, [cp, sz]),
            "hrt_coop_caps": (u32, []),
            "hrt_event_record": (ctypes.c_int, [u32]),
            "hrt_event_elapsed_ms": (f32, [u32, u32]),
            "hrt_graph_begin": (ctypes.c_int, []),
            "hrt_graph_end": (i64, []),
            "hrt_graph_launch": (ctypes.c_int, [i64]),
            "hrt_graph_destroy": (ctypes.c_int, [i64]),
            "hrt_reduce_workspace": (i64, [vp]),
            "hrt_ln_bwd_noalloc": (ctypes.c_int, [vp, i32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        self.lib = lib
        self._ids = {}
        self.check(lib.hrt_init(), "hrt_init")

    def last_error(self):
        buf = ctypes.create_string_buffer(4096)
        self.lib.hrt_last_error(buf, len(buf))
        return buf.value.decode(errors="replace")

    def check(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: {self.last_error()}")

    def kernel(self, name):
        k = self._ids.get(name)
        if k is None:
            k = self.lib.hrt_kernel_index(name.encode())
            if k < 0:
                raise KeyError(f"kernel {name!r} is not registered")
            self._ids[name] = k
        return k

    def dispatch(self, name, args):
        """Queue operator kernel `name` with a Structure argument block (the kernel sizes its own grid)."""
        self.check(self.lib.hrt_dispatch(self.kernel(name), ctypes.byref(args), ctypes.sizeof(args), 0, 0, 0), name)

    def batch(self, pairs):
        """A prepared sequence of (kernel name, Structure) launches for run_batch (keeps the blocks alive)."""
        n = len(pairs)
        vp = ctypes.c_void_p
        ids = (u32 * n)(*[self.kernel(k) for k, _ in pairs])
        ptrs = (vp * n)(*[ctypes.addressof(a) for _, a in pairs])
        lens = (u32 * n)(*[ctypes.sizeof(a) for _, a in pairs])
        return (ids, ptrs, lens, n, [a for _, a in pairs])

    def run_batch(self, b):
        """Queue a prepared sequence with one hrt_dispatch_batch call."""
        rc = self.lib.hrt_dispatch_batch(b[0], b[1], b[2], b[3])
        if rc != 0:
            raise RuntimeError(f"hrt_dispatch_batch failed at launch {-rc - 1}: {self.last_error()}")

    def ln_bwd_noalloc(self, args, dtype):
        """hrt_ln_bwd_noalloc: layer_norm backward with the partial sums in the library's scratch array."""
        self.check(self.lib.hrt_ln_bwd_noalloc(ctypes.byref(args), dtype), "hrt_ln_bwd_noalloc")

    def synchronize(self):
        self.check(self.lib.hrt_synchronize(), "hrt_synchronize")

    def event_record(self, slot):
        self.check(self.lib.hrt_event_record(slot), "hrt_event_record")

    def elapsed_ms(self, a, b):
        ms = self.lib.hrt_event_elapsed_ms(a, b)
        if ms < 0:
            raise RuntimeError("hrt_event_elapsed_ms failed: " + self.last_error())
        return ms

    def graph(self, enqueue):
        """Record everything `enqueue()` dispatches into a HIP graph; returns its id."""
        self.check(self.lib.hrt_graph_begin(), "hrt_graph_begin")
        try:
            enqueue()
        finally:
            gid = self.lib.hrt_graph_end()
        if gid < 0:
            raise RuntimeError("hrt_graph_end failed: " + self.last_error())
        return gid

    def graph_launch(self, gid):
        self.check(self.lib.hrt_graph_launch(gid), "hrt_graph_launch")

    def graph_destroy(self, gid):
        self.check(self.lib.hrt_graph_destroy(gid), "hrt_graph_destroy")
