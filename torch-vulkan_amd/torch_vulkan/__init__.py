"""MI355X-native "vk" device for PyTorch: the torch_vulkan API over HIP and hand-written gfx950 kernels.

`import torch_vulkan` loads the C++ shim (which registers the PrivateUse1 operators: mm/bmm/addmm/
baddbmm, fused SDPA forward+backward, softmax (+backward, _safe_softmax), layer_norm (+backward), copies
and fills), renames PrivateUse1 to "vk" and installs the `torch.vk` module, so training code written for
the reference `torch_vulkan` package (torch_vulkan/__init__.py:1-270) runs unchanged: tensors move with
`.to("vk")`, every other op falls back to the CPU, and the counters below report which path ran.

The native libraries are built in-tree by `torch-vulkan_amd/build.py`; there is no pure-Python
substitute, so a missing build is an ImportError.
"""

import importlib
import os
import sys
import types

import torch

_THIS_DIR = os.path.dirname(os.path.abspath(__file__))


def _load_extension():
    if _THIS_DIR not in sys.path:
        sys.path.insert(0, _THIS_DIR)
    try:
        return importlib.import_module("torch_vulkan_C")
    except ImportError as e:  # no silent fallback: the device does not exist without its native code
        raise ImportError(
            f"torch_vulkan: the native extension is not built ({e}); run `python torch-vulkan_amd/build.py`"
        ) from e


_C = _load_extension()


def is_available() -> bool:
    return True


def device_count() -> int:
    return 1


def current_device() -> int:
    return 0


def set_device(device) -> None:
    return None


def synchronize(device=None) -> None:
    _C.synchronize()


def device_name() -> str:
    return _C.device_name()


def live_bytes() -> int:
    return _C.live_bytes()


def memory_info() -> dict:
    """Device memory in bytes: budget (what this process can still reach: free + own reservation), usage
    (all processes) and heap (device total)."""
    budget, usage, heap = _C.memory_info()
    return {"budget": budget, "usage": usage, "heap": heap}


def peak_live_bytes() -> int:
    """High-water mark of live device bytes since reset_peak_live_bytes()."""
    return _C.peak_live_bytes()


def reset_peak_live_bytes() -> None:
    _C.reset_peak_live_bytes()


def set_memory_limit(megabytes: int) -> None:
    """Cap the device memory reserved by this process (MiB, 0 = no cap); exceeding it raises an OOM
    RuntimeError.  Also settable with VKT_MEM_LIMIT_MB at import time."""
    _C.set_memory_limit(int(megabytes) << 20)


def set_fused_attention(mode: str) -> None:
    """Policy of the fused F.scaled_dot_product_attention: "auto" (default), "on" or "off".  auto uses it
    for bf16/f16 and, for f32, when the score matrix would be >= 256 MiB.  Env: VKT_FUSED_ATTN=0/1."""
    _C.set_fused_attention({"off": 0, "on": 1, "auto": 2}[mode])


def kernel_counts() -> dict:
    return dict(_C.kernel_counts())


def validation_errors() -> int:
    return _C.validation_errors()


def empty_cache() -> None:
    _C.empty_cache()


def reserved_bytes() -> int:
    return _C.reserved_bytes()


def live_blocks() -> int:
    return _C.live_blocks()


def slab_count() -> int:
    return _C.slab_count()


def manual_seed(seed: int) -> None:
    # random numbers are drawn on the CPU and copied, as in the reference
    return None


def manual_seed_all(seed: int) -> None:
    return None


def seed() -> None:
    return None


def _is_in_bad_fork() -> bool:
    return False


def get_amp_supported_dtype():
    return [torch.bfloat16, torch.float16]


class device:  # noqa: N801  same name and use as torch.cuda.device
    def __init__(self, device=None):
        self.idx = device

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


def get_rng_state(device="vk") -> torch.Tensor:
    return torch.zeros(1, dtype=torch.uint8)


def set_rng_state(new_state, device="vk") -> None:
    return None


# Names of the runtime counters (include/hrt.h, hrt_stat) as stats() reports them: (key, index, scale).
_RUNTIME_COUNTERS = (
    ("dispatch_s", 0, 1e-9), ("dispatch_n", 1, 1.0), ("transfer_s", 2, 1e-9), ("transfer_n", 3, 1.0),
    ("pipeline_create_s", 4, 1e-9), ("upload_MB", 5, 1.0 / 2**20), ("download_MB", 6, 1.0 / 2**20),
    ("gpu_wait_s", 7, 1e-9),
)


def stats() -> dict:
    """Host-side runtime counters: time spent queueing kernels and in transfers, their counts, kernel-table
    set-up time, bytes moved, time waiting for the GPU, and the time spent in CPU fallbacks."""
    raw = _C.runtime_counters()
    out = {key: raw[i] * scale for key, i, scale in _RUNTIME_COUNTERS}
    out["fallback_s"] = sum(fallback_time_by_op().values())
    return out


def fallback_time_by_op() -> dict:
    return dict(_C.fallback_time_by_op())


def profile() -> str:
    """Per-kernel GPU time ("name\tms\tcount" lines) when HRT_PROFILE=1 was set at start-up."""
    return _C.profile()


def _report_at_exit():
    """VKT_STATS=1 / HRT_PROFILE=1: a summary of where the time went, printed when the process ends."""
    lines = ["runtime " + " ".join(f"{k}={v:.3g}" for k, v in stats().items())]
    slow = sorted(fallback_time_by_op().items(), key=lambda kv: kv[1], reverse=True)
    if slow:
        lines.append("CPU fallbacks by time " + " ".join(f"{k}={v:.3g}s" for k, v in slow[:8]))
    busy = sorted(kernel_counts().items(), key=lambda kv: kv[1], reverse=True)
    lines.append("GPU operators by count " + " ".join(f"{k}={n}" for k, n in busy[:8]))
    prof = [row.split("\t") for row in profile().splitlines() if row]
    if prof:
        total = sum(float(r[1]) for r in prof) or 1.0
        lines.append(f"kernel time {total:.1f} ms")
        lines += [f"  {name:34s} {float(ms):9.1f} ms {100 * float(ms) / total:5.1f}%  x{n}" for name, ms, n in prof[:18]]
    print("\n".join("[torch_vulkan] " + l for l in lines))


if os.environ.get("VKT_STATS") or os.environ.get("HRT_PROFILE"):
    import atexit

    atexit.register(_report_at_exit)


def coop_caps() -> int:
    """Matrix-core kernels available (bit0 = f16, bit1 = bf16): 3 on gfx950."""
    return _C.coop_caps()


def set_coop_enabled(on: bool) -> None:
    """Switch the matrix-core (MFMA) kernels on/off; off routes bf16/f16 to the FMA kernels.
    Env: VKT_NO_COOP=1."""
    _C.set_coop_enabled(bool(on))


def empty_pinned(shape, dtype=torch.float32) -> torch.Tensor:
    """An uninitialised CPU tensor in pinned (page-locked) host memory of the vk runtime.  Copies between it
    and a dense vk tensor of the same dtype and shape with non_blocking=True are asynchronous: uploads run
    on the runtime's copy stream and overlap kernels that do not touch their destination (the kernels that
    do wait for them); downloads are valid after torch_vulkan.synchronize().  The block-swap path:
    frozen weights kept here and streamed into a ring of device buffers each step."""
    return _C.empty_pinned(list(shape), dtype)


def is_pinned(t: torch.Tensor) -> bool:
    """True if CPU tensor t lies in vk pinned host memory (what t.is_pinned(device="vk") answers, without
    PyTorch's deprecation warning for the device argument)."""
    return bool(_C.is_pinned(t))


def pin_memory(t: torch.Tensor) -> torch.Tensor:
    """A copy of CPU tensor t in vk pinned host memory (see empty_pinned); t itself if it already is."""
    if is_pinned(t):
        return t
    out = _C.empty_pinned(list(t.shape), t.dtype)
    out.copy_(t)
    return out


def dequant_int8(q, scale, out_dtype=torch.bfloat16):
    """Weight-only int8 dequant: out[r, c] = float(q[r, c]) * float(scale[r, c // 64]) rounded to out_dtype.

    q: int8 [rows, cols]; scale: bfloat16 [rows, ceil(cols / 64)] (64-column blocks per row).  On vk
    tensors this runs the dq8 kernel; CPU tensors get the same closed form in PyTorch, as the reference's
    function does (torch_vulkan/__init__.py:193-205).
    """
    if q.device.type == "vk":
        return _C.dequant_int8(q.contiguous(), scale.contiguous(), out_dtype)
    # each row padded to whole 64-element blocks, every block times its scale in float32, rounded once
    rows, cols = q.shape
    nb = scale.shape[1]
    blocks = torch.zeros((rows, nb * 64), dtype=torch.float32)
    blocks[:, :cols] = q.float()
    prod = blocks.view(rows, nb, 64) * scale.float().unsqueeze(-1)
    return prod.view(rows, nb * 64)[:, :cols].to(out_dtype)


def dequant_int8_linear(x, q, scale, bias=None):
    """Fused int8 weight-only linear: x @ dequant_int8(q, scale, x.dtype).T (+ bias), x bf16/f16 on vk.

    The dequantized weight never reaches memory; its values are bit-identical to dequant_int8's."""
    if x.device.type != "vk":
        raise RuntimeError("dequant_int8_linear: x must be a vk tensor")
    return _C.dequant_int8_linear(x, q.contiguous(), scale.contiguous(), bias)


def event_record(slot: int) -> None:
    """Record HIP event `slot` (0..1023) on the runtime's stream (the stream every vk kernel runs on)."""
    _C.event_record(int(slot))


def event_elapsed_ms(start_slot: int, end_slot: int) -> float:
    """Milliseconds between two recorded slots (waits for the later one)."""
    return _C.event_elapsed_ms(int(start_slot), int(end_slot))


def fallback_counts() -> dict:
    return dict(_C.fallback_counts())


def reset_fallback_counts() -> None:
    _C.reset_counts()


def set_inline_backward(on: bool = True) -> None:
    """Run autograd's backward on the calling thread (PyTorch's thread-local
    torch.autograd.set_multithreading_enabled(False)), for the thread that calls this.  PyTorch otherwise
    hands the work of every non-CPU device to a per-device worker thread and waits for it; the vk device
    has one stream, so that thread adds only a cross-thread handoff: on MI355X a backward() call costs
    ~49 us of host time on vk that way against ~24 us inline, which left the GPU idle in short steps.
    Gradients are the same either way.  Opt-in, because it changes the calling thread's autograd state
    (and CUDA or other devices' backward on that thread would run inline too): call it on the thread that
    runs the training loop, or set VKT_INLINE_BACKWARD=1 to apply it to the importing thread at import."""
    torch._C._set_multithreading_enabled(not on)


def _register():
    # Keep nn.Parameter identity when modules move to vk (optimizers built before .to() keep working).
    torch.__future__.set_swap_module_params_on_conversion(True)
    # "vulkan" is taken by PyTorch's own inference backend, hence "vk".
    torch.utils.rename_privateuse1_backend("vk")
    module = types.ModuleType("torch.vk")
    for name in (
        "is_available",
        "device_count",
        "current_device",
        "set_device",
        "synchronize",
        "empty_cache",
        "manual_seed",
        "manual_seed_all",
        "seed",
        "_is_in_bad_fork",
        "get_amp_supported_dtype",
        "device",
        "get_rng_state",
        "set_rng_state",
        "memory_info",
        "set_memory_limit",
        "peak_live_bytes",
        "reset_peak_live_bytes",
        "empty_pinned",
        "pin_memory",
        "is_pinned",
    ):
        setattr(module, name, globals()[name])
    torch._register_device_module("vk", module)


_register()
if os.environ.get("VKT_INLINE_BACKWARD") == "1":
    set_inline_backward(True)


def set_coop_range(lo: int = 0, hi: int = 2**64 - 1, kind: int = 0) -> None:
    """Debug: only matrix-core-eligible GEMM calls numbered [lo, hi) use MFMA (others the FMA kernel);
    kind 0 = all, 1 = bmm only, 2 = mm only.  For bisecting a bad call."""
    _C.set_coop_range(int(lo), int(hi), int(kind))


def reset_coop_calls() -> None:
    _C.reset_coop_calls()


def coop_calls() -> int:
    return _C.coop_calls()


if os.environ.get("VKT_MEM_LIMIT_MB"):
    set_memory_limit(int(os.environ["VKT_MEM_LIMIT_MB"]))
