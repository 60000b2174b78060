"""Build the C restatement of the oracle (test infrastructure): oracle/_build/liboracle.so.

The reference's own implementation cannot be built here (Rust + Vulkan runtime, GLSL shaders, a C++ shim
that links the Rust library), so there is no oracle/_ref build: the restatement is pinned by the
reference's golden vectors, float64 torch and closed forms in tests/ instead."""

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_build", "liboracle.so")


def build():
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    tmp = OUT + ".tmp"
    subprocess.run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-o", tmp, os.path.join(HERE, "csrc", "oracle.c")],
                   check=True)
    os.replace(tmp, OUT)
    return OUT


def load():
    """ctypes handle of liboracle.so (built on demand)."""
    import ctypes

    if not os.path.exists(OUT):
        build()
    lib = ctypes.CDLL(OUT)
    i64, vp = ctypes.c_int64, ctypes.c_void_p
    lib.oracle_round_bf16.argtypes = [vp, vp, i64]
    lib.oracle_round_f16.argtypes = [vp, vp, i64]
    lib.oracle_dequant_int8.argtypes = [vp, vp, i64, i64, ctypes.c_int, vp]
    return lib


if __name__ == "__main__":
    print(build())
