"""Build recipe of the MI355X "vk" backend (in-tree; the products travel with the source tree).

Products (written into torch-vulkan_amd/torch_vulkan/):
  libhrt.so        — the C-ABI runtime (include/hrt.h) plus every gfx950 kernel, built by hipcc;
  torch_vulkan_C*.so — the PyTorch PrivateUse1 shim, a plain C++ extension built by g++ against the
                       installed torch headers and linked to libhrt.so (no hipify, no HIP headers).

Usage:  python torch-vulkan_amd/build.py [--jobs N] [--only hrt|shim]
"""

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig

PKG_ROOT = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
OUT_DIR = os.path.join(PKG_ROOT, "torch_vulkan")
BUILD_DIR = os.path.join(PKG_ROOT, "_build")
INCLUDE = os.path.join(REPO, "include")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in generated code (they have produced silent wrong results on
# this hardware pool); the host pass warns that it does not know the feature, which is harmless.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-I", INCLUDE,
]

HRT_SOURCES = [
    "hrt/runtime.cpp",
    "kernels/ew.hip",
    "kernels/ew_map.hip",
    "kernels/reduce.hip",
    "kernels/conv_norm.hip",
    "kernels/conv3x3.hip",
    "kernels/dq8.hip",
    "kernels/gemm.hip",
    "kernels/gemm_mfma.hip",
    "kernels/rows.hip",
    "kernels/attn_fwd.hip",
    "kernels/attn_bwd.hip",
    "kernels/attn_f32.hip",
]
SHIM_SOURCES = [
    "shim/device.cpp",
    "shim/fallback.cpp",
    "shim/bindings.cpp",
    "shim/autocast.cpp",
    "shim/op_gemm.cpp",
    "shim/op_attention.cpp",
    "shim/op_rows.cpp",
    "shim/op_reduce.cpp",
    "shim/op_quant.cpp",
    "shim/op_ew.cpp",
    "shim/op_image.cpp",
]


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines() if "is not a recognized feature for this target" not in l)
    if p.returncode != 0:
        raise RuntimeError("build step failed:\n" + " ".join(cmd) + "\n" + out)
    return out


def _obj(src, tag):
    return os.path.join(BUILD_DIR, tag, src.replace("/", "_").rsplit(".", 1)[0] + ".o")


def build_hrt(jobs):
    srcs = [s for s in HRT_SOURCES if os.path.exists(os.path.join(CSRC, s))]
    os.makedirs(os.path.join(BUILD_DIR, "hrt"), exist_ok=True)
    cmds = []
    for s in srcs:
        lang = ["-x", "hip"] if s.endswith(".hip") else []
        cmds.append([HIPCC, *HIP_FLAGS, *lang, "-c", os.path.join(CSRC, s), "-o", _obj(s, "hrt")])
    with cf.ThreadPoolExecutor(jobs) as ex:
        for out in ex.map(_run, cmds):
            if out.strip():
                print(out)
    so = os.path.join(OUT_DIR, "libhrt.so")
    tmp = so + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *[_obj(s, "hrt") for s in srcs]])
    os.replace(tmp, so)
    return so


def _torch_flags():
    import torch
    import torch.utils.cpp_extension as ce

    inc = []
    for d in ce.include_paths():
        inc += ["-isystem", d]
    inc += ["-isystem", sysconfig.get_paths()["include"]]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    defs = [f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_EXTENSION_NAME=torch_vulkan_C", "-DTORCH_API_INCLUDE_EXTENSION_H"]
    libdir = ce.library_paths()[0]
    return inc, defs, libdir


def build_shim(jobs):
    inc, defs, libdir = _torch_flags()
    os.makedirs(os.path.join(BUILD_DIR, "shim"), exist_ok=True)
    cxx = os.environ.get("CXX", "g++")
    flags = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function", "-Wno-sign-compare", *defs, *inc, "-I", INCLUDE]
    cmds = [[cxx, *flags, "-c", os.path.join(CSRC, s), "-o", _obj(s, "shim")] for s in SHIM_SOURCES]
    with cf.ThreadPoolExecutor(jobs) as ex:
        for out in ex.map(_run, cmds):
            if out.strip():
                print(out)
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    so = os.path.join(OUT_DIR, "torch_vulkan_C" + suffix)
    tmp = so + ".tmp"
    _run([cxx, "-shared", "-o", tmp, *[_obj(s, "shim") for s in SHIM_SOURCES], "-L", libdir, "-lc10", "-ltorch", "-ltorch_cpu",
          "-ltorch_python", "-L", OUT_DIR, "-lhrt", "-Wl,-rpath,$ORIGIN", "-Wl,-rpath," + libdir])
    os.replace(tmp, so)
    return so


def build(jobs=None, only=None):
    jobs = jobs or min(16, os.cpu_count() or 4)
    built = []
    if only in (None, "hrt"):
        built.append(build_hrt(jobs))
    if only in (None, "shim"):
        built.append(build_shim(jobs))
    return built


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--only", choices=["hrt", "shim"], default=None)
    a = ap.parse_args()
    for p in build(a.jobs, a.only):
        print("built", os.path.relpath(p, REPO))
