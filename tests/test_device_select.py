"""Explicit device selection with HRT_DEVICE (the reference's VKRT_DEVICE, vkrt/src/lib.rs:241-262, tested
by tests/test_device_select.py of the reference): an index, or a case-insensitive substring of a device's
name; anything else fails at initialisation with the list of devices.  The variable is read once when the
runtime initialises, so every case runs in a freshly spawned child process."""

import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROBE = "import torch_vulkan; print('NAME=' + torch_vulkan.device_name())"


def run(value):
    env = dict(os.environ)
    env.pop("HRT_DEVICE", None)
    if value is not None:
        env["HRT_DEVICE"] = value
    env["PYTHONPATH"] = os.pathsep.join([REPO, os.path.join(REPO, "torch-vulkan_amd"), env.get("PYTHONPATH", "")])
    print("child with HRT_DEVICE =", value, flush=True)
    return subprocess.run([sys.executable, "-c", PROBE], capture_output=True, text=True, env=env, timeout=300)


def name_of(r):
    return next((line[5:] for line in r.stdout.splitlines() if line.startswith("NAME=")), None)


def test_default_index_and_name_substring_select_the_same_device():
    default = run(None)
    assert default.returncode == 0 and name_of(default), default.stderr[-600:]
    by_index = run("0")
    assert name_of(by_index) == name_of(default)
    arch = name_of(default).split("(")[-1].split(":")[0].upper()  # e.g. "GFX950", matched case-insensitively
    assert name_of(run(f"  {arch} ")) == name_of(default)


@pytest.mark.parametrize("bad", ["no-such-gpu-xyz", "99", "-1"])
def test_unknown_name_or_index_fails_with_the_device_list(bad):
    r = run(bad)
    assert r.returncode != 0 and name_of(r) is None
    text = r.stdout + r.stderr
    assert "HRT_DEVICE" in text and "0: " in text and "does not name a device" in text, text[-600:]
