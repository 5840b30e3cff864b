"""The per-device, thread-safe set-up guard (csrc/once_per_device.h) behind
the decode kernel's hipFuncSetAttribute: compiled on its own with the host
compiler and driven from several threads over several device ids (CPU)."""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_once_per_device(tmp_path):
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        pytest.skip("no C++ compiler")
    exe = str(tmp_path / "once_per_device_test")
    subprocess.run([cxx, "-std=c++17", "-O2", "-Wall", "-Werror", "-pthread",
                    "-I", os.path.join(REPO, "acestep.cpp_amd", "csrc"),
                    os.path.join(REPO, "tests", "c", "once_per_device_test.cpp"), "-o", exe], check=True)
    out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    kv = dict(line.split(" ", 1) for line in out.strip().splitlines())
    assert "bad_return" not in kv
    # 1600 concurrent calls over 4 devices: one setting per device
    assert [kv[f"dev{d}"] for d in range(4)] == ["1", "1", "1", "1"]
    # a failed setting (7) is retried, then remembered
    assert kv["retry"] == "7 0 0 2"
    # a new device id grows the table; device 0 stays done
    assert kv["grow"] == "0 0 1 1"


def test_decode_launch_uses_the_guard():
    src = open(os.path.join(REPO, "acestep.cpp_amd", "csrc", "fa_decode.hip")).read()
    assert "static OncePerDevice attr;" in src
    assert "static bool attr_set" not in src
