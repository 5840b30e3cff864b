"""The C-ABI library: it loads without a GPU, exports every entry point that
include/mxfa.h declares, and its supports_op logic (descriptor checks only,
no device access) accepts the reference's call-site layouts and rejects what
the kernels do not handle."""
from __future__ import annotations

import os
import re

import pytest

from conftest import REPO


def _declared_symbols():
    text = open(os.path.join(REPO, "include", "mxfa.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mxfa_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    import mxfa

    declared = _declared_symbols()
    assert declared == sorted(mxfa.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(mxfa.lib, name), name
    assert mxfa.version() >= 100
    assert mxfa.status_string(0) == "ok"
    assert mxfa.status_string(-2) == "unsupported"


def test_calibration_library_loads():
    # bench.py's streaming-read calibration lives in its own library, beside
    # the engine and outside its ABI
    import ctypes

    import torch  # noqa: F401  (one HIP runtime: torch's, loaded first)

    lib = ctypes.CDLL(os.path.join(REPO, "acestep.cpp_amd", "lib", "libmxfa_calib.so"))
    assert hasattr(lib, "mxfa_calib_stream_read")
    # argument checks run before any device call
    lib.mxfa_calib_stream_read.restype = ctypes.c_int
    lib.mxfa_calib_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int,
                                           ctypes.c_void_p]
    assert lib.mxfa_calib_stream_read(None, 16, None, 1, None) != 0
    assert lib.mxfa_calib_stream_read(1 << 20, 15, 1 << 21, 1, None) != 0


def _dev(view, fake_ptr=1 << 20):
    import mxfa

    return mxfa.DeviceView(view.type, tuple(view.ne), tuple(view.nb), fake_ptr)


@pytest.mark.parametrize("name", ["c1", "c3", "c4x"])
def test_supports_reference_layouts(name):
    import mxfa
    from mxfa import cases

    kw = {"c3": dict(max_seq=1024, lmin=100, lmax=1024), "c4x": dict(S=300)}.get(name, {})
    c = cases.BUILDERS[name](**kw)
    q, k, v = _dev(c.q), _dev(c.k), _dev(c.v)
    m = _dev(c.mask) if c.mask is not None else None
    assert mxfa.supports(q, k, v, m, c.scale)
    assert mxfa.supports(q, k, v, None, c.scale)


def test_supports_rejections():
    import mxfa
    from mxfa import cases

    c = cases.c1()
    q, k, v, m = _dev(c.q), _dev(c.k), _dev(c.v), _dev(c.mask)
    ok = mxfa.supports(q, k, v, m, c.scale)
    assert ok
    D64 = mxfa.DeviceView(k.type, (64,) + k.ne[1:], k.nb, k.ptr)
    assert not mxfa.supports(q, D64, v, m, c.scale)                    # head size
    f32k = mxfa.DeviceView(0, k.ne, (4, 512) + k.nb[2:], k.ptr)
    assert not mxfa.supports(q, f32k, v, m, c.scale)                   # K type
    mixed = mxfa.DeviceView(30, v.ne, v.nb, v.ptr)
    assert not mxfa.supports(q, k, mixed, m, c.scale)                  # K/V type mix
    badm = mxfa.DeviceView(0, m.ne, (4,) + m.nb[1:], m.ptr)
    assert not mxfa.supports(q, k, v, badm, c.scale)                   # mask type
    short = mxfa.DeviceView(1, (100,) + m.ne[1:], m.nb, m.ptr)
    assert not mxfa.supports(q, k, v, short, c.scale)                  # mask narrower than Skv
    gqa = mxfa.DeviceView(k.type, k.ne[:2] + (3, 1), k.nb, k.ptr)
    assert not mxfa.supports(q, gqa, gqa, m, c.scale)                  # 16 % 3 != 0
    unal = mxfa.DeviceView(q.type, q.ne, q.nb, q.ptr + 4)
    assert not mxfa.supports(unal, k, v, m, c.scale)                   # alignment
    assert not mxfa.supports(q, k, v, m, float("nan"))                 # scale
    assert not mxfa.supports(q, k, v, m, c.scale, prec=3)              # prec
    assert "prec" in mxfa.last_error()
    dst_bad = mxfa.DeviceView(0, (128, 16, 1, 1), (4, 512, 4096, 4096 * 2), 1 << 21)
    assert not mxfa.supports(q, k, v, m, c.scale, dst=dst_bad)         # non-contiguous dst
    dst_ok = mxfa.DeviceView(0, (128, 16, 1, 1), (4, 512, 8192, 8192), 1 << 21)
    assert mxfa.supports(q, k, v, m, c.scale, dst=dst_ok)


def test_one_hip_runtime_whatever_the_import_order():
    """torch bundles its own HIP runtime; libmxfa.so must bind to that one
    even when mxfa is imported before torch (two runtimes in one process
    crash torch's device calls)."""
    import subprocess
    import sys

    code = ("import sys, re; sys.path.insert(0, {pkg!r}); import mxfa, torch; "
            "print(len(set(re.findall(r'\\S*libamdhip64\\S*', open('/proc/self/maps').read()))))")
    out = subprocess.run([sys.executable, "-c", code.format(pkg=os.path.join(REPO, "acestep.cpp_amd"))],
                         capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    assert out.stdout.strip().splitlines()[-1] == "1", out.stdout
