"""include/mxfa_ggml.h compiled against a mock struct ggml_tensor (CPU):
the adapter reads src[0..3], op_params and the node itself into the C ABI
descriptors exactly, rejects attention sinks, and its supports_op wrapper
reaches libmxfa's mxfa_supports (descriptor checks only, no device)."""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBDIR = os.path.join(REPO, "acestep.cpp_amd", "lib")


@pytest.fixture(scope="module")
def exe(tmp_path_factory):
    if not os.path.exists(os.path.join(LIBDIR, "libmxfa.so")):
        pytest.skip("libmxfa.so not built")
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    out = str(tmp_path_factory.mktemp("adapter") / "ggml_adapter_mock")
    subprocess.run([cc, "-std=c11", "-Wall", "-Werror", "-I", os.path.join(REPO, "include"),
                    os.path.join(REPO, "tests", "c", "ggml_adapter_mock.c"), "-L", LIBDIR, "-lmxfa",
                    "-Wl,-rpath," + LIBDIR, "-o", out], check=True)
    return out


def run(exe, *args):
    r = subprocess.run([exe, *args], check=True, capture_output=True, text=True)
    return dict(line.split(" ", 1) for line in r.stdout.strip().splitlines())


def test_unpack_fields_and_params(exe):
    o = run(exe, "mask")
    assert o["unpack"] == "0"
    assert o["q"] == "type=0 ne=128,1,32,8 nb=4,16384,512,16384 data=0x100000"
    assert o["k"] == "type=1 ne=128,8192,8,8 nb=2,256,2097152,16777216 data=0x200000"
    assert o["v"] == "type=1 ne=128,8192,8,8 nb=2,256,2097152,16777216 data=0x300000"
    assert o["mask"] == "type=1 ne=8192,1,1,8 nb=2,16384,16384,16384 data=0x400000"
    assert o["dst"] == "type=0 ne=128,32,1,8 nb=4,512,16384,16384 data=0x500000"
    assert o["params"] == "scale=0.0883883461 max_bias=0 softcap=0 prec=10"
    assert o["supports"] == "1"


def test_null_mask_and_sinks(exe):
    o = run(exe)
    assert o["mask"] == "NULL" and o["supports"] == "1"
    o = run(exe, "sinks")
    assert o["unpack"] == "-2" and o["supports"] == "0"


def test_set_rows_node(exe):
    """A batched-decode cache write node: supported; a non-integer row-id
    tensor is not; a node without row ids is rejected without a launch."""
    o = run(exe)
    assert o["set_rows_supports"] == "1"
    assert o["set_rows_bad_ids"] == "0"
    assert o["set_rows_no_ids"] == "0 -1"


def test_norm_rope_node(exe):
    """The pre-attention step as one custom node: sources in the documented
    order, Q out as the node, row ids optional; wrong position type and a
    missing cache source are refused without a launch."""
    o = run(exe)
    assert o["nr_unpack"] == "0"
    assert o["nr_q"] == "type=0 ne=128,32,7,1 nb=4,512,16384,114688 data=0x800000"
    assert o["nr_kcache"] == "type=1 ne=128,2048,8,1 nb=2,256,524288,4194304 data=0xd00000"
    assert o["nr_qout"] == "type=1 ne=128,32,7,1 nb=2,256,8192,57344 data=0x1000000"
    assert o["nr_rows"] == "type=27 ne=7,1,1,1 nb=8,56,56,56 data=0xf00000"
    assert o["nr_supports"] == "1"
    assert o["nr_bad_pos"] == "0"
    assert o["nr_no_rows"] == "1"
    assert o["nr_no_cache"] == "0 -1"
