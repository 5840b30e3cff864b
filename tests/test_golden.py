"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the seeded inputs regenerate bit-exactly from Philox4x32-10 and the
reference-layout builders, and the oracle reproduces the stored outputs
bit-exactly (fp64 exact form, ggml algorithm with fp32 and with fp16 V
accumulator).  GPU: libmxfa on the stored inputs meets the parity bar
against the stored gate and exact outputs."""
from __future__ import annotations

import glob
import json
import os
import sys

import numpy as np
import pytest

from conftest import MAX_ABS_TOL, ROW_COS_TOL, row_metrics

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))


def load(path):
    from mxfa.cases import FaCase, HostView

    z = np.load(path, allow_pickle=False)
    meta = json.loads(bytes(z["meta"]).decode())
    spec = meta["spec"]
    kt = spec["kv_type"]
    q = HostView(0, tuple(meta["q"]["ne"]), tuple(meta["q"]["nb"]), z["q"])
    kb = z["k"] if kt == 8 else z["k"].view(np.uint16)
    vb = z["v"] if kt == 8 else z["v"].view(np.uint16)
    k = HostView(kt, tuple(meta["k"]["ne"]), tuple(meta["k"]["nb"]), kb)
    v = HostView(kt, tuple(meta["v"]["ne"]), tuple(meta["v"]["nb"]), vb)
    m = None
    if meta["mask"] is not None:
        m = HostView(1, tuple(meta["mask"]["ne"]), tuple(meta["mask"]["nb"]), z["mask"])
    c = FaCase(spec["name"], q, k, v, m, meta["scale"], max_bias=spec.get("max_bias", 0.0),
               softcap=spec.get("softcap", 0.0))
    return c, spec, {n: z[n] for n in ("out_exact", "out_gate", "out_strict")}


def test_fixtures_present():
    assert len(FIXTURES) >= 5


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p)[:-4])
def test_inputs_regenerate(path):
    sys.path.insert(0, os.path.join(HERE, "golden"))
    import make_golden

    c, spec, _ = load(path)
    r = make_golden.make_case(**spec)
    assert np.array_equal(c.q.buf, r.q.buf)
    assert np.array_equal(c.k.buf.view(np.uint8), r.k.buf.view(np.uint8))
    assert np.array_equal(c.v.buf.view(np.uint8), r.v.buf.view(np.uint8))
    if c.mask is not None:
        assert np.array_equal(c.mask.buf, r.mask.buf)


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p)[:-4])
def test_oracle_reproduces_fixture(path, oracle_lib):
    import oracle

    c, _, out = load(path)
    args = (c.q, c.k, c.v, c.mask, c.scale, c.max_bias, c.softcap)
    assert np.array_equal(oracle.fa_exact(*args, q_round=True), out["out_exact"])
    assert np.array_equal(oracle.fa_ggml(*args, acc_f32=True), out["out_gate"])
    assert np.array_equal(oracle.fa_ggml(*args), out["out_strict"])
    # the gate and exact forms agree to well inside the GPU bar
    mg = row_metrics(out["out_gate"], out["out_exact"])
    assert mg["max_abs"] < 1e-5 and mg["min_cos"] > 0.999999


@pytest.mark.gpu
@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p)[:-4])
def test_gpu_matches_fixture(path):
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mxfa

    c, spec, out = load(path)
    print(f"[golden] {spec['name']}", flush=True)
    dm = mxfa.upload(c.mask) if c.mask is not None else None
    o = mxfa.flash_attn_ext(mxfa.upload(c.q), mxfa.upload(c.k), mxfa.upload(c.v), dm, c.scale, c.max_bias,
                            c.softcap)
    torch.cuda.synchronize()
    got = mxfa.output_tensor(o).cpu().numpy()
    tol = MAX_ABS_TOL
    for ref in ("out_gate", "out_exact"):
        m = row_metrics(got, out[ref])
        assert m["max_abs"] <= tol and m["min_cos"] >= ROW_COS_TOL, (spec["name"], ref, m)
