#!/usr/bin/env python3
"""Writes the golden fixtures of tests/golden/ (run from the repo root).

Each fixture is a small seeded attention case in the layouts the reference
hands to ggml_flash_attn_ext, with the expected outputs:
  out_exact   fp64 two-pass softmax on the same rounded Q (oracle fa_exact)
  out_gate    ggml CPU algorithm with an fp32 V accumulator (the GPU gate)
  out_strict  ggml CPU algorithm as it runs (fp16 V accumulator for F16 V)
ggml itself is not available (its submodule is empty in the reference), so
these outputs come from the C restatement in oracle/ after it passed the
closed-form and invariant checks of tests/test_oracle.py; the fixtures pin
that state so later changes to the oracle or the kernels are caught.
Inputs are Philox4x32-10 N(0,1) (acestep.cpp_amd/mxfa/synth.py), seed and
streams recorded per fixture.  Stored with numpy.savez (no pickled objects).
"""
from __future__ import annotations

import json
import math
import os
import sys

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(REPO, "acestep.cpp_amd"))
sys.path.insert(0, os.path.join(REPO, "oracle"))

from mxfa import synth  # noqa: E402
from mxfa.cases import FaCase, HostView, quantize_q8_0, to_bf16_bits, to_f16_bits  # noqa: E402

D = 128
OUT_DIR = os.path.dirname(os.path.abspath(__file__))


def make_case(name, seed, B, Sq, Nh, Nkv, Skv, kv_type, mask, softcap=0.0, max_bias=0.0):
    q = synth.normal(seed, 0, 0, D * Sq * Nh * B).astype(np.float32)
    # permuted Q view as the LM builds it: memory [B, Sq, Nh, D]
    qv = HostView(0, (D, Sq, Nh, B), (4, 4 * D * Nh, 4 * D, 4 * D * Nh * Sq), q)
    kf = synth.normal(seed, 1, 0, D * Skv * Nkv * B)
    vf = synth.normal(seed, 2, 0, D * Skv * Nkv * B)
    if kv_type == 8:
        kb, vb = quantize_q8_0(kf), quantize_q8_0(vf)
        row = D // 32 * 34
        nb = (34, row, row * Skv, row * Skv * Nkv)
    else:
        conv = to_bf16_bits if kv_type == 30 else to_f16_bits
        kb, vb = conv(kf), conv(vf)
        nb = (2, 2 * D, 2 * D * Skv, 2 * D * Skv * Nkv)
    kv = HostView(kv_type, (D, Skv, Nkv, B), nb, kb)
    vv = HostView(kv_type, (D, Skv, Nkv, B), nb, vb)
    mv = None
    if mask == "causal":
        allowed = np.arange(Skv)[None, :] <= (Skv - Sq + np.arange(Sq))[:, None]
        vals = np.broadcast_to(np.where(allowed, 0.0, -np.inf), (B, 1, Sq, Skv))
    elif mask == "random":
        u = synth.uniform_u32(seed, 4, 0, B * Sq * Skv).reshape(B, 1, Sq, Skv)
        g = synth.normal(seed, 3, 0, B * Sq * Skv).reshape(B, 1, Sq, Skv)
        vals = np.where(u % 10 < 3, -np.inf, 0.5 * g)
        vals[..., 0] = 0.0       # every row keeps a live key
    elif mask == "zero":
        vals = np.zeros((B, 1, Sq, Skv))
    else:
        vals = None
    if vals is not None:
        if max_bias > 0:
            vals = np.where(np.isneginf(vals), vals, -np.abs(vals) * 3)
        bits = np.asarray(vals, dtype=np.float32).astype(np.float16).view(np.uint16).reshape(-1).copy()
        mv = HostView(1, (Skv, Sq, 1, B), (2, 2 * Skv, 2 * Skv * Sq, 2 * Skv * Sq), bits)
    return FaCase(name, qv, kv, vv, mv, 1.0 / math.sqrt(D), max_bias=max_bias, softcap=softcap,
                  meta=dict(seed=seed, streams=dict(q=0, k=1, v=2, mask_values=3, mask_keep=4)))


CASES = [
    dict(name="decode_gqa_mask", seed=2001, B=2, Sq=1, Nh=8, Nkv=2, Skv=77, kv_type=1, mask="random"),
    dict(name="short_rows_f16", seed=2002, B=1, Sq=5, Nh=4, Nkv=4, Skv=33, kv_type=1, mask=None),
    dict(name="prefill_causal", seed=2003, B=1, Sq=64, Nh=2, Nkv=1, Skv=64, kv_type=1, mask="causal"),
    dict(name="q8_0_decode", seed=2004, B=1, Sq=2, Nh=4, Nkv=2, Skv=100, kv_type=8, mask="zero"),
    dict(name="bf16_softcap_alibi", seed=2005, B=1, Sq=3, Nh=8, Nkv=4, Skv=50, kv_type=30, mask="random",
         softcap=30.0, max_bias=8.0),
]


def main():
    import oracle

    oracle.build()
    for spec in CASES:
        c = make_case(**spec)
        args = (c.q, c.k, c.v, c.mask, c.scale, c.max_bias, c.softcap)
        exact = oracle.fa_exact(*args, q_round=True, n_threads=1)
        gate = oracle.fa_ggml(*args, n_threads=1, acc_f32=True)
        strict = oracle.fa_ggml(*args, n_threads=1)
        meta = dict(spec=spec, scale=c.scale, q=dict(ne=c.q.ne, nb=c.q.nb), k=dict(ne=c.k.ne, nb=c.k.nb),
                    v=dict(ne=c.v.ne, nb=c.v.nb),
                    mask=None if c.mask is None else dict(ne=c.mask.ne, nb=c.mask.nb),
                    rng=c.meta)
        arrays = dict(meta=np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8),
                      q=c.q.buf, k=c.k.buf.view(np.uint8), v=c.v.buf.view(np.uint8),
                      out_exact=exact, out_gate=gate, out_strict=strict)
        if c.mask is not None:
            arrays["mask"] = c.mask.buf
        path = os.path.join(OUT_DIR, spec["name"] + ".npz")
        np.savez_compressed(path, **arrays)
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
