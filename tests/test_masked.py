"""Structured masks (mxfa_flash_attn_ext_masked), CPU side.

The structured form stands for the dense F16 mask the reference builds on the
host.  These tests pin `cases.dense_mask_bits` (the dense form the GPU tests
compare against) to the reference's own mask loops, restated here as plain
loops over (query, key) -- a transposed index, an off-by-one at the causal
diagonal or the window edge, or a length compared with <= fails them -- and
check the C ABI's supports_op for the structured entry point (descriptor and
spec checks only, no device)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

NEG = 0xFC00


def _loops_causal(Sq, Skv, pos0):
    # src/qwen3-lm.h:600-607 (and qwen3-enc.h:431-435 with pos0 = 0)
    m = np.empty((Sq, Skv), dtype=np.uint16)
    for i in range(Sq):
        for j in range(Skv):
            m[i, j] = 0 if j <= pos0 + i else NEG
    return m


def _loops_lengths(Skv, kvl):
    # src/qwen3-lm.h:875-881: one query row per sequence, 0 for j < kv_len
    return np.array([0 if j < kvl else NEG for j in range(Skv)], dtype=np.uint16)


def _loops_window(S, win):
    # src/dit-sampler.h:273-283 (win <= 0 or S <= win: every key live)
    m = np.empty((S, S), dtype=np.uint16)
    for qi in range(S):
        for ki in range(S):
            dist = qi - ki if qi > ki else ki - qi
            m[qi, ki] = 0 if (win <= 0 or S <= win or dist <= win) else NEG
    return m


def _loops_pad(S, enc_S, re):
    # src/dit-sampler.h:299-305: value depends on the key only
    m = np.empty((S, enc_S), dtype=np.uint16)
    for qi in range(S):
        for ki in range(enc_S):
            m[qi, ki] = 0 if ki < re else NEG
    return m


def test_dense_form_matches_reference_loops():
    from mxfa import cases as C

    for Sq, Skv, pos0 in ((1, 300, 299), (7, 256, 100), (40, 40, 0)):
        got = C.dense_mask_bits(dict(causal=True, pos0=pos0), Sq, Skv, 1)[0, 0]
        np.testing.assert_array_equal(got, _loops_causal(Sq, Skv, pos0))
    lens = [5, 256, 1, 0]
    got = C.dense_mask_bits(dict(lengths=lens), 1, 256, 4)
    for b, L in enumerate(lens):
        np.testing.assert_array_equal(got[b, 0, 0], _loops_lengths(256, L))
    for S, win in ((50, 7), (33, 0), (20, 40)):
        spec = dict(window=win) if (win > 0 and S > win) else {}
        got = C.dense_mask_bits(spec, S, S, 1)[0, 0]
        np.testing.assert_array_equal(got, _loops_window(S, win))
    got = C.dense_mask_bits(dict(lengths=[17, 30]), 9, 32, 2)
    np.testing.assert_array_equal(got[0, 0], _loops_pad(9, 32, 17))
    np.testing.assert_array_equal(got[1, 0], _loops_pad(9, 32, 30))
    # flags combine as a conjunction
    got = C.dense_mask_bits(dict(causal=True, window=3, lengths=[12], pos0=4), 6, 16, 1)[0, 0]
    exp = np.where((_loops_causal(6, 16, 4) == 0) & (np.abs(np.arange(6)[:, None] + 4 - np.arange(16)[None, :]) <= 3)
                   & (np.arange(16)[None, :] < 12), 0, NEG)
    np.testing.assert_array_equal(got, exp)


def test_structured_specs_of_the_benchmark_cases():
    """The structured form of each masked benchmark case reproduces the mask
    the case builder laid out like the reference."""
    from mxfa import cases as C

    builds = [C.c1(), C.c2(n_tokens=256), C.lm_batch("t", N=4, max_seq=512, lmin=10, lmax=500),
              C.dit_cross("t", S=64), C.dit_self("t", S=300, window=64)]
    for c in builds:
        spec = C.structured_spec(c)
        d = C.with_dense_mask(c, spec)
        Sq, Skv, B = int(c.q.ne[1]), int(c.k.ne[1]), int(c.q.ne[3])
        own = c.mask.buf.reshape(int(c.mask.ne[3]), Sq, int(c.mask.ne[0]))[..., :Skv]
        mine = d.mask.buf.reshape(B, Sq, Skv)
        for b in range(B):
            np.testing.assert_array_equal(own[b % own.shape[0]], mine[b], err_msg=c.name)
    assert C.structured_spec(C.dit_self("t", S=64)) == {}


def _dev(view, ptr=1 << 20):
    import mxfa

    return mxfa.DeviceView(view.type, tuple(view.ne), tuple(view.nb), ptr)


def test_supports_masked():
    import mxfa
    from mxfa import cases as C

    c = C.c2(n_tokens=256)
    q, k, v = _dev(c.q), _dev(c.k), _dev(c.v)
    ok = lambda sp: mxfa.supports_masked(q, k, v, sp, c.scale)  # noqa: E731
    assert ok(mxfa.mask_spec(causal=True, pos0=0))
    assert ok(mxfa.mask_spec())                                    # no mask
    assert ok(mxfa.mask_spec(window=128, lengths=[100]))
    bad = mxfa.mask_spec(causal=True)
    bad.flags = 16
    assert not ok(bad) and "flags" in mxfa.last_error()
    # device-resident lengths / pos0 (MXFA_MASK_DEVICE): accepted without
    # reading them on the host (placeholder device addresses)
    dv = mxfa.mask_spec(causal=True)
    dv.flags |= mxfa.MASK_DEVICE
    dv.dev_pos0 = 1 << 20
    assert ok(dv)
    dl = mxfa.mask_spec(lengths=[7])
    dl.flags |= mxfa.MASK_DEVICE
    dl.lengths = ctypes.cast(ctypes.c_void_p(1 << 20), ctypes.POINTER(ctypes.c_int32))
    assert ok(dl)
    dl.lengths = None
    assert not ok(dl)
    assert not ok(mxfa.mask_spec(window=-1))
    assert not ok(mxfa.mask_spec(causal=True, pos0=-5))
    assert not ok(mxfa.mask_spec(lengths=[1, 2, 3]))                # neither 1 nor B = 1
    assert not ok(mxfa.mask_spec(lengths=[-1]))
    nolen = mxfa.mask_spec(lengths=[4])
    nolen.lengths = None
    assert not ok(nolen)
    cb = C.lm_batch("t", N=8, max_seq=1024, lmin=100, lmax=1024)
    qb, kb, vb = _dev(cb.q), _dev(cb.k), _dev(cb.v)
    assert mxfa.supports_masked(qb, kb, vb, mxfa.mask_spec(lengths=cb.meta["lengths"]), cb.scale)
