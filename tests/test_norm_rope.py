"""Pre-attention fusion (mxfa_qk_norm_rope), CPU side: the oracle's
restatement of ggml's rms_norm and NEOX rope (oracle/fa_oracle.c,
ora_qk_norm_rope) pinned by what the mathematics fixes, and the C ABI's
argument checks.

ggml is absent from the reference checkout and its tests hold no vectors for
these ops, so the pins are closed forms chosen so that a plausible mistake
fails one of them: rope at position 0 is the identity (a wrong theta_0);
rows after rms_norm have unit RMS and the weight multiplies each dimension
(a dropped weight or eps in the wrong place); each rotated pair keeps its
norm (a sign error in the rotation); a one-hot input rotates into dimension
i + 64 with angle p * base^(-2i/128) (GPT-J pairing (2i, 2i+1) or a wrong
frequency exponent); rotations compose by relative position (a transposed
angle); V passes through untouched or clamped.  The no-RoPE form (DiT
cross-attention, ora_qk_norm) equals the rotating form at position 0 bit for
bit (rope at position 0 multiplies by cos 0 = 1 and adds sin 0 = 0 terms).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

BASE = 1_000_000.0
EPS = 1e-6


def _ora():
    import oracle

    oracle.build()
    return oracle


def _rows(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def test_position_zero_is_rms_norm_times_weight():
    o = _ora()
    q, k = _rows((1, 1, 3, 128), 1), _rows((1, 1, 2, 128), 2)
    w = np.linspace(0.5, 2.0, 128).astype(np.float32)
    qo, ko, _ = o.qk_norm_rope(q, k, k, w, w, np.array([0]), EPS, BASE)
    for x, y in ((q, qo), (k, ko)):
        rms = np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + EPS)
        np.testing.assert_allclose(y, (x / rms) * w, rtol=2e-6, atol=1e-6)
    # with unit weights the rows have unit RMS
    qo1, _, _ = o.qk_norm_rope(q, k, k, np.ones(128), np.ones(128), np.array([0]), EPS, BASE)
    np.testing.assert_allclose(np.sqrt((qo1.astype(np.float64) ** 2).mean(-1)), 1.0, atol=2e-6)


def test_rotation_keeps_pair_norms():
    o = _ora()
    q = _rows((2, 5, 4, 128), 3)
    ones = np.ones(128, dtype=np.float32)
    pos = np.array([0, 1, 17, 300, 8191], dtype=np.int32)
    q0, _, _ = o.qk_norm_rope(q, q[:, :, :1], q[:, :, :1], ones, ones, np.zeros(5, np.int32), EPS, BASE)
    qp, _, _ = o.qk_norm_rope(q, q[:, :, :1], q[:, :, :1], ones, ones, pos, EPS, BASE)
    n0 = q0[..., :64] ** 2 + q0[..., 64:] ** 2
    n1 = qp[..., :64] ** 2 + qp[..., 64:] ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("i", [0, 1, 7, 63])
@pytest.mark.parametrize("p", [1, 3, 250])
def test_neox_pairing_and_frequency(i, p):
    """One-hot at dimension i: after rms_norm it holds sqrt(128); rope turns
    it into sqrt(128) * (cos a, sin a) at dimensions (i, i + 64), a = p *
    base^(-2i/128), and leaves every other dimension at 0."""
    o = _ora()
    x = np.zeros((1, 1, 1, 128), dtype=np.float32)
    x[..., i] = 1.0
    ones = np.ones(128, dtype=np.float32)
    y, _, _ = o.qk_norm_rope(x, x, x, ones, ones, np.array([p]), 0.0, BASE)
    a = p * BASE ** (-2.0 * i / 128)
    r = np.sqrt(128.0)
    exp = np.zeros(128)
    exp[i], exp[i + 64] = r * np.cos(a), r * np.sin(a)
    # float theta (repeated products) and float cos/sin: a few ulps of the angle
    np.testing.assert_allclose(y[0, 0, 0], exp, atol=r * (1e-6 + 3e-7 * p))


def test_relative_position():
    """<R(p) a, R(p + d) b> = <R(0) a, R(d) b>: attention scores depend on
    the distance only."""
    o = _ora()
    a, b = _rows((1, 1, 1, 128), 5), _rows((1, 1, 1, 128), 6)
    ones = np.ones(128, dtype=np.float32)

    def rot(x, p):
        y, _, _ = o.qk_norm_rope(x, x, x, ones, ones, np.array([p]), EPS, BASE)
        return y[0, 0, 0].astype(np.float64)

    for p, d in ((0, 5), (100, 5), (1000, 37)):
        s0 = rot(a, 0) @ rot(b, d)
        s1 = rot(a, p) @ rot(b, p + d)
        assert abs(s0 - s1) < 2e-3 * (1 + abs(s0)), (p, d, s0, s1)


def test_v_passthrough_and_clamp_and_batch_positions():
    o = _ora()
    v = _rows((2, 3, 2, 128), 7) * 1e5
    q = _rows((2, 3, 4, 128), 8)
    ones = np.ones(128, dtype=np.float32)
    pos = np.array([[0, 1, 2], [10, 11, 12]], dtype=np.int32)
    _, _, vo = o.qk_norm_rope(q, v, v, ones, ones, pos, EPS, BASE, clamp_v=False)
    np.testing.assert_array_equal(vo, v)
    _, _, vc = o.qk_norm_rope(q, v, v, ones, ones, pos, EPS, BASE, clamp_v=True)
    np.testing.assert_array_equal(vc, np.clip(v, -65504.0, 65504.0))
    # per-batch positions: batch 1 at position 10 equals batch 0 run at 10
    qa, _, _ = o.qk_norm_rope(q, v, v, ones, ones, pos, EPS, BASE)
    qb, _, _ = o.qk_norm_rope(q[1:], v[1:], v[1:], ones, ones, np.array([10, 11, 12]), EPS, BASE)
    np.testing.assert_array_equal(qa[1], qb[0])


def _dev(t, ne, nb, typ, ptr=1 << 20):
    import mxfa

    return mxfa.DeviceView(typ, ne, nb, ptr)


def test_abi_argument_checks():
    """Malformed calls are rejected before anything is launched (no device
    is touched: every check precedes the launch)."""
    import mxfa

    D, Nh, Nkv, S = 128, 4, 2, 8
    q = _dev(0, (D, Nh, S, 1), (4, 4 * D, 4 * D * Nh, 4 * D * Nh * S), 0)
    k = _dev(0, (D, Nkv, S, 1), (4, 4 * D, 4 * D * Nkv, 4 * D * Nkv * S), 0)
    w = _dev(0, (D, 1, 1, 1), (4, 4 * D, 4 * D, 4 * D), 0)
    pos = _dev(0, (S, 1, 1, 1), (4, 4 * S, 4 * S, 4 * S), 26)
    qo = _dev(0, (D, Nh, S, 1), (2, 2 * D, 2 * D * Nh, 2 * D * Nh * S), 1)
    ko = _dev(0, (D, 64, Nkv, 1), (2, 2 * D, 2 * D * 64, 2 * D * 64 * Nkv), 1)
    bad = dict(q=q, k=k, v=k, qn=w, kn=w, pos=pos, qo=qo, ko=ko, vo=ko)

    def call(**kw):
        a = dict(bad)
        a.update(kw)
        try:
            mxfa.qk_norm_rope(a["q"], a["k"], a["v"], a["qn"], a["kn"], a["pos"], EPS, BASE, a["qo"], a["ko"],
                              a["vo"], stream=0)
        except mxfa.MxfaError as e:
            return e.status
        return 0

    assert call(q=mxfa.DeviceView(0, (64, Nh, S, 1), q.nb, q.ptr)) == mxfa.ERR_UNSUPPORTED   # head size
    assert call(pos=mxfa.DeviceView(26, (S - 1, 1, 1, 1), pos.nb, pos.ptr)) == mxfa.ERR_INVALID
    assert call(qo=mxfa.DeviceView(0, qo.ne, (4,) + qo.nb[1:], qo.ptr)) == mxfa.ERR_UNSUPPORTED   # F32 out
    assert call(ko=mxfa.DeviceView(1, (D, S - 1, Nkv, 1), ko.nb, ko.ptr),
                vo=mxfa.DeviceView(1, (D, S - 1, Nkv, 1), ko.nb, ko.ptr)) == mxfa.ERR_INVALID    # too few rows
    assert call(kn=mxfa.DeviceView(0, (64, 1, 1, 1), w.nb, w.ptr)) == mxfa.ERR_INVALID
    # rows are read in 16-byte pieces: a misaligned view is left to the op chain
    assert call(q=mxfa.DeviceView(0, q.ne, q.nb, q.ptr + 4)) == mxfa.ERR_UNSUPPORTED
    assert call(qn=mxfa.DeviceView(0, w.ne, w.nb, w.ptr + 4)) == mxfa.ERR_UNSUPPORTED
    # the supports query answers without launching (descriptors only)
    P = ctypes.POINTER(mxfa.MxfaTensor)
    descs = [t.desc() for t in (q, k, k, w, w, pos, qo, ko, ko)]
    prm = mxfa.MxfaNormRopeParams(EPS, BASE, 0)
    ref = [ctypes.byref(d) for d in descs]
    assert mxfa.lib.mxfa_qk_norm_rope_supports(ref[0], ref[1], ref[2], ref[3], ref[4], ref[5], ctypes.byref(prm),
                                               ref[6], ref[7], ref[8], None) == 1
    bad_pos = mxfa.DeviceView(27, pos.ne, (8, 8 * S, 8 * S, 8 * S), pos.ptr).desc()
    assert mxfa.lib.mxfa_qk_norm_rope_supports(ref[0], ref[1], ref[2], ref[3], ref[4], ctypes.byref(bad_pos),
                                               ctypes.byref(prm), ref[6], ref[7], ref[8], None) == 0


def test_norm_without_rope_is_position_zero():
    """ora_qk_norm (the QK-norm of DiT cross-attention, no RoPE,
    dit-graph.h:326-333) equals the rotating chain at position 0, bit for
    bit, and normalises each row to unit RMS times the weight."""
    o = _ora()
    q, k = _rows((2, 3, 4, 128), 11) * 3, _rows((2, 3, 2, 128), 12)
    w = np.linspace(0.25, 3.0, 128).astype(np.float32)
    qo, ko, _ = o.qk_norm_rope(q, k, k, w, w, np.zeros(3, np.int32), EPS, BASE)
    np.testing.assert_array_equal(o.qk_norm(q, w, EPS), qo)
    np.testing.assert_array_equal(o.qk_norm(k, w, EPS), ko)
    y = o.qk_norm(q, np.ones(128, np.float32), EPS)
    np.testing.assert_allclose(np.sqrt((y.astype(np.float64) ** 2).mean(-1)), 1.0, atol=2e-6)
    # scale invariance of rms_norm (eps negligible)
    np.testing.assert_allclose(o.qk_norm(q * 8, w, 0.0), o.qk_norm(q, w, 0.0), rtol=1e-6, atol=1e-7)


def test_abi_cross_attention_form():
    """positions = NULL: no rotation, and K/V may hold enc_S tokens next to
    Q's S (the DiT cross-attention chain, dit-graph.h:317-346); with
    positions given the token counts must agree."""
    import mxfa

    D, Nh, Nkv, S, E = 128, 4, 2, 8, 5
    q = _dev(0, (D, Nh, S, 1), (4, 4 * D, 4 * D * Nh, 4 * D * Nh * S), 0)
    k = _dev(0, (D, Nkv, E, 1), (4, 4 * D, 4 * D * Nkv, 4 * D * Nkv * E), 0)
    w = _dev(0, (D, 1, 1, 1), (4, 4 * D, 4 * D, 4 * D), 0)
    pos = _dev(0, (S, 1, 1, 1), (4, 4 * S, 4 * S, 4 * S), 26)
    qo = _dev(0, (D, Nh, S, 1), (2, 2 * D, 2 * D * Nh, 2 * D * Nh * S), 1)
    ko = _dev(0, (D, E, Nkv, 1), (2, 2 * D, 2 * D * E, 2 * D * E * Nkv), 1)
    P = ctypes.POINTER(mxfa.MxfaTensor)
    prm = mxfa.MxfaNormRopeParams(EPS, BASE, 0)

    def sup(pos_view, kk=k, kout=ko, rows=None):
        d = [t.desc() for t in (q, kk, kk, w, w)]
        dp = pos_view.desc() if pos_view is not None else None
        o = [t.desc() for t in (qo, kout, kout)]
        r = [ctypes.byref(x) for x in d]
        ro = [ctypes.byref(x) for x in o]
        return mxfa.lib.mxfa_qk_norm_rope_supports(r[0], r[1], r[2], r[3], r[4],
                                                   ctypes.byref(dp) if dp is not None else None,
                                                   ctypes.byref(prm), ro[0], ro[1], ro[2],
                                                   ctypes.byref(rows.desc()) if rows is not None else None)

    assert sup(None) == 1                 # no RoPE, 5 K/V tokens against 8 queries
    assert sup(pos) == 0                  # RoPE needs one position per token of every row
    short = _dev(0, (D, E - 1, Nkv, 1), ko.nb, 1)
    assert sup(None, kout=short) == 0     # too few K/V rows
    rows_e = _dev(0, (E, 1, 1, 1), (8, 8 * E, 8 * E, 8 * E), 27)
    rows_s = _dev(0, (S, 1, 1, 1), (8, 8 * S, 8 * S, 8 * S), 27)
    assert sup(None, rows=rows_e) == 1    # row ids count K/V tokens
    assert sup(None, rows=rows_s) == 0
