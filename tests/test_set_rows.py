"""KV-cache write (GGML_OP_SET_ROWS): the CPU oracle pinned, the host-side
case builders, and libmxfa's supports_op for the node (descriptor checks
only, no device).

ggml's set_rows lives in the un-vendored ggml submodule, and the reference's
tests hold no vectors for it, so the oracle (oracle/fa_oracle.c,
ora_set_rows) is pinned here by what the mathematics and the reference's
call sites fix:
  * F16 conversion = numpy's IEEE binary16 cast (round to nearest even);
  * BF16 conversion = an independent frexp/rint restatement of round to
    nearest even at 8 significant bits;
  * Q8_0 = error bound |x - q*d| <= d/2 per value, |q| <= 127 with 127 at the
    block's amax, d = fp16(amax/127), and a known tie (x*127/amax = 2.5 -> 2:
    round half to even, as ggml's AVX2/NEON quantisers do), and against the
    numpy quantiser of mxfa.cases;
  * placement = the two reference layouts written out as array assignments
    (src/qwen3-lm.h:453-454: cache[:, rows[i], h] = k[:, i, h];
    :776-777: sets[:, rows[s], h, s] = k_new[:, 0, h, s]), rows not named
    keep their bytes, a row id broadcast per head (R1 > 1), I32 ids, and
    out-of-range ids skipped and counted.
"""
from __future__ import annotations

import numpy as np
import pytest

D = 128


def _ora():
    import oracle

    oracle.build()
    return oracle


def _host(t, ne, nb, buf, offset=0):
    import oracle

    return oracle.HostTensor(t, tuple(ne), tuple(nb), buf, offset)


def _bf16_rne_independent(x: np.ndarray) -> np.ndarray:
    """x rounded to 8 significant bits (round half to even), as float32."""
    x = x.astype(np.float64)
    m, e = np.frexp(x)                      # x = m * 2^e, 0.5 <= |m| < 1
    r = np.rint(m * 256.0) / 256.0          # 8 significant bits
    return np.ldexp(r, e).astype(np.float32)


def _rows_f32(n, seed=0, scale=1.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(n) * scale).astype(np.float32)


def test_f16_rows_match_numpy_rne():
    o = _ora()
    S, Nkv, M = 7, 3, 11
    x = _rows_f32(D * S * Nkv, 1, 300.0)
    # include values at the fp16 overflow edge, tiny subnormals and exact ties
    x[:6] = [65504.0, 65520.0, 1e-6, -6e-8, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11]
    src = _host(o.F32, (D, S, Nkv, 1), (4, 4 * D, 4 * D * S, 4 * D * S * Nkv), x)
    rows = np.array([3, 0, 10, 5, 1, 7, 2], dtype=np.int64)
    rv = _host(o.I64, (S, 1, 1, 1), (8, 8 * S, 8 * S, 8 * S), rows)
    cache = np.full(D * M * Nkv, 0x1234, dtype=np.uint16)
    dst = _host(o.F16, (D, M, Nkv, 1), (2, 2 * D, 2 * D * M, 2 * D * M * Nkv), cache)
    assert o.set_rows(dst, src, rv) == 0
    got = cache.reshape(Nkv, M, D)
    with np.errstate(over="ignore"):          # 65520 rounds to inf, as intended
        ref = x.reshape(Nkv, S, D).astype(np.float16).view(np.uint16)
    for i, r in enumerate(rows):
        np.testing.assert_array_equal(got[:, r, :], ref[:, i, :])
    untouched = sorted(set(range(M)) - set(rows.tolist()))
    assert (got[:, untouched, :] == 0x1234).all()


def test_bf16_rows_match_independent_rounding():
    o = _ora()
    S, Nkv, M = 5, 2, 5
    x = _rows_f32(D * S * Nkv, 2, 10.0)
    x[0] = 1.0 + 2.0 ** -8            # exact tie -> even (1.0)
    x[1] = 1.0 + 3 * 2.0 ** -8        # exact tie -> even (1 + 2^-6)
    src = _host(o.F32, (D, S, Nkv, 1), (4, 4 * D, 4 * D * S, 4 * D * S * Nkv), x)
    rows = np.arange(S, dtype=np.int32)[::-1].copy()
    rv = _host(o.I32, (S, 1, 1, 1), (4, 4 * S, 4 * S, 4 * S), rows)
    cache = np.zeros(D * M * Nkv, dtype=np.uint16)
    dst = _host(o.BF16, (D, M, Nkv, 1), (2, 2 * D, 2 * D * M, 2 * D * M * Nkv), cache)
    assert o.set_rows(dst, src, rv) == 0
    got = (cache.astype(np.uint32) << 16).view(np.float32).reshape(Nkv, M, D)
    ref = _bf16_rne_independent(x).reshape(Nkv, S, D)
    for i, r in enumerate(rows):
        np.testing.assert_array_equal(got[:, r, :], ref[:, i, :])
    assert got[0, rows[0], 0] == 1.0 and got[0, rows[0], 1] == 1.0 + 2.0 ** -6


def test_q8_0_rows_bounds_and_ties():
    o = _ora()
    from mxfa import cases as C

    S, Nkv, M = 6, 2, 9
    x = _rows_f32(D * S * Nkv, 3, 4.0)
    # block 0 of row 0: amax 127 -> id = 1, so 2.5 and -3.5 are exact ties
    x[:32] = 0.25
    x[0], x[1], x[2] = 127.0, 2.5, -3.5
    x[32:64] = 0.0                   # all-zero block: d = 0, q = 0
    src = _host(o.F32, (D, S, Nkv, 1), (4, 4 * D, 4 * D * S, 4 * D * S * Nkv), x)
    rows = np.array([8, 0, 4, 2, 6, 1], dtype=np.int64)
    rv = _host(o.I64, (S, 1, 1, 1), (8, 8 * S, 8 * S, 8 * S), rows)
    rb = D // 32 * 34
    cache = np.full(rb * M * Nkv, 0xAB, dtype=np.uint8)
    dst = _host(o.Q8_0, (D, M, Nkv, 1), (34, rb, rb * M, rb * M * Nkv), cache)
    assert o.set_rows(dst, src, rv) == 0
    got = cache.reshape(Nkv, M, D // 32, 34)
    xs = x.reshape(Nkv, S, D // 32, 32)
    for h in range(Nkv):
        for i, r in enumerate(rows):
            for b in range(D // 32):
                blk = got[h, r, b]
                d = blk[:2].view(np.float16)[0]
                q = blk[2:].view(np.int8).astype(np.int64)
                xb = xs[h, i, b]
                amax = np.abs(xb).max()
                assert d == np.float16(np.float32(amax) / np.float32(127.0))
                if amax == 0:
                    assert (q == 0).all()
                    continue
                assert np.abs(q).max() == 127 and q[np.argmax(np.abs(xb))] == np.sign(xb[np.argmax(np.abs(xb))]) * 127
                # |x - q*amax/127| <= amax/254 (plus float slack)
                err = np.abs(xb.astype(np.float64) - q * (amax / 127.0))
                assert err.max() <= amax / 254.0 * (1 + 1e-6)
            np.testing.assert_array_equal(got[h, r].reshape(-1), C.quantize_q8_0(xs[h, i].reshape(-1)))
    q0 = got[0, rows[0], 0, 2:].view(np.int8)
    assert q0[0] == 127 and q0[1] == 2 and q0[2] == -4      # half to even: 2.5 -> 2, -3.5 -> -4
    untouched = sorted(set(range(M)) - set(rows.tolist()))
    assert (got[:, untouched] == 0xAB).all()


def test_reference_layout_single():
    """src/qwen3-lm.h:448-454 written as an array assignment."""
    o = _ora()
    from mxfa import cases as C

    c = C.kv_write_single("t", seed=5, n_tokens=37, kv_pos=100, Nkv=4, max_seq=256, cache_type=C.TYPE_F32)
    before = c.dst.buf.copy()
    assert o.set_rows(c.dst, c.src, c.rows) == 0
    cache = c.dst.buf.view(np.float32).reshape(4, 256, D)
    k = c.src.buf.reshape(4, 37, D)
    exp = before.view(np.float32).reshape(4, 256, D).copy()
    exp[:, 100:137, :] = k
    np.testing.assert_array_equal(cache.view(np.uint32), exp.view(np.uint32))


def test_reference_layout_batched_sets():
    """src/qwen3-lm.h:760-777: one row per set at its own position, the view
    starting at set s0, sets outside [s0, s0+N) untouched."""
    o = _ora()
    from mxfa import cases as C

    N, Nkv, M, s0, n_sets = 4, 2, 64, 1, 6
    pos = [5, 63, 0, 5]
    c = C.kv_write_batch("t", seed=6, N=N, Nkv=Nkv, max_seq=M, n_sets=n_sets, s0=s0, positions=pos,
                         cache_type=C.TYPE_F16)
    before = c.dst.buf.copy().view(np.uint16).reshape(n_sets, Nkv, M, D)
    assert o.set_rows(c.dst, c.src, c.rows) == 0
    got = c.dst.buf.view(np.uint16).reshape(n_sets, Nkv, M, D)
    kn = c.src.buf.reshape(N, Nkv, 1, D)
    exp = before.copy()
    for s in range(N):
        exp[s0 + s, :, pos[s], :] = kn[s, :, 0, :].astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, exp)


def test_per_head_ids_and_out_of_range():
    """R1 = Nkv (one id per head), I32 ids, ids past the cache skipped."""
    o = _ora()
    S, Nkv, M = 3, 2, 8
    x = _rows_f32(D * S * Nkv, 7)
    src = _host(o.F32, (D, S, Nkv, 1), (4, 4 * D, 4 * D * S, 4 * D * S * Nkv), x)
    ids = np.array([[1, 4, 9], [2, -1, 0]], dtype=np.int32)        # [Nkv][S]; 9 and -1 out of range
    rv = _host(o.I32, (S, Nkv, 1, 1), (4, 4 * S, 4 * S * Nkv, 4 * S * Nkv), ids)
    cache = np.zeros(D * M * Nkv, dtype=np.float32)
    dst = _host(o.F32, (D, M, Nkv, 1), (4, 4 * D, 4 * D * M, 4 * D * M * Nkv), cache)
    assert o.set_rows(dst, src, rv) == 2
    got = cache.reshape(Nkv, M, D)
    xs = x.reshape(Nkv, S, D)
    np.testing.assert_array_equal(got[0, 1], xs[0, 0])
    np.testing.assert_array_equal(got[0, 4], xs[0, 1])
    np.testing.assert_array_equal(got[1, 2], xs[1, 0])
    np.testing.assert_array_equal(got[1, 0], xs[1, 2])
    written = {(0, 1), (0, 4), (1, 2), (1, 0)}
    for h in range(Nkv):
        for r in range(M):
            if (h, r) not in written:
                assert (got[h, r] == 0).all()


def test_oracle_rejects_malformed_nodes():
    o = _ora()
    x = np.zeros(D * 4, dtype=np.float32)
    src = _host(o.F32, (D, 4, 1, 1), (4, 4 * D, 16 * D, 16 * D), x)
    ids = np.zeros(3, dtype=np.int64)
    bad_rows = _host(o.I64, (3, 1, 1, 1), (8, 24, 24, 24), ids)      # ne0 != src ne1
    cache = np.zeros(D * 8, dtype=np.float32)
    dst = _host(o.F32, (D, 8, 1, 1), (4, 4 * D, 32 * D, 32 * D), cache)
    with pytest.raises(ValueError):
        o.set_rows(dst, src, bad_rows)
    f64_rows = _host(28, (4, 1, 1, 1), (8, 32, 32, 32), np.zeros(4, dtype=np.int64))
    with pytest.raises(ValueError):
        o.set_rows(dst, src, f64_rows)


# -- supports_op of the C ABI (descriptor checks only) -------------------------

def _dev(view, ptr=1 << 20):
    import mxfa

    return mxfa.DeviceView(view.type, tuple(view.ne), tuple(view.nb), ptr)


@pytest.mark.parametrize("name", ["kw2", "kw3", "kw5"])
def test_set_rows_supports_reference_layouts(name):
    import mxfa
    from mxfa import cases as C

    kw = {"kw2": dict(n_tokens=64, max_seq=256), "kw5": dict(n_tokens=64, max_seq=256),
          "kw3": dict(max_seq=256)}[name]
    c = C.SET_ROWS_BUILDERS[name](**kw)
    assert mxfa.set_rows_supports(_dev(c.dst), _dev(c.src, 1 << 24), _dev(c.rows, 1 << 26)), mxfa.last_error()


def test_set_rows_supports_rejections():
    import mxfa
    from mxfa import cases as C

    c = C.kv_write_single("t", n_tokens=16, max_seq=64, Nkv=2)
    d, s, r = _dev(c.dst), _dev(c.src, 1 << 24), _dev(c.rows, 1 << 26)
    assert mxfa.set_rows_supports(d, s, r)
    ok = lambda **kw: mxfa.set_rows_supports(kw.get("d", d), kw.get("s", s), kw.get("r", r))  # noqa: E731
    assert not ok(s=mxfa.DeviceView(1, s.ne, (2,) + s.nb[1:], s.ptr))                 # F16 source
    assert not ok(r=mxfa.DeviceView(28, r.ne, r.nb, r.ptr))                             # id type
    assert not ok(r=mxfa.DeviceView(r.type, (15,) + r.ne[1:], r.nb, r.ptr))             # n mismatch
    assert not ok(r=mxfa.DeviceView(r.type, (16, 3, 1, 1), r.nb, r.ptr))                # 2 % 3 != 0
    assert not ok(d=mxfa.DeviceView(d.type, (64,) + d.ne[1:], d.nb, d.ptr))             # row length
    assert not ok(d=mxfa.DeviceView(d.type, d.ne[:2] + (4, 1), d.nb, d.ptr))            # head count
    assert not ok(s=mxfa.DeviceView(s.type, s.ne, s.nb, s.ptr + 4))                     # alignment
    assert not ok(d=mxfa.DeviceView(6, d.ne, d.nb, d.ptr))                              # dst type
    assert "type" in mxfa.last_error()
    # an empty source is a well-formed no-op
    empty_s = mxfa.DeviceView(s.type, (D, 0, 2, 1), s.nb, 0)
    empty_r = mxfa.DeviceView(r.type, (0, 1, 1, 1), r.nb, 0)
    assert ok(s=empty_s, r=empty_r)
