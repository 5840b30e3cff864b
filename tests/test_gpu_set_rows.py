"""GPU parity of the KV-cache write (GGML_OP_SET_ROWS): libmxfa's set_rows
kernel, called through the C ABI (mxfa.set_rows -> mxfa_set_rows), against
the CPU oracle (ora_set_rows) on the same bytes.  The bar is bit-exact: the
whole destination buffer (written rows and the rows the write must leave
alone) is compared byte for byte.

At the benchmark's full sizes the check is a property that needs no oracle
pass: the rows gathered back out of the cache equal torch's own F16 cast of
the source (IEEE round to nearest even), and every other row is unchanged.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
D = 128


@pytest.fixture(scope="module")
def mx():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mxfa

    return mxfa


def _run_both(mx, c, label):
    """Runs the write on the GPU and in the oracle; returns (gpu bytes,
    oracle bytes, skipped rows)."""
    import oracle
    import torch

    print(f"[set_rows] {label}: src{tuple(c.src.ne)} dst{tuple(c.dst.ne)} t{c.dst.type} "
          f"rows{tuple(c.rows.ne)} t{c.rows.type}", flush=True)
    dd, ds, dr = mx.upload(c.dst), mx.upload(c.src), mx.upload(c.rows)
    mx.set_rows(dd, ds, dr)
    torch.cuda.synchronize()
    got = dd.owner.cpu().numpy()
    ref_buf = np.ascontiguousarray(c.dst.buf).view(np.uint8).reshape(-1).copy()
    ref_view = oracle.HostTensor(c.dst.type, tuple(c.dst.ne), tuple(c.dst.nb), ref_buf, c.dst.offset)
    skipped = oracle.set_rows(ref_view, c.src, c.rows)
    return got, ref_buf, skipped


@pytest.mark.parametrize("ctype", ["f32", "f16", "bf16", "q8_0"])
@pytest.mark.parametrize("rtype", ["i64", "i32"])
def test_single_sequence_write(mx, ctype, rtype):
    from mxfa import cases as C

    t = {"f32": C.TYPE_F32, "f16": C.TYPE_F16, "bf16": C.TYPE_BF16, "q8_0": C.TYPE_Q8_0}[ctype]
    r = C.TYPE_I64 if rtype == "i64" else C.TYPE_I32
    c = C.kv_write_single("t", seed=11, n_tokens=300, kv_pos=77, Nkv=8, max_seq=512, cache_type=t, row_type=r)
    got, ref, skipped = _run_both(mx, c, f"single {ctype} {rtype}")
    assert skipped == 0
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("ctype", ["f16", "q8_0"])
def test_decode_token_write(mx, ctype):
    """One token at the end of a 512-row window (C1's write)."""
    from mxfa import cases as C

    t = C.TYPE_F16 if ctype == "f16" else C.TYPE_Q8_0
    c = C.kv_write_single("t", seed=12, n_tokens=1, kv_pos=511, Nkv=8, max_seq=8192, cache_type=t)
    got, ref, _ = _run_both(mx, c, f"decode {ctype}")
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("ctype", ["f16", "bf16", "q8_0"])
def test_batched_sets_write(mx, ctype):
    """C3's write: N sets from s0, one position each, view offset into the
    4D cache; sets outside the view untouched."""
    from mxfa import cases as C

    t = {"f16": C.TYPE_F16, "bf16": C.TYPE_BF16, "q8_0": C.TYPE_Q8_0}[ctype]
    c = C.kv_write_batch("t", seed=13, N=8, Nkv=8, max_seq=1024, n_sets=11, s0=2, cache_type=t)
    got, ref, _ = _run_both(mx, c, f"batched {ctype}")
    np.testing.assert_array_equal(got, ref)


def test_per_head_ids_and_out_of_range(mx):
    """Row ids per KV head (R1 = Nkv), I32, some outside the cache: those
    rows are skipped on both sides."""
    import oracle
    from mxfa import cases as C

    c = C.kv_write_single("t", seed=14, n_tokens=40, kv_pos=0, Nkv=4, max_seq=64, cache_type=C.TYPE_F16)
    rng = np.random.default_rng(14)
    ids = rng.integers(-3, 70, size=(4, 40)).astype(np.int32)
    ids[0, :] = np.arange(40)          # one clean head
    rows = oracle.HostTensor(C.TYPE_I32, (40, 4, 1, 1), (4, 160, 640, 640), ids)
    c = C.SetRowsCase("t", c.dst, c.src, rows)
    got, ref, skipped = _run_both(mx, c, "per-head ids")
    assert skipped == int(((ids < 0) | (ids >= 64)).sum()) > 0
    # duplicate ids within a head race (unspecified order, as in ggml): compare
    # only the rows that exactly one source row names
    M = 64
    g = got.view(np.uint16).reshape(4, M, D)
    r = ref.view(np.uint16).reshape(4, M, D)
    for h in range(4):
        vals, counts = np.unique(ids[h][(ids[h] >= 0) & (ids[h] < M)], return_counts=True)
        single = set(vals[counts == 1].tolist())
        for row in range(M):
            if row in single or row not in vals:
                np.testing.assert_array_equal(g[h, row], r[h, row], err_msg=f"head {h} row {row}")


def test_broadcast_over_batches(mx):
    """Row ids [n, 1, R2] broadcast over ne3 (ne3 % R2 == 0, R2 < ne3)."""
    import oracle
    from mxfa import cases as C

    S, Nkv, B, M = 17, 2, 4, 40
    x = np.random.default_rng(15).standard_normal(D * S * Nkv * B).astype(np.float32)
    src = oracle.HostTensor(C.TYPE_F32, (D, S, Nkv, B), (4, 4 * D, 4 * D * S, 4 * D * S * Nkv), x)
    ids = np.stack([np.arange(S) + 3, np.arange(S)[::-1] + 20]).astype(np.int64)   # R2 = 2
    rows = oracle.HostTensor(C.TYPE_I64, (S, 1, 2, 1), (8, 8 * S, 8 * S, 16 * S), ids)
    cache = np.random.default_rng(16).integers(0, 2 ** 16, size=D * M * Nkv * B).astype(np.uint16)
    dst = oracle.HostTensor(C.TYPE_F16, (D, M, Nkv, B), (2, 2 * D, 2 * D * M, 2 * D * M * Nkv), cache)
    got, ref, skipped = _run_both(mx, C.SetRowsCase("t", dst, src, rows), "broadcast R2")
    assert skipped == 0
    np.testing.assert_array_equal(got, ref)


def test_empty_source_is_a_noop(mx):
    import torch

    buf = torch.zeros(D * 8, dtype=torch.float16, device="cuda")
    dst = mx.DeviceView(1, (D, 8, 1, 1), (2, 2 * D, 16 * D, 16 * D), buf.data_ptr(), buf)
    src = mx.DeviceView(0, (D, 0, 1, 1), (4, 4 * D, 0, 0), 0)
    rows = mx.DeviceView(27, (0, 1, 1, 1), (8, 0, 0, 0), 0)
    mx.set_rows(dst, src, rows)
    torch.cuda.synchronize()
    assert (buf == 0).all()


def test_full_size_prefill_write_property(mx):
    """kw2 at full size (2048 tokens x 8 heads into a 2048-row cache, then the
    same rows into a larger cache at an offset): gathered rows == torch's
    RNE cast of the source, other rows unchanged."""
    import torch
    from mxfa import cases as C

    for kv_pos, max_seq in ((0, 2048), (3000, 8192)):
        c = C.kv_write_single("kw2", n_tokens=2048, kv_pos=kv_pos, Nkv=8, max_seq=max_seq)
        print(f"[set_rows] full-size kw2 at {kv_pos} of {max_seq}", flush=True)
        dd, ds, dr = mx.upload(c.dst), mx.upload(c.src), mx.upload(c.rows)
        before = dd.owner.clone()
        mx.set_rows(dd, ds, dr)
        torch.cuda.synchronize()
        cache = dd.owner.view(torch.int16).view(8, max_seq, D)
        src = ds.owner.view(torch.float32).view(8, 2048, D)
        exp = src.to(torch.float16).view(torch.int16)
        assert torch.equal(cache[:, kv_pos:kv_pos + 2048], exp)
        old = before.view(torch.int16).view(8, max_seq, D)
        assert torch.equal(cache[:, :kv_pos], old[:, :kv_pos])
        assert torch.equal(cache[:, kv_pos + 2048:], old[:, kv_pos + 2048:])


def test_rejected_node_launches_nothing(mx):
    """A malformed node raises MxfaError and leaves the cache untouched."""
    import torch

    buf = torch.zeros(D * 8, dtype=torch.float16, device="cuda")
    src_t = torch.ones(D * 4, dtype=torch.float32, device="cuda")
    ids = torch.arange(3, dtype=torch.int64, device="cuda")
    dst = mx.DeviceView(1, (D, 8, 1, 1), (2, 2 * D, 16 * D, 16 * D), buf.data_ptr(), buf)
    src = mx.DeviceView(0, (D, 4, 1, 1), (4, 4 * D, 16 * D, 16 * D), src_t.data_ptr(), src_t)
    rows = mx.DeviceView(27, (3, 1, 1, 1), (8, 24, 24, 24), ids.data_ptr(), ids)
    with pytest.raises(mx.MxfaError):
        mx.set_rows(dst, src, rows)
    torch.cuda.synchronize()
    assert (buf == 0).all()
