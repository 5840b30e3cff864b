"""GPU parity of the pre-attention fusion (mxfa_qk_norm_rope) and of
attention over the 16-bit Q it writes.

The reference's layer runs rms_norm, mul, rope_ext, cont, clamp, set_rows as
separate ops (src/qwen3-lm.h:418-454, src/dit-graph.h:177-225) and hands
attention an F32 Q that ggml converts to K's type.  Checked here:
  * the fused kernel against the oracle (oracle/fa_oracle.c ora_qk_norm_rope)
    cast to the 16-bit type: every value within one 16-bit ulp (plus a few
    float ulps of its rotated pair's magnitude, for cancellation), V
    bit-exact, at most 1% of Q/K values off by that ulp (device cosf/sinf and
    the summation tree of the double sum differ from the host's in the last
    float bits, which moves a value across a 16-bit rounding boundary
    rarely); cache rows not named by `rows` keep their contents and
    out-of-range ids are skipped;
  * attention with Q stored in K's 16-bit type equals attention with the F32
    Q it was rounded from, bit for bit (ggml rounds Q to K's type to the
    nearest even before the KQ product, and so does the F32 path here);
  * the whole pipeline (fused kernel, then attention on its outputs) against
    the oracle's F32 chain at the attention bar: max-abs <= 2e-3, per-row
    cosine >= 0.9999.
"""
from __future__ import annotations

import zlib

import numpy as np
import pytest

from conftest import MAX_ABS_TOL, ROW_COS_TOL, row_metrics

pytestmark = pytest.mark.gpu
D = 128
EPS = 1e-6
BASE = 1_000_000.0


@pytest.fixture(scope="module")
def mx():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mxfa

    return mxfa


def _to16(x, out_type):
    from mxfa import cases as C

    return C.to_bf16_bits(x) if out_type == C.TYPE_BF16 else C.to_f16_bits(x)


def _from16(bits, out_type):
    from mxfa import cases as C

    bits = np.asarray(bits, dtype=np.uint16)
    if out_type == C.TYPE_BF16:
        return (bits.astype(np.uint32) << 16).view(np.float32)
    return bits.view(np.float16).astype(np.float32)


def _ulp16(x, out_type):
    """One ulp of the 16-bit type at the magnitude of x (float32 array)."""
    from mxfa import cases as C

    mant, emin = (7, -126) if out_type == C.TYPE_BF16 else (10, -14)
    e = np.frexp(np.abs(x).astype(np.float64))[1] - 1
    e = np.maximum(e, emin)
    return np.ldexp(1.0, e - mant)


class Layer:
    """Device buffers of one layer's pre-attention step: a fused QKV
    projection output [B, S, Nh + 2 Nkv, 128] F32 (q, k, v are strided views
    of it, as the reference's reshapes of the projection are), Q out
    [B, S, Nh, 128], caches [B, Nkv, max_seq, 128] of the 16-bit type."""

    def __init__(self, mx, seed, B, S, Nh, Nkv, max_seq, out_type, pos, rows=None, rows_i64=True, x_scale=3.0):
        import torch

        self.mx, self.B, self.S, self.Nh, self.Nkv, self.max_seq, self.ot = mx, B, S, Nh, Nkv, max_seq, out_type
        rng = np.random.default_rng(seed)
        H = Nh + 2 * Nkv
        self.x = (rng.standard_normal((B, S, H, D)) * x_scale).astype(np.float32)
        self.qw = (1.0 + 0.3 * rng.standard_normal(D)).astype(np.float32)
        self.kw = (1.0 + 0.3 * rng.standard_normal(D)).astype(np.float32)
        self.pos = np.asarray(pos, dtype=np.int32)           # [S] or [B, S]
        self.rows = None if rows is None else np.asarray(rows, dtype=np.int64 if rows_i64 else np.int32)  # [R, S]
        # a warm cache: rows the step does not write hold earlier keys/values
        self.sentinel = _to16((rng.standard_normal((B, Nkv, max_seq, D)) * 0.5).astype(np.float32), out_type)
        dev = "cuda"
        self.dx = torch.from_numpy(self.x).to(dev)
        self.dqw, self.dkw = torch.from_numpy(self.qw).to(dev), torch.from_numpy(self.kw).to(dev)
        self.dpos = torch.from_numpy(self.pos).to(dev)
        self.drows = None if self.rows is None else torch.from_numpy(self.rows).to(dev)
        self.qo = torch.zeros((B, S, Nh, D), dtype=torch.int16, device=dev)
        self.kc = torch.from_numpy(self.sentinel.view(np.int16).copy()).to(dev)
        self.vc = torch.from_numpy(self.sentinel.view(np.int16).copy()).to(dev)

    def views(self):
        mx, B, S, Nh, Nkv, ms, ot = self.mx, self.B, self.S, self.Nh, self.Nkv, self.max_seq, self.ot
        H = Nh + 2 * Nkv
        xnb = (4, 4 * D, 4 * D * H, 4 * D * H * S)
        base = self.dx.data_ptr()
        q = mx.DeviceView(0, (D, Nh, S, B), xnb, base, self.dx)
        k = mx.DeviceView(0, (D, Nkv, S, B), xnb, base + 4 * D * Nh, self.dx)
        v = mx.DeviceView(0, (D, Nkv, S, B), xnb, base + 4 * D * (Nh + Nkv), self.dx)
        wnb = (4, 4 * D, 4 * D, 4 * D)
        qw = mx.DeviceView(0, (D, 1, 1, 1), wnb, self.dqw.data_ptr(), self.dqw)
        kw = mx.DeviceView(0, (D, 1, 1, 1), wnb, self.dkw.data_ptr(), self.dkw)
        pr = 1 if self.pos.ndim == 1 else B
        pos = mx.DeviceView(26, (S, pr, 1, 1), (4, 4 * S, 4 * S * pr, 4 * S * pr), self.dpos.data_ptr(), self.dpos)
        qo = mx.DeviceView(ot, (D, Nh, S, B), (2, 2 * D, 2 * D * Nh, 2 * D * Nh * S), self.qo.data_ptr(), self.qo)
        cnb = (2, 2 * D, 2 * D * ms, 2 * D * ms * Nkv)
        ko = mx.DeviceView(ot, (D, ms, Nkv, B), cnb, self.kc.data_ptr(), self.kc)
        vo = mx.DeviceView(ot, (D, ms, Nkv, B), cnb, self.vc.data_ptr(), self.vc)
        rows = None
        if self.rows is not None:
            R = self.rows.shape[0]
            es = self.rows.itemsize
            rows = mx.DeviceView(27 if es == 8 else 26, (S, R, 1, 1), (es, es * S, es * S * R, es * S * R),
                                 self.drows.data_ptr(), self.drows)
        return q, k, v, qw, kw, pos, qo, ko, vo, rows

    def run(self, clamp_v=False):
        q, k, v, qw, kw, pos, qo, ko, vo, rows = self.views()
        self.mx.qk_norm_rope(q, k, v, qw, kw, pos, EPS, BASE, qo, ko, vo, rows, clamp_v=clamp_v)

    def oracle(self, clamp_v=False):
        import oracle

        Nh, Nkv = self.Nh, self.Nkv
        q, k, v = self.x[:, :, :Nh], self.x[:, :, Nh:Nh + Nkv], self.x[:, :, Nh + Nkv:]
        return oracle.qk_norm_rope(q, k, v, self.qw, self.kw, self.pos, EPS, BASE, clamp_v=clamp_v)

    def expected_caches(self, ko, vo):
        """The caches as the reference's set_rows leaves them (16-bit bits)."""
        B, S, ms = self.B, self.S, self.max_seq
        ek, ev = self.sentinel.copy(), self.sentinel.copy()
        written = np.zeros((B, ms), dtype=bool)
        for b in range(B):
            for s in range(S):
                r = s if self.rows is None else int(self.rows[b % self.rows.shape[0], s])
                if not 0 <= r < ms:
                    continue
                ek[b, :, r] = _to16(ko[b, s], self.ot)
                ev[b, :, r] = _to16(vo[b, s], self.ot)
                written[b, r] = True
        return ek, ev, written


def _check_close16(got_bits, ref_f32, ot, label, max_frac=0.01):
    """Each value within one 16-bit ulp of the oracle's rounded value plus
    2^-20 of its rotated pair's magnitude m = |(y_i, y_i+64)|: the rotation
    y_i = x_i cos - x_i+64 sin can cancel, and then an ulp of cosf/sinf
    (device vs host libm) is |m| 2^-24 absolute, many ulps of a small y_i."""
    got = _from16(got_bits, ot)
    exp = _from16(_to16(ref_f32, ot), ot)
    diff = np.abs(got.astype(np.float64) - exp)
    r = np.asarray(ref_f32, dtype=np.float64)
    m = np.sqrt(r[..., :64] ** 2 + r[..., 64:] ** 2)
    slack = np.ldexp(np.concatenate([m, m], axis=-1), -20)
    ulp = np.maximum(_ulp16(got, ot), _ulp16(exp, ot)) + slack
    assert np.all(diff <= ulp), (label, float(diff.max()), np.argwhere(diff > ulp)[:4])
    frac = float(np.mean(diff > 0))
    print(f"[norm_rope] {label}: {frac * 100:.3f}% of values one ulp off", flush=True)
    assert frac <= max_frac, (label, frac)


CASES = [
    # label, B, S, Nh, Nkv, max_seq, rows-kind
    ("lm prefill 300 at 200", 1, 300, 16, 8, 1024, "contig"),
    ("lm decode batch", 4, 1, 32, 8, 4096, "per_batch"),
    ("cfg pair shared rows", 2, 7, 16, 8, 512, "shared"),
    ("dit self no rows", 2, 64, 16, 16, 64, None),
    ("wide token, two passes", 4, 3, 64, 4, 128, "shared"),   # 72 rows per token: two 48-row passes
]


@pytest.mark.parametrize("out_type", [1, 30])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_fused_vs_oracle(mx, case, out_type):
    import torch

    label, B, S, Nh, Nkv, ms, kind = case
    rng = np.random.default_rng(zlib.crc32(label.encode()))
    if kind == "contig":
        pos = np.arange(200, 200 + S)
        rows = pos[None, :].copy()
        rows[0, 5] = ms             # out of range: skipped
        rows[0, 9] = -1
    elif kind == "per_batch":
        pos = rng.integers(0, ms, size=(B, S))
        rows = pos.copy()           # [B, 1]: one row per sequence
    elif kind == "shared":
        pos = np.arange(100, 100 + S)
        rows = rng.permutation(ms)[:S][None, :]   # one row set broadcast over the batch
    else:
        pos = np.arange(S)
        rows = None
    for i64 in ((True, False) if rows is not None else (True,)):
        print(f"[norm_rope] {label} out={out_type} rows_i64={i64}", flush=True)
        L = Layer(mx, 7 + B * S, B, S, Nh, Nkv, ms, out_type, pos, rows, rows_i64=i64)
        L.run()
        torch.cuda.synchronize()
        qo, ko, vo = L.oracle()
        got_q = L.qo.cpu().numpy().view(np.uint16)
        _check_close16(got_q, qo, out_type, f"{label} Q")
        ek, ev, written = L.expected_caches(ko, vo)
        gk = L.kc.cpu().numpy().view(np.uint16)
        gv = L.vc.cpu().numpy().view(np.uint16)
        # rows nobody wrote keep their contents
        keep = ~written
        assert np.array_equal(gk.transpose(0, 2, 1, 3)[keep], ek.transpose(0, 2, 1, 3)[keep]), label
        assert np.array_equal(gv.transpose(0, 2, 1, 3)[keep], ev.transpose(0, 2, 1, 3)[keep]), label
        # V is a cast: bit-exact
        assert np.array_equal(gv, ev), label
        kb = gk.transpose(0, 2, 1, 3)[written]
        kref = _from16(ek.transpose(0, 2, 1, 3)[written], out_type)
        _check_close16(kb, kref, out_type, f"{label} K")


def test_v_clamp(mx):
    import torch

    L = Layer(mx, 11, 1, 16, 4, 2, 64, 1, np.arange(16), None, x_scale=1e5)
    L.run(clamp_v=True)
    torch.cuda.synchronize()
    _, _, vo = L.oracle(clamp_v=True)
    ek, ev, _ = L.expected_caches(vo, vo)
    gv = L.vc.cpu().numpy().view(np.uint16)
    assert np.array_equal(gv, ev)
    assert np.isfinite(_from16(gv, 1)).all()


# ---------------------------------------------------------------------------
# attention on a 16-bit Q
# ---------------------------------------------------------------------------

def _q16_view(mx, case, dq):
    """The F16/BF16 twin of an F32 Q view: same element layout, rounded to
    nearest even, strides halved."""
    import torch

    from mxfa import cases as C

    q32 = np.ascontiguousarray(case.q.buf).view(np.float32)
    bits = _to16(q32, case.k.type)
    t = torch.from_numpy(bits.view(np.int16)).to("cuda")
    nb = tuple(int(x) // 2 for x in case.q.nb)
    assert case.q.offset % 4 == 0
    return mx.DeviceView(case.k.type, tuple(case.q.ne), nb, t.data_ptr() + case.q.offset // 2, t)


def _fa(mx, dq, dk, dv, dm, case, spec=None):
    import torch

    if spec is None:
        out = mx.flash_attn_ext(dq, dk, dv, dm, case.scale, case.max_bias, case.softcap)
    else:
        out = mx.flash_attn_ext_masked(dq, dk, dv, mx.mask_spec(**spec), case.scale, case.max_bias, case.softcap)
    torch.cuda.synchronize()
    return mx.output_tensor(out).cpu().numpy()


def _q16_cases():
    from mxfa import cases as C
    from test_gpu_parity import _rand_case

    return [
        ("C2 prefill", C.c2(), None),
        ("C2 structured", C.c2(), "spec"),
        ("C1 decode", C.c1(), None),
        ("C3 batch decode", C.c3(), None),
        ("bf16 prefill", _rand_case(610, B=2, Sq=200, Nh=8, Nkv=2, Skv=336, kv_type=30), None),
        ("bf16 decode", _rand_case(611, B=3, Sq=2, Nh=8, Nkv=4, Skv=700, kv_type=30), None),
        ("softcap alibi", _rand_case(612, B=1, Sq=130, Nh=8, Nkv=2, Skv=300, softcap=30.0, max_bias=8.0), None),
        # the kernel with 48 queries per wave (no mask; masks over <= 4 key tiles)
        ("C4 self (wide)", C.c4_self(), None),
        ("C4 cross (wide)", C.c4_cross(), None),
        ("C4 cross structured (wide)", C.c4_cross(), "spec"),
        ("no mask odd shape (wide)", _rand_case(613, B=2, Bk=1, Sq=385, Nh=8, Nkv=2, Skv=333, mask=None), None),
    ]


def test_fa_16bit_q_equals_f32_q(mx):
    from mxfa import cases as C

    for label, case, spec in _q16_cases():
        print(f"[q16] {label}: q{tuple(case.q.ne)} k{tuple(case.k.ne)} t{case.k.type}", flush=True)
        dq, dk, dv = mx.upload(case.q), mx.upload(case.k), mx.upload(case.v)
        dm = mx.upload(case.mask) if case.mask is not None else None
        sp = C.structured_spec(case) if spec else None
        ref = _fa(mx, dq, dk, dv, dm, case, sp)
        got = _fa(mx, _q16_view(mx, case, dq), dk, dv, dm, case, sp)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (label, np.abs(got - ref).max())


def test_q16_type_rules(mx):
    """Q must be F32 or K's own 16-bit type; a Q8_0 cache takes F32 Q only."""
    from mxfa import cases as C
    from test_gpu_parity import _rand_case

    c = _rand_case(620, B=1, Sq=4, Nh=4, Nkv=4, Skv=256, kv_type=30)
    dq, dk, dv = mx.upload(c.q), mx.upload(c.k), mx.upload(c.v)
    q16 = _q16_view(mx, c, dq)
    wrong = mx.DeviceView(C.TYPE_F16, q16.ne, q16.nb, q16.ptr, q16.owner)   # F16 Q, BF16 K
    with pytest.raises(mx.MxfaError) as e:
        mx.flash_attn_ext(wrong, dk, dv, None, c.scale)
    assert e.value.status == mx.ERR_UNSUPPORTED
    c8 = C.lm_batch_q8("t", N=1, L=256)
    dq8, dk8, dv8 = mx.upload(c8.q), mx.upload(c8.k), mx.upload(c8.v)
    f16q = mx.DeviceView(C.TYPE_F16, dq8.ne, tuple(x // 2 for x in dq8.nb), dq8.ptr, dq8.owner)
    with pytest.raises(mx.MxfaError) as e:
        mx.flash_attn_ext(f16q, dk8, dv8, None, c8.scale)
    assert e.value.status == mx.ERR_UNSUPPORTED


# ---------------------------------------------------------------------------
# the pipeline: fused pre-attention step, then attention on its outputs
# ---------------------------------------------------------------------------

def _pipeline(mx, L, n_kv_pad, spec, label):
    """Attention over the caches the fused kernel wrote, Q from q_out viewed
    [D, S, Nh, B] (the reference's permute), against the oracle's F32 chain:
    ora_qk_norm_rope, the caches' 16-bit rows, fa_ggml on the F32 Q with the
    dense form of the mask."""
    import torch

    import oracle
    from mxfa import cases as C

    B, S, Nh, Nkv, ms, ot = L.B, L.S, L.Nh, L.Nkv, L.max_seq, L.ot
    L.run()
    _, _, _, _, _, _, qo, ko, vo, _ = L.views()
    q16 = mx.DeviceView(ot, (D, S, Nh, B), (2, 2 * D * Nh, 2 * D, 2 * D * Nh * S), qo.ptr, qo.owner)
    kwin = mx.DeviceView(ot, (D, n_kv_pad, Nkv, B), ko.nb, ko.ptr, ko.owner)
    vwin = mx.DeviceView(ot, (D, n_kv_pad, Nkv, B), vo.nb, vo.ptr, vo.owner)
    out = mx.flash_attn_ext_masked(q16, kwin, vwin, mx.mask_spec(**spec), 1.0 / D ** 0.5)
    torch.cuda.synchronize()
    got = mx.output_tensor(out).cpu().numpy()

    qr, kr, vr = L.oracle()
    ek, ev, _ = L.expected_caches(kr, vr)           # 16-bit caches from the oracle's rows
    qbuf = np.ascontiguousarray(qr)                 # [B, S, Nh, D]
    qv = C.HostView(C.TYPE_F32, (D, S, Nh, B), (4, 4 * D * Nh, 4 * D, 4 * D * Nh * S), qbuf)
    cnb = (2, 2 * D, 2 * D * ms, 2 * D * ms * Nkv)
    kv = C.HostView(ot, (D, n_kv_pad, Nkv, B), cnb, ek.reshape(-1))
    vv = C.HostView(ot, (D, n_kv_pad, Nkv, B), cnb, ev.reshape(-1))
    case = C.with_dense_mask(C.FaCase(label, qv, kv, vv, None, 1.0 / D ** 0.5), spec)
    ref = oracle.fa_ggml(case.q, case.k, case.v, case.mask, case.scale, acc_f32=True)
    m = row_metrics(got, ref)
    print(f"[pipeline] {label}: max_abs={m['max_abs']:.3e} min_cos={m['min_cos']:.7f}", flush=True)
    tol = MAX_ABS_TOL
    assert m["max_abs"] <= tol and m["min_cos"] >= ROW_COS_TOL, (label, m)


@pytest.mark.parametrize("out_type", [1, 30])
def test_pipeline_prefill(mx, out_type):
    """A prompt of 300 tokens continued at position 200 (LM prefill with a
    warm cache): causal mask from position 200."""
    S, kv_pos, ms = 300, 200, 1024
    pos = np.arange(kv_pos, kv_pos + S)
    L = Layer(mx, 21, 1, S, 16, 8, ms, out_type, pos, pos[None, :])
    _pipeline(mx, L, 512, dict(causal=True, pos0=kv_pos), f"prefill t{out_type}")


def test_pipeline_batched_decode(mx):
    """Batched decode: one token per sequence at its own position, written
    to its own row; each sequence attends over its first pos + 1 rows."""
    B, ms = 4, 2048
    pos = np.array([[1500], [37], [0], [1023]])
    L = Layer(mx, 22, B, 1, 32, 8, ms, 1, pos, pos.reshape(B, 1))
    # rows never written hold the sentinel: the lengths mask excludes them
    _pipeline(mx, L, 1536, dict(lengths=[int(p) + 1 for p in pos[:, 0]]), "batched decode")


@pytest.mark.parametrize("out_type", [1, 30])
@pytest.mark.parametrize("S,E", [(300, 77), (64, 300)])
def test_cross_attention_chain(mx, out_type, S, E):
    """DiT cross-attention's pre-attention step (src/dit-graph.h:317-346):
    QK-norm on S queries and on enc_S = E encoder keys (fewer keys than
    queries, and more: the kernel's grid follows the larger count and
    switches off the rows of the other), no RoPE (positions = NULL), V cast;
    Q out [128, Nh, S, B], K/V [128, enc_S, Nkv, B].  The kernel's rows against the oracle's (ora_qk_norm) cast to 16
    bits, V bit-exact; then attention on its 16-bit Q with the encoder
    padding mask against the oracle's F32 chain at the attention bar."""
    import torch

    import oracle
    from mxfa import cases as C

    B, Nh, Nkv = 2, 16, 8
    rng = np.random.default_rng(4242 + out_type + S)
    xq = (rng.standard_normal((B, S, Nh, D)) * 3).astype(np.float32)      # projection [D, Nh, S, B]
    xkv = (rng.standard_normal((B, E, 2 * Nkv, D)) * 3).astype(np.float32)  # fused K|V [D, 2 Nkv, E, B]
    qw = (1.0 + 0.3 * rng.standard_normal(D)).astype(np.float32)
    kw = (1.0 + 0.3 * rng.standard_normal(D)).astype(np.float32)
    dq, dkv = torch.from_numpy(xq).cuda(), torch.from_numpy(xkv).cuda()
    dqw, dkw = torch.from_numpy(qw).cuda(), torch.from_numpy(kw).cuda()
    qo = torch.zeros((B, S, Nh, D), dtype=torch.int16, device="cuda")
    ko = torch.zeros((B, Nkv, E, D), dtype=torch.int16, device="cuda")
    vo = torch.zeros_like(ko)
    V = mx.DeviceView
    qv = V(0, (D, Nh, S, B), (4, 4 * D, 4 * D * Nh, 4 * D * Nh * S), dq.data_ptr(), dq)
    kvnb = (4, 4 * D, 4 * D * 2 * Nkv, 4 * D * 2 * Nkv * E)
    kv_ = V(0, (D, Nkv, E, B), kvnb, dkv.data_ptr(), dkv)
    vv_ = V(0, (D, Nkv, E, B), kvnb, dkv.data_ptr() + 4 * D * Nkv, dkv)
    wnb = (4, 4 * D, 4 * D, 4 * D)
    onb = (2, 2 * D, 2 * D * E, 2 * D * E * Nkv)
    print(f"[cross] pre-attention S={S} enc_S={E} type={out_type}", flush=True)
    mx.qk_norm_rope(qv, kv_, vv_, V(0, (D, 1, 1, 1), wnb, dqw.data_ptr(), dqw),
                    V(0, (D, 1, 1, 1), wnb, dkw.data_ptr(), dkw), None, EPS, BASE,
                    V(out_type, (D, Nh, S, B), (2, 2 * D, 2 * D * Nh, 2 * D * Nh * S), qo.data_ptr(), qo),
                    V(out_type, (D, E, Nkv, B), onb, ko.data_ptr(), ko),
                    V(out_type, (D, E, Nkv, B), onb, vo.data_ptr(), vo))
    torch.cuda.synchronize()
    rq = oracle.qk_norm(xq, qw, EPS)                                    # [B, S, Nh, D]
    rk = oracle.qk_norm(xkv[:, :, :Nkv], kw, EPS).transpose(0, 2, 1, 3)  # [B, Nkv, E, D]
    rv = xkv[:, :, Nkv:].transpose(0, 2, 1, 3)
    for label, got, ref in (("q", qo, rq), ("k", ko, rk), ("v", vo, rv)):
        g = got.cpu().numpy().view(np.uint16)
        r16 = _to16(np.ascontiguousarray(ref), out_type)
        if label == "v":
            assert np.array_equal(g, r16), label
            continue
        diff = np.abs(_from16(g, out_type).astype(np.float64) - _from16(r16, out_type))
        tol = _ulp16(_from16(r16, out_type), out_type)
        assert np.all(diff <= tol), (label, float(diff.max()))
        assert np.mean(g != r16) <= 0.01, (label, float(np.mean(g != r16)))

    # attention over the step's outputs: Q is the permuted view [D, S, Nh, B]
    pads = [0, 31]
    live = np.arange(E)[None, :] < (E - np.asarray(pads))[:, None]                 # [B, E]
    mbits = np.broadcast_to(np.where(live, 0, 0xFC00).astype(np.uint16)[:, None, :], (B, S, E)).copy()
    dmask = torch.from_numpy(mbits.view(np.int16)).cuda()
    q16 = V(out_type, (D, S, Nh, B), (2, 2 * D * Nh, 2 * D, 2 * D * Nh * S), qo.data_ptr(), qo)
    kvnb16 = (2, 2 * D, 2 * D * E, 2 * D * E * Nkv)
    out = mx.flash_attn_ext(q16, V(out_type, (D, E, Nkv, B), kvnb16, ko.data_ptr(), ko),
                            V(out_type, (D, E, Nkv, B), kvnb16, vo.data_ptr(), vo),
                            V(1, (E, S, 1, B), (2, 2 * E, 2 * E * S, 2 * E * S), dmask.data_ptr(), dmask),
                            1.0 / D ** 0.5)
    torch.cuda.synchronize()
    got = mx.output_tensor(out).cpu().numpy()
    qh = C.HostView(0, (D, S, Nh, B), (4, 4 * D * Nh, 4 * D, 4 * D * Nh * S), np.ascontiguousarray(rq).reshape(-1))
    kh = C.HostView(out_type, (D, E, Nkv, B), kvnb16, ko.cpu().numpy().view(np.uint16).reshape(-1))
    vh = C.HostView(out_type, (D, E, Nkv, B), kvnb16, vo.cpu().numpy().view(np.uint16).reshape(-1))
    mh = C.HostView(1, (E, S, 1, B), (2, 2 * E, 2 * E * S, 2 * E * S), mbits.reshape(-1))
    ref = oracle.fa_ggml(qh, kh, vh, mh, 1.0 / D ** 0.5, acc_f32=True)
    m = row_metrics(got, ref)
    print(f"[cross] chain type={out_type}: max_abs={m['max_abs']:.3e} min_cos={m['min_cos']:.7f}", flush=True)
    assert m["max_abs"] <= MAX_ABS_TOL and m["min_cos"] >= ROW_COS_TOL, m


def test_cross_chain_rows_more_keys_than_queries(mx):
    """The cross form with enc_S = 300 > S = 64 and explicit cache rows:
    encoder token e of batch b goes to row rows[e, b % 2] of a 400-row K/V
    view; rows no token names keep their bytes."""
    import torch

    import oracle

    B, S, E, Nh, Nkv, M = 2, 64, 300, 8, 4, 400
    rng = np.random.default_rng(977)
    xq = (rng.standard_normal((B, S, Nh, D)) * 3).astype(np.float32)
    xkv = (rng.standard_normal((B, E, 2 * Nkv, D)) * 3).astype(np.float32)
    qw = (1.0 + 0.3 * rng.standard_normal(D)).astype(np.float32)
    kw = (1.0 + 0.3 * rng.standard_normal(D)).astype(np.float32)
    rows = np.stack([rng.permutation(M)[:E] for _ in range(2)], axis=1).astype(np.int64)   # [E, 2]
    dq, dkv = torch.from_numpy(xq).cuda(), torch.from_numpy(xkv).cuda()
    dqw, dkw = torch.from_numpy(qw).cuda(), torch.from_numpy(kw).cuda()
    drows = torch.from_numpy(np.ascontiguousarray(rows.T)).cuda()   # memory [2][E]: ne = (E, 2)
    qo = torch.zeros((B, S, Nh, D), dtype=torch.int16, device="cuda")
    sentinel = 0x1234
    ko = torch.full((B, Nkv, M, D), sentinel, dtype=torch.int16, device="cuda")
    vo = torch.full_like(ko, sentinel)
    V = mx.DeviceView
    kvnb = (4, 4 * D, 4 * D * 2 * Nkv, 4 * D * 2 * Nkv * E)
    wnb = (4, 4 * D, 4 * D, 4 * D)
    onb = (2, 2 * D, 2 * D * M, 2 * D * M * Nkv)
    print(f"[cross] rows: S={S} enc_S={E} M={M}", flush=True)
    mx.qk_norm_rope(V(0, (D, Nh, S, B), (4, 4 * D, 4 * D * Nh, 4 * D * Nh * S), dq.data_ptr(), dq),
                    V(0, (D, Nkv, E, B), kvnb, dkv.data_ptr(), dkv),
                    V(0, (D, Nkv, E, B), kvnb, dkv.data_ptr() + 4 * D * Nkv, dkv),
                    V(0, (D, 1, 1, 1), wnb, dqw.data_ptr(), dqw), V(0, (D, 1, 1, 1), wnb, dkw.data_ptr(), dkw),
                    None, EPS, BASE,
                    V(1, (D, Nh, S, B), (2, 2 * D, 2 * D * Nh, 2 * D * Nh * S), qo.data_ptr(), qo),
                    V(1, (D, M, Nkv, B), onb, ko.data_ptr(), ko), V(1, (D, M, Nkv, B), onb, vo.data_ptr(), vo),
                    V(27, (E, 2, 1, 1), (8, 8 * E, 16 * E, 16 * E), drows.data_ptr(), drows))
    torch.cuda.synchronize()
    rq = oracle.qk_norm(xq, qw, EPS)
    rk = oracle.qk_norm(xkv[:, :, :Nkv], kw, EPS)      # [B, E, Nkv, D]
    rv = xkv[:, :, Nkv:]
    g = qo.cpu().numpy().view(np.uint16)
    r16 = _to16(np.ascontiguousarray(rq), 1)
    assert np.all(np.abs(_from16(g, 1).astype(np.float64) - _from16(r16, 1)) <= _ulp16(_from16(r16, 1), 1))
    kh, vh = ko.cpu().numpy().view(np.uint16), vo.cpu().numpy().view(np.uint16)
    named = np.zeros((B, M), dtype=bool)
    for b in range(B):
        for e in range(E):
            r = rows[e, b % 2]
            named[b, r] = True
            gk, rk16 = kh[b, :, r], _to16(np.ascontiguousarray(rk[b, e]), 1)
            assert np.all(np.abs(_from16(gk, 1).astype(np.float64) - _from16(rk16, 1)) <= _ulp16(_from16(rk16, 1), 1)), (b, e)
            assert np.array_equal(vh[b, :, r], _to16(np.ascontiguousarray(rv[b, e]), 1)), (b, e)
    for b in range(B):
        assert np.all(kh[b][:, ~named[b]] == sentinel) and np.all(vh[b][:, ~named[b]] == sentinel), b
