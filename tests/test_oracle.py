"""Pins the CPU oracle (oracle/fa_oracle.c) before it is trusted.

The reference has no flash_attn_ext golden vectors (every committed log ran
with FA disabled, reference tests/debug-dit-cossim.py:147) and ggml itself is
absent (empty submodule), so the oracle is pinned by:
  * library routines: numpy float16 (IEEE RNE) for the fp16 codec, torch
    bfloat16 for the bf16 codec (the RNG's published Philox KAT vectors are
    checked in tests/test_synth.py);
  * an independent numpy fp64 implementation in matrix form (the reference's
    own non-FA statement of the op: qwen3-enc.h:101-112 / dit-graph.h:123-134
    and the PyTorch restatement tests/debug-lm-logits.py:100-115) that reads
    the ggml views through numpy strides instead of the oracle's pointer
    arithmetic;
  * closed forms that a plausible mistake breaks: Skv = 1, one unmasked key,
    uniform V, key permutation, scale 0, fully masked rows, zero mask vs NULL
    mask, GQA head map, batch broadcast, ALiBi slopes of power-of-2 heads;
  * the oracle's scalar and AVX2 forms agreeing bit for bit.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import row_metrics

F32, F16, Q8_0, BF16 = 0, 1, 8, 30


# ---------------------------------------------------------------------------
# independent numpy reference
# ---------------------------------------------------------------------------

def view_to_array(t) -> np.ndarray:
    """float64 array indexed [i3, i2, i1, i0] from a ggml view over host bytes."""
    raw = np.ascontiguousarray(t.buf).view(np.uint8).reshape(-1)
    ne0, ne1, ne2, ne3 = (int(x) for x in t.ne)
    nb0, nb1, nb2, nb3 = (int(x) for x in t.nb)
    if t.type == Q8_0:
        rowb = ne0 // 32 * 34
    else:
        rowb = ne0 * {F32: 4, F16: 2, BF16: 2}[t.type]
    rows = np.lib.stride_tricks.as_strided(raw[t.offset:], shape=(ne3, ne2, ne1, rowb),
                                           strides=(nb3, nb2, nb1, 1))
    rows = np.ascontiguousarray(rows)
    if t.type == F32:
        return rows.view(np.float32).astype(np.float64)
    if t.type == F16:
        return rows.view(np.float16).astype(np.float64)
    if t.type == BF16:
        return (rows.view(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    blk = rows.reshape(ne3, ne2, ne1, ne0 // 32, 34)
    d = np.ascontiguousarray(blk[..., :2]).view(np.float16).astype(np.float64)
    qv = np.ascontiguousarray(blk[..., 2:]).view(np.int8).astype(np.float64)
    return (qv * d).reshape(ne3, ne2, ne1, ne0)


def numpy_fa(case_q, case_k, case_v, mask, scale, max_bias=0.0, softcap=0.0, q_round=None):
    """Matrix-form fp64 attention with ggml semantics; returns [B, Sq, Nh, DV]."""
    Q = view_to_array(case_q)          # [B, Nh, Sq, D]
    K = view_to_array(case_k)          # [Bk, Nkv, Skv, D]
    V = view_to_array(case_v)
    if q_round == "f16":
        Q = Q.astype(np.float16).astype(np.float64)
    B, Nh, Sq, _ = Q.shape
    Bk, Nkv, Skv, _ = K.shape
    G, rk3 = Nh // Nkv, B // Bk
    if mask is not None:
        Mv = view_to_array(mask)[:, :, :Sq, :Skv]   # [Bm, Hm, Sq, Skv]
    n_head_log2 = 2 ** int(math.floor(math.log2(Nh)))
    m0 = 2.0 ** (-max_bias / n_head_log2)
    m1 = 2.0 ** (-(max_bias / 2.0) / n_head_log2)
    out = np.zeros((B, Sq, Nh, V.shape[-1]))
    for b in range(B):
        for h in range(Nh):
            slope = 1.0
            if max_bias > 0:
                slope = m0 ** (h + 1) if h < n_head_log2 else m1 ** (2 * (h - n_head_log2) + 1)
            kk = K[b // rk3, h // G]
            vv = V[b // rk3, h // G]
            s = Q[b, h] @ kk.T * scale
            if softcap:
                s = softcap * np.tanh(s / softcap)
            if mask is not None:
                mv = Mv[b % Mv.shape[0], h % Mv.shape[1]] * slope
                s = np.where(np.isneginf(mv), -np.inf, s + np.where(np.isneginf(mv), 0.0, mv))
            mx = np.max(s, axis=1, keepdims=True)
            ok = np.isfinite(mx)
            p = np.where(ok, np.exp(s - np.where(ok, mx, 0.0)), 0.0)
            den = p.sum(axis=1, keepdims=True)
            o = np.where(den > 0, (p @ vv) / np.where(den > 0, den, 1.0), 0.0)
            out[b, :, h, :] = o
    return out


def make_view(type_, arr4, layout="contig"):
    """Host view of logical array [ne3, ne2, ne1, ne0] (float values),
    optionally stored with dims 1/2 swapped in memory ("perm")."""
    from mxfa.cases import HostView, to_f16_bits, to_bf16_bits, quantize_q8_0

    arr4 = np.asarray(arr4, dtype=np.float32)
    ne3, ne2, ne1, ne0 = arr4.shape
    if type_ == Q8_0:
        buf = quantize_q8_0(arr4.reshape(-1))
        rowb = ne0 // 32 * 34
        nb = (34, rowb, rowb * ne1, rowb * ne1 * ne2)
        return HostView(Q8_0, (ne0, ne1, ne2, ne3), nb, buf)
    esz = 4 if type_ == F32 else 2
    conv = {F32: lambda x: x.astype(np.float32), F16: to_f16_bits, BF16: to_bf16_bits}[type_]
    if layout == "perm":
        mem = np.ascontiguousarray(arr4.transpose(0, 2, 1, 3))   # [ne3, ne1, ne2, ne0]
        nb = (esz, ne2 * ne0 * esz, ne0 * esz, ne0 * ne1 * ne2 * esz)
    else:
        mem = arr4
        nb = (esz, ne0 * esz, ne0 * ne1 * esz, ne0 * ne1 * ne2 * esz)
    return HostView(type_, (ne0, ne1, ne2, ne3), nb, conv(mem).reshape(-1))


def mask_view(allowed, extra=None):
    """F16 mask view from bool [Bm, Hm, Sq, Skv] (+ optional finite values)."""
    from mxfa.cases import HostView

    vals = np.where(allowed, 0.0, -np.inf).astype(np.float32)
    if extra is not None:
        vals = np.where(allowed, extra, vals).astype(np.float32)
    Bm, Hm, Sq, Skv = vals.shape
    bits = vals.astype(np.float16).view(np.uint16).reshape(-1)
    return HostView(F16, (Skv, Sq, Hm, Bm), (2, 2 * Skv, 2 * Skv * Sq, 2 * Skv * Sq * Hm), bits)


def rnd(rng, *shape):
    return rng.standard_normal(shape).astype(np.float32)


# ---------------------------------------------------------------------------
# codecs
# ---------------------------------------------------------------------------

def test_fp16_decode_exhaustive(oracle_lib):
    h = np.arange(65536, dtype=np.uint16)
    got = oracle_lib.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_fp16_encode_matches_numpy(oracle_lib):
    rng = np.random.default_rng(0)
    # every fp16 value, midpoints (ties), neighbours, random magnitudes, specials
    h = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    h = h[np.isfinite(h)]
    mids = ((h[:-1].astype(np.float64) + h[1:].astype(np.float64)) / 2).astype(np.float32)
    near = np.concatenate([np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf))])
    rand = (rng.standard_normal(200000) * np.exp2(rng.integers(-30, 20, 200000))).astype(np.float32)
    spec = np.array([0.0, -0.0, np.inf, -np.inf, 65504, 65519.99, 65520, 1e-8, 2.0 ** -25, 2.0 ** -24,
                     3 * 2.0 ** -26, 1e30, -1e30], dtype=np.float32)
    x = np.concatenate([h, mids, near, rand, spec])
    got = oracle_lib.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    nanb = oracle_lib.f32_to_f16_bits(np.array([np.nan], dtype=np.float32))
    assert np.isnan(nanb.view(np.float16)[0])


def test_bf16_codec_matches_torch(oracle_lib):
    import torch

    rng = np.random.default_rng(1)
    x = (rng.standard_normal(300000) * np.exp2(rng.integers(-60, 60, 300000))).astype(np.float32)
    u = rng.integers(0, 2 ** 32, 100000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = np.concatenate([x, u[np.isfinite(u)], np.array([0.0, -0.0, np.inf, -np.inf], np.float32)])
    got = oracle_lib.f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    back = oracle_lib.bf16_bits_to_f32(got)
    assert np.array_equal(back.view(np.uint32), got.astype(np.uint32) << 16)
    from mxfa.cases import to_bf16_bits

    assert np.array_equal(to_bf16_bits(x), ref)


def test_q8_0_quantiser_matches_package_and_closed_form(oracle_lib):
    from mxfa.cases import quantize_q8_0

    rng = np.random.default_rng(2)
    x = rnd(rng, 64 * 32) * 3
    x[:32] = 0.0                      # all-zero block
    x[32:64] = np.linspace(-1, 1, 32)  # exact ties would be measure-zero
    q_or = oracle_lib.quantize_q8_0(x)
    q_pk = quantize_q8_0(x)
    assert np.array_equal(q_or, q_pk)
    blk = q_or.reshape(-1, 34)
    d = blk[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
    qv = blk[:, 2:].view(np.int8).astype(np.float32)
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float16).astype(np.float32))
    assert np.abs(qv).max() <= 127
    deq = oracle_lib.dequantize_q8_0(q_or, x.size).reshape(-1, 32)
    assert np.array_equal(deq, qv * d[:, None])
    # reconstruction within half a step, plus 127 times the fp16 rounding
    # error of d (relative 2^-11): 0.5*d + 127*d*2^-11 < 0.57*d
    err = np.abs(deq - x.reshape(-1, 32))
    assert np.all(err <= 0.57 * amax[:, None] / 127 + 1e-7)


def test_dot_and_mad_kernels(oracle_lib):
    rng = np.random.default_rng(3)
    for n in (128, 96, 130):
        x = rnd(rng, n).astype(np.float16)
        y = rnd(rng, n).astype(np.float16)
        got = oracle_lib.lib().ora_dot_f16(n, x.ctypes.data, y.ctypes.data)
        ref = float(np.dot(x.astype(np.float64), y.astype(np.float64)))
        bound = 2 * n * 2.0 ** -24 * float(np.dot(np.abs(x.astype(np.float64)), np.abs(y.astype(np.float64))))
        assert abs(got - ref) <= bound + 1e-7
    # mad_f16: y <- fp16(fma(x, v, y)), one fp16 rounding per element
    x = rnd(rng, 128).astype(np.float16)
    y = rnd(rng, 128).astype(np.float16)
    v = np.float32(0.37)
    yy = y.copy()
    oracle_lib.lib().ora_mad_f16(128, yy.ctypes.data, x.ctypes.data, float(v))
    exact = x.astype(np.float64) * np.float64(v) + y.astype(np.float64)
    ref = exact.astype(np.float32).astype(np.float16)
    ulp = np.abs(np.spacing(ref.astype(np.float16))).astype(np.float64)
    assert np.all(np.abs(yy.astype(np.float64) - ref.astype(np.float64)) <= ulp)


# ---------------------------------------------------------------------------
# the attention oracles
# ---------------------------------------------------------------------------

def _small_case(rng, B=2, Sq=5, Nh=4, Nkv=2, Skv=37, kv_type=F16, q_layout="perm", Bk=None):
    Bk = B if Bk is None else Bk
    q = make_view(F32, rnd(rng, B, Nh, Sq, 128), q_layout)
    k = make_view(kv_type, rnd(rng, Bk, Nkv, Skv, 128))
    v = make_view(kv_type, rnd(rng, Bk, Nkv, Skv, 128))
    return q, k, v


@pytest.mark.parametrize("kv_type", [F16, BF16, Q8_0])
@pytest.mark.parametrize("with_mask", [False, True])
def test_exact_oracle_matches_numpy(oracle_lib, kv_type, with_mask):
    rng = np.random.default_rng(10 + kv_type + with_mask)
    B, Sq, Nh, Nkv, Skv = 2, 5, 4, 2, 37
    q, k, v = _small_case(rng, B, Sq, Nh, Nkv, Skv, kv_type)
    mask = None
    if with_mask:
        allowed = rng.random((B, 1, Sq, Skv)) > 0.3
        allowed[0, 0, 2, :] = False          # fully masked row
        extra = (rng.standard_normal((B, 1, Sq, Skv)) * 0.5).astype(np.float32)
        mask = mask_view(allowed, extra)
    scale = 1 / math.sqrt(128)
    got = oracle_lib.fa_exact(q, k, v, mask, scale)
    ref = numpy_fa(q, k, v, mask, scale)
    assert np.max(np.abs(got - ref)) < 1e-12
    if with_mask:
        assert np.all(got[0, 2] == 0.0)
    # ggml-semantics oracle against exact maths on the same rounded Q: an
    # fp32 accumulator (BF16/Q8_0 V) leaves only fp32 rounding; the fp16
    # running accumulator of F16 V costs up to ~1 fp16 ulp of the (unnormalised)
    # accumulator, i.e. a few 1e-3 on these short rows with |o| ~ 0.3
    gg = oracle_lib.fa_ggml(q, k, v, mask, scale)
    refq = oracle_lib.fa_exact(q, k, v, mask, scale, q_round=True)
    m = row_metrics(gg, refq)
    if kv_type == F16:
        assert m["max_abs"] < 5e-3 and m["min_cos"] > 0.9999, m
    else:
        assert m["max_abs"] < 1e-5 and m["min_cos"] > 0.9999999, m


def test_head_map_output_layout_and_broadcast(oracle_lib):
    """Skv = 1 => O = V0 of the mapped KV head / batch.  Distinct V per
    (kv batch, kv head) pins the GQA map (kv = h // (Nh/Nkv)), the KV batch
    broadcast (kb = b // (B/Bk)) and the permuted output [DV, Nh, Sq, B]."""
    B, Bk, Nh, Nkv, Sq = 4, 2, 6, 3, 3
    rng = np.random.default_rng(20)
    q = make_view(F32, rnd(rng, B, Nh, Sq, 128), "perm")
    kv = np.zeros((Bk, Nkv, 1, 128), np.float32)
    for bk in range(Bk):
        for g in range(Nkv):
            kv[bk, g, 0, :] = (bk * 10 + g + 1) + np.arange(128) / 256.0
    k = make_view(F16, rnd(rng, Bk, Nkv, 1, 128))
    v = make_view(F16, kv)
    for fn in (oracle_lib.fa_ggml, oracle_lib.fa_exact):
        out = fn(q, k, v, None, 0.1)
        for b in range(B):
            for i in range(Sq):
                for h in range(Nh):
                    exp = kv[b // (B // Bk), h // (Nh // Nkv), 0].astype(np.float16).astype(np.float64)
                    assert np.array_equal(out[b, i, h].astype(np.float64), exp), (fn, b, i, h)


def test_special_cases(oracle_lib):
    rng = np.random.default_rng(21)
    B, Sq, Nh, Nkv, Skv = 1, 4, 2, 2, 50
    q, k, _ = _small_case(rng, B, Sq, Nh, Nkv, Skv)
    scale = 1 / math.sqrt(128)
    # uniform V => O = V row
    row = rnd(rng, 128)
    vu = make_view(F16, np.broadcast_to(row, (B, Nkv, Skv, 128)).copy())
    rowh = row.astype(np.float16).astype(np.float64)
    ex = oracle_lib.fa_exact(q, k, vu, None, scale)
    assert np.max(np.abs(ex - rowh)) < 1e-12
    gg = oracle_lib.fa_ggml(q, k, vu, None, scale)
    # fp16 running accumulator: relative drift of a few 1e-3 over 50 keys
    assert np.max(np.abs(gg - rowh)) < 5e-3 * np.max(np.abs(rowh))
    # one unmasked key => O = that V row (both oracles, exactly)
    vv = rnd(rng, B, Nkv, Skv, 128)
    v = make_view(F16, vv)
    allowed = np.zeros((B, 1, Sq, Skv), bool)
    for i in range(Sq):
        allowed[0, 0, i, 7 * i + 3] = True
    m = mask_view(allowed)
    for fn in (oracle_lib.fa_ggml, oracle_lib.fa_exact):
        out = fn(q, k, v, m, scale)
        for i in range(Sq):
            for h in range(Nh):
                exp = vv[0, h, 7 * i + 3].astype(np.float16).astype(np.float64)
                assert np.array_equal(out[0, i, h].astype(np.float64), exp)
    # scale 0 => mean of the unmasked V rows
    allowed = rng.random((B, 1, Sq, Skv)) > 0.5
    m = mask_view(allowed)
    ex = oracle_lib.fa_exact(q, k, v, m, 0.0)
    vh = vv.astype(np.float16).astype(np.float64)
    for i in range(Sq):
        for h in range(Nh):
            exp = vh[0, h, allowed[0, 0, i]].mean(axis=0)
            assert np.max(np.abs(ex[0, i, h] - exp)) < 1e-12
    # all-zero mask == NULL mask, bit for bit (both oracles)
    zero = mask_view(np.ones((B, 1, Sq, Skv), bool))
    for fn in (oracle_lib.fa_ggml, oracle_lib.fa_exact):
        assert np.array_equal(fn(q, k, v, zero, scale), fn(q, k, v, None, scale))
    # fully masked rows => 0
    none = mask_view(np.zeros((B, 1, Sq, Skv), bool))
    for fn in (oracle_lib.fa_ggml, oracle_lib.fa_exact):
        assert np.all(fn(q, k, v, none, scale) == 0.0)


def test_key_permutation_invariance(oracle_lib):
    rng = np.random.default_rng(22)
    B, Sq, Nh, Nkv, Skv = 1, 3, 2, 1, 64
    qa = rnd(rng, B, Nh, Sq, 128)
    ka = rnd(rng, B, Nkv, Skv, 128)
    va = rnd(rng, B, Nkv, Skv, 128)
    perm = rng.permutation(Skv)
    q = make_view(F32, qa)
    o1 = oracle_lib.fa_exact(q, make_view(F16, ka), make_view(F16, va), None, 0.09)
    o2 = oracle_lib.fa_exact(q, make_view(F16, ka[:, :, perm]), make_view(F16, va[:, :, perm]), None, 0.09)
    assert np.max(np.abs(o1 - o2)) < 1e-12
    g1 = oracle_lib.fa_ggml(q, make_view(F16, ka), make_view(F16, va), None, 0.09)
    g2 = oracle_lib.fa_ggml(q, make_view(F16, ka[:, :, perm]), make_view(F16, va[:, :, perm]), None, 0.09)
    # the fp16 running accumulator depends on key order: close, not equal
    assert np.max(np.abs(g1 - g2)) < 5e-3 and row_metrics(g1, g2)["min_cos"] > 0.9999


def test_alibi_and_softcap(oracle_lib):
    rng = np.random.default_rng(23)
    B, Sq, Nh, Nkv, Skv = 1, 3, 16, 16, 40
    q, k, v = _small_case(rng, B, Sq, Nh, Nkv, Skv)
    # ALiBi: for 16 heads (a power of two) slope(h) = 2^(-max_bias*(h+1)/16);
    # with a mask row of -j (distance) the bias is -slope*j
    allowed = np.ones((B, 1, Sq, Skv), bool)
    dist = -np.broadcast_to(np.arange(Skv, dtype=np.float32), (B, 1, Sq, Skv)).copy()
    m = mask_view(allowed, dist)
    out = oracle_lib.fa_exact(q, k, v, m, 0.05, max_bias=8.0)
    ref = numpy_fa(q, k, v, m, 0.05, max_bias=8.0)
    assert np.max(np.abs(out - ref)) < 1e-12
    Q = view_to_array(q)
    K = view_to_array(k)
    V = view_to_array(v)
    for h in (0, 5, 15):
        slope = 2.0 ** (-8.0 * (h + 1) / 16)
        s = Q[0, h] @ K[0, h].T * 0.05 - slope * np.arange(Skv)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        exp = (p @ V[0, h]) / p.sum(axis=1, keepdims=True)
        assert np.max(np.abs(out[0, :, h] - exp)) < 1e-12
    # softcap c: s -> c * tanh(s / c) before the mask
    out = oracle_lib.fa_exact(q, k, v, None, 0.2, softcap=2.0)
    for h in (0, 7):
        s = 2.0 * np.tanh(Q[0, h] @ K[0, h].T * 0.2 / 2.0)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        exp = (p @ V[0, h]) / p.sum(axis=1, keepdims=True)
        assert np.max(np.abs(out[0, :, h] - exp)) < 1e-12
    gg = oracle_lib.fa_ggml(q, k, v, m, 0.05, max_bias=8.0)
    assert row_metrics(gg, oracle_lib.fa_exact(q, k, v, m, 0.05, max_bias=8.0, q_round=True))["min_cos"] > 0.9999


def test_simd_and_scalar_forms_agree(oracle_lib):
    L = oracle_lib.lib()
    if not L.ora_simd_available():
        pytest.skip("host has no AVX2/FMA/F16C")
    rng = np.random.default_rng(24)
    q, k, v = _small_case(rng, 2, 6, 4, 2, 300)
    allowed = rng.random((2, 1, 6, 300)) > 0.2
    m = mask_view(allowed)
    cases = [(q, k, v)]
    kb = _small_case(np.random.default_rng(26), 2, 6, 4, 2, 300, kv_type=BF16)
    cases.append(kb)
    for qq, kk, vv in cases:
        for acc in (False, True):
            a = oracle_lib.fa_ggml(qq, kk, vv, m, 0.088, acc_f32=acc)
            L.ora_set_force_scalar(1)
            try:
                b = oracle_lib.fa_ggml(qq, kk, vv, m, 0.088, acc_f32=acc)
            finally:
                L.ora_set_force_scalar(0)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (kk.type, acc)


def test_ggml_semantics_fp16_accumulation_is_visible(oracle_lib):
    """The ggml CPU kernel accumulates V in fp16 when V is F16 (what the
    reference calls audible drift, src/dit.h:260-261).  The oracle must show
    that rounding: against the exact result at 4096 keys it is measurably
    off (yet still close), whereas BF16 V (fp32 accumulator) is not."""
    rng = np.random.default_rng(25)
    q, k, v = _small_case(rng, 1, 4, 2, 1, 4096)
    scale = 1 / math.sqrt(128)
    gg = oracle_lib.fa_ggml(q, k, v, None, scale)
    ex = oracle_lib.fa_exact(q, k, v, None, scale, q_round=True)
    m = row_metrics(gg, ex)
    assert 1e-6 < m["max_abs"] < 2e-3
    assert m["min_cos"] > 0.999
