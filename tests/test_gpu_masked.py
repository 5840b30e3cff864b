"""GPU parity of structured masks (mxfa_flash_attn_ext_masked).

Each case runs the structured call through the C ABI and compares it with:
  * the dense call (mxfa_flash_attn_ext with the equivalent F16 mask): on
    the prefill kernel the two take the same tile classes and the same
    arithmetic, so the outputs must be bit-identical; on the decode kernel
    the structured call cuts its splits from the live lengths, so the split
    merge adds in another order and the bar is the parity bar;
  * the CPU oracle on the dense form (fa_ggml with an fp32 accumulator):
    max-abs <= 2e-3 and per-row cosine >= 0.9999 (every K/V type, bf16 included).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import MAX_ABS_TOL, ROW_COS_TOL, row_metrics
from test_gpu_parity import _rand_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mx():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mxfa

    return mxfa


def _run(mx, case, spec=None):
    """Structured call when `spec` (mask_spec kwargs) is given, else dense."""
    import torch

    dq, dk, dv = mx.upload(case.q), mx.upload(case.k), mx.upload(case.v)
    if spec is None:
        dm = mx.upload(case.mask) if case.mask is not None else None
        out = mx.flash_attn_ext(dq, dk, dv, dm, case.scale, case.max_bias, case.softcap)
    else:
        out = mx.flash_attn_ext_masked(dq, dk, dv, mx.mask_spec(**spec), case.scale, case.max_bias, case.softcap)
    torch.cuda.synchronize()
    return mx.output_tensor(out).cpu().numpy()


def check(mx, case, spec, label, bitwise):
    import oracle
    from mxfa import cases as C

    dense = C.with_dense_mask(case, spec)
    print(f"[masked] {label}: q{tuple(case.q.ne)} k{tuple(case.k.ne)} t{case.k.type} spec={spec if len(str(spec)) < 80 else '...'}",
          flush=True)
    got = _run(mx, case, spec)
    assert not np.isnan(got).any()
    ref = _run(mx, dense)
    if bitwise:
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (label, np.abs(got - ref).max())
    gate = oracle.fa_ggml(dense.q, dense.k, dense.v, dense.mask, dense.scale, dense.max_bias, dense.softcap,
                          acc_f32=True)
    m = row_metrics(got, gate)
    md = row_metrics(got, ref)
    print(f"[masked] {label}: vs oracle max_abs={m['max_abs']:.3e} min_cos={m['min_cos']:.7f} | "
          f"vs dense max_abs={md['max_abs']:.3e}", flush=True)
    tol = MAX_ABS_TOL
    assert m["max_abs"] <= tol and m["min_cos"] >= ROW_COS_TOL, (label, m)
    return got


# ---------------------------------------------------------------------------
# the reference's masks in structured form
# ---------------------------------------------------------------------------

def test_c2_causal_prefill(mx):
    from mxfa import cases as C

    c = C.c2()
    check(mx, c, C.structured_spec(c), "C2 causal 2048", bitwise=True)


def test_causal_continuation_prefill(mx):
    """A prompt continued at kv_pos > 0 (the causal diagonal shifted)."""
    from mxfa import cases as C

    c = C.lm_single("t", n_tokens=300, kv_pos=700, Nh=16, Nkv=8, max_seq=2048)
    check(mx, c, C.structured_spec(c), "causal at kv_pos 700", bitwise=True)


def test_dit_sliding_window_prefill(mx):
    from mxfa import cases as C

    c = C.dit_self("t", S=1024, window=128)
    check(mx, c, C.structured_spec(c), "DiT window 128", bitwise=True)


def test_dit_cross_padding_prefill(mx):
    from mxfa import cases as C

    c = C.c4_cross()
    check(mx, c, C.structured_spec(c), "C4 cross padding", bitwise=True)


def test_c1_causal_decode(mx):
    from mxfa import cases as C

    c = C.c1()
    check(mx, c, C.structured_spec(c), "C1 decode", bitwise=False)


def test_c3_lengths_decode(mx):
    """Per-sequence lengths: the host cuts the splits from the live lengths."""
    from mxfa import cases as C

    c = C.c3()
    print("[masked] C3 lengths", c.meta["lengths"], flush=True)
    check(mx, c, C.structured_spec(c), "C3 lengths", bitwise=False)


def test_q8_0_lengths_decode(mx):
    from mxfa import cases as C

    c = C.lm_batch_q8("t", N=4, L=2048)
    spec = dict(lengths=[2048, 100, 1, 1500])
    check(mx, c, spec, "Q8_0 lengths", bitwise=False)


# ---------------------------------------------------------------------------
# combinations and edges, random data
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("Sq", [1, 5, 64, 200])
def test_combined_flags(mx, Sq):
    """causal + window + lengths together, per-batch lengths, GQA; Sq < 64
    runs the decode kernel, Sq >= 64 the prefill kernel."""
    c = _rand_case(400 + Sq, B=3, Sq=Sq, Nh=8, Nkv=2, Skv=640, mask=None)
    spec = dict(causal=True, pos0=640 - Sq, window=300, lengths=[640, 500, 37])
    check(mx, c, spec, f"combined Sq={Sq}", bitwise=Sq >= 64)


@pytest.mark.parametrize("kv_type", [30, 8])
def test_other_kv_types(mx, kv_type):
    c = _rand_case(500 + kv_type, B=2, Sq=3, Nh=8, Nkv=4, Skv=400, kv_type=kv_type, mask=None)
    check(mx, c, dict(causal=True, pos0=397, lengths=[400, 250]), f"kv type {kv_type}", bitwise=False)


def test_bf16_prefill_window(mx):
    c = _rand_case(510, B=1, Sq=300, Nh=4, Nkv=2, Skv=300, kv_type=30, mask=None)
    check(mx, c, dict(window=50), "bf16 window prefill", bitwise=True)


def test_empty_rows_and_long_lengths(mx):
    """A batch with length 0 (every row fully masked -> 0), lengths past Skv
    (clamped), window 0 (each query sees its own position only)."""
    for Sq in (2, 130):
        c = _rand_case(520 + Sq, B=3, Sq=Sq, Nh=4, Nkv=4, Skv=256, mask=None)
        got = check(mx, c, dict(lengths=[0, 10_000, 256]), f"lengths 0 / large Sq={Sq}", bitwise=Sq >= 64)
        assert np.all(got[0] == 0.0)
        c = _rand_case(530 + Sq, B=1, Sq=Sq, Nh=4, Nkv=4, Skv=256, mask=None)
        check(mx, c, dict(window=0, pos0=7), f"window 0 Sq={Sq}", bitwise=Sq >= 64)


def test_softcap_alibi(mx):
    c = _rand_case(540, B=1, Sq=130, Nh=8, Nkv=2, Skv=300, mask=None, softcap=30.0, max_bias=8.0)
    check(mx, c, dict(causal=True, pos0=170), "softcap + alibi prefill", bitwise=True)
    c = _rand_case(541, B=1, Sq=4, Nh=8, Nkv=2, Skv=300, mask=None, softcap=30.0, max_bias=8.0)
    check(mx, c, dict(causal=True, pos0=296), "softcap + alibi decode", bitwise=False)


@pytest.mark.parametrize("B,Sq", [(3, 20), (22, 12)])
def test_decode_split_grids(mx, B, Sq):
    """Decode with host lengths, several row tiles per (batch, kv head):
    3 batches x 5 row tiles use the grid that lists the live splits
    ((batch, row tile, split) major, kv head minor); 22 batches x 3 row
    tiles (66 streams, more than the list takes) use the dense grid whose
    workgroups past their stream's last split return at once."""
    rng = np.random.default_rng(600 + B)
    c = _rand_case(600 + B + Sq, B=B, Sq=Sq, Nh=8, Nkv=2, Skv=900, mask=None)
    lengths = [int(x) for x in rng.integers(0, 901, size=B)]
    lengths[0] = 900
    spec = dict(causal=True, pos0=900 - Sq, lengths=lengths)
    check(mx, c, spec, f"decode grids B={B} Sq={Sq}", bitwise=False)


@pytest.mark.parametrize("i,spec", list(enumerate([
    dict(causal=True),
    dict(window=40, pos0=60),
    dict(causal=True, window=70, pos0=20, lengths=[200, 150, 37]),
])))
def test_short_kv_wide_structured(mx, i, spec):
    """Calls of at most 4 key tiles run the kernel with 48 queries per wave
    in both forms (dense and structured), whose tile ranges and classes are
    taken over the same 128-query class tiles: 300 queries (a partial second
    192-query tile) over 200 keys, GQA 4:1, rows masked out entirely."""
    c = _rand_case(550 + i, B=3, Sq=300, Nh=8, Nkv=2, Skv=200, mask=None)
    check(mx, c, spec, f"short K/V wide {spec}", bitwise=True)
