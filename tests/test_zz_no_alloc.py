"""GPU: the allocation-free entry point (mxfa_flash_attn_ext_noalloc) against
mxfa_flash_attn_ext through the C ABI.

The two run the same kernels; the allocation-free one keeps the split-KV
partials, split tickets and mask tile classes in the library's fixed
per-GPU scratch array instead of the stream's grow-only workspace.  Each
case makes two calls in a row, the second smaller than the first (the
scratch keeps the first call's contents), and every output must equal the
workspace entry point's bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mx():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import mxfa

    return mxfa


def _both(mx, case):
    import torch

    dq, dk, dv = mx.upload(case.q), mx.upload(case.k), mx.upload(case.v)
    dm = mx.upload(case.mask) if case.mask is not None else None
    ref = mx.flash_attn_ext(dq, dk, dv, dm, case.scale, case.max_bias, case.softcap)
    torch.cuda.synchronize()
    got = mx.flash_attn_ext_noalloc(dq, dk, dv, dm, case.scale, case.max_bias, case.softcap)
    torch.cuda.synchronize()
    return mx.output_tensor(got).cpu().numpy(), mx.output_tensor(ref).cpu().numpy()


def test_noalloc_decode_matches_workspace_entry(mx):
    """Split-KV decode (partials and tickets in the scratch): C3's batched
    CFG decode, then a smaller batch with shorter sequences."""
    from mxfa import cases as C

    for label, case in (("C3", C.c3()),
                        ("small", C.lm_batch("na", N=2, Nh=16, Nkv=8, max_seq=2048, lengths=[700, 1900]))):
        print(f"[noalloc] decode {label}: q{tuple(case.q.ne)} k{tuple(case.k.ne)}", flush=True)
        got, ref = _both(mx, case)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (label, float(np.abs(got - ref).max()))


def test_noalloc_prefill_matches_workspace_entry(mx):
    """Prefill with a dense mask (tile classes in the scratch): a causal
    prompt of 1000 tokens, then a smaller one of 300 at an offset."""
    from mxfa import cases as C

    for label, case in (("c2-1000", C.c2(n_tokens=1000)),
                        ("c1-300", C.lm_single("np", n_tokens=300, kv_pos=211, Nh=16, Nkv=8, max_seq=1024))):
        print(f"[noalloc] prefill {label}: q{tuple(case.q.ne)} k{tuple(case.k.ne)}", flush=True)
        got, ref = _both(mx, case)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (label, float(np.abs(got - ref).max()))


def test_noalloc_wide_prefill_matches_workspace_entry(mx):
    """The kernel with 48 queries per wave under a dense mask (its tile
    classes in the scratch): C4 cross at full size, then a smaller random
    mask over 4 key tiles."""
    from mxfa import cases as C
    from test_gpu_parity import _rand_case

    for label, case in (("c4x", C.c4_cross()),
                        ("wide-300", _rand_case(814, B=1, Sq=300, Nh=8, Nkv=2, Skv=200, mask="random"))):
        print(f"[noalloc] wide prefill {label}: q{tuple(case.q.ne)} k{tuple(case.k.ne)}", flush=True)
        got, ref = _both(mx, case)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (label, float(np.abs(got - ref).max()))


def test_noalloc_q8_0_prefill_matches_workspace_entry(mx):
    """Prefill over a Q8_0 cache (tile classes and the F16 staging of K and
    V in the scratch; Q is quantised to Q8_0 on load): two calls, the second
    smaller."""
    from test_gpu_parity import _rand_case

    for label, case in (("q8-300", _rand_case(811, B=2, Sq=300, Nh=8, Nkv=2, Skv=516, kv_type=8, mask="causal")),
                        ("q8-96", _rand_case(812, B=1, Sq=96, Nh=8, Nkv=2, Skv=188, kv_type=8))):
        print(f"[noalloc] q8_0 prefill {label}: q{tuple(case.q.ne)} k{tuple(case.k.ne)}", flush=True)
        got, ref = _both(mx, case)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (label, float(np.abs(got - ref).max()))


def test_noalloc_q8_0_prompt_larger_than_the_staging(mx):
    """C2's prompt over a Q8_0 cache (16384 K/V rows: 8 MiB of F16 staging,
    more than the scratch holds) runs through the decode kernel, which
    stages nothing, at the parity bar against the oracle; then a small
    Q8_0 prompt, whose staging fits, takes the prefill kernel again and
    equals the workspace entry point bit for bit."""
    import oracle
    import torch

    from conftest import MAX_ABS_TOL, ROW_COS_TOL, row_metrics
    from mxfa import cases as C
    from test_gpu_parity import _rand_case

    case = C.c2_q8()
    print(f"[noalloc] c2q8: q{tuple(case.q.ne)} k{tuple(case.k.ne)}", flush=True)
    dq, dk, dv, dm = mx.upload(case.q), mx.upload(case.k), mx.upload(case.v), mx.upload(case.mask)
    out = mx.flash_attn_ext_noalloc(dq, dk, dv, dm, case.scale)
    torch.cuda.synchronize()
    got = mx.output_tensor(out).cpu().numpy()
    gate = oracle.fa_ggml(case.q, case.k, case.v, case.mask, case.scale, acc_f32=True)
    m = row_metrics(got, gate)
    print(f"[noalloc] c2q8 vs gate: max_abs={m['max_abs']:.3e} min_cos={m['min_cos']:.7f}", flush=True)
    assert m["max_abs"] <= MAX_ABS_TOL and m["min_cos"] >= ROW_COS_TOL, m
    small = _rand_case(813, B=1, Sq=128, Nh=8, Nkv=2, Skv=300, kv_type=8, mask="causal")
    got, ref = _both(mx, small)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), float(np.abs(got - ref).max())


def test_noalloc_allocates_nothing_in_the_engine(mx):
    """The engine's own workspaces do not grow for allocation-free calls."""
    import torch

    from mxfa import cases as C

    case = C.lm_batch("nz", N=4, Nh=32, Nkv=8, max_seq=4096, lmin=3000, lmax=4096)
    dq, dk, dv, dm = mx.upload(case.q), mx.upload(case.k), mx.upload(case.v), mx.upload(case.mask)
    out = mx.flash_attn_ext_noalloc(dq, dk, dv, dm, case.scale)
    torch.cuda.synchronize()
    live0, ret0 = mx.workspace_info()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        mx.flash_attn_ext_noalloc(dq, dk, dv, dm, case.scale, dst=out, stream=s.cuda_stream)
    torch.cuda.synchronize()
    assert mx.workspace_info() == (live0, ret0)
