"""GPU regression: device addresses whose low 32-bit word is >= 2^31.

The kernels build buffer resources from 64-bit base addresses that are made
wave-uniform with v_readfirstlane, whose builtin returns a signed int.  Each
half must be widened as an unsigned value: a sign-extended low word >= 2^31
would overwrite the high word and point the resource at an unmapped address.
Where torch places a tensor decides whether a call sees such an address, so
this test places every operand (Q, K, V, mask, output) explicitly, once at
low words >= 2^31 and once below, inside one 4 GiB + 32 MiB device buffer,
and checks each call against the CPU oracle at the parity bar.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import MAX_ABS_TOL, ROW_COS_TOL, row_metrics
from test_gpu_parity import _rand_case

pytestmark = pytest.mark.gpu

WINDOW = 1 << 32
SLOT = 4 << 20            # one operand per 4 MiB of the window


@pytest.fixture(scope="module")
def big():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.empty(WINDOW + 8 * SLOT, dtype=torch.uint8, device="cuda")


def _offset(base, low_word):
    """Byte offset into the buffer at which the address's low word equals
    `low_word` (always < 2^32, so the operand fits in the buffer)."""
    return (low_word - (base & 0xFFFFFFFF)) % WINDOW


def _place(mx, big, view, low_word):
    import torch

    raw = np.ascontiguousarray(view.buf).view(np.uint8).reshape(-1)
    assert raw.size <= SLOT
    off = _offset(big.data_ptr(), low_word)
    big[off:off + raw.size].copy_(torch.from_numpy(raw))
    ptr = big.data_ptr() + off + int(view.offset)
    assert (ptr & 0xFFFFFFFF) == low_word + int(view.offset)
    return mx.DeviceView(view.type, tuple(view.ne), tuple(view.nb), ptr, big)


@pytest.mark.parametrize("high", [True, False], ids=["low-word-ge-2^31", "low-word-lt-2^31"])
@pytest.mark.parametrize("shape", ["prefill-mask", "prefill-causal", "decode-mask"])
def test_operands_at_high_low_words(big, high, shape):
    import mxfa as mx
    import oracle
    import torch

    if shape == "prefill-mask":       # MFMA prefill + mask tile classifier
        c = _rand_case(301, B=2, Sq=200, Nh=8, Nkv=2, Skv=320)
    elif shape == "prefill-causal":
        c = _rand_case(302, B=1, Sq=256, Nh=4, Nkv=1, Skv=256, mask="causal")
    else:                             # split-KV decode kernel
        c = _rand_case(303, B=2, Sq=5, Nh=8, Nkv=2, Skv=320)
    start = 0xC0000000 if high else 0x40000000
    print(f"[addr] {shape} low words from {start:#x}", flush=True)
    dq = _place(mx, big, c.q, start)
    dk = _place(mx, big, c.k, start + SLOT)
    dv = _place(mx, big, c.v, start + 2 * SLOT)
    dm = _place(mx, big, c.mask, start + 3 * SLOT)
    B, Sq, Nh, DV = c.out_shape
    off = _offset(big.data_ptr(), start + 4 * SLOT)
    assert B * Sq * Nh * DV * 4 <= SLOT
    dst = mx.DeviceView(0, (DV, Nh, Sq, B), (4, 4 * DV, 4 * DV * Nh, 4 * DV * Nh * Sq), big.data_ptr() + off, big)
    mx.flash_attn_ext(dq, dk, dv, dm, c.scale, dst=dst)
    torch.cuda.synchronize()
    got = big[off:off + B * Sq * Nh * DV * 4].cpu().numpy().view(np.float32).reshape(B, Sq, Nh, DV)
    gate = oracle.fa_ggml(c.q, c.k, c.v, c.mask, c.scale, acc_f32=True)
    m = row_metrics(got, gate)
    print(f"[addr] {shape}: max_abs={m['max_abs']:.3e} min_cos={m['min_cos']:.7f}", flush=True)
    assert m["max_abs"] <= MAX_ABS_TOL and m["min_cos"] >= ROW_COS_TOL, m


@pytest.mark.parametrize("high", [True, False], ids=["low-word-ge-2^31", "low-word-lt-2^31"])
def test_set_rows_at_high_low_words(big, high):
    import mxfa as mx
    import oracle
    import torch
    from mxfa import cases as C

    c = C.kv_write_single("t", seed=21, n_tokens=100, kv_pos=10, Nkv=4, max_seq=256, cache_type=C.TYPE_Q8_0)
    start = 0xD0000000 if high else 0x50000000
    print(f"[addr] set_rows low words from {start:#x}", flush=True)
    dd = _place(mx, big, c.dst, start)
    ds = _place(mx, big, c.src, start + SLOT)
    dr = _place(mx, big, c.rows, start + 2 * SLOT)
    mx.set_rows(dd, ds, dr)
    torch.cuda.synchronize()
    off = _offset(big.data_ptr(), start)
    n = c.dst.buf.view(np.uint8).size
    got = big[off:off + n].cpu().numpy()
    ref = np.ascontiguousarray(c.dst.buf).view(np.uint8).reshape(-1).copy()
    oracle.set_rows(oracle.HostTensor(c.dst.type, c.dst.ne, c.dst.nb, ref), c.src, c.rows)
    np.testing.assert_array_equal(got, ref)
