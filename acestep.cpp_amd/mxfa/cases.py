"""Workload builders: the five attention configurations of the benchmark,
laid out exactly as acestep.cpp hands them to ggml_flash_attn_ext.

Each builder returns an `FaCase` whose tensors are ggml views (`HostView`:
type id, ne, nb over a host byte buffer) reproducing the reference's views:

* LM single-sequence attention (src/qwen3-lm.h:434-466): Q is the permuted
  view [D, S, Nh] of the RoPE output [D, Nh, S] (nb1 = Nh*D*4, nb2 = D*4);
  K/V are [D, n_kv_pad, Nkv] windows of the F16 cache [D, max_seq, Nkv]
  (nb1 = 2D, nb2 = 2D*max_seq); the mask is the causal F16 [n_kv_pad, S]
  built at :597-610 (0 if j <= kv_pos + i, else -inf).
* LM batched CFG decode (src/qwen3-lm.h:780-794): Q contiguous [D, 1, Nh, N];
  K/V the 4D view [D, n_kv_pad, Nkv, N] of the [D, max_seq, Nkv, n_sets]
  cache; the mask [n_kv_pad, 1, 1, N] is 0 for j < kv_len of each sequence
  (:872-883); n_kv_pad = min(pad256(max kv_len), max_seq) (:654-658).
  The cache is zero-filled at allocation (:255-258) and written only at the
  valid positions.
* DiT self-attention (src/dit-graph.h:207-231): Q the permuted view
  [D, S, Nh, N] of [D, Nh, S, N] (nb1 = Nh*D*4, nb2 = D*4); K/V contiguous
  F16 [D, S, Nkv, N] (ggml_cast of the permuted view); no mask on the
  full-attention layers (:575).
* DiT cross-attention (src/dit-graph.h:317-352): Q contiguous [D, S, Nh, N]
  (rms_norm output); K/V F16 [D, enc_S, Nkv, N]; mask [enc_S, S, 1, N] with
  -inf on the padded encoder positions, uncond slots copying the cond masks
  (src/dit-sampler.h:290-309).

Values are N(0,1) from Philox4x32-10 (synth.py) with a fixed seed per config
and fixed stream ids per tensor (q 0, k 1, v 2, lengths 3, pads 4).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from . import synth

TYPE_F32, TYPE_F16, TYPE_Q8_0, TYPE_BF16 = 0, 1, 8, 30
D = 128
SEEDS = {"c1": 1001, "c2": 1002, "c3": 1003, "c4s": 1004, "c4x": 1005, "c5": 1006,
         "kw2": 1102, "kw3": 1103, "kw5": 1105}


@dataclass
class HostView:
    type: int
    ne: tuple
    nb: tuple
    buf: np.ndarray
    offset: int = 0

    def ptr(self) -> int:
        return self.buf.ctypes.data + self.offset


@dataclass
class FaCase:
    name: str
    q: HostView
    k: HostView
    v: HostView
    mask: Optional[HostView]
    scale: float
    max_bias: float = 0.0
    softcap: float = 0.0
    meta: dict = field(default_factory=dict)

    @property
    def out_shape(self):
        """[B, Sq, Nh, DV] (row-major view of ggml's [DV, Nh, Sq, B])."""
        return (int(self.q.ne[3]), int(self.q.ne[1]), int(self.q.ne[2]), int(self.v.ne[0]))


# -- element codecs (library routines: numpy float16 is IEEE RNE) -----------

def to_f16_bits(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 64).astype(np.uint16)
    return r


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """ggml block_q8_0 bytes (fp16 d + 32 int8) for a float array whose size
    is a multiple of 32: d = amax/127, q = round_half_even(x * 127/amax)."""
    xb = np.asarray(x, dtype=np.float32).reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(amax != 0, np.float32(127.0) / amax, np.float32(0.0)).astype(np.float32)
    qv = np.rint(xb * idv[:, None]).astype(np.int8)
    out = np.empty((xb.shape[0], 34), dtype=np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = qv.view(np.uint8)
    return out.reshape(-1)


def f16_mask_value(allowed: np.ndarray) -> np.ndarray:
    """0 where allowed, -inf elsewhere, as fp16 bits."""
    return np.where(allowed, np.uint16(0x0000), np.uint16(0xFC00)).astype(np.uint16)


def _contig_nb(ne, esize):
    nb = [esize]
    for i in range(1, 4):
        nb.append(nb[-1] * ne[i - 1])
    return tuple(nb)


def _kv16(values_f32: np.ndarray, kv_type: int) -> np.ndarray:
    return to_bf16_bits(values_f32) if kv_type == TYPE_BF16 else to_f16_bits(values_f32)


# -- builders ----------------------------------------------------------------

def lm_single(name="c1", seed=None, n_tokens=1, kv_pos=511, Nh=16, Nkv=8, max_seq=8192,
              mask_mode="causal", kv_type=TYPE_F16) -> FaCase:
    """LM attention through qw3lm_forward: n_tokens new tokens at kv_pos.

    C1 = defaults (Qwen3-0.6B decode, KV length 512, all-zero mask row).
    C2 = lm_single("c2", n_tokens=2048, kv_pos=0, Nh=32, Nkv=8, max_seq=2048).
    mask_mode: "causal" (the reference's mask) or "none" (NULL mask).
    """
    seed = SEEDS.get(name, 1000) if seed is None else seed
    kv_len = kv_pos + n_tokens
    assert kv_len <= max_seq
    n_kv_pad = min(-(-kv_len // 256) * 256, max_seq)
    S = n_tokens
    # Q: RoPE output [D, Nh, S] contiguous, viewed as [D, S, Nh].
    qbuf = synth.normal(seed, synth.STREAM_Q, 0, D * Nh * S)
    q = HostView(TYPE_F32, (D, S, Nh, 1), (4, Nh * D * 4, D * 4, Nh * D * S * 4), qbuf)
    # Cache [D, max_seq, Nkv] zero-filled; rows [0, kv_len) hold data.
    kc = np.zeros(Nkv * max_seq * D, dtype=np.uint16)
    vc = np.zeros(Nkv * max_seq * D, dtype=np.uint16)
    for g in range(Nkv):
        st = D * max_seq * g
        kc[st:st + D * kv_len] = _kv16(synth.normal(seed, synth.STREAM_K, st, D * kv_len), kv_type)
        vc[st:st + D * kv_len] = _kv16(synth.normal(seed, synth.STREAM_V, st, D * kv_len), kv_type)
    kvnb = (2, 2 * D, 2 * D * max_seq, 2 * D * max_seq * Nkv)
    k = HostView(kv_type, (D, n_kv_pad, Nkv, 1), kvnb, kc)
    v = HostView(kv_type, (D, n_kv_pad, Nkv, 1), kvnb, vc)
    mask = None
    if mask_mode == "causal":
        j = np.arange(n_kv_pad)[None, :]
        i = np.arange(S)[:, None]
        mb = f16_mask_value(j <= kv_pos + i).reshape(-1)
        mask = HostView(TYPE_F16, (n_kv_pad, S, 1, 1), (2, 2 * n_kv_pad, 2 * n_kv_pad * S, 2 * n_kv_pad * S), mb)
    return FaCase(name, q, k, v, mask, 1.0 / math.sqrt(D),
                  meta=dict(seed=seed, kv_pos=kv_pos, kv_len=kv_len, n_kv_pad=n_kv_pad, max_seq=max_seq,
                            Nh=Nh, Nkv=Nkv, S=S, kind="lm_single"))


def c1(**kw) -> FaCase:
    """Qwen3-0.6B-shaped decode: 1 token, 16/8 heads, KV length 512."""
    return lm_single("c1", **kw)


def c2(n_tokens=2048, **kw) -> FaCase:
    """Qwen3-4B-shaped causal prefill: 2048 tokens, 32/8 heads, 2048-slot cache."""
    return lm_single("c2", n_tokens=n_tokens, kv_pos=0, Nh=32, Nkv=8, max_seq=max(n_tokens, 256), **kw)


def lm_batch(name="c3", seed=None, N=8, Nh=32, Nkv=8, max_seq=8192, lmin=1024, lmax=8192,
             lengths=None, kv_type=TYPE_F16) -> FaCase:
    """Batched CFG decode through qw3lm_forward_batch: N sequences (cond
    [0, N/2), uncond [N/2, N)), one query token each.  kv_len per sequence is
    uniform in [lmin, lmax] (stream 3) unless `lengths` is given."""
    seed = SEEDS.get(name, 1000) if seed is None else seed
    if lengths is None:
        lengths = synth.uniform_int(seed, synth.STREAM_LEN, 0, N, lmin, lmax)
    lengths = np.asarray(lengths, dtype=np.int64)
    assert lengths.max() <= max_seq and lengths.min() >= 1
    n_kv_pad = int(min(-(-int(lengths.max()) // 256) * 256, max_seq))
    qbuf = synth.normal(seed, synth.STREAM_Q, 0, D * Nh * N)
    q = HostView(TYPE_F32, (D, 1, Nh, N), _contig_nb((D, 1, Nh, N), 4), qbuf)
    kc = np.zeros(N * Nkv * max_seq * D, dtype=np.uint16)
    vc = np.zeros(N * Nkv * max_seq * D, dtype=np.uint16)
    for s in range(N):
        L = int(lengths[s])
        for g in range(Nkv):
            st = D * max_seq * (g + Nkv * s)
            kc[st:st + D * L] = _kv16(synth.normal(seed, synth.STREAM_K, st, D * L), kv_type)
            vc[st:st + D * L] = _kv16(synth.normal(seed, synth.STREAM_V, st, D * L), kv_type)
    kvnb = (2, 2 * D, 2 * D * max_seq, 2 * D * max_seq * Nkv)
    k = HostView(kv_type, (D, n_kv_pad, Nkv, N), kvnb, kc)
    v = HostView(kv_type, (D, n_kv_pad, Nkv, N), kvnb, vc)
    j = np.arange(n_kv_pad)[None, :]
    mb = f16_mask_value(j < lengths[:, None]).reshape(-1)
    mask = HostView(TYPE_F16, (n_kv_pad, 1, 1, N), (2, 2 * n_kv_pad, 2 * n_kv_pad, 2 * n_kv_pad), mb)
    return FaCase(name, q, k, v, mask, 1.0 / math.sqrt(D),
                  meta=dict(seed=seed, lengths=lengths.tolist(), n_kv_pad=n_kv_pad, max_seq=max_seq, N=N,
                            Nh=Nh, Nkv=Nkv, kind="lm_batch"))


def c3(**kw) -> FaCase:
    """Qwen3-4B-shaped batched CFG decode: 8 sequences, lengths U[1024, 8192]."""
    return lm_batch("c3", **kw)


def dit_self(name="c4s", seed=None, B=2, S=3000, Nh=16, Nkv=16, kv_type=TYPE_F16, window=0) -> FaCase:
    """DiT self-attention over B = 2N (CFG) batches.  window > 0 adds the
    sliding-window mask of the even layers (|qi - ki| <= window)."""
    seed = SEEDS.get(name, 1000) if seed is None else seed
    qbuf = synth.normal(seed, synth.STREAM_Q, 0, D * Nh * S * B)   # [D, Nh, S, B] memory
    q = HostView(TYPE_F32, (D, S, Nh, B), (4, Nh * D * 4, D * 4, Nh * D * S * 4), qbuf)
    n = D * S * Nkv * B
    kb = _kv16(synth.normal(seed, synth.STREAM_K, 0, n), kv_type)
    vb = _kv16(synth.normal(seed, synth.STREAM_V, 0, n), kv_type)
    kvne = (D, S, Nkv, B)
    k = HostView(kv_type, kvne, _contig_nb(kvne, 2), kb)
    v = HostView(kv_type, kvne, _contig_nb(kvne, 2), vb)
    mask = None
    if window > 0:
        qi = np.arange(S)[:, None]
        ki = np.arange(S)[None, :]
        allowed = (S <= window) | (np.abs(qi - ki) <= window)
        plane = f16_mask_value(allowed).reshape(-1)
        mb = np.tile(plane, B)
        mask = HostView(TYPE_F16, (S, S, 1, B), (2, 2 * S, 2 * S * S, 2 * S * S), mb)
    return FaCase(name, q, k, v, mask, 1.0 / math.sqrt(D),
                  meta=dict(seed=seed, B=B, S=S, Nh=Nh, Nkv=Nkv, window=window, kind="dit_self"))


def c4_self(**kw) -> FaCase:
    return dit_self("c4s", **kw)


def dit_cross(name="c4x", seed=None, B=2, S=3000, Nh=16, Nkv=16, enc_S=256, pad_max=128, pads=None,
              kv_type=TYPE_F16) -> FaCase:
    """DiT cross-attention: S queries against enc_S encoder tokens; the last
    pad_b keys of real sample b are masked (pad_b uniform in {0..pad_max},
    stream 4); uncond slots [B/2, B) copy the cond masks."""
    seed = SEEDS.get(name, 1000) if seed is None else seed
    n_real = max(B // 2, 1)
    if pads is None:
        pads = synth.uniform_int(seed, synth.STREAM_PAD, 0, n_real, 0, pad_max)
    pads = np.asarray(pads, dtype=np.int64)
    pads_b = np.concatenate([pads, pads])[:B] if B > 1 else pads[:1]
    qbuf = synth.normal(seed, synth.STREAM_Q, 0, D * S * Nh * B)
    qne = (D, S, Nh, B)
    q = HostView(TYPE_F32, qne, _contig_nb(qne, 4), qbuf)
    n = D * enc_S * Nkv * B
    kb = _kv16(synth.normal(seed, synth.STREAM_K, 0, n), kv_type)
    vb = _kv16(synth.normal(seed, synth.STREAM_V, 0, n), kv_type)
    kvne = (D, enc_S, Nkv, B)
    k = HostView(kv_type, kvne, _contig_nb(kvne, 2), kb)
    v = HostView(kv_type, kvne, _contig_nb(kvne, 2), vb)
    ki = np.arange(enc_S)
    planes = [np.broadcast_to(f16_mask_value(ki < enc_S - int(p))[None, :], (S, enc_S)).reshape(-1)
              for p in pads_b]
    mb = np.concatenate(planes)
    mask = HostView(TYPE_F16, (enc_S, S, 1, B), (2, 2 * enc_S, 2 * enc_S * S, 2 * enc_S * S), mb)
    return FaCase(name, q, k, v, mask, 1.0 / math.sqrt(D),
                  meta=dict(seed=seed, B=B, S=S, Nh=Nh, Nkv=Nkv, enc_S=enc_S, pads=pads_b.tolist(),
                            kind="dit_cross"))


def c4_cross(**kw) -> FaCase:
    return dit_cross("c4x", **kw)


def lm_batch_q8(name="c5", seed=None, N=4, Nh=32, Nkv=8, L=8192, max_seq=None, zero_mask=True) -> FaCase:
    """Batched decode over a Q8_0 KV cache (rows of 128 = 4 blocks of 34 B),
    quantised from N(0,1) fp32; every sequence has kv_len = L."""
    seed = SEEDS.get(name, 1000) if seed is None else seed
    max_seq = L if max_seq is None else max_seq
    n_kv_pad = min(-(-L // 256) * 256, max_seq)
    qbuf = synth.normal(seed, synth.STREAM_Q, 0, D * Nh * N)
    q = HostView(TYPE_F32, (D, 1, Nh, N), _contig_nb((D, 1, Nh, N), 4), qbuf)
    row = D // 32 * 34
    kc = np.zeros(N * Nkv * max_seq * row, dtype=np.uint8)
    vc = np.zeros(N * Nkv * max_seq * row, dtype=np.uint8)
    for s in range(N):
        for g in range(Nkv):
            st = D * max_seq * (g + Nkv * s)
            bst = row * max_seq * (g + Nkv * s)
            kc[bst:bst + row * L] = quantize_q8_0(synth.normal(seed, synth.STREAM_K, st, D * L))
            vc[bst:bst + row * L] = quantize_q8_0(synth.normal(seed, synth.STREAM_V, st, D * L))
    kvnb = (34, row, row * max_seq, row * max_seq * Nkv)
    k = HostView(TYPE_Q8_0, (D, n_kv_pad, Nkv, N), kvnb, kc)
    v = HostView(TYPE_Q8_0, (D, n_kv_pad, Nkv, N), kvnb, vc)
    mask = None
    if zero_mask:
        j = np.arange(n_kv_pad)[None, :]
        mb = f16_mask_value(np.broadcast_to(j < L, (N, n_kv_pad))).reshape(-1)
        mask = HostView(TYPE_F16, (n_kv_pad, 1, 1, N), (2, 2 * n_kv_pad, 2 * n_kv_pad, 2 * n_kv_pad), mb)
    return FaCase(name, q, k, v, mask, 1.0 / math.sqrt(D),
                  meta=dict(seed=seed, N=N, Nh=Nh, Nkv=Nkv, L=L, n_kv_pad=n_kv_pad, kind="lm_batch_q8"))


def c5(**kw) -> FaCase:
    return lm_batch_q8("c5", **kw)


def c4_self8(**kw) -> FaCase:
    """C4 self with the real DiT's 16 / 8 heads (the config lists 16 / 16)."""
    return dit_self("c4s8", seed=SEEDS["c4s"], Nkv=8, **kw)


def c4_cross8(**kw) -> FaCase:
    """C4 cross with 16 / 8 heads."""
    return dit_cross("c4x8", seed=SEEDS["c4x"], Nkv=8, **kw)


def c4_self_window(**kw) -> FaCase:
    """The DiT's sliding-window self-attention layer at C4's size: every even
    layer (layer_type 0) reads the window mask sa_mask_sw [S, S, 1, N]
    (dit-graph.h:522-524, :574-576) built at dit-sampler.h:262-289 with the
    GGUF's acestep.sliding_window (dit.h:286; 128 in the reference's runs)."""
    return dit_self("c4sw", seed=SEEDS["c4s"], window=128, **kw)


def c4_self_window8(**kw) -> FaCase:
    """The window layer with the real DiT's 16 / 8 heads."""
    return dit_self("c4sw8", seed=SEEDS["c4s"], Nkv=8, window=128, **kw)


def c2_q8(n_tokens=2048, **kw) -> FaCase:
    """C2's prompt over a Q8_0 cache (the prompt path of qwen3-lm.h with a
    Q8_0 cache type): the same Q, mask and N(0,1) K/V rows as C2, the K/V
    rows quantised to Q8_0 (rows of 128 = 4 blocks of 34 B)."""
    base = c2(n_tokens=n_tokens, **kw)
    m = base.meta
    Nkv, max_seq, kv_len, seed = m["Nkv"], m["max_seq"], m["kv_len"], m["seed"]
    row = D // 32 * 34
    bufs = []
    for stream in (synth.STREAM_K, synth.STREAM_V):
        f = np.zeros(Nkv * max_seq * D, dtype=np.float32)
        for g in range(Nkv):
            st = D * max_seq * g
            f[st:st + D * kv_len] = synth.normal(seed, stream, st, D * kv_len)
        bufs.append(quantize_q8_0(f))
    kvnb = (34, row, row * max_seq, row * max_seq * Nkv)
    k = HostView(TYPE_Q8_0, base.k.ne, kvnb, bufs[0])
    v = HostView(TYPE_Q8_0, base.v.ne, kvnb, bufs[1])
    return FaCase("c2q8", base.q, k, v, base.mask, base.scale, meta=dict(m, kind="lm_single_q8"))


BUILDERS = {"c1": c1, "c2": c2, "c3": c3, "c4s": c4_self, "c4x": c4_cross, "c5": c5, "c4s8": c4_self8,
            "c4x8": c4_cross8, "c2q8": c2_q8, "c4sw": c4_self_window, "c4sw8": c4_self_window8}


def with_q16(case: FaCase) -> FaCase:
    """A copy of `case` whose Q is stored in K's 16-bit type (F16 / BF16),
    rounded to nearest even, same element layout: what the fused
    pre-attention step hands attention (mxfa_qk_norm_rope)."""
    assert case.k.type in (TYPE_F16, TYPE_BF16) and case.q.type == TYPE_F32 and case.q.offset % 4 == 0
    bits = _kv16(np.ascontiguousarray(case.q.buf).view(np.float32), case.k.type)
    q = HostView(case.k.type, tuple(case.q.ne), tuple(int(x) // 2 for x in case.q.nb), bits, case.q.offset // 2)
    return FaCase(case.name, q, case.k, case.v, case.mask, case.scale, case.max_bias, case.softcap, dict(case.meta))


def norm_rope_work(B: int, S: int, Nh: int, Nkv: int, rows_i64: bool = True, Skv: Optional[int] = None) -> dict:
    """Algorithmic bytes of one fused pre-attention call (mxfa_qk_norm_rope):
    every F32 row of Q, K and V read once, its 16-bit row written once, the
    positions and row ids read once (the two 512 B weights are noise).  The
    reference's op chain (rms_norm, mul, rope, cont, clamp, set_rows, and
    attention's F32 Q read) moves several times that.  Skv given: the
    cross-attention form (no RoPE, no positions or row ids, Skv K/V
    tokens)."""
    if Skv is not None:
        n = (Nh * S + 2 * Nkv * Skv) * B
        rd, wr = n * 4 * D, n * 2 * D
        return dict(rows=n, read_bytes=rd, write_bytes=wr, id_bytes=0, bytes=rd + wr)
    n = (Nh + 2 * Nkv) * S * B
    rd, wr = n * 4 * D, n * 2 * D
    ids = S * B * 4 + S * B * (8 if rows_i64 else 4)
    return dict(rows=n, read_bytes=rd, write_bytes=wr, id_bytes=ids, bytes=rd + wr + ids)


# -- structured masks ------------------------------------------------------------

def structured_spec(case: FaCase) -> dict:
    """The structured mask (keyword arguments of mxfa.mask_spec) that stands
    for the dense mask the reference builds for this case: causal from the
    query position (qwen3-lm.h:597-610), per-sequence lengths
    (qwen3-lm.h:872-883, dit-sampler.h:296-309), the sliding window
    (dit-sampler.h:262-289); {} for an unmasked case."""
    m = case.meta
    kind = m.get("kind")
    if case.mask is None:
        return {}
    if kind == "lm_single":
        return dict(causal=True, pos0=int(m["kv_pos"]))
    if kind == "lm_batch":
        return dict(lengths=[int(x) for x in m["lengths"]])
    if kind == "dit_cross":
        return dict(lengths=[int(m["enc_S"]) - int(p) for p in m["pads"]])
    if kind == "dit_self" and m.get("window", 0) > 0 and m["S"] > m["window"]:
        return dict(window=int(m["window"]))
    raise ValueError(f"no structured form for case {case.name} ({kind})")


def dense_mask_bits(spec: dict, Sq: int, Skv: int, B: int) -> np.ndarray:
    """The dense F16 mask [B][1][Sq][Skv] (uint16 bits: 0 live, -inf dead)
    that a structured mask (mask_spec keyword arguments) stands for."""
    i = np.arange(Sq)[:, None] + int(spec.get("pos0", 0))
    j = np.arange(Skv)[None, :]
    lengths = spec.get("lengths")
    out = np.empty((B, 1, Sq, Skv), dtype=np.uint16)
    for b in range(B):
        live = np.ones((Sq, Skv), dtype=bool)
        if lengths is not None:
            live &= j < lengths[b % len(lengths)]
        if spec.get("causal"):
            live &= j <= i
        if spec.get("window") is not None:
            live &= np.abs(i - j) <= spec["window"]
        out[b, 0] = np.where(live, np.uint16(0), np.uint16(0xFC00))
    return out


def with_dense_mask(case: FaCase, spec: dict) -> FaCase:
    """A copy of `case` whose mask is the dense form of `spec` ([Skv, Sq, 1, B])."""
    Sq, Skv, B = int(case.q.ne[1]), int(case.k.ne[1]), int(case.q.ne[3])
    bits = dense_mask_bits(spec, Sq, Skv, B).reshape(-1)
    m = HostView(TYPE_F16, (Skv, Sq, 1, B), (2, 2 * Skv, 2 * Skv * Sq, 2 * Skv * Sq), bits)
    return FaCase(case.name, case.q, case.k, case.v, m, case.scale, case.max_bias, case.softcap, dict(case.meta))


# -- KV-cache write (GGML_OP_SET_ROWS) -------------------------------------------

TYPE_I32, TYPE_I64 = 26, 27


@dataclass
class SetRowsCase:
    name: str
    dst: HostView          # the cache view set_rows writes into
    src: HostView          # F32 rows
    rows: HostView         # I64 / I32 row ids
    meta: dict = field(default_factory=dict)


def _cache_fill(seed, n_bytes):
    """Random bytes standing for whatever the cache held before the write
    (rows the write does not name must keep them)."""
    return synth.uniform_u32(seed, synth.STREAM_PAD, 0, -(-n_bytes // 4)).view(np.uint8)[:n_bytes].copy()


def kv_write_single(name="kw2", seed=None, n_tokens=2048, kv_pos=0, Nkv=8, max_seq=2048,
                    cache_type=TYPE_F16, row_type=TYPE_I64) -> SetRowsCase:
    """qw3lm_build_attn's cache write (src/qwen3-lm.h:448-454): the
    contiguous F32 [D, S, Nkv] rows (ggml_cont of the permuted RoPE output,
    :433-436) go to rows kv_pos .. kv_pos+S-1 of the [D, max_seq, Nkv] cache;
    kv_rows is I64 [S] (:528-530), broadcast over Nkv."""
    seed = SEEDS.get(name, 1100) if seed is None else seed
    S = n_tokens
    assert kv_pos + S <= max_seq
    src = HostView(TYPE_F32, (D, S, Nkv, 1), _contig_nb((D, S, Nkv, 1), 4),
                   synth.normal(seed, synth.STREAM_K, 0, D * S * Nkv))
    idt = np.int64 if row_type == TYPE_I64 else np.int32
    rows = np.arange(kv_pos, kv_pos + S, dtype=idt)
    rv = HostView(row_type, (S, 1, 1, 1), _contig_nb((S, 1, 1, 1), rows.itemsize), rows)
    rb = _type_row_bytes(cache_type, D)
    dnb = (_type_row_bytes(cache_type, 1) if cache_type != TYPE_Q8_0 else 34, rb, rb * max_seq, rb * max_seq * Nkv)
    dst = HostView(cache_type, (D, max_seq, Nkv, 1), dnb, _cache_fill(seed, rb * max_seq * Nkv))
    return SetRowsCase(name, dst, src, rv, meta=dict(seed=seed, S=S, kv_pos=kv_pos, Nkv=Nkv, max_seq=max_seq,
                                                     kind="kv_write_single"))


def kv_write_batch(name="kw3", seed=None, N=8, Nkv=8, max_seq=8192, n_sets=None, s0=0, positions=None,
                   cache_type=TYPE_F16) -> SetRowsCase:
    """qw3lm_forward_batch's cache write (src/qwen3-lm.h:760-777): one new
    token per sequence; dst is the 4D view [D, max_seq, Nkv, N] of the
    [D, max_seq, Nkv, n_sets] cache starting at set s0, src the F32
    [D, 1, Nkv, N] rows, kv_rows I64 [1, 1, N] one position per set
    (:699-701), broadcast over Nkv."""
    seed = SEEDS.get(name, 1101) if seed is None else seed
    n_sets = N + s0 if n_sets is None else n_sets
    assert s0 + N <= n_sets
    if positions is None:
        positions = synth.uniform_int(seed, synth.STREAM_LEN, 0, N, 0, max_seq - 1)
    positions = np.asarray(positions, dtype=np.int64)
    src = HostView(TYPE_F32, (D, 1, Nkv, N), _contig_nb((D, 1, Nkv, N), 4),
                   synth.normal(seed, synth.STREAM_K, 0, D * Nkv * N))
    rv = HostView(TYPE_I64, (1, 1, N, 1), (8, 8, 8, 8 * N), positions.copy())
    rb = _type_row_bytes(cache_type, D)
    nb = (_type_row_bytes(cache_type, 1) if cache_type != TYPE_Q8_0 else 34, rb, rb * max_seq, rb * max_seq * Nkv)
    buf = _cache_fill(seed, nb[3] * n_sets)
    dst = HostView(cache_type, (D, max_seq, Nkv, N), nb, buf, offset=s0 * nb[3])
    return SetRowsCase(name, dst, src, rv, meta=dict(seed=seed, N=N, Nkv=Nkv, max_seq=max_seq, s0=s0,
                                                     positions=positions.tolist(), kind="kv_write_batch"))


def kw2(**kw) -> SetRowsCase:
    """C2's cache write: 2048 prompt tokens x 8 KV heads into the F16 cache."""
    return kv_write_single("kw2", **kw)


def kw3(**kw) -> SetRowsCase:
    """C3's cache write: one token for each of 8 sequences, 8 KV heads."""
    return kv_write_batch("kw3", **kw)


def kw5(**kw) -> SetRowsCase:
    """C2's cache write into a Q8_0 cache (quantised on the fly)."""
    kw.setdefault("cache_type", TYPE_Q8_0)
    return kv_write_single("kw5", **kw)


SET_ROWS_BUILDERS = {"kw2": kw2, "kw3": kw3, "kw5": kw5}


def set_rows_work(case: SetRowsCase) -> dict:
    """Algorithmic bytes of one set_rows call: every F32 source row read once,
    its converted row written once, the row ids read once."""
    n = int(case.src.ne[1] * case.src.ne[2] * case.src.ne[3])
    r = case.rows
    rd = n * 4 * D
    wr = n * _type_row_bytes(case.dst.type, D)
    ids = int(r.ne[0] * r.ne[1] * r.ne[2]) * (8 if r.type == TYPE_I64 else 4)
    return dict(rows=n, read_bytes=rd, write_bytes=wr, id_bytes=ids, bytes=rd + wr + ids)


# -- work accounting -----------------------------------------------------------

def _type_row_bytes(t: int, ne0: int) -> int:
    return {TYPE_F32: 4 * ne0, TYPE_F16: 2 * ne0, TYPE_BF16: 2 * ne0, TYPE_Q8_0: ne0 // 32 * 34}[t]


def _mask_alive(case: FaCase) -> np.ndarray:
    """bool [Bm3, Nm2, Sq, Skv]: key allowed for (mask batch, mask head, query)."""
    Sq, Skv = int(case.q.ne[1]), int(case.k.ne[1])
    if case.mask is None:
        return np.ones((1, 1, Sq, Skv), dtype=bool)
    m = case.mask
    n2, n3 = int(m.ne[2]), int(m.ne[3])
    out = np.empty((n3, n2, Sq, Skv), dtype=bool)
    raw = m.buf.view(np.uint8)
    for i3 in range(n3):
        for i2 in range(n2):
            for i1 in range(Sq):
                off = m.offset + i1 * m.nb[1] + i2 * m.nb[2] + i3 * m.nb[3]
                row = raw[off:off + 2 * Skv].view(np.uint16)
                out[i3, i2, i1] = row != 0xFC00
    return out


def work(case: FaCase) -> dict:
    """Algorithmic work of one call:
    flops     = 4*D per unmasked (query, key) pair per q head (QK^T + PV);
    kv_bytes  = K+V rows with at least one unmasked query, once per
                (batch, KV head) -- what a decode kernel must stream;
    bytes     = Q (as typed) + kv_bytes + mask + O."""
    Sq, Nh, B = int(case.q.ne[1]), int(case.q.ne[2]), int(case.q.ne[3])
    Skv, Nkv, Bk = int(case.k.ne[1]), int(case.k.ne[2]), int(case.k.ne[3])
    G, rk3 = Nh // Nkv, B // Bk
    alive = _mask_alive(case)
    n3, n2 = alive.shape[0], alive.shape[1]
    pairs = 0
    kv_rows = 0
    for b in range(B):
        for h in range(Nh):
            pairs += int(alive[b % n3, h % n2].sum())
    for bk in range(Bk):
        for g in range(Nkv):
            any_key = np.zeros(Skv, dtype=bool)
            for b in range(bk * rk3, (bk + 1) * rk3):
                for h in range(g * G, (g + 1) * G):
                    any_key |= alive[b % n3, h % n2].any(axis=0)
            kv_rows += int(any_key.sum())
    row_kv = _type_row_bytes(case.k.type, D) + _type_row_bytes(case.v.type, D)
    kv_bytes = kv_rows * row_kv
    q_bytes = _type_row_bytes(case.q.type, D) * Sq * Nh * B
    o_bytes = D * Sq * Nh * B * 4
    m_bytes = 0 if case.mask is None else int(case.mask.ne[2] * case.mask.ne[3]) * Sq * Skv * 2
    return dict(flops=4 * D * pairs, pairs=pairs, kv_bytes=kv_bytes,
                bytes=q_bytes + kv_bytes + m_bytes + o_bytes, q_bytes=q_bytes, o_bytes=o_bytes,
                mask_bytes=m_bytes)
