"""Seeded synthetic inputs: Philox4x32-10 + Box-Muller.

Written from the published description of Philox (J. Salmon, M. Moraes,
R. Dror, D. Shaw, "Parallel Random Numbers: As Easy as 1, 2, 3", SC'11):
10 rounds of

    (c0, c1, c2, c3) -> (hi(M1*c2) ^ c1 ^ k0, lo(M1*c2), hi(M0*c0) ^ c3 ^ k1, lo(M0*c0))

with multipliers M0 = 0xD2511F53, M1 = 0xCD9E8D57 and the key bumped by the
Weyl constants (0x9E3779B9, 0xBB67AE85) between rounds.  Normals come from
the textbook Box-Muller transform of two uniforms u = (x + 0.5) / 2^32.

Element e of a stream is the (e % 4)-th normal of counter block
(e // 4 low 32 bits, e // 4 high 32 bits, stream id, 0) under key (seed low,
seed high).  Any sub-range of a stream can be generated independently, so
large tensors (a 128 MiB KV cache) are generated only where they are written.
"""
from __future__ import annotations

import numpy as np

M0 = np.uint64(0xD2511F53)
M1 = np.uint64(0xCD9E8D57)
W0 = 0x9E3779B9
W1 = 0xBB67AE85
_MASK32 = np.uint64(0xFFFFFFFF)
_SH32 = np.uint64(32)

# Stream ids per tensor, fixed for every config.
STREAM_Q, STREAM_K, STREAM_V, STREAM_LEN, STREAM_PAD = 0, 1, 2, 3, 4


def philox4x32_10(c0, c1, c2, c3, k0: int, k1: int):
    """Vectorised Philox4x32-10.  c* are uint32-valued arrays, k* ints."""
    c0 = np.asarray(c0, dtype=np.uint64)
    c1 = np.asarray(c1, dtype=np.uint64)
    c2 = np.asarray(c2, dtype=np.uint64)
    c3 = np.asarray(c3, dtype=np.uint64)
    k0 &= 0xFFFFFFFF
    k1 &= 0xFFFFFFFF
    for r in range(10):
        if r:
            k0 = (k0 + W0) & 0xFFFFFFFF
            k1 = (k1 + W1) & 0xFFFFFFFF
        p0 = M0 * c0
        p1 = M1 * c2
        c0, c1, c2, c3 = ((p1 >> _SH32) ^ c1 ^ np.uint64(k0), p1 & _MASK32,
                          (p0 >> _SH32) ^ c3 ^ np.uint64(k1), p0 & _MASK32)
    return (c0.astype(np.uint32), c1.astype(np.uint32), c2.astype(np.uint32), c3.astype(np.uint32))


def _blocks(seed: int, stream: int, b0: int, nblk: int):
    idx = np.arange(b0, b0 + nblk, dtype=np.uint64)
    return philox4x32_10(idx & _MASK32, idx >> _SH32, np.full(nblk, stream, dtype=np.uint64),
                         np.zeros(nblk, dtype=np.uint64), seed & 0xFFFFFFFF, seed >> 32)


def uniform_u32(seed: int, stream: int, start: int, n: int) -> np.ndarray:
    """Raw 32-bit outputs for elements [start, start+n) of a stream."""
    b0, b1 = start // 4, (start + n + 3) // 4
    x = np.stack(_blocks(seed, stream, b0, b1 - b0), axis=1).reshape(-1)
    off = start - 4 * b0
    return x[off:off + n]


def normal(seed: int, stream: int, start: int, n: int, chunk: int = 1 << 22) -> np.ndarray:
    """N(0,1) float32 for elements [start, start+n) of a stream."""
    out = np.empty(n, dtype=np.float32)
    pos = 0
    while pos < n:
        m = min(chunk, n - pos)
        s = start + pos
        b0, b1 = s // 4, (s + m + 3) // 4
        x0, x1, x2, x3 = _blocks(seed, stream, b0, b1 - b0)
        inv = 1.0 / 4294967296.0
        u = [(x.astype(np.float64) + 0.5) * inv for x in (x0, x1, x2, x3)]
        r01 = np.sqrt(-2.0 * np.log(u[0]))
        r23 = np.sqrt(-2.0 * np.log(u[2]))
        t01 = 2.0 * np.pi * u[1]
        t23 = 2.0 * np.pi * u[3]
        z = np.stack([r01 * np.cos(t01), r01 * np.sin(t01), r23 * np.cos(t23), r23 * np.sin(t23)], axis=1)
        z = z.reshape(-1)
        off = s - 4 * b0
        out[pos:pos + m] = z[off:off + m]
        pos += m
    return out


def uniform_int(seed: int, stream: int, start: int, n: int, lo: int, hi: int) -> np.ndarray:
    """Integers uniform in [lo, hi] (inclusive)."""
    u = (uniform_u32(seed, stream, start, n).astype(np.float64) + 0.5) / 4294967296.0
    return (lo + np.floor(u * (hi - lo + 1))).astype(np.int64)
