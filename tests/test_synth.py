"""Pins the seeded input generator (acestep.cpp_amd/mxfa/synth.py).

* Philox4x32-10 against the published known-answer vectors of the Random123
  distribution (the reference implementation of Salmon et al., SC'11,
  `kat_vectors`, the three philox4x32 10-round lines: all-zero, all-ones and
  the pi-digit counter/key).
* Box-Muller: every normal is the closed form of its two uniforms, so a
  swapped cos/sin, a wrong offset or a mis-ordered counter block fails.
* Stream layout: any sub-range of a stream equals the same slice of the whole.
"""
from __future__ import annotations

import math

import numpy as np

from mxfa import synth

# counter (c0..c3), key (k0, k1), expected output (x0..x3)
KAT = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF),
     (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


def test_philox_known_answers():
    for ctr, key, want in KAT:
        got = synth.philox4x32_10(*[np.array([c], dtype=np.uint64) for c in ctr], *key)
        assert tuple(int(x[0]) for x in got) == want, (ctr, key)


def test_philox_vectorised_matches_scalar_calls():
    c = np.arange(5, dtype=np.uint64)
    vec = synth.philox4x32_10(c, c + 7, c * 3, c ^ 5, 123, 456)
    for i in range(5):
        one = synth.philox4x32_10(*[np.array([int(x)], dtype=np.uint64) for x in (i, i + 7, 3 * i, i ^ 5)], 123, 456)
        assert all(int(vec[j][i]) == int(one[j][0]) for j in range(4))


def test_box_muller_closed_form():
    seed, stream = 1002, 1
    u = synth.uniform_u32(seed, stream, 0, 16).astype(np.float64)
    z = synth.normal(seed, stream, 0, 16)
    for blk in range(4):
        x = (u[4 * blk:4 * blk + 4] + 0.5) / 2.0 ** 32
        r01, r23 = math.sqrt(-2 * math.log(x[0])), math.sqrt(-2 * math.log(x[2]))
        want = [r01 * math.cos(2 * math.pi * x[1]), r01 * math.sin(2 * math.pi * x[1]),
                r23 * math.cos(2 * math.pi * x[3]), r23 * math.sin(2 * math.pi * x[3])]
        assert np.array_equal(z[4 * blk:4 * blk + 4], np.asarray(want, dtype=np.float32))


def test_stream_slices_and_moments():
    whole = synth.normal(7, 2, 0, 1 << 16)
    assert np.array_equal(synth.normal(7, 2, 1234, 999), whole[1234:1234 + 999])
    assert np.array_equal(synth.normal(7, 2, 3, 5, chunk=2), whole[3:8])
    assert abs(float(whole.mean())) < 0.02 and abs(float(whole.var()) - 1.0) < 0.02
    ints = synth.uniform_int(7, 3, 0, 4096, 1024, 8192)
    assert ints.min() >= 1024 and ints.max() <= 8192
