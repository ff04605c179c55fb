"""Pins oracle/philox.py, the checker of the device replay sampler.

* philox4x32_10 against the known-answer vectors the generator's authors
  publish with their reference implementation (Random123, kat_vectors:
  counter / key / expected output for the all-zero, all-one and pi-digit
  inputs).
* The 64-bit multiply-high against Python's exact integers.
* replay_indices: every index is the floor of word * count / 2^64 of the
  Philox word built from (row, draw, stream), recomputed here with Python
  integers; ranges and the 64-bit draw/seed split.
"""

import numpy as np
import pytest

from oracle import philox as PH

KAT = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF),
     (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("counter,key,expected", KAT)
def test_philox_known_answers(counter, key, expected):
    got = PH.philox4x32_10(tuple(np.uint32(c) for c in counter), key)
    assert tuple(int(v) for v in got) == expected


def test_philox_is_elementwise_over_arrays():
    counters = np.array([[0, 0, 0, 0], [0xFFFFFFFF] * 4, [0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344]],
                        dtype=np.uint32)
    # one key per call: compare the vectorized first row against the scalar known answer
    got = PH.philox4x32_10(tuple(counters[:1, i] for i in range(4)), KAT[0][1])
    assert tuple(int(v[0]) for v in got) == KAT[0][2]


def test_mulhi64_exact():
    rng = np.random.default_rng(0)
    a = rng.integers(0, 2**63, 1000, dtype=np.uint64) * np.uint64(2) + rng.integers(0, 2, 1000, dtype=np.uint64)
    b = rng.integers(0, 2**63, 1000, dtype=np.uint64)
    got = PH._mulhi64(a, b)
    expected = [(int(x) * int(y)) >> 64 for x, y in zip(a, b)]
    assert [int(v) for v in got] == expected
    assert int(PH._mulhi64(np.uint64(2**64 - 1), np.uint64(2**64 - 1))) == 2**64 - 2


@pytest.mark.parametrize("seed,draw,stream_id,count", [(1, 0, 1, 1_048_576), (2**40 + 3, 2**33 + 5, 23, 1000),
                                                       (9, 7, 1, 1)])
def test_replay_indices_follow_the_definition(seed, draw, stream_id, count):
    n = 64
    got = PH.replay_indices(seed, draw, stream_id, count, n)
    for i in range(n):
        counter = (i & 0xFFFFFFFF, i >> 32, draw & 0xFFFFFFFF, (stream_id ^ (((draw >> 32) << 16) & 0xFFFFFFFF)))
        x, y, _, _ = (int(v) for v in PH.philox4x32_10(tuple(np.uint32(c) for c in counter),
                                                        (seed & 0xFFFFFFFF, seed >> 32)))
        assert got[i] == (((x << 32) | y) * count) >> 64
    assert got.min() >= 0 and got.max() < count


def test_replay_indices_cover_the_range_uniformly():
    bins = 97
    got = PH.replay_indices(5, 0, 1, bins, 200_000)
    counts = np.bincount(got, minlength=bins)
    expected = got.size / bins
    chi2 = float(((counts - expected) ** 2 / expected).sum())
    assert abs(chi2 - (bins - 1)) < 6 * np.sqrt(2 * (bins - 1))
