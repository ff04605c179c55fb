"""Philox-4x32-10 counter-based generator in NumPy (TEST INFRASTRUCTURE ONLY).

Restates the published algorithm (Salmon, Moraes, Dror, Shaw, "Parallel random
numbers: as easy as 1, 2, 3", SC 2011): ten rounds of two 32x32->64-bit
multiplies with the constants 0xD2511F53 / 0xCD9E8D57 and a Weyl key schedule
with increments 0x9E3779B9 / 0xBB67AE85.  Pinned in tests/test_oracle.py by
the authors' known-answer vectors.

On top of it, the replay index draw that the MI355X library uses in place of
the reference's samplers (robolearn/flashsac/replay.py:179-183 draws with
torch.randint, robolearn/warp/_flash_replay.py:116-129 with Warp's rejection
sampler; the two reference learners already draw different streams, so parity
is defined on the indices themselves):

    counter = (i mod 2^32, i >> 32, draw mod 2^32, stream_id ^ ((draw >> 32) << 16))
    key     = (seed mod 2^32, seed >> 32)
    (x, y, _, _) = philox(counter, key);  idx[i] = ((x << 32 | y) * count) >> 64

Only tests/ import this module, as the checker of the device sampler.
"""

import numpy as np

M0, M1 = 0xD2511F53, 0xCD9E8D57
W0, W1 = 0x9E3779B9, 0xBB67AE85
MASK32 = np.uint64(0xFFFFFFFF)


def philox4x32_10(counter, key):
    """counter: 4 uint32 arrays (broadcastable); key: 2 uint32 values.  Returns 4 uint32 arrays."""
    c0, c1, c2, c3 = (np.asarray(c, dtype=np.uint64) & MASK32 for c in counter)
    k0, k1 = (np.uint64(int(k) & 0xFFFFFFFF) for k in key)
    for round_index in range(10):
        if round_index:
            k0 = (k0 + np.uint64(W0)) & MASK32
            k1 = (k1 + np.uint64(W1)) & MASK32
        p0 = np.uint64(M0) * c0
        p1 = np.uint64(M1) * c2
        hi0, lo0 = p0 >> np.uint64(32), p0 & MASK32
        hi1, lo1 = p1 >> np.uint64(32), p1 & MASK32
        c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
    return tuple(c.astype(np.uint32) for c in (c0, c1, c2, c3))


def _mulhi64(a, b):
    """High 64 bits of the 128-bit products a * b (uint64 arrays), exact."""
    a = np.asarray(a, dtype=np.uint64)
    b = np.asarray(b, dtype=np.uint64)
    a_lo, a_hi = a & MASK32, a >> np.uint64(32)
    b_lo, b_hi = b & MASK32, b >> np.uint64(32)
    lo_lo = a_lo * b_lo
    hi_lo = a_hi * b_lo
    lo_hi = a_lo * b_hi
    hi_hi = a_hi * b_hi
    cross = (lo_lo >> np.uint64(32)) + (hi_lo & MASK32) + (lo_hi & MASK32)
    return hi_hi + (hi_lo >> np.uint64(32)) + (lo_hi >> np.uint64(32)) + (cross >> np.uint64(32))


def replay_indices(seed: int, draw: int, stream_id: int, count: int, n: int) -> np.ndarray:
    """The n int64 replay indices in [0, count) of one update's draw."""
    i = np.arange(n, dtype=np.uint64)
    draw_hi = (int(draw) >> 32) & 0xFFFFFFFF
    counter = (i & MASK32, i >> np.uint64(32), np.uint64(int(draw) & 0xFFFFFFFF),
               np.uint64((int(stream_id) ^ ((draw_hi << 16) & 0xFFFFFFFF)) & 0xFFFFFFFF))
    x, y, _, _ = philox4x32_10(counter, (int(seed) & 0xFFFFFFFF, (int(seed) >> 32) & 0xFFFFFFFF))
    word = (x.astype(np.uint64) << np.uint64(32)) | y.astype(np.uint64)
    return _mulhi64(word, np.uint64(count)).astype(np.int64)
