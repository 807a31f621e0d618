"""CPU checker of the keyed random numbers (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

The reference has no counterpart: its Engine shares one generator across requests (engine.py:41,
126-133). The speculative Engine of forgeserve_amd keys each request's draws instead; this module
states that stream in numpy so the tests can check the kernel bit for bit (uniforms) and to a few
ulps (Exp(1), whose log1p is not correctly rounded on either side).

Philox4x32-10 as published by Salmon, Moraes, Dror and Shaw ("Parallel random numbers: as easy as
1, 2, 3", SC'11): ten rounds of two 32x32->64 multiplies with M0 = 0xD2511F53, M1 = 0xCD9E8D57 and key
increments W0 = 0x9E3779B9, W1 = 0xBB67AE85. Pinned in tests/test_oracle.py by the known-answer
vectors of the authors' Random123 distribution (counter/key all zeros, all ones, and the pi digits).

Mapping (the kernel's, forgeserve_amd/csrc/rng.hip): counter (j // 2, slot, 0, 0), key (low, high 32
bits of the row key); column 2i takes words (w0, w1), column 2i+1 (w2, w3); uniform = (w_a >> 8) *
2^-24; Exp(1) = -log1p(-t), t = (1 + (w_a >> 9) * 2^-23) * 2^-(1 + clz32(w_b)).
"""

import numpy as np

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = np.uint64(0x9E3779B9), np.uint64(0xBB67AE85)
MASK = np.uint64(0xFFFFFFFF)


def philox4x32_10(c0, c1, c2, c3, k0, k1):
    """Elementwise Philox4x32-10 over numpy arrays (any broadcastable shapes) -> four uint32 arrays."""
    c0, c1, c2, c3 = (np.asarray(x, dtype=np.uint64) & MASK for x in (c0, c1, c2, c3))
    k0, k1 = (np.asarray(x, dtype=np.uint64) & MASK for x in (k0, k1))
    for _ in range(10):
        p0 = M0 * c0
        p1 = M1 * c2
        c0, c1, c2, c3 = ((p1 >> np.uint64(32)) ^ c1 ^ k0) & MASK, p1 & MASK, \
                         ((p0 >> np.uint64(32)) ^ c3 ^ k1) & MASK, p0 & MASK
        k0 = (k0 + W0) & MASK
        k1 = (k1 + W1) & MASK
    return tuple(x.astype(np.uint32) for x in (c0, c1, c2, c3))


def words(key: int, slot: int, n: int):
    """The two words (a, b) behind columns 0..n-1 of (key, slot): uint32 arrays of length n."""
    pair = np.arange((n + 1) // 2, dtype=np.uint64)
    key = int(key) & 0xFFFFFFFFFFFFFFFF
    w0, w1, w2, w3 = philox4x32_10(pair, slot, 0, 0, key & 0xFFFFFFFF, key >> 32)
    a = np.stack([w0, w2], 1).reshape(-1)[:n]
    b = np.stack([w1, w3], 1).reshape(-1)[:n]
    return a, b


def uniform(key: int, slot: int, n: int) -> np.ndarray:
    a, _ = words(key, slot, n)
    return ((a >> np.uint32(8)).astype(np.float32) * np.float32(2.0 ** -24)).astype(np.float32)


def clz32(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.uint64)
    out = np.full(x.shape, 32, dtype=np.int64)
    nz = x != 0
    out[nz] = 31 - np.floor(np.log2(x[nz].astype(np.float64))).astype(np.int64)
    return out


def exponential(key: int, slot: int, n: int) -> np.ndarray:
    """Exp(1) variates in float64 (the exact value the float32 kernel rounds)."""
    a, b = words(key, slot, n)
    mant = 1.0 + (a >> np.uint32(9)).astype(np.float64) * 2.0 ** -23
    t = np.ldexp(mant, -(1 + clz32(b)))
    return -np.log1p(-t)
