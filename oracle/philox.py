"""Philox4x32-10 counter-based generator (oracle side).

The reference draws its acceptance uniforms with ``torch.rand(1)``
(nano_sglang/decode/speculative.py:150) and its resamples with
``torch.multinomial`` (speculative.py:162); neither stream is reproducible
across devices.  The verify step instead takes *supplied* uniforms, and this
module fixes how they are made so that the CPU oracle and the HIP kernel see
the same numbers:

* block function: Philox4x32 with 10 rounds, multipliers 0xD2511F53 /
  0xCD9E8D57 and Weyl key increments 0x9E3779B9 / 0xBB67AE85
  (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3",
  SC'11);
* uniform ``n`` of stream ``s`` under ``seed``: word ``n % 4`` of
  ``philox(ctr=[lo32(n//4), hi32(n//4), s, 0], key=[lo32(seed), hi32(seed)])``;
* word -> float: ``u = (w >> 8) * 2**-24`` which lies in [0, 1) and is exact
  in float32.

Pinning: ``philox4x32_10`` is checked against the Random123 known-answer
vectors (tests/golden/philox_kat.json); the uniform mapping is exact integer
arithmetic checked against hand-computed values in the tests.
"""

from __future__ import annotations

import numpy as np

M0 = np.uint64(0xD2511F53)
M1 = np.uint64(0xCD9E8D57)
W0 = np.uint32(0x9E3779B9)
W1 = np.uint32(0xBB67AE85)
_MASK32 = np.uint64(0xFFFFFFFF)


def _mulhilo(a: np.uint64, b: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    p = b.astype(np.uint64) * a
    return (p >> np.uint64(32)).astype(np.uint32), (p & _MASK32).astype(np.uint32)


def philox4x32_10(ctr: np.ndarray, key: np.ndarray) -> np.ndarray:
    """Vectorised Philox4x32-10.

    ctr: uint32 array of shape (..., 4); key: uint32 array of shape (..., 2)
    (broadcastable).  Returns uint32 (..., 4).
    """
    ctr = np.asarray(ctr, dtype=np.uint32)
    key = np.asarray(key, dtype=np.uint32)
    c0, c1, c2, c3 = (ctr[..., i].copy() for i in range(4))
    k0 = np.broadcast_to(key[..., 0], c0.shape).astype(np.uint32)
    k1 = np.broadcast_to(key[..., 1], c0.shape).astype(np.uint32)
    with np.errstate(over="ignore"):
        for r in range(10):
            if r > 0:
                k0 = (k0 + W0).astype(np.uint32)
                k1 = (k1 + W1).astype(np.uint32)
            hi0, lo0 = _mulhilo(M0, c0)
            hi1, lo1 = _mulhilo(M1, c2)
            c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
    return np.stack([c0, c1, c2, c3], axis=-1)


def philox_words(seed: int, stream: int, offset: int, n: int) -> np.ndarray:
    """Raw 32-bit words ``offset .. offset+n-1`` of stream ``stream``."""
    idx = np.arange(offset, offset + n, dtype=np.uint64)
    blk = idx // np.uint64(4)
    ctr = np.zeros((n, 4), dtype=np.uint32)
    ctr[:, 0] = (blk & _MASK32).astype(np.uint32)
    ctr[:, 1] = (blk >> np.uint64(32)).astype(np.uint32)
    ctr[:, 2] = np.uint32(stream & 0xFFFFFFFF)
    key = np.array([seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF], dtype=np.uint32)
    out = philox4x32_10(ctr, key)
    return out[np.arange(n), (idx % np.uint64(4)).astype(np.int64)]


def words_to_uniform(w: np.ndarray) -> np.ndarray:
    """u = (w >> 8) * 2^-24, in [0, 1), exact in float32."""
    return ((np.asarray(w, dtype=np.uint32) >> np.uint32(8)).astype(np.float32)
            * np.float32(2.0 ** -24))


def philox_uniforms(seed: int, stream: int, offset: int, n: int) -> np.ndarray:
    """float32 uniforms ``offset .. offset+n-1`` of ``stream`` under ``seed``."""
    return words_to_uniform(philox_words(seed, stream, offset, n))
