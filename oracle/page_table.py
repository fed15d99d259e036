"""CSR page table and flat-slot arithmetic (oracle side).

Restates nano_sglang/engine/engine.py:419-448 (the FlashInfer path's metadata
builder) and the slot rule used by the KV scatter at
nano_sglang/model/causal_lm.py:335-338:

* ``kv_indices``   = concatenation of every request's block table (int32);
* ``kv_indptr``    = running page counts, ``int32[B+1]``;
* ``last_page_len`` = ``L % P`` or ``P`` when that is 0 (engine.py:434-435);
* flat slot of absolute position ``pos`` = ``block[pos // P] * P + pos % P``
  (engine.py:438-443), int64.

Pinning: exact integer arithmetic, checked in tests against hand-worked
examples (L < P, L a multiple of P, several requests) and against a brute-force
walk that reconstructs every token's (block, offset) pair.
"""

from __future__ import annotations

import numpy as np


def build_csr(block_tables: list[list[int]], kv_lens: list[int], page_size: int):
    """engine.py:424-447 -> (kv_indptr, kv_indices, kv_last_page_len)."""
    indptr = [0]
    indices: list[int] = []
    last = []
    for bt, L in zip(block_tables, kv_lens):
        need = (L + page_size - 1) // page_size
        if len(bt) < need:
            raise ValueError(f"block table holds {len(bt)} pages, {need} needed for {L} tokens")
        indices.extend(bt[:need])
        indptr.append(indptr[-1] + need)
        lpl = L % page_size
        last.append(lpl if lpl > 0 else page_size)
    return (np.asarray(indptr, np.int32), np.asarray(indices, np.int32),
            np.asarray(last, np.int32))


def kv_len_from_csr(kv_indptr: np.ndarray, last_page_len: np.ndarray, page_size: int) -> np.ndarray:
    """Inverse of the last_page_len rule: L_b = (pages_b - 1) * P + last_b."""
    pages = np.diff(kv_indptr.astype(np.int64))
    return np.where(pages > 0, (pages - 1) * page_size + last_page_len.astype(np.int64), 0)


def slot_of(block_table: list[int] | np.ndarray, pos: int, page_size: int) -> int:
    """engine.py:440-442: flat slot index of absolute position ``pos``."""
    return int(block_table[pos // page_size]) * page_size + pos % page_size


def write_indices(block_tables, starts, counts, page_size: int) -> np.ndarray:
    """engine.py:437-443: flat write slots for ``counts[b]`` tokens from ``starts[b]``."""
    out = []
    for bt, s, n in zip(block_tables, starts, counts):
        out.extend(slot_of(bt, s + t, page_size) for t in range(n))
    return np.asarray(out, np.int64)
