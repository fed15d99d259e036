"""Pins oracle/page_table.py by hand-worked cases and a brute-force walk."""
import numpy as np

from oracle.page_table import build_csr, kv_len_from_csr, slot_of, write_indices


def test_last_page_len_rule():
    indptr, idx, last = build_csr([[5], [7, 2], [9, 1, 4]], [3, 32, 33], 16)
    assert indptr.tolist() == [0, 1, 3, 6]
    assert idx.tolist() == [5, 7, 2, 9, 1, 4]
    assert last.tolist() == [3, 16, 1]  # L%P, or P when L%P == 0
    assert kv_len_from_csr(indptr, last, 16).tolist() == [3, 32, 33]


def test_extra_pages_are_not_listed():
    indptr, idx, _ = build_csr([[4, 8, 15]], [16], 16)
    assert idx.tolist() == [4]


def test_slots_bruteforce():
    rng = np.random.default_rng(0)
    P = 16
    bt = rng.permutation(100)[:7].tolist()
    for pos in range(7 * P):
        s = slot_of(bt, pos, P)
        assert s // P == bt[pos // P] and s % P == pos % P
    w = write_indices([bt, bt[::-1]], [3, 40], [5, 2], P)
    assert w.tolist() == [slot_of(bt, p, P) for p in range(3, 8)] + \
        [slot_of(bt[::-1], p, P) for p in (40, 41)]
