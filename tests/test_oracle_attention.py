"""Pins oracle/verify_attention.py.

* brute-force scalar loops on tiny shapes (independent code path);
* torch SDPA with the explicit bottom-right mask, the library routine the
  reference's own packed fallback calls (nano_sglang/model/causal_lm.py:392-415);
* invariants: page permutation, L < P, L % P == 0, q_len = 1 decode,
  uniform keys -> mean of the visible values;
* a planted page swap in the oracle input must be caught by the comparison.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.verify_attention import verify_attention, verify_attention_bruteforce
from tests._attn_cases import make_batch


def _run(c, **kw):
    return verify_attention(c["q"], c["k"], c["v"], c["qo_indptr"], c["kv_indptr"],
                            c["kv_indices"], c["kv_last_page_len"], **kw)


@pytest.mark.parametrize("causal", [True, False])
def test_matches_bruteforce_tiny(causal):
    c = make_batch(1, q_lens=[3, 1, 2], kv_lens=[5, 19, 16], Hq=4, Hkv=2, D=8, P=4)
    a = _run(c, causal=causal)
    b = verify_attention_bruteforce(c["q"], c["k"], c["v"], c["qo_indptr"], c["kv_indptr"],
                                    c["kv_indices"], c["kv_last_page_len"], causal=causal)
    np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-12)


def test_matches_torch_sdpa_bottom_right():
    c = make_batch(2, q_lens=[5] * 4, kv_lens=[100, 17, 64, 301], Hq=14, Hkv=2, D=64)
    out = _run(c)
    P = 16
    for b in range(4):
        q0, q1 = c["qo_indptr"][b], c["qo_indptr"][b + 1]
        pages = c["kv_indices"][c["kv_indptr"][b]:c["kv_indptr"][b + 1]]
        L = (len(pages) - 1) * P + c["kv_last_page_len"][b]
        kb = torch.from_numpy(c["k"][pages].reshape(-1, 2, 64)[:L]).double()
        vb = torch.from_numpy(c["v"][pages].reshape(-1, 2, 64)[:L]).double()
        qb = torch.from_numpy(c["q"][q0:q1]).double()
        ql = q1 - q0
        row = torch.arange(ql)[:, None]
        col = torch.arange(L)[None, :]
        mask = torch.where(col <= (L - ql) + row, 0.0, float("-inf")).double()
        ref = F.scaled_dot_product_attention(
            qb.transpose(0, 1)[None], kb.transpose(0, 1)[None], vb.transpose(0, 1)[None],
            attn_mask=mask, scale=1 / 8.0, enable_gqa=True)[0].transpose(0, 1)
        np.testing.assert_allclose(out[q0:q1], ref.numpy(), rtol=1e-9, atol=1e-12)


def test_page_permutation_invariance():
    c = make_batch(3, q_lens=[5, 5], kv_lens=[70, 33], Hq=8, Hkv=2, D=16)
    a = _run(c)
    N = c["k"].shape[0]
    perm = np.random.default_rng(9).permutation(N)   # new physical location of page p
    k2 = np.empty_like(c["k"]); v2 = np.empty_like(c["v"])
    k2[perm] = c["k"]; v2[perm] = c["v"]
    c2 = dict(c, k=k2, v=v2, kv_indices=perm[c["kv_indices"]].astype(np.int32))
    np.testing.assert_allclose(_run(c2), a, rtol=0, atol=0)


def test_planted_page_swap_is_caught():
    c = make_batch(4, q_lens=[5], kv_lens=[64], Hq=4, Hkv=1, D=16)
    a = _run(c)
    bad = c["kv_indices"].copy()
    bad[[0, 3]] = bad[[3, 0]]          # moves keys across the causal boundary
    b = _run(dict(c, kv_indices=bad))
    assert np.abs(a - b).max() > 2e-3
    unused = sorted(set(range(c["k"].shape[0])) - set(c["kv_indices"].tolist()))
    bad = c["kv_indices"].copy()
    bad[1] = unused[0]                 # one page replaced by a foreign page
    b = _run(dict(c, kv_indices=bad))
    assert np.abs(a - b).max() > 2e-3


def test_q_len_one_is_full_decode():
    c = make_batch(5, q_lens=[1, 1], kv_lens=[9, 40], Hq=4, Hkv=2, D=8)
    np.testing.assert_allclose(_run(c, causal=True), _run(c, causal=False), rtol=0, atol=0)


def test_uniform_keys_average_visible_values():
    c = make_batch(6, q_lens=[3], kv_lens=[10], Hq=2, Hkv=1, D=4, P=4)
    c["k"][:] = 0.25  # every score equal -> softmax uniform over visible columns
    out = _run(c)
    pages = c["kv_indices"]
    vv = c["v"][pages].reshape(-1, 1, 4)[:10, 0]
    for r in range(3):
        vis = 10 - 3 + r + 1
        np.testing.assert_allclose(out[r, 0], vv[:vis].astype(np.float64).mean(0), rtol=1e-12)


def test_partial_and_full_last_page():
    for L in (7, 16, 32):
        c = make_batch(7, q_lens=[1], kv_lens=[L], Hq=2, Hkv=1, D=8)
        assert int(c["kv_last_page_len"][0]) == (L % 16 or 16)
        a = _run(c)
        b = verify_attention_bruteforce(c["q"], c["k"], c["v"], c["qo_indptr"], c["kv_indptr"],
                                        c["kv_indices"], c["kv_last_page_len"])
        np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-12)
