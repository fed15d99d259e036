"""Ragged multi-query paged attention (oracle side).

Semantics restated from the reference's own PyTorch fallbacks for the packed
path, which define what FlashInfer's ``BatchPrefillWithPagedKVCacheWrapper``
with ``causal=True`` computes at nano_sglang/model/causal_lm.py:340:

* per request, ``scores = q . k^T * sm_scale`` with ``sm_scale = 1/sqrt(D)``
  (causal_lm.py:374, 452);
* bottom-right causal mask: query row ``r`` of a request with ``q_len`` query
  tokens and ``L`` KV tokens sees columns ``c <= (L - q_len) + r``
  (causal_lm.py:403-412, 459-463); with ``causal=False`` it sees all ``L``;
* GQA: query head ``hq`` reads KV head ``hq // (Hq / Hkv)``
  (``repeat_interleave`` at causal_lm.py:443-445);
* softmax in fp32 or better (causal_lm.py:467), then ``P . V``.

KV comes from the NHD paged pool ``[num_pages, P, Hkv, D]`` through the CSR
page table (engine.py:419-448); the request's tokens are its pages in table
order, truncated to ``L = (pages - 1) * P + last_page_len``.

This restatement accumulates in float64 and does not round P to bf16; the
kernel's bf16 rounding of P is covered by the test tolerance.

Pinning: brute-force scalar loops on tiny shapes, ``torch.nn.functional.
scaled_dot_product_attention`` with the explicit bottom-right mask (the
library routine the reference itself calls, causal_lm.py:392-415), and
invariants (page permutation, L < P, L multiple of P, q_len = 1 decode,
uniform keys -> mean of visible values) -- see tests/test_oracle_attention.py.
"""

from __future__ import annotations

import numpy as np


def gather_request_kv(k_cache: np.ndarray, v_cache: np.ndarray, kv_indices: np.ndarray,
                      kv_indptr: np.ndarray, last_page_len: np.ndarray, b: int):
    """Contiguous (L, Hkv, D) K and V of request ``b`` (paged_kv_cache.py:139-162)."""
    P = k_cache.shape[1]
    pages = kv_indices[kv_indptr[b]:kv_indptr[b + 1]]
    if len(pages) == 0:
        return k_cache[:0, 0], v_cache[:0, 0]
    L = (len(pages) - 1) * P + int(last_page_len[b])
    k = k_cache[pages].reshape(len(pages) * P, *k_cache.shape[2:])[:L]
    v = v_cache[pages].reshape(len(pages) * P, *v_cache.shape[2:])[:L]
    return k, v


def verify_attention(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                     qo_indptr: np.ndarray, kv_indptr: np.ndarray, kv_indices: np.ndarray,
                     kv_last_page_len: np.ndarray, sm_scale: float | None = None,
                     causal: bool = True) -> np.ndarray:
    """q: (T, Hq, D); caches: (N, P, Hkv, D). Returns float64 (T, Hq, D)."""
    q = np.asarray(q, np.float64)
    T, Hq, D = q.shape
    Hkv = k_cache.shape[2]
    if Hq % Hkv:
        raise ValueError("num_qo_heads must be a multiple of num_kv_heads")
    G = Hq // Hkv
    scale = 1.0 / np.sqrt(D) if sm_scale is None else float(sm_scale)
    out = np.zeros((T, Hq, D), np.float64)
    B = len(qo_indptr) - 1
    for b in range(B):
        q0, q1 = int(qo_indptr[b]), int(qo_indptr[b + 1])
        ql = q1 - q0
        if ql == 0:
            continue
        kb, vb = gather_request_kv(k_cache, v_cache, kv_indices, kv_indptr, kv_last_page_len, b)
        kb = np.asarray(kb, np.float64)
        vb = np.asarray(vb, np.float64)
        L = kb.shape[0]
        if L < ql:
            raise ValueError(f"request {b}: kv length {L} < query length {ql}")
        kh = np.repeat(kb, G, axis=1).transpose(1, 0, 2)  # (Hq, L, D)
        vh = np.repeat(vb, G, axis=1).transpose(1, 0, 2)
        qh = q[q0:q1].transpose(1, 0, 2)                   # (Hq, ql, D)
        s = np.einsum("hqd,hkd->hqk", qh, kh) * scale
        if causal:
            row = np.arange(ql)[:, None]
            col = np.arange(L)[None, :]
            s = np.where(col <= (L - ql) + row, s, -np.inf)
        s = s - s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        out[q0:q1] = np.einsum("hqk,hkd->hqd", p, vh).transpose(1, 0, 2)
    return out


def verify_attention_bruteforce(q, k_cache, v_cache, qo_indptr, kv_indptr, kv_indices,
                                kv_last_page_len, sm_scale=None, causal=True):
    """Scalar-loop restatement for tiny shapes; walks pages token by token."""
    T, Hq, D = q.shape
    N, P, Hkv, _ = k_cache.shape
    G = Hq // Hkv
    scale = 1.0 / np.sqrt(D) if sm_scale is None else float(sm_scale)
    out = np.zeros((T, Hq, D))
    for b in range(len(qo_indptr) - 1):
        q0, q1 = int(qo_indptr[b]), int(qo_indptr[b + 1])
        ql = q1 - q0
        npg = int(kv_indptr[b + 1] - kv_indptr[b])
        L = (npg - 1) * P + int(kv_last_page_len[b]) if npg else 0
        toks = []
        for j in range(L):
            page = int(kv_indices[kv_indptr[b] + j // P])
            toks.append((page, j % P))
        for r in range(ql):
            for hq in range(Hq):
                h = hq // G
                lim = (L - ql) + r if causal else L - 1
                sc = []
                for j in range(L):
                    if j > lim:
                        continue
                    pg, sl = toks[j]
                    dot = 0.0
                    for d in range(D):
                        dot += float(q[q0 + r, hq, d]) * float(k_cache[pg, sl, h, d])
                    sc.append((j, dot * scale))
                m = max(x for _, x in sc)
                w = [(j, np.exp(x - m)) for j, x in sc]
                z = sum(x for _, x in w)
                for d in range(D):
                    acc = 0.0
                    for j, x in w:
                        pg, sl = toks[j]
                        acc += x * float(v_cache[pg, sl, h, d])
                    out[q0 + r, hq, d] = acc / z
    return out
