"""Seeded synthetic inputs for the verify-step workloads (host side, numpy).

* :func:`verify_attention_batch` -- paged verify attention: B requests with
  q_len query tokens each, KV lengths uniform in [min_len, max_len] (the q_len
  verify positions included), pages drawn as a seeded permutation of a pool
  that is filled with noise, Q ~ N(0,1), K, V ~ kv_scale * N(0,1), bf16.
  Defaults: batch 32, 5 query tokens (k = 4 drafts + bonus), 14 q / 2 kv
  heads, head dim 64, page size 16, lengths 100..640, 8000-page pool.
* :func:`acceptance_batch` -- fused acceptance: draft logits 2 * N(0,1),
  target rows 0..k-1 = draft + 0.5 * N(0,1), target row k = 2 * N + 0.5 * N,
  all rounded to bf16; draft tokens sampled from softmax(draft / T).
  Defaults: batch 64, k = 4, vocab 151936, T = 0.8.

Values are rounded to bf16 and returned as float32 numpy arrays (exactly
representable in bf16), plus int32 page-table arrays in the CSR layout of
nano_sglang/engine/engine.py:419-448.
"""

from __future__ import annotations

import numpy as np


def _bf16_round(x: np.ndarray) -> np.ndarray:
    """Round finite float32 to the nearest bf16 (ties to even), returned as
    float32.  In uint32 arithmetic: a finite float's bits are at most
    0xFF7FFFFF, so adding at most 0x8000 cannot wrap."""
    u = np.array(x, dtype=np.float32, copy=True).view(np.uint32)
    r = (u >> 16) & np.uint32(1)
    r += np.uint32(0x7FFF)
    u += r
    u &= np.uint32(0xFFFF0000)
    return u.view(np.float32)


def verify_attention_batch(batch=32, q_len=5, num_qo_heads=14, num_kv_heads=2, head_dim=64,
                           page_size=16, min_len=100, max_len=640, num_pages=8000,
                           kv_scale=0.5, seed=0, kv_lens=None, q_lens=None):
    rng = np.random.default_rng(seed)
    if kv_lens is None:
        kv_lens = rng.integers(min_len, max_len + 1, size=batch)
    kv_lens = np.asarray(kv_lens, np.int64)
    if q_lens is None:
        q_lens = np.full(batch, q_len, np.int64)
    q_lens = np.asarray(q_lens, np.int64)
    need = (kv_lens + page_size - 1) // page_size
    if need.sum() > num_pages:
        raise ValueError(f"{need.sum()} pages needed, pool has {num_pages}")
    perm = rng.permutation(num_pages).astype(np.int32)
    kv_indices = perm[:need.sum()].copy()
    kv_indptr = np.zeros(batch + 1, np.int32)
    kv_indptr[1:] = np.cumsum(need)
    qo_indptr = np.zeros(batch + 1, np.int32)
    qo_indptr[1:] = np.cumsum(q_lens)
    last = np.where(kv_lens % page_size == 0, page_size, kv_lens % page_size).astype(np.int32)
    q = _bf16_round(rng.standard_normal((int(qo_indptr[-1]), num_qo_heads, head_dim),
                                        dtype=np.float32))
    shape = (num_pages, page_size, num_kv_heads, head_dim)
    k = _bf16_round(kv_scale * rng.standard_normal(shape, dtype=np.float32))
    v = _bf16_round(kv_scale * rng.standard_normal(shape, dtype=np.float32))
    return dict(q=q, k=k, v=v, qo_indptr=qo_indptr, kv_indptr=kv_indptr, kv_indices=kv_indices,
                kv_last_page_len=last, kv_lens=kv_lens, q_lens=q_lens, page_size=page_size,
                sm_scale=1.0 / np.sqrt(head_dim))


def acceptance_batch(batch=64, k=4, vocab=151936, temperature=0.8, seed=0):
    rng = np.random.default_rng(seed)
    draft = _bf16_round(2.0 * rng.standard_normal((batch, k, vocab), dtype=np.float32))
    target = np.empty((batch, k + 1, vocab), np.float32)
    target[:, :k] = draft + 0.5 * rng.standard_normal((batch, k, vocab), dtype=np.float32)
    target[:, k] = 2.0 * rng.standard_normal((batch, vocab), dtype=np.float32) \
        + 0.5 * rng.standard_normal((batch, vocab), dtype=np.float32)
    target = _bf16_round(target)
    tokens = np.empty((batch, k), np.int64)
    u = rng.random((batch, k))
    for b in range(batch):
        for i in range(k):
            x = draft[b, i].astype(np.float64) / temperature
            p = np.exp(x - x.max())
            c = np.cumsum(p)
            tokens[b, i] = min(int(np.searchsorted(c, u[b, i] * c[-1], side="right")), vocab - 1)
    return dict(target=target, draft=draft, draft_tokens=tokens, temperature=temperature)


def acceptance_page_table(batch=64, k=4, page_size=16, num_pages=8000, min_len=100,
                          max_len=640, seed=0):
    """Page table of an acceptance call: request b's verify window sits at
    positions start_b .. start_b + k (start_b = L_b - k - 1 with L_b uniform in
    [min_len, max_len], the verify-attention workload's KV lengths), on pages
    drawn as a seeded permutation of the pool.  Returns (start_pos int32 [B],
    kv_indptr int32 [B+1], kv_indices int32) for the rollback slots."""
    rng = np.random.default_rng(seed)
    L = rng.integers(max(min_len, k + 1), max_len + 1, size=batch)
    start = (L - k - 1).astype(np.int32)
    need = (L + page_size - 1) // page_size
    if need.sum() > num_pages:
        raise ValueError(f"{need.sum()} pages needed, pool has {num_pages}")
    indptr = np.zeros(batch + 1, np.int32)
    indptr[1:] = np.cumsum(need)
    indices = rng.permutation(num_pages).astype(np.int32)[:indptr[-1]].copy()
    return start, indptr, indices


def algorithmic_bytes_verify_attention(kv_lens, q_total, num_qo_heads, num_kv_heads, head_dim,
                                       batch, num_pages_listed, elem=2):
    """KV bytes (every visible K and V row once) + Q in + O out + page-table ints."""
    kv = int(np.sum(kv_lens)) * num_kv_heads * head_dim * 2 * elem
    qo = 2 * int(q_total) * num_qo_heads * head_dim * elem
    meta = 4 * (int(num_pages_listed) + 2 * (batch + 1) + batch)
    return kv + qo + meta


def algorithmic_bytes_acceptance(batch, k, vocab, greedy, elem=2):
    rows = batch * (k + 1) + (0 if greedy else batch * k)
    return rows * vocab * elem
