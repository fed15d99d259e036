"""Acceptance / rejection sampling, residual resample, bonus token and
KV-slot rollback for one verify step (oracle side).

Restates nano_sglang/decode/speculative.py:130-196 with the three parity
decisions the verify step is built to (each one differs from the literal
reference code on purpose, for the reason given):

1. Greedy (``temperature < 1e-6``, the reference's greedy test in
   nano_sglang/engine/sampling.py:44) uses the T->0 limit of the ratio test:
   draft token ``d_i`` is accepted iff it equals ``argmax(target row i)``
   (lowest index on ties, like ``torch.argmax``, sampling.py:45); the first
   mismatch emits that argmax; if all ``k`` match, the bonus is
   ``argmax(target row k)`` (speculative.py:174-182).  The reference's T=0
   path still draws ``torch.rand`` against T=1 softmaxes
   (speculative.py:91-92, 139, 150), which is not deterministic.
2. Stochastic: ``p = softmax(logits / T)`` in float64 here (speculative.py:90,
   135); accept ``d_i`` iff ``u_i < min(1, p_t(d_i) / p_d(d_i))`` with strict
   ``<`` (speculative.py:145-151) and ``p_d(d_i) == 0 -> accept``
   (speculative.py:147-148); stop at the first rejection (speculative.py:172).
3. On rejection at position ``i`` the token is drawn from the textbook
   residual ``max(0, p_t - p_d) / sum`` (Leviathan et al. 2023, Alg. 1; Chen
   et al. 2023) by inverse CDF with the supplied uniform ``u_k``; if the sum
   is 0 it falls back to sampling ``p_t`` (mirrors speculative.py:163-169).
   The reference's own expression at speculative.py:156-158 is identically
   zero for T > 0 and so always takes that fallback.

Inverse CDF: the token is the smallest ``j`` with ``cumsum(w)[j] > u * sum(w)``;
if rounding leaves no such ``j``, the last ``j`` with ``w_j > 0``.

Rollback (the reference's ``reset_draft_cache`` is a no-op,
speculative.py:186-196): the verify forward wrote KV for positions
``start .. start+k``; after emitting ``n`` tokens the positions
``start+n .. start+k`` (``k+1-n`` of them) hold rejected tokens.  Their flat
slots are ``kv_indices[kv_indptr[b] + pos // P] * P + pos % P``
(nano_sglang/engine/engine.py:438-443).

Pinning: hand-worked known-answer cases (all-match, first mismatch,
all-equal logits -> index 0, V=3/V=4 stochastic cases with closed-form
probabilities), brute-force enumeration on tiny V, and the speculative-
sampling theorem (the emitted-token distribution equals ``p_t``) by a
chi-square test over many uniforms -- see tests/test_oracle_acceptance.py.
"""

from __future__ import annotations

import numpy as np

GREEDY_EPS = 1e-6  # nano_sglang/engine/sampling.py:44


def softmax64(logits: np.ndarray, temperature: float) -> np.ndarray:
    x = np.asarray(logits, np.float64) / float(temperature)
    x = x - x.max(axis=-1, keepdims=True)
    e = np.exp(x)
    return e / e.sum(axis=-1, keepdims=True)


def residual_weights(pt: np.ndarray, pd: np.ndarray) -> np.ndarray:
    """Unnormalised residual max(0, p_t - p_d); p_t itself when that is all 0
    (the fallback of speculative.py:163-169)."""
    r = np.maximum(0.0, pt - pd)
    return r if r.sum() > 0 else pt


def inverse_cdf(w: np.ndarray, u: float) -> tuple[int, float]:
    """Smallest j with cumsum(w)[j] > u*sum(w).  Returns (j, margin) where
    margin is the distance of u*sum(w) from the nearest boundary of the chosen
    bucket, relative to sum(w)."""
    c = np.cumsum(w)
    s = c[-1]
    target = u * s
    j = int(np.searchsorted(c, target, side="right"))
    if j >= len(w):
        nz = np.nonzero(w > 0)[0]
        j = int(nz[-1])
    lo = c[j - 1] if j > 0 else 0.0
    margin = min(abs(target - lo), abs(c[j] - target)) / s if s > 0 else np.inf
    return j, float(margin)


def accept_request(target_logits: np.ndarray, draft_logits: np.ndarray | None,
                   draft_tokens: np.ndarray, uniforms: np.ndarray, temperature: float):
    """One request.  target_logits (k+1, V); draft_logits (k, V) or None (greedy);
    draft_tokens (k,); uniforms (k+1,).  Returns (emitted list, margin) where
    margin is the smallest decision margin (|min(1,ratio) - u| for every ratio
    test made, and the inverse-CDF margin for the sampled token); inf for greedy.
    """
    k = len(draft_tokens)
    greedy = temperature < GREEDY_EPS
    if greedy:
        a = np.argmax(np.asarray(target_logits, np.float64), axis=-1)  # first max index
        out = []
        for i in range(k):
            if int(draft_tokens[i]) == int(a[i]):
                out.append(int(draft_tokens[i]))
            else:
                out.append(int(a[i]))
                return out, np.inf
        out.append(int(a[k]))
        return out, np.inf

    margin = np.inf
    out = []
    for i in range(k):
        pt = softmax64(target_logits[i], temperature)
        pd = softmax64(draft_logits[i], temperature)
        x = int(draft_tokens[i])
        u = float(uniforms[i])
        if pd[x] > 0:
            thr = min(1.0, pt[x] / pd[x])
            margin = min(margin, abs(thr - u))
            acc = u < thr
        else:
            acc = True
        if acc:
            out.append(x)
            continue
        w = residual_weights(pt, pd)
        tok, m2 = inverse_cdf(w, float(uniforms[k]))
        out.append(tok)
        return out, min(margin, m2)
    pt = softmax64(target_logits[k], temperature)
    tok, m2 = inverse_cdf(pt, float(uniforms[k]))
    out.append(tok)
    return out, min(margin, m2)


def rollback_slots(num_emitted: int, k: int, start_pos: int, kv_indices: np.ndarray,
                   kv_indptr: np.ndarray, b: int, page_size: int) -> list[int]:
    """Slots of the rejected verify positions start+n .. start+k."""
    slots = []
    for pos in range(start_pos + num_emitted, start_pos + k + 1):
        page = int(kv_indices[int(kv_indptr[b]) + pos // page_size])
        slots.append(page * page_size + pos % page_size)
    return slots


def spec_accept(target_logits, draft_logits, draft_tokens, uniforms, temperature,
                kv_indptr=None, kv_indices=None, start_pos=None, page_size=16):
    """Batched oracle.  Shapes: target (B, k+1, V), draft (B, k, V) or None,
    draft_tokens (B, k), uniforms (B, k+1).

    Returns dict with num_emitted int32 (B,), emitted int64 (B, k+1) padded
    -1, rollback int64 (B, k) padded -1 (all -1 without a page table), and
    margin float64 (B,).
    """
    target_logits = np.asarray(target_logits)
    B, k1, V = target_logits.shape
    k = k1 - 1
    n_out = np.zeros(B, np.int32)
    emitted = np.full((B, k + 1), -1, np.int64)
    rb = np.full((B, max(k, 1)), -1, np.int64)[:, :k]
    margin = np.full(B, np.inf)
    if uniforms is None:  # greedy needs none
        uniforms = np.zeros((B, k + 1), np.float32)
    for b in range(B):
        dl = None if draft_logits is None else np.asarray(draft_logits[b])
        out, m = accept_request(target_logits[b], dl, np.asarray(draft_tokens[b]),
                                np.asarray(uniforms[b]), temperature)
        n_out[b] = len(out)
        emitted[b, :len(out)] = out
        margin[b] = m
        if kv_indptr is not None:
            s = rollback_slots(len(out), k, int(start_pos[b]), kv_indices, kv_indptr, b, page_size)
            rb[b, :len(s)] = s
    return {"num_emitted": n_out, "emitted": emitted, "rollback": rb, "margin": margin}
