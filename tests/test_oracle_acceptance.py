"""Pins oracle/acceptance.py by known answers, brute force and the
speculative-sampling theorem (emitted tokens are distributed as p_target)."""
import numpy as np
import pytest

import oracle.acceptance as acc
from oracle.acceptance import accept_request, spec_accept


def _log(p):
    return np.log(np.asarray(p, np.float64))


def test_greedy_all_match_emits_bonus():
    t = np.zeros((4, 6)); t[0, 2] = t[1, 5] = t[2, 0] = 1; t[3, 4] = 2
    out, _ = accept_request(t, None, np.array([2, 5, 0]), np.zeros(4), 0.0)
    assert out == [2, 5, 0, 4]


def test_greedy_first_mismatch():
    t = np.zeros((4, 6)); t[0, 2] = t[1, 5] = t[2, 0] = 1; t[3, 4] = 2
    out, _ = accept_request(t, None, np.array([2, 1, 0]), np.zeros(4), 0.0)
    assert out == [2, 5]
    out, _ = accept_request(t, None, np.array([3, 5, 0]), np.zeros(4), 0.0)
    assert out == [2]


def test_greedy_ties_take_lowest_index():
    t = np.zeros((3, 7))  # all-equal logits -> argmax 0
    out, _ = accept_request(t, None, np.array([0, 0]), np.zeros(3), 0.0)
    assert out == [0, 0, 0]
    t[1, [3, 5]] = 1.0  # tie between 3 and 5 -> 3
    out, _ = accept_request(t, None, np.array([0, 5]), np.zeros(3), 0.0)
    assert out == [0, 3]


def test_stochastic_known_answers_v3():
    tl = np.stack([_log([0.5, 0.3, 0.2]), _log([0.1, 0.6, 0.3])])
    dl = _log([[0.2, 0.3, 0.5]])
    # ratio p_t/p_d = 0.2/0.5 = 0.4
    assert accept_request(tl, dl, np.array([2]), np.array([0.39, 0.65]), 1.0)[0] == [2, 1]
    assert accept_request(tl, dl, np.array([2]), np.array([0.39, 0.05]), 1.0)[0] == [2, 0]
    # rejected: residual max(0, pt - pd) = [0.3, 0, 0] -> token 0 for any u
    for u1 in (0.0, 0.5, 0.999):
        assert accept_request(tl, dl, np.array([2]), np.array([0.41, u1]), 1.0)[0] == [0]
    tl = np.stack([_log([0.4, 0.4, 0.2]), _log([1 / 3] * 3)])
    dl = _log([[0.1, 0.2, 0.7]])
    # residual [0.3, 0.2, 0] / 0.5 -> cdf [0.6, 1.0]
    assert accept_request(tl, dl, np.array([2]), np.array([0.5, 0.59]), 1.0)[0] == [0]
    assert accept_request(tl, dl, np.array([2]), np.array([0.5, 0.61]), 1.0)[0] == [1]


def test_temperature_divides_logits():
    # T = 0.5 squares the probabilities (before renormalising)
    tl = np.stack([_log([0.6, 0.4]), _log([0.5, 0.5])])
    dl = _log([[0.4, 0.6]])
    # p_t(T) = [.36,.16]/.52 ; p_d(T) = [.16,.36]/.52 ; ratio for token 1 = .16/.36
    thr = 0.16 / 0.36
    assert accept_request(tl, dl, np.array([1]), np.array([thr - 1e-3, 0.0]), 0.5)[0][0] == 1
    assert accept_request(tl, dl, np.array([1]), np.array([thr + 1e-3, 0.0]), 0.5)[0] == [0]


def test_zero_draft_probability_accepts():
    tl = np.stack([_log([0.5, 0.5]), _log([0.5, 0.5])])
    dl = np.array([[0.0, -1e4]])
    assert accept_request(tl, dl, np.array([1]), np.array([0.999, 0.0]), 1.0)[0] == [1, 0]


def test_equal_distributions_always_accept():
    rng = np.random.default_rng(0)
    l = rng.normal(size=(3, 50))
    u = rng.random((200, 3))
    for uu in u:
        out, _ = accept_request(l, l[:2], np.array([7, 9]), uu, 0.8)
        assert out[:2] == [7, 9] and len(out) == 3


def test_rollback_slots():
    P = 4
    kv_indices = np.array([10, 3, 7], np.int32)
    kv_indptr = np.array([0, 3], np.int32)
    # k = 4, start 5: verify positions 5..9; n = 2 emitted -> rejected 7, 8, 9
    assert acc.rollback_slots(2, 4, 5, kv_indices, kv_indptr, 0, P) == [3 * 4 + 3, 7 * 4 + 0, 7 * 4 + 1]
    assert acc.rollback_slots(5, 4, 5, kv_indices, kv_indptr, 0, P) == []


def _emit_histogram(pt, pd, n, seed):
    """First emitted token over n draws with k = 1 and the draft token drawn
    from p_d by inverse CDF."""
    rng = np.random.default_rng(seed)
    V = len(pt)
    tl = np.stack([np.log(pt), np.log(pt)])
    dl = np.log(pd)[None]
    cd = np.cumsum(pd)
    hist = np.zeros(V)
    for _ in range(n):
        x = min(int(np.searchsorted(cd, rng.random() * cd[-1], side="right")), V - 1)
        out, _ = accept_request(tl, dl, np.array([x]), rng.random(2), 1.0)
        hist[out[0]] += 1
    return hist


def _chi2_pvalue(hist, p):
    from scipy.stats import chisquare
    return chisquare(hist, p * hist.sum()).pvalue


def test_emitted_distribution_is_target():
    pt = np.array([0.35, 0.05, 0.3, 0.1, 0.2])
    pd = np.array([0.1, 0.4, 0.1, 0.3, 0.1])
    assert _chi2_pvalue(_emit_histogram(pt, pd, 20000, 1), pt) > 1e-3


def test_planted_residual_error_fails_theorem(monkeypatch):
    pt = np.array([0.35, 0.05, 0.3, 0.1, 0.2])
    pd = np.array([0.1, 0.4, 0.1, 0.3, 0.1])
    # a plausible mistake: resample from p_t instead of the residual
    monkeypatch.setattr(acc, "residual_weights", lambda a, b: a)
    assert _chi2_pvalue(_emit_histogram(pt, pd, 20000, 1), pt) < 1e-6


def test_batched_matches_per_request():
    rng = np.random.default_rng(3)
    B, k, V = 5, 4, 40
    dl = 2 * rng.standard_normal((B, k, V))
    tl = np.concatenate([dl + 0.5 * rng.standard_normal((B, k, V)),
                         2 * rng.standard_normal((B, 1, V))], axis=1)
    dt = rng.integers(0, V, (B, k))
    u = rng.random((B, k + 1)).astype(np.float32)
    res = spec_accept(tl, dl, dt, u, 0.8)
    for b in range(B):
        out, _ = accept_request(tl[b], dl[b], dt[b], u[b], 0.8)
        assert res["num_emitted"][b] == len(out)
        assert res["emitted"][b, :len(out)].tolist() == out
        assert (res["emitted"][b, len(out):] == -1).all()


def test_greedy_batched_needs_no_uniforms():
    t = np.zeros((2, 3, 5)); t[:, :, 1] = 1
    res = spec_accept(t, None, np.array([[1, 1], [1, 2]]), None, 0.0)
    assert res["num_emitted"].tolist() == [3, 2]
