"""Temperature / top-k / top-p sampling (oracle side).

TEST INFRASTRUCTURE ONLY (see the package docstring).

Restates nano_sglang/engine/sampling.py:25-50 (``sample_token``: argmax when
T < 1e-6) and :71-88 (``_sample_pytorch``), in the exact arithmetic the HIP
sampler evaluates:

* logits / T; top-k keeps every logit >= the k-th largest (:75-78, ties kept);
* top-p (:80-85): tokens in descending-logit order, ``p = softmax``; sorted
  position i is dropped when its exclusive cumulative ``sum_{j<i} p_j >=
  top_p``; among equal logits the lower vocabulary index comes first (torch's
  sort leaves that order unspecified);
* the draw (:87-88, ``multinomial``) is an inverse CDF in vocabulary order
  with a supplied uniform.

Weights are ``w = 2^(fma(x, c, -max*c))`` with ``c = f32(log2(e) / T)``, held
in 2^-40 fixed point (uint64), so all masses are exact integer sums; the
top-p comparison is ``(double)prefix < f64(top_p) * (double)Z_k``; the draw
takes the first index whose inclusive kept prefix exceeds
``floor(u * (double)Z_kept)``.  The one inexact step is ``exp2`` (the GPU's
``v_exp_f32`` may differ by an ulp), so GPU parity is exact except where a
decision lies within that rounding of a boundary -- ``sample`` returns the
relative margin for that test.

Pinning (tests/test_oracle_sampling.py): hand-worked examples of the
reference's masks (ties at the top-k threshold kept, a tie group split by
the top-p boundary); the reference's mask expressions evaluated in float64 by
torch on random logits; top_k = 1 / tiny top_p reduce to argmax; the
inverse CDF's token frequencies over a uniform grid follow the kept weights.
"""

from __future__ import annotations

import numpy as np

LOG2E_F32 = np.float32(1.4426950408889634)
FIX = float(2 ** 40)


def order_keys(x: np.ndarray) -> np.ndarray:
    """Order-preserving unsigned keys of bf16 (uint16 bits) or fp32 values
    (-0 == +0), as the kernel's radix selection uses."""
    x = np.asarray(x)
    if x.dtype == np.float32:
        b = x.view(np.uint32).astype(np.uint64)
        b = np.where(b == 0x80000000, 0, b)
        return np.where(b & 0x80000000, ~b & 0xFFFFFFFF, b | 0x80000000).astype(np.int64)
    if x.dtype == np.uint16:      # bf16 bits
        b = x.astype(np.uint32)
        b = np.where(b == 0x8000, 0, b)
        return np.where(b & 0x8000, ~b & 0xFFFF, b | 0x8000).astype(np.int64)
    raise TypeError("fp32 values or bf16 bits (uint16)")


def values_f32(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x)
    if x.dtype == np.uint16:
        return (x.astype(np.uint32) << 16).view(np.float32)
    return x.astype(np.float32)


def fixed_weights(x: np.ndarray, temperature: float) -> np.ndarray:
    """2^-40 fixed-point weights 2^(fma(x, c, -max*c)), uint64."""
    v = values_f32(x)
    c = np.float32(LOG2E_F32 / np.float32(temperature))
    M = v[np.argmax(order_keys(x))]
    mc = np.float32(M * c)
    t = (v.astype(np.float64) * np.float64(c) - np.float64(mc)).astype(np.float32)
    w = np.exp2(t.astype(np.float64)).astype(np.float32)
    return np.floor(w.astype(np.float64) * FIX).astype(np.uint64)


def kept_mask(x: np.ndarray, temperature: float, top_k: int = 0, top_p: float = 1.0,
              W: np.ndarray | None = None):
    """Tokens the reference's filters keep (sampling.py:75-85).

    Returns (mask, margin): margin = the smallest relative distance of a
    top-p exclusive prefix from top_p * Z_k (inf without top-p)."""
    keys = order_keys(x)
    V = keys.shape[0]
    W = fixed_weights(x, temperature) if W is None else W
    order = np.lexsort((np.arange(V), -keys))          # descending key, ascending index
    kept = np.ones(V, bool)
    if 0 < top_k < V:
        kept &= keys >= keys[order[top_k - 1]]
    margin = np.inf
    p = np.float64(np.float32(top_p))
    if p < 1.0:
        ordk = order[kept[order]]
        Wk = W[ordk]
        zk = float(int(Wk.sum(dtype=np.uint64)))
        pz = p * zk
        excl = np.concatenate([[0], np.cumsum(Wk, dtype=np.uint64)[:-1]]).astype(np.float64)
        keep = excl < pz
        kept = np.zeros(V, bool)
        kept[ordk[keep]] = True
        margin = float(np.min(np.abs(excl - pz)) / zk)
    return kept, margin


def sample(x: np.ndarray, temperature: float, top_k: int, top_p: float, u: float):
    """One draw (sampling.py:25-50, 71-88).  Returns (token, margin): margin is
    the smallest relative distance of a decision from its boundary."""
    keys = order_keys(x)
    if temperature < 1e-6:
        return int(np.argmax(keys)), np.inf             # first index of the max
    W = fixed_weights(x, temperature)
    kept, m_p = kept_mask(x, temperature, top_k, top_p, W)
    Wk = np.where(kept, W, np.uint64(0))
    incl = np.cumsum(Wk, dtype=np.uint64)
    Z = int(incl[-1])
    if Z == 0:
        return -1, np.inf
    target = int(np.float64(np.float32(u)) * float(Z))
    if target >= Z:
        target = Z - 1
    tok = int(np.searchsorted(incl, np.uint64(target), side="right"))
    excl = int(incl[tok]) - int(Wk[tok])
    m_draw = min(target - excl, int(incl[tok]) - 1 - target) / Z
    return tok, min(m_p, m_draw)
