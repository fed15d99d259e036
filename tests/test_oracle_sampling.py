"""Pins the sampling oracle (oracle/sampling.py) to the reference's rules
(nano_sglang/engine/sampling.py:25-50, 71-88) on the CPU."""
import numpy as np
import pytest
import torch

from oracle import sampling as osm


def _f32(v):
    return np.asarray(v, np.float32)


def test_hand_worked_masks():
    # logits [2, 1, 1, 0, -1] at T = 1: p ~ [.5206, .1915, .1915, .0705, .0259];
    # descending order with the tie in index order: 0, 1, 2, 3, 4;
    # exclusive cumulatives: 0, .5206, .7121, .9036, .9741
    x = _f32([2, 1, 1, 0, -1])
    m, _ = osm.kept_mask(x, 1.0, 0, 0.6)
    assert m.tolist() == [True, True, False, False, False]     # the tie group is split
    m, _ = osm.kept_mask(x, 1.0, 0, 0.8)
    assert m.tolist() == [True, True, True, False, False]
    m, _ = osm.kept_mask(x, 1.0, 2, 1.0)                       # 2nd largest is 1: ties kept
    assert m.tolist() == [True, True, True, False, False]
    m, _ = osm.kept_mask(x, 1.0, 4, 1.0)
    assert m.tolist() == [True, True, True, True, False]
    # top-k then top-p on the renormalised survivors: p' ~ [.5761, .2119, .2119]
    m, _ = osm.kept_mask(x, 1.0, 2, 0.6)
    assert m.tolist() == [True, True, False, False, False]
    m, _ = osm.kept_mask(x, 1.0, 2, 0.57)
    assert m.tolist() == [True, False, False, False, False]
    # temperature sharpens: T = 0.5 -> p ~ [.7658, .1036, .1036, .0140, .0019]
    m, _ = osm.kept_mask(x, 0.5, 0, 0.8)
    assert m.tolist() == [True, True, False, False, False]
    # no filter keeps everything; top_k >= V is off
    assert osm.kept_mask(x, 1.0, 0, 1.0)[0].all() and osm.kept_mask(x, 1.0, 9, 1.0)[0].all()


def _reference_mask_f64(logits, T, top_k, top_p):
    """The reference's mask expressions (sampling.py:75-85) in float64 torch."""
    lg = torch.from_numpy(logits.astype(np.float64))[None] / T
    if top_k > 0:
        kth = torch.topk(lg, min(top_k, lg.size(-1)), dim=-1).values[:, -1:]
        lg = lg.masked_fill(lg < kth, float("-inf"))
    if top_p < 1.0:
        sl, si = torch.sort(lg, descending=True, dim=-1, stable=True)
        cp = torch.cumsum(torch.softmax(sl, -1), -1)
        mask = cp - torch.softmax(sl, -1) >= top_p
        sl[mask] = float("-inf")
        lg = sl.scatter(1, si, sl)
    return torch.isfinite(lg[0]).numpy()


@pytest.mark.parametrize("seed", range(6))
def test_masks_agree_with_the_reference_expressions(seed):
    rng = np.random.default_rng(seed)
    V = int(rng.integers(50, 3000))
    x = (rng.standard_normal(V) * rng.choice([0.5, 2.0, 6.0])).astype(np.float32)
    checked = 0
    for T in (0.7, 1.0, 1.6):
        for top_k, top_p in ((0, 0.9), (0, 0.5), (20, 1.0), (200, 0.95), (7, 0.3), (1, 1.0)):
            mine, margin = osm.kept_mask(x, T, top_k, top_p)
            if margin < 1e-5:
                continue
            np.testing.assert_array_equal(mine, _reference_mask_f64(x, T, top_k, top_p))
            checked += 1
    assert checked >= 12


def test_degenerate_filters_reduce_to_argmax():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(1000) * 3).astype(np.float32)
    x[417] = x.max() + 1
    for u in (0.0, 0.3, 0.999):
        assert osm.sample(x, 1.0, 1, 1.0, u)[0] == 417
        assert osm.sample(x, 1.0, 0, 1e-7, u)[0] == 417
    # ties at the max: top_k = 1 keeps all of them, a tiny top_p only the first
    x[[12, 417, 900]] = x.max()
    assert osm.kept_mask(x, 1.0, 1, 1.0)[0].nonzero()[0].tolist() == [12, 417, 900]
    assert osm.kept_mask(x, 1.0, 0, 1e-7)[0].nonzero()[0].tolist() == [12]
    assert osm.sample(x, 0.0, 0, 1.0, 0.5)[0] == 12             # greedy: first max index


def test_inverse_cdf_frequencies_follow_the_kept_weights():
    x = _f32([0.3, 1.2, -0.5, 1.2, 0.0, 2.0, -3.0, 0.9])
    for top_k, top_p in ((0, 1.0), (3, 1.0), (0, 0.7), (5, 0.9)):
        kept, _ = osm.kept_mask(x, 0.8, top_k, top_p)
        W = osm.fixed_weights(x, 0.8).astype(np.float64) * kept
        n = 8000
        counts = np.zeros(len(x))
        for i in range(n):
            counts[osm.sample(x, 0.8, top_k, top_p, (i + 0.5) / n)[0]] += 1
        np.testing.assert_allclose(counts / n, W / W.sum(), atol=2e-4)
        assert (counts[~kept] == 0).all()


def test_bf16_bits_and_keys():
    v = torch.tensor([-1.5, -0.0, 0.0, 2.0, -3.0e38, 1e-3]).bfloat16()
    bits = v.view(torch.int16).numpy().view(np.uint16)
    k = osm.order_keys(bits)
    assert k[1] == k[2]                                        # -0 == +0
    assert np.argsort(k, kind="stable").tolist() == [4, 0, 1, 2, 5, 3]
    np.testing.assert_array_equal(osm.values_f32(bits), v.float().numpy())
