"""nsg_sample (temperature / top-k / top-p sampling) and the acceptance
kernel's bonus hand-off on the GPU, against the sampling oracle
(oracle/sampling.py; reference nano_sglang/engine/sampling.py:25-50, 71-88).

Bar: the same token as the oracle for every draw whose decisions (the top-p
boundary and the inverse-CDF draw) lie more than 1e-6 (relative mass) from a
boundary -- the one inexact step shared by both sides is exp2, whose last-ulp
differences move any mass by at most about 1.2e-7 relative."""
import numpy as np
import pytest
import torch

from nanosglang_amd import kernels
from oracle import sampling as osm

pytestmark = pytest.mark.gpu
MARGIN = 1e-6


def _rows(seed, R, V, kind):
    g = torch.Generator().manual_seed(seed)
    scale = {"narrow": 0.5, "normal": 2.0, "wide": 6.0, "ties": 2.0}[kind]
    x = torch.randn(R, V, generator=g) * scale
    if kind == "ties":
        x = torch.round(x * 4) / 4          # many equal logits around every threshold
    return x


def _oracle_rows(x, dtype):
    if dtype == torch.bfloat16:
        return x.bfloat16().view(torch.int16).numpy().view(np.uint16)
    return x.float().numpy()


def _check(x_dev, x_np, T, top_k, top_p, u):
    got = kernels.sample(x_dev, T, top_k, top_p, u.cuda() if u is not None else None).cpu()
    compared = 0
    for r in range(x_np.shape[0]):
        tok, margin = osm.sample(x_np[r], T, top_k, top_p, float(u[r]) if u is not None else 0.)
        if margin < MARGIN:
            continue
        assert int(got[r]) == tok, (r, T, top_k, top_p, int(got[r]), tok, margin)
        compared += 1
    return compared


CASES = [(1.0, 0, 1.0), (0.8, 0, 0.9), (1.0, 50, 1.0), (0.7, 40, 0.8), (1.3, 0, 0.3),
         (1.0, 1, 1.0), (0.6, 1000, 0.95), (1.0, 0, 1e-4)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("V,kind", [(151936, "normal"), (151936, "ties"), (4099, "wide"),
                                    (50257, "narrow"), (64, "ties")])
def test_sample_matches_oracle(dtype, V, kind):
    R = 12
    x = _rows(V + R, R, V, kind)
    x_dev = x.to(dtype).cuda()
    x_np = _oracle_rows(x, dtype)
    g = torch.Generator().manual_seed(V)
    total = 0
    for i, (T, top_k, top_p) in enumerate(CASES):
        u = torch.rand(R, generator=g)
        print(f"case: dtype {dtype} V {V} {kind} T {T} top_k {top_k} top_p {top_p}", flush=True)
        total += _check(x_dev, x_np, T, top_k, top_p, u)
    assert total >= 0.8 * R * len(CASES)


def test_sample_greedy_is_the_first_argmax():
    x = torch.randn(5, 1000)
    x[2, [10, 500, 999]] = 9.0
    x[4] = 0.0
    x[4, 7] = -0.0
    for dtype in (torch.bfloat16, torch.float32):
        got = kernels.sample(x.to(dtype).cuda(), 0.0).cpu()
        ref = [osm.sample(r, 0.0, 0, 1.0, 0.0)[0] for r in _oracle_rows(x, dtype)]
        assert got.tolist() == ref
        assert got[2] == 10 and got[4] == 0


@pytest.mark.parametrize("top_k,top_p", [(0, 0.9), (30, 1.0), (30, 0.6), (0, 0.2)])
def test_sample_uniform_grid_stays_in_the_kept_set(top_k, top_p):
    """One row, many uniforms: every token kept by the oracle's mask, and the
    same draws as the oracle."""
    V, R = 32000, 512
    x = _rows(7, 1, V, "ties")[0]
    x_np = _oracle_rows(x[None], torch.bfloat16)[0]
    kept, margin = osm.kept_mask(x_np, 0.9, top_k, top_p)
    assert margin > MARGIN
    xs = x.bfloat16().cuda()[None].expand(R, V).contiguous()
    u = (torch.arange(R, dtype=torch.float32) + 0.5) / R
    got = kernels.sample(xs, 0.9, top_k, top_p, u.cuda()).cpu().numpy()
    assert kept[got].all()
    ref = np.array([osm.sample(x_np, 0.9, top_k, top_p, float(v)) for v in u], dtype=object)
    ok = np.array([m >= MARGIN for _, m in ref])
    assert ok.mean() > 0.9
    np.testing.assert_array_equal(got[ok], np.array([t for t, _ in ref])[ok])


def test_sample_strided_rows_and_row_count_one():
    V = 5000
    x = _rows(3, 6, 3 * V, "normal").view(6, 3, V)
    base = x.bfloat16().cuda()
    view = base[:, 1, :]                            # row stride 3V, unaligned start
    u = torch.rand(6, generator=torch.Generator().manual_seed(1))
    x_np = _oracle_rows(x[:, 1, :].contiguous(), torch.bfloat16)
    assert _check(view, x_np, 0.9, 20, 0.9, u) >= 5
    one = kernels.sample(view[2:3], 0.9, 20, 0.9, u[2:3].cuda()).cpu()
    tok, m = osm.sample(x_np[2], 0.9, 20, 0.9, float(u[2]))
    if m >= MARGIN:
        assert int(one[0]) == tok


def test_sample_repeated_calls_are_identical():
    """The workspace needs no clearing: a second call (after a call of another
    shape through the same workspace) gives the same tokens."""
    x = _rows(11, 16, 151936, "normal").bfloat16().cuda()
    u = torch.rand(16, device="cuda")
    a = kernels.sample(x, 1.0, 50, 0.9, u)
    kernels.sample(x[:3, :1000], 0.5, 5, 0.5, u[:3])
    b = kernels.sample(x, 1.0, 50, 0.9, u)
    assert torch.equal(a, b)


def test_accept_takes_the_bonus_token_after_full_acceptance():
    B, k, V = 6, 3, 3000
    g = torch.Generator().manual_seed(5)
    tl = (torch.randn(B, k + 1, V, generator=g) * 2).bfloat16().cuda()
    dl = tl[:, :k].clone()                          # draft == target: ratio 1, all accepted
    drafts = torch.randint(0, V, (B, k), generator=g).cuda()
    u = torch.rand(B, k + 1, generator=g).cuda()
    bonus = kernels.sample(tl[:, k], 0.8, 20, 0.9, u[:, k].contiguous())
    n, em, _ = kernels.spec_accept(tl, dl, drafts, u, 0.8, bonus_tokens=bonus)
    assert (n.cpu() == k + 1).all()
    assert torch.equal(em[:, :k].cpu(), drafts.cpu())
    assert torch.equal(em[:, k].cpu(), bonus.cpu())
    # a rejection keeps the residual draw: the result equals the call without bonus
    dl2 = (torch.randn(B, k, V, generator=g) * 2).bfloat16().cuda()
    n1, em1, _ = kernels.spec_accept(tl, dl2, drafts, u, 0.8, bonus_tokens=bonus)
    n0, em0, _ = kernels.spec_accept(tl, dl2, drafts, u, 0.8)
    assert torch.equal(n1, n0)
    full = n0 == k + 1
    assert torch.equal(em1[~full], em0[~full])
    assert torch.equal(em1[full, k], bonus[full])
