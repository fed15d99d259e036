"""GPU parity of KV slot writes / clears and of the Philox uniform kernel."""
import numpy as np
import pytest
import torch

from oracle.page_table import write_indices
from oracle.philox import philox_uniforms

pytestmark = pytest.mark.gpu


def test_philox_matches_oracle_bitwise():
    from nanosglang_amd.kernels import philox_uniform
    for seed, stream, off, n in [(0, 0, 0, 1000), (12345, 7, 1001, 333), (2**40 + 3, 2, 2**33 + 1, 77)]:
        got = philox_uniform(seed, stream, off, n, "cuda").cpu().numpy()
        assert np.array_equal(got, philox_uniforms(seed, stream, off, n)), (seed, stream, off)


def test_kv_write_matches_index_put():
    from nanosglang_amd.kernels import kv_write
    rng = np.random.default_rng(0)
    N, P, Hkv, D = 50, 16, 2, 64
    kc = torch.randn(N, P, Hkv, D, device="cuda").bfloat16()
    vc = torch.randn(N, P, Hkv, D, device="cuda").bfloat16()
    tables = [rng.permutation(N)[:4].tolist(), rng.permutation(N)[:3].tolist()]
    slots = write_indices(tables, [10, 30], [5, 9], P)
    T = len(slots)
    qkv = torch.randn(T, (14 + 2 * Hkv) * D, device="cuda").bfloat16()   # fused projection rows
    k = qkv[:, 14 * D:(14 + Hkv) * D].view(T, Hkv, D)
    v = qkv[:, (14 + Hkv) * D:].view(T, Hkv, D)
    ref_k, ref_v = kc.clone(), vc.clone()
    s = torch.from_numpy(slots).cuda()
    ref_k.view(-1, Hkv, D)[s] = k
    ref_v.view(-1, Hkv, D)[s] = v
    kv_write(k, v, s, kc, vc)
    torch.cuda.synchronize()
    assert torch.equal(kc, ref_k) and torch.equal(vc, ref_v)


def test_kv_write_skips_negative_slots():
    from nanosglang_amd.kernels import kv_write
    kc = torch.zeros(4, 16, 1, 64, device="cuda", dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    k = torch.ones(3, 1, 64, device="cuda", dtype=torch.bfloat16)
    kv_write(k, k, torch.tensor([5, -1, 17], device="cuda"), kc, vc)
    torch.cuda.synchronize()
    flat = kc.view(-1, 64)
    assert flat[5].eq(1).all() and flat[17].eq(1).all() and flat.sum() == 128


def test_kv_clear_slots_all_layers():
    from nanosglang_amd.kernels import kv_clear_slots
    kc = torch.ones(3, 8, 16, 2, 64, device="cuda", dtype=torch.bfloat16)
    vc = torch.ones_like(kc)
    slots = torch.tensor([3, -1, 40, 127], device="cuda")
    kv_clear_slots(slots, kc, vc)
    torch.cuda.synchronize()
    flat = kc.view(3, -1, 2, 64)
    for s in (3, 40, 127):
        assert flat[:, s].eq(0).all()
    assert flat.float().sum().item() == 3 * (128 - 3) * 128
    assert torch.equal(kc, vc)
