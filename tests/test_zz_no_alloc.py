"""The allocation-free acceptance entry point (nsg_spec_accept_noalloc),
called through the C ABI: its outputs equal nsg_spec_accept's bit for bit,
greedy and stochastic, on two calls in a row -- the second with a smaller
input, so the static scratch holds the first call's contents when it runs --
and the device error flags reach the caller's word; an input whose workspace
exceeds the static scratch is refused without a launch; the scratch reset
leaves it working."""
import ctypes as C

import numpy as np
import pytest
import torch

from nanosglang_amd import _native, workloads
from oracle.philox import philox_uniforms

pytestmark = pytest.mark.gpu


def _dev(x, dtype):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda").to(dtype)


def _inputs(B, k, V, seed):
    a = workloads.acceptance_batch(batch=B, k=k, vocab=V, temperature=0.8, seed=seed)
    start, indptr, indices = workloads.acceptance_page_table(batch=B, k=k, seed=seed)
    return dict(t=_dev(a["target"], torch.bfloat16), d=_dev(a["draft"], torch.bfloat16),
                x=_dev(a["draft_tokens"], torch.int64),
                u=_dev(philox_uniforms(seed, 0, 0, B * (k + 1)).reshape(B, k + 1),
                       torch.float32),
                indptr=_dev(indptr, torch.int32), indices=_dev(indices, torch.int32),
                start=_dev(start, torch.int32), B=B, k=k, V=V)


def _call(lib, inp, temperature, noalloc, ws=None, flags=None):
    B, k, V = inp["B"], inp["k"], inp["V"]
    greedy = temperature < 1e-6
    n = torch.full((B,), -7, dtype=torch.int32, device="cuda")
    em = torch.full((B, k + 1), -7, dtype=torch.int64, device="cuda")
    rb = torch.full((B, k), -7, dtype=torch.int64, device="cuda")
    t, d = inp["t"], inp["d"]
    args = [t.data_ptr(), t.stride(0), t.stride(1), None if greedy else d.data_ptr(),
            d.stride(0), d.stride(1), 0, inp["x"].data_ptr(),
            None if greedy else inp["u"].data_ptr(), None, B, k, V, temperature,
            inp["indptr"].data_ptr(), inp["indices"].data_ptr(), inp["start"].data_ptr(), 16,
            n.data_ptr(), em.data_ptr(), rb.data_ptr()]
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.nsg_spec_accept_noalloc(*args, None if flags is None else flags.data_ptr(),
                                         stream)
        _native.check(rc, "nsg_spec_accept_noalloc")
    else:
        rc = lib.nsg_spec_accept(*args, ws.data_ptr(), ws.numel(), stream)
        _native.check(rc, "nsg_spec_accept")
    torch.cuda.synchronize()
    return n.cpu().numpy(), em.cpu().numpy(), rb.cpu().numpy()


@pytest.mark.parametrize("temperature", [0.8, 0.0])
def test_noalloc_equals_spec_accept_on_two_calls(temperature):
    lib = _native.load()
    print(f"case: nsg_spec_accept_noalloc T={temperature}", flush=True)
    for B, k, V, seed in ((64, 4, 151936, 31), (8, 3, 20000, 32)):   # second call smaller
        inp = _inputs(B, k, V, seed)
        ws = torch.zeros(lib.nsg_spec_accept_workspace_bytes(B, k, V), dtype=torch.uint8,
                         device="cuda")
        ref = _call(lib, inp, temperature, False, ws=ws)
        flags = torch.zeros(1, dtype=torch.int32, device="cuda")
        got = _call(lib, inp, temperature, True, flags=flags)
        for r, g in zip(ref, got):
            np.testing.assert_array_equal(g, r)
        assert (got[0] >= 1).all() and (got[0] <= k + 1).all()
        assert int(flags.item()) == 0
        print(f"  B={B} k={k} V={V}: equal, mean emitted {got[0].mean():.2f}", flush=True)


def test_noalloc_reports_flags_and_refuses_oversized_inputs():
    lib = _native.load()
    inp = _inputs(4, 3, 1000, 33)
    bad = inp["x"].clone()
    bad[1, 0] = 1000                                      # outside the vocabulary
    inp["x"] = bad
    flags = torch.zeros(1, dtype=torch.int32, device="cuda")
    n, em, _ = _call(lib, inp, 0.8, True, flags=flags)
    assert int(flags.item()) == 4
    assert n[1] == 1 and 0 <= em[1, 0] < 1000
    n2, _, _ = _call(lib, inp, 0.8, True, flags=None)     # no caller word: not reported
    np.testing.assert_array_equal(n2, n)
    cap = lib.nsg_spec_accept_noalloc_max_bytes()
    assert cap == 8 << 20
    B = 4096
    assert lib.nsg_spec_accept_workspace_bytes(B, 8, 151936) > cap
    dummy = torch.zeros(16, dtype=torch.int64, device="cuda")
    p = dummy.data_ptr()
    rc = lib.nsg_spec_accept_noalloc(p, 9 * 151936, 151936, p, 8 * 151936, 151936, 0, p, p,
                                     None, B, 8, 151936, 0.8, None, None, None, 16, p, p, None,
                                     None, torch.cuda.current_stream().cuda_stream)
    assert rc == 3                                        # NSG_ERR_WORKSPACE, nothing launched
    assert b"static scratch" in lib.nsg_last_error()


def test_noalloc_reset_leaves_a_working_scratch():
    """nsg_spec_accept_noalloc_reset (the recovery after flag bit 3) zeroes
    the static scratch with a fill kernel: calls after it still equal
    nsg_spec_accept, stochastic then greedy."""
    lib = _native.load()
    print("case: nsg_spec_accept_noalloc_reset", flush=True)
    stream = torch.cuda.current_stream().cuda_stream
    for temperature in (0.8, 0.0):
        _native.check(lib.nsg_spec_accept_noalloc_reset(stream), "nsg_spec_accept_noalloc_reset")
        inp = _inputs(16, 4, 20000, 35)
        ws = torch.zeros(lib.nsg_spec_accept_workspace_bytes(16, 4, 20000), dtype=torch.uint8,
                         device="cuda")
        ref = _call(lib, inp, temperature, False, ws=ws)
        got = _call(lib, inp, temperature, True)
        for r, g in zip(ref, got):
            np.testing.assert_array_equal(g, r)
