"""The torch operators (torch.ops.nsg.*) on the GPU run the same kernels as
the host wrappers: each result equals the wrapper's bit for bit (the
wrappers' results are checked against the oracle elsewhere), and one
attention call checks the operator itself against the oracle.  The plan /
run pair replays inside a captured HIP graph."""
import numpy as np
import pytest
import torch

from nanosglang_amd import kernels, ops, workloads
from oracle.verify_attention import verify_attention as oracle_attention

pytestmark = pytest.mark.gpu


def _dev(x, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda").to(dtype)


def _attn_inputs(seed, batch=12):
    c = workloads.verify_attention_batch(batch=batch, num_pages=600, seed=seed)
    i32 = torch.int32
    return c, dict(q=_dev(c["q"]), k=_dev(c["k"]), v=_dev(c["v"]),
                   qo=_dev(c["qo_indptr"], i32), kvp=_dev(c["kv_indptr"], i32),
                   idx=_dev(c["kv_indices"], i32), last=_dev(c["kv_last_page_len"], i32))


def test_verify_attention_operator_equals_the_wrapper_and_the_oracle():
    print("case: nsg::verify_attention, batch 12", flush=True)
    c, t = _attn_inputs(1)
    got = torch.ops.nsg.verify_attention(t["q"], t["k"], t["v"], t["qo"], t["kvp"], t["idx"],
                                         t["last"])
    ws = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    w = kernels.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(t["qo"], t["kvp"], t["idx"], t["last"], 14, 2, 64, 16)
    ref = w.run(t["q"], (t["k"], t["v"]))
    assert torch.equal(got, ref)
    o = oracle_attention(c["q"], c["k"], c["v"], c["qo_indptr"], c["kv_indptr"],
                         c["kv_indices"], c["kv_last_page_len"], c["sm_scale"], True)
    g = got.float().cpu().numpy()
    assert (np.abs(g - o) <= 2e-3 + 2.0 ** -8 * np.abs(o)).all()


def test_plan_and_run_operators_replay_in_a_graph():
    print("case: nsg::verify_attention_plan / _run, eager and graph", flush=True)
    c, t = _attn_inputs(2)
    rec, work_h = torch.ops.nsg.verify_attention_plan(
        torch.from_numpy(c["qo_indptr"]), torch.from_numpy(c["kv_indptr"]),
        torch.from_numpy(c["kv_last_page_len"]), 14, 2, 64, 16)
    work = work_h.cuda()
    ws = torch.zeros(ops.plan_workspace_bytes(rec), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(t["q"])

    def run(q):
        torch.ops.nsg.verify_attention_run(rec, work, q, t["k"], t["v"], t["qo"], t["kvp"],
                                           t["idx"], t["last"], 0.125, True, ws, out)

    run(t["q"])
    ref = torch.ops.nsg.verify_attention(t["q"], t["k"], t["v"], t["qo"], t["kvp"], t["idx"],
                                         t["last"])
    assert torch.equal(out, ref)
    q_static = t["q"].clone()
    run(q_static)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run(q_static)
    gen = torch.Generator(device="cuda").manual_seed(5)
    for rep in range(3):
        q_new = torch.randn(q_static.shape, generator=gen, device="cuda").bfloat16()
        q_static.copy_(q_new)
        g.replay()
        torch.cuda.synchronize()
        want = torch.ops.nsg.verify_attention(q_new, t["k"], t["v"], t["qo"], t["kvp"],
                                              t["idx"], t["last"])
        assert torch.equal(out, want), rep


def test_run_operator_checks_shapes_against_the_plan():
    c, t = _attn_inputs(3)
    rec, work_h = torch.ops.nsg.verify_attention_plan(
        torch.from_numpy(c["qo_indptr"]), torch.from_numpy(c["kv_indptr"]),
        torch.from_numpy(c["kv_last_page_len"]), 14, 2, 64, 16)
    work = work_h.cuda()
    ws = torch.zeros(ops.plan_workspace_bytes(rec), dtype=torch.uint8, device="cuda")
    short_q = t["q"][:-1].contiguous()
    with pytest.raises(ValueError, match="as planned"):
        torch.ops.nsg.verify_attention_run(rec, work, short_q, t["k"], t["v"], t["qo"], t["kvp"],
                                           t["idx"], t["last"], 0.125, True, ws,
                                           torch.empty_like(short_q))
    with pytest.raises(ValueError, match="page ids"):
        torch.ops.nsg.verify_attention_run(rec, work, t["q"], t["k"], t["v"], t["qo"], t["kvp"],
                                           t["idx"][:-1].contiguous(), t["last"], 0.125, True,
                                           ws, torch.empty_like(t["q"]))
    with pytest.raises(ValueError, match="workspace"):
        torch.ops.nsg.verify_attention_run(rec, work, t["q"], t["k"], t["v"], t["qo"], t["kvp"],
                                           t["idx"], t["last"], 0.125, True, ws[:16],
                                           torch.empty_like(t["q"]))


@pytest.mark.parametrize("temperature", [0.0, 0.8])
def test_spec_accept_and_sample_operators_equal_the_wrappers(temperature):
    print(f"case: nsg::spec_accept / nsg::sample, T={temperature}", flush=True)
    a = workloads.acceptance_batch(batch=8, k=4, vocab=5000, seed=4)
    tl, dl = _dev(a["target"]), _dev(a["draft"])
    toks = _dev(a["draft_tokens"], torch.int64)
    u = torch.rand(8, 5, generator=torch.Generator().manual_seed(4)).cuda()
    greedy = temperature < 1e-6
    args = (tl, None if greedy else dl, toks, None if greedy else u, temperature)
    got = torch.ops.nsg.spec_accept(*args)
    ref = kernels.spec_accept(*args)
    for x, y in zip(got, ref):
        assert torch.equal(x, y)
    s = torch.ops.nsg.sample(tl[:, 0], temperature, 20, 0.9, None if greedy else u[:, 0])
    assert torch.equal(s, kernels.sample(tl[:, 0], temperature, 20, 0.9,
                                         None if greedy else u[:, 0]))


def test_kv_write_operators_equal_the_wrappers():
    print("case: nsg::kv_write / nsg::rope_kv_write", flush=True)
    T, Hq, Hkv, D, N, P = 9, 14, 2, 64, 32, 16
    g = torch.Generator(device="cuda").manual_seed(6)
    qkv = torch.randn(T, (Hq + 2 * Hkv) * D, generator=g, device="cuda").bfloat16()
    pos = torch.randint(0, 500, (T,), generator=g, device="cuda")
    slots = torch.randperm(N * P, generator=g, device="cuda")[:T]
    inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    ang = torch.arange(512, dtype=torch.float64)[:, None] * inv[None]
    cos, sin = ang.cos().float().cuda(), ang.sin().float().cuda()
    caches = [torch.zeros(N, P, Hkv, D, dtype=torch.bfloat16, device="cuda") for _ in range(4)]
    q1 = torch.ops.nsg.rope_kv_write(qkv, Hq, Hkv, D, pos, cos, sin, slots, caches[0], caches[1])
    q2 = kernels.rope_kv_write(qkv, Hq, Hkv, D, pos, cos, sin, slots, caches[2], caches[3])
    assert torch.equal(q1, q2)
    assert torch.equal(caches[0], caches[2]) and torch.equal(caches[1], caches[3])
    k = torch.randn(T, Hkv, D, generator=g, device="cuda").bfloat16()
    v = torch.randn(T, Hkv, D, generator=g, device="cuda").bfloat16()
    torch.ops.nsg.kv_write(k, v, slots, caches[0], caches[1])
    kernels.kv_write(k, v, slots, caches[2], caches[3])
    assert torch.equal(caches[0], caches[2]) and torch.equal(caches[1], caches[3])
    flat = caches[0].view(-1, Hkv, D)
    assert torch.equal(flat[slots], k)


def _accept_args(B, k, V, seed, T=0.8):
    a = workloads.acceptance_batch(batch=B, k=k, vocab=V, seed=seed)
    u = torch.rand(B, k + 1, generator=torch.Generator().manual_seed(seed)).cuda()
    return (_dev(a["target"]), _dev(a["draft"]), _dev(a["draft_tokens"], torch.int64), u, T)


def test_spec_accept_operator_graph_keeps_its_workspace_after_growth():
    """A graph captured around nsg::spec_accept keeps using the per-stream
    workspace it was captured with: after a larger eager call on the same
    stream grows that workspace, every replay still equals a call on a fresh
    workspace (the replaced buffer stays allocated), and so does the larger
    call."""
    print("case: nsg::spec_accept captured, then its workspace grown", flush=True)
    small, big = _accept_args(8, 4, 5000, 31), _accept_args(64, 4, 151936, 32)
    ref_small = kernels.spec_accept(*small, workspace=kernels.AcceptWorkspace("cuda"))
    ref_big = kernels.spec_accept(*big, workspace=kernels.AcceptWorkspace("cuda"))
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        torch.ops.nsg.spec_accept(*small)            # creates the stream's workspace
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            out = torch.ops.nsg.spec_accept(*small)
        for rep in range(3):
            got_big = torch.ops.nsg.spec_accept(*big)  # the first one grows the workspace
            g.replay()
            s.synchronize()
            for x, y in zip(out, ref_small):
                assert torch.equal(x, y), rep
            for x, y in zip(got_big, ref_big):
                assert torch.equal(x, y), rep
        assert torch.ops.nsg.spec_accept_check_flags(torch.device("cuda", 0)) == 0
    del g
    torch.cuda.synchronize()


def test_spec_accept_operator_refuses_to_grow_its_workspace_under_capture():
    """A first nsg::spec_accept call on a stream that is being captured would
    allocate its workspace from the graph's private pool: it raises instead,
    before any kernel is enqueued."""
    print("case: nsg::spec_accept workspace growth under capture", flush=True)
    args = _accept_args(8, 4, 5000, 33)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with pytest.raises(RuntimeError, match="being captured"):
            with torch.cuda.graph(g, stream=s):
                torch.ops.nsg.spec_accept(*args)
    del g
    torch.cuda.synchronize()


def test_spec_accept_check_flags_operator_reports_device_errors():
    """nsg::spec_accept_check_flags returns and clears the error bits of the
    current stream's acceptance workspace: a draft token outside the
    vocabulary sets bit 2 (that request is rejected at position 0)."""
    print("case: nsg::spec_accept_check_flags", flush=True)
    dev = torch.device("cuda", 0)
    tl, dl, dt, u, T = _accept_args(8, 4, 5000, 34)
    torch.ops.nsg.spec_accept(tl, dl, dt, u, T)
    assert torch.ops.nsg.spec_accept_check_flags(dev) == 0
    bad = dt.clone()
    bad[3, 0] = 5000
    n, em, _ = torch.ops.nsg.spec_accept(tl, dl, bad, u, T)
    assert torch.ops.nsg.spec_accept_check_flags(dev) == 4
    assert torch.ops.nsg.spec_accept_check_flags(dev) == 0
    assert int(n[3]) == 1 and 0 <= int(em[3, 0]) < 5000
