"""GPU parity of the fused acceptance kernel against the oracle.

Greedy: num_emitted / emitted / rollback bit-exact.
Stochastic (same supplied uniforms): bit-exact except requests whose oracle
decision margin is below 1e-5 (|min(1, ratio) - u| for a ratio test, or the
distance of u * sum from a CDF boundary relative to the sum); those must be
rare and are counted.
"""
import numpy as np
import pytest
import torch

from nanosglang_amd import workloads
from oracle.acceptance import spec_accept as oracle_accept
from oracle.philox import philox_uniforms

pytestmark = pytest.mark.gpu
MARGIN = 1e-5


def _dev(x, dtype):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda").to(dtype)


def _page_table(B, k, seed, P=16):
    rng = np.random.default_rng(seed)
    start = rng.integers(0, 300, size=B).astype(np.int32)
    npg = (start + k + 1 + P - 1) // P
    perm = rng.permutation(int(npg.sum()) + 50).astype(np.int32)
    indptr = np.zeros(B + 1, np.int32)
    indptr[1:] = np.cumsum(npg)
    return start, indptr, perm[:indptr[-1]].copy()


def _run(a, temperature, uniforms, dtype=torch.bfloat16, with_pt=True, seed=0, P=16):
    from nanosglang_amd.kernels import spec_accept
    B, k1, V = a["target"].shape
    k = k1 - 1
    start, indptr, indices = _page_table(B, k, seed, P)
    greedy = temperature < 1e-6
    n, em, rb = spec_accept(
        _dev(a["target"], dtype), None if greedy else _dev(a["draft"], dtype),
        _dev(a["draft_tokens"], torch.int64) if k else None,
        None if greedy else _dev(uniforms, torch.float32), temperature,
        *((_dev(indptr, torch.int32), _dev(indices, torch.int32), _dev(start, torch.int32))
          if with_pt else (None, None, None)), page_size=P)
    torch.cuda.synchronize()
    ref = oracle_accept(a["target"], None if greedy else a["draft"], a["draft_tokens"],
                        uniforms, temperature, indptr if with_pt else None, indices,
                        start, P)
    return n.cpu().numpy(), em.cpu().numpy(), rb.cpu().numpy(), ref


def _uniforms(B, k, seed):
    return philox_uniforms(seed, 0, 0, B * (k + 1)).reshape(B, k + 1)


def _assert_exact(n, em, rb, ref):
    assert np.array_equal(n, ref["num_emitted"])
    assert np.array_equal(em, ref["emitted"])
    assert np.array_equal(rb, ref["rollback"])


def _assert_stochastic(n, em, rb, ref, max_exempt_frac=0.02):
    bad = np.nonzero((n != ref["num_emitted"]) | (em != ref["emitted"]).any(1)
                     | (rb != ref["rollback"]).any(1))[0]
    exempt = [b for b in bad if ref["margin"][b] < MARGIN]
    print(f"  mismatches {len(bad)}, all within margin: {len(exempt) == len(bad)}", flush=True)
    assert len(exempt) == len(bad), [(int(b), ref["margin"][b]) for b in bad]
    assert len(bad) <= max(1, max_exempt_frac * len(n))


def test_greedy_c3_shape():
    a = workloads.acceptance_batch(seed=0)                 # B=64, k=4, V=151936
    n, em, rb, ref = _run(a, 0.0, None)
    print(f"  mean emitted {n.mean():.2f}", flush=True)
    _assert_exact(n, em, rb, ref)


def test_greedy_accepts_when_drafts_are_target_argmax():
    a = workloads.acceptance_batch(batch=8, k=4, vocab=5000, seed=1)
    a["draft_tokens"] = a["target"][:, :4].argmax(-1)
    n, em, rb, ref = _run(a, 0.0, None)
    assert (n == 5).all() and (rb == -1).all()
    _assert_exact(n, em, rb, ref)


def test_greedy_ties_lowest_index():
    a = workloads.acceptance_batch(batch=4, k=2, vocab=4096, seed=2)
    a["target"][:] = 0.0
    a["target"][0, 0, [7, 3000]] = 1.0     # tie across chunks -> 7
    a["target"][1, 0, [100, 101]] = 5.0
    a["target"][3, 0] = -1.0               # -0 and +0 tie (the kernel's keys rank them equal)
    a["target"][3, 0, 5] = -0.0
    a["target"][3, 0, 4000] = 0.0
    a["target"][2, 1] = -0.0               # a row of -0 only -> column 0
    a["draft_tokens"][:] = 0
    n, em, rb, ref = _run(a, 0.0, None)
    _assert_exact(n, em, rb, ref)
    assert em[0, 0] == 7 and em[1, 0] == 100 and em[2, 0] == 0 and em[3, 0] == 5
    assert n[2] >= 2 and em[2, 1] == 0


def test_stochastic_c3_shape():
    a = workloads.acceptance_batch(seed=0)                 # T = 0.8
    u = _uniforms(64, 4, 123)
    n, em, rb, ref = _run(a, 0.8, u)
    print(f"  mean emitted {n.mean():.2f}, resample rows {(n < 5).sum()}", flush=True)
    _assert_stochastic(n, em, rb, ref)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_stochastic_many_seeds_small_vocab(seed):
    a = workloads.acceptance_batch(batch=256, k=4, vocab=1000, temperature=1.0, seed=seed)
    u = _uniforms(256, 4, seed)
    n, em, rb, ref = _run(a, 1.0, u, seed=seed)
    _assert_stochastic(n, em, rb, ref)


def test_stochastic_fp32_logits_and_k8():
    a = workloads.acceptance_batch(batch=16, k=8, vocab=12289, temperature=1.0, seed=4)
    u = _uniforms(16, 8, 4)
    n, em, rb, ref = _run(a, 1.0, u, dtype=torch.float32)
    _assert_stochastic(n, em, rb, ref)


@pytest.mark.parametrize("vocab", [3001, 3000])   # 3000: the one-launch tail (V % 8 == 0)
def test_k0_samples_one_token(vocab):
    a = workloads.acceptance_batch(batch=32, k=0, vocab=vocab, temperature=0.7, seed=5)
    u = _uniforms(32, 0, 5)
    n, em, rb, ref = _run(a, 0.7, u, with_pt=False)
    assert (n == 1).all()
    _assert_stochastic(n, em, rb, ref)
    n, em, rb, ref = _run(a, 0.0, None, with_pt=False)
    _assert_exact(n, em, rb, ref)


def test_identical_distributions_always_accept():
    a = workloads.acceptance_batch(batch=16, k=4, vocab=2048, temperature=1.0, seed=6)
    a["target"][:, :4] = a["draft"]
    u = _uniforms(16, 4, 6)
    n, em, rb, ref = _run(a, 1.0, u)
    assert (n == 5).all()
    _assert_stochastic(n, em, rb, ref)


def test_rollback_without_page_table_is_minus_one():
    a = workloads.acceptance_batch(batch=4, k=4, vocab=999, seed=7)
    n, em, rb, ref = _run(a, 0.0, None, with_pt=False)
    assert (rb == -1).all()


@pytest.mark.parametrize("temperature", [0.0, 0.8])
def test_bad_device_inputs_set_flags_and_keep_outputs_defined(temperature):
    """Draft tokens outside the vocabulary are rejected and set flag bit 2;
    rolled-back positions past a request's pages get slot -1 and set bit 1;
    nsg_spec_accept_check_flags returns the flags and clears them."""
    from nanosglang_amd.kernels import AcceptWorkspace, spec_accept
    B, k, V = 4, 3, 1000
    a = workloads.acceptance_batch(batch=B, k=k, vocab=V, seed=9)
    greedy = temperature < 1e-6
    ws = AcceptWorkspace("cuda")
    start, indptr, indices = _page_table(B, k, 9)
    t, d = _dev(a["target"], torch.bfloat16), _dev(a["draft"], torch.bfloat16)
    u = _dev(_uniforms(B, k, 9), torch.float32)

    def call(tokens, start):
        n, em, rb = spec_accept(t, None if greedy else d, _dev(tokens, torch.int64),
                                None if greedy else u, temperature, _dev(indptr, torch.int32),
                                _dev(indices, torch.int32), _dev(start, torch.int32),
                                page_size=16, workspace=ws)
        return n.cpu().numpy(), em.cpu().numpy(), rb.cpu().numpy()

    n0, em0, rb0 = call(a["draft_tokens"], start)
    assert ws.check_flags() == 0
    bad = a["draft_tokens"].copy()
    bad[1, 0] = V
    bad[2, 0] = -1
    n, em, rb = call(bad, start)
    assert ws.check_flags() == 4
    assert ws.check_flags() == 0                     # cleared by the read
    for b in (1, 2):                                 # rejected at position 0
        assert n[b] == 1 and 0 <= em[b, 0] < V and (em[b, 1:] == -1).all()
        assert (rb[b] >= 0).all()
    np.testing.assert_array_equal(n[[0, 3]], n0[[0, 3]])
    np.testing.assert_array_equal(em[[0, 3]], em0[[0, 3]])
    # request 1's verify positions lie past its pages: every rollback slot -1
    past = start.copy()
    past[1] = (indptr[2] - indptr[1]) * 16
    n, em, rb = call(bad, past)
    assert ws.check_flags() == 4 | 2
    assert n[1] == 1 and (rb[1] == -1).all()


def test_check_flags_after_bit3_zeroes_the_whole_workspace():
    """Recovery after flag bit 3 (a hand-off wait gave up, which can leave
    published slots anywhere in the workspace body): with the body dirtied
    from the host and bit 3 set -- no kernel runs on the dirty workspace --
    check_flags returns the bit and leaves every byte zero, and the next call
    equals one on a fresh workspace."""
    from nanosglang_amd.kernels import AcceptWorkspace, spec_accept
    print("case: acceptance workspace recovery after bit 3", flush=True)
    B, k, V = 16, 4, 20000
    a = workloads.acceptance_batch(batch=B, k=k, vocab=V, seed=13)
    args = (_dev(a["target"], torch.bfloat16), _dev(a["draft"], torch.bfloat16),
            _dev(a["draft_tokens"], torch.int64), _dev(_uniforms(B, k, 13), torch.float32), 0.8)
    ws = AcceptWorkspace("cuda")
    buf = ws.get(_native_lib().nsg_spec_accept_workspace_bytes(B, k, V))
    buf.fill_(0x5A)
    buf[:4].view(torch.int32).fill_(8)
    assert ws.check_flags() == 8
    assert int((ws.buf != 0).sum()) == 0
    got = spec_accept(*args, workspace=ws)
    ref = spec_accept(*args, workspace=AcceptWorkspace("cuda"))
    for x, y in zip(got, ref):
        assert torch.equal(x, y)
    assert ws.check_flags() == 0


def test_calls_on_two_streams_use_separate_default_workspaces():
    """Stochastic calls enqueued on two streams at once, each with the
    default workspace: the same results as the calls one after the other."""
    from nanosglang_amd.kernels import spec_accept
    B, k, V = 16, 4, 20000
    inputs = []
    for seed in (11, 12):
        a = workloads.acceptance_batch(batch=B, k=k, vocab=V, seed=seed)
        inputs.append((_dev(a["target"], torch.bfloat16), _dev(a["draft"], torch.bfloat16),
                       _dev(a["draft_tokens"], torch.int64),
                       _dev(_uniforms(B, k, seed), torch.float32)))
    ref = [spec_accept(t, d, x, u, 0.8) for t, d, x, u in inputs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [None, None]
    for rep in range(3):
        for i, s in enumerate(streams):
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                outs[i] = spec_accept(*inputs[i][:3], inputs[i][3], 0.8)
        torch.cuda.synchronize()
        for i in range(2):
            for x, y in zip(outs[i], ref[i]):
                assert torch.equal(x, y), (rep, i)


def test_bad_arguments_raise():
    from nanosglang_amd.kernels import spec_accept
    t = torch.zeros(2, 5, 100, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        spec_accept(t, None, torch.zeros(2, 4, dtype=torch.int64, device="cuda"),
                    None, 0.8)                          # stochastic without draft logits
    with pytest.raises(TypeError):
        spec_accept(t.half(), None, torch.zeros(2, 4, dtype=torch.int64, device="cuda"),
                    None, 0.0)


def test_greedy_large_shape_full_size_closed_form():
    """The large shape's acceptance (64 requests, k = 8, vocab 128,256, bf16),
    greedy: the closed form -- drafts accepted while each equals the first
    argmax of its target row, then that argmax emitted -- with drafts that
    match a random prefix of every request."""
    from nanosglang_amd.kernels import spec_accept
    B, k, V = 64, 8, 128256
    print("case: greedy acceptance, large shape", flush=True)
    g = torch.Generator(device="cuda").manual_seed(22)
    tl = (2 * torch.randn(B, k + 1, V, generator=g, device="cuda")).bfloat16()
    am = tl.float().argmax(-1).cpu().numpy()          # first maximal index
    rng = np.random.default_rng(22)
    prefix = rng.integers(0, k + 1, B)
    drafts = rng.integers(0, V, (B, k))
    for b in range(B):
        drafts[b, :prefix[b]] = am[b, :prefix[b]]
        if prefix[b] < k and drafts[b, prefix[b]] == am[b, prefix[b]]:
            drafts[b, prefix[b]] = (am[b, prefix[b]] + 1) % V
    n, em, rb = spec_accept(tl, None, _dev(drafts, torch.int64), None, 0.0)
    n, em = n.cpu().numpy(), em.cpu().numpy()
    from nanosglang_amd.kernels import _accept_ws
    assert _accept_ws("cuda").check_flags() == 0
    np.testing.assert_array_equal(n, prefix + 1)
    for b in range(B):
        j = prefix[b]
        assert list(em[b, :j]) == list(drafts[b, :j])
        assert em[b, j] == am[b, j]
        assert (em[b, j + 1:] == -1).all()


def test_stochastic_large_shape_full_size_properties():
    """The large shape's stochastic acceptance (64 requests, k = 8, vocab
    128,256, T = 1, bf16) through properties that need no full oracle run:
    accepted drafts are emitted unchanged; every decided ratio test agrees
    with u vs min(1, p_t / p_d) recomputed in float64 (or lies within 1e-5 of
    it); a token drawn after a rejection lies in the residual's support
    (p_t > p_d).  Identical draft and target rows accept all k drafts."""
    from nanosglang_amd.kernels import spec_accept
    B, k, V, T = 64, 8, 128256, 1.0
    print("case: stochastic acceptance, large shape", flush=True)
    g = torch.Generator(device="cuda").manual_seed(23)
    dl = (2 * torch.randn(B, k, V, generator=g, device="cuda")).bfloat16()
    tl = torch.empty(B, k + 1, V, dtype=torch.bfloat16, device="cuda")
    tl[:, :k] = (dl.float() + 0.5 * torch.randn(B, k, V, generator=g, device="cuda")).bfloat16()
    tl[:, k] = (2 * torch.randn(B, V, generator=g, device="cuda")).bfloat16()
    pd = torch.softmax(dl.double() / T, -1)
    drafts = torch.multinomial(pd.view(-1, V).float(), 1, generator=g).view(B, k)
    u = torch.from_numpy(_uniforms(B, k, 23)).cuda()
    n, em, _ = spec_accept(tl, dl, drafts, u, T)
    n, em = n.cpu().numpy(), em.cpu().numpy()
    lpt = torch.log_softmax(tl.double() / T, -1)
    lpd = torch.log_softmax(dl.double() / T, -1)
    d_h, u_h = drafts.cpu().numpy(), u.cpu().numpy()
    ratio = torch.exp(lpt[:, :k].gather(-1, drafts[..., None]) -
                      lpd.gather(-1, drafts[..., None]))[..., 0].clamp(max=1.0).cpu().numpy()
    rejected = 0
    for b in range(B):
        j = n[b] - 1
        assert 0 <= j <= k
        assert list(em[b, :j]) == list(d_h[b, :j])
        for i in range(j):                                # accepted: u < min(1, ratio)
            assert u_h[b, i] < ratio[b, i] or abs(u_h[b, i] - ratio[b, i]) < MARGIN
        if j < k:                                         # rejected at j
            rejected += 1
            assert u_h[b, j] >= ratio[b, j] or abs(u_h[b, j] - ratio[b, j]) < MARGIN
            x = int(em[b, j])
            assert 0 <= x < V
            assert lpt[b, j, x] > lpd[b, j, x] - 1e-9     # residual support
        assert (em[b, j + 1:] == -1).all()
    print(f"  rejections {rejected} / {B}", flush=True)
    assert rejected > 0
    tl[:, :k] = dl                                        # identical distributions
    n, _, _ = spec_accept(tl, dl, drafts, u, T)
    assert (n.cpu().numpy() == k + 1).all()


def test_stochastic_large_shape_full_size_oracle():
    """The large shape's stochastic acceptance at full size (64 requests,
    k = 8, vocab 128,256, T = 1, bf16 logits, rollback slots from a page
    table) against the float64 oracle, to the bar of the acceptance shape:
    bit-exact except requests whose decision margin is below 1e-5."""
    print("case: stochastic acceptance, large shape, oracle", flush=True)
    a = workloads.acceptance_batch(batch=64, k=8, vocab=128256, temperature=1.0, seed=24)
    u = _uniforms(64, 8, 24)
    n, em, rb, ref = _run(a, 1.0, u, seed=24)
    print(f"  mean emitted {n.mean():.2f}, resample rows {(n < 9).sum()}", flush=True)
    _assert_stochastic(n, em, rb, ref)


def test_sampler_and_acceptance_interleaved_on_their_own_workspaces():
    """The captured engine step interleaves filtered draws (nsg_sample) with
    acceptance calls, each kind on its own workspace: the acceptance flags
    read back as zero and every acceptance result equals a call on a fresh
    workspace (the hand-off slots are left zero after every call)."""
    from nanosglang_amd.kernels import AcceptWorkspace, sample, spec_accept
    B, k, V = 8, 4, 20000
    a = workloads.acceptance_batch(batch=B, k=k, vocab=V, seed=25)
    ws, sws = AcceptWorkspace("cuda"), AcceptWorkspace("cuda")
    t, d = _dev(a["target"], torch.bfloat16), _dev(a["draft"], torch.bfloat16)
    u = _dev(_uniforms(B, k, 25), torch.float32)
    dt = _dev(a["draft_tokens"], torch.int64)
    fresh = [spec_accept(t, d, dt, u, 0.8, workspace=AcceptWorkspace("cuda")),
             spec_accept(t, None, dt, None, 0.0, workspace=AcceptWorkspace("cuda"))]
    for _ in range(3):
        sample(t[:, 0], 0.8, top_k=50, top_p=0.9, uniforms=u[:, 0].contiguous(), workspace=sws)
        got = [spec_accept(t, d, dt, u, 0.8, workspace=ws)]
        sample(t[:, 0], 0.8, top_k=50, uniforms=u[:, 0].contiguous(), workspace=sws)
        got.append(spec_accept(t, None, dt, None, 0.0, workspace=ws))
        assert ws.check_flags() == 0
        for g, f in zip(got, fresh):
            for x, y in zip(g, f):
                assert torch.equal(x, y)


def test_one_workspace_across_shapes_and_modes_ends_zero():
    """Acceptance calls of different batch, k, vocabulary and mode on one
    workspace: each equals the same call on a fresh workspace, and after every
    call the workspace (past the flag word) is all zero again -- the kernels'
    hand-off slots must read zero at the start of any later call, whatever
    layout the previous call used."""
    from nanosglang_amd.kernels import AcceptWorkspace, spec_accept
    ws = AcceptWorkspace("cuda")
    cases = [(16, 8, 12288, 1.0), (32, 0, 3000, 0.7), (64, 4, 20000, 0.8), (8, 3, 3001, 0.9),
             (32, 0, 3000, 0.7), (16, 8, 12288, 0.0), (64, 4, 20000, 0.0), (8, 3, 3001, 1.0)]
    ws.get(max(_native_lib().nsg_spec_accept_workspace_bytes(B, k, V) for B, k, V, _ in cases))
    for i, (B, k, V, T) in enumerate(cases):
        a = workloads.acceptance_batch(batch=B, k=k, vocab=V, temperature=max(T, 0.5), seed=40 + i)
        start, indptr, indices = _page_table(B, k, 40 + i)
        args = (_dev(a["target"], torch.bfloat16), _dev(a["draft"], torch.bfloat16) if T else None,
                _dev(a["draft_tokens"], torch.int64) if k else None,
                _dev(_uniforms(B, k, 40 + i), torch.float32) if T else None, T,
                _dev(indptr, torch.int32), _dev(indices, torch.int32), _dev(start, torch.int32))
        got = spec_accept(*args, workspace=ws)
        ref = spec_accept(*args, workspace=AcceptWorkspace("cuda"))
        torch.cuda.synchronize()
        for x, y in zip(got, ref):
            assert torch.equal(x, y), (i, B, k, V, T)
        assert ws.check_flags() == 0
        assert int((ws.buf.view(torch.int32)[1:] != 0).sum()) == 0, (i, B, k, V, T)


def _native_lib():
    from nanosglang_amd import _native
    return _native.load()


@pytest.mark.parametrize("B,k,V,match", [(64, 4, 151936, 0.0), (64, 4, 151936, 0.8),
                                         (32, 4, 5000, 0.7),
                                         (8, 8, 3001, 1.0), (5, 0, 999, 0.0)])
def test_greedy_from_target_tokens_equals_greedy_on_logits(B, k, V, match):
    """nsg_spec_accept_greedy_tokens on each target row's first argmax gives
    the outputs and rollback slots of the greedy acceptance on the logits
    (and of the oracle), bit for bit; ``match``: the share of drafts set to
    the target's own argmax, so that accepted prefixes of every length
    occur."""
    from nanosglang_amd.kernels import spec_accept_greedy_tokens
    print(f"case: greedy from tokens B={B} k={k} V={V} match={match}", flush=True)
    a = workloads.acceptance_batch(batch=B, k=k, vocab=V, seed=B + k)
    am = a["target"].argmax(-1)
    rng = np.random.default_rng(B)
    if k:
        take = rng.random((B, k)) < match
        a["draft_tokens"] = np.where(take, am[:, :k], a["draft_tokens"])
    n, em, rb, ref = _run(a, 0.0, None, seed=B)
    _assert_exact(n, em, rb, ref)
    if 0.5 <= match < 1.0:      # accepted prefixes of several lengths occurred
        assert len(set(n.tolist())) >= 3 and (n > 1).sum() >= B // 4, np.bincount(n)
    start, indptr, indices = _page_table(B, k, B)
    n2, em2, rb2 = spec_accept_greedy_tokens(
        _dev(am, torch.int64), _dev(a["draft_tokens"], torch.int64) if k else None, V,
        _dev(indptr, torch.int32), _dev(indices, torch.int32), _dev(start, torch.int32),
        page_size=16)
    torch.cuda.synchronize()
    _assert_exact(n2.cpu().numpy(), em2.cpu().numpy(), rb2.cpu().numpy(), ref)
    if k:
        # drafts as rows of a position-major (k + 1) x B id buffer: strides (1, B)
        ids = torch.zeros(k + 1, B, dtype=torch.int64, device="cuda")
        ids[1:] = _dev(a["draft_tokens"], torch.int64).t()
        n3, em3, rb3 = spec_accept_greedy_tokens(
            _dev(am, torch.int64), ids[1:].t(), V, _dev(indptr, torch.int32),
            _dev(indices, torch.int32), _dev(start, torch.int32), page_size=16)
        torch.cuda.synchronize()
        _assert_exact(n3.cpu().numpy(), em3.cpu().numpy(), rb3.cpu().numpy(), ref)


def test_greedy_from_target_tokens_flags():
    """Out-of-vocabulary drafts never match and set bit 2, rolled-back
    positions past the pages get -1 and set bit 1, in the workspace's flag
    word, as in the logits form."""
    from nanosglang_amd.kernels import AcceptWorkspace, spec_accept_greedy_tokens
    print("case: greedy from tokens flags", flush=True)
    B, k, V = 4, 3, 1000
    a = workloads.acceptance_batch(batch=B, k=k, vocab=V, seed=9)
    am = a["target"].argmax(-1)
    ws = AcceptWorkspace("cuda")
    start, indptr, indices = _page_table(B, k, 9)
    bad = am[:, :k].copy()
    bad[1, 0] = V
    bad[2, 0] = (am[2, 0] + 1) % V              # rejected: positions 1..k roll back
    past = start.copy()
    past[2] = (indptr[3] - indptr[2]) * 16
    n, em, rb = spec_accept_greedy_tokens(
        _dev(am, torch.int64), _dev(bad, torch.int64), V, _dev(indptr, torch.int32),
        _dev(indices, torch.int32), _dev(past, torch.int32), page_size=16, workspace=ws)
    n, em, rb = n.cpu().numpy(), em.cpu().numpy(), rb.cpu().numpy()
    assert ws.check_flags() == 4 | 2
    assert n[1] == 1 and em[1, 0] == am[1, 0] and (em[1, 1:] == -1).all()
    assert n[0] == k + 1 and n[3] == k + 1 and (em[0] == am[0]).all()
    assert n[2] == 1 and (rb[2] == -1).all()
    assert (rb[1] >= 0).all() and (rb[0] == -1).all()
