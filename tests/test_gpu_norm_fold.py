"""GPU numerics of the RMSNorm folded into the linears around it
(nsg_row_sumsq, nsg_linear_fold, nsg_linear_rope_kv_fold) against plain
PyTorch fp32 references of the same ops:

* partial sums of squares (one per 16 columns of a row) of bf16 rows;
* producer (o_proj / down_proj): y = bf16(residual + bf16(x W^T)) written to
  the residual buffer, with the partial sums of squares of the new rows;
* consumer (gate/up with SwiGLU, q/k/v with RoPE + KV write): x holds the
  un-normalised rows, W the norm weight folded into its columns, and each
  row of x W^T is scaled by rsqrt(mean(x^2) + eps) before the epilogue;
* the lm_head with the final norm folded in (logits and greedy tokens):
  bit-exact against the plain lm_head on rows whose scale is a power of two,
  within bf16 rounding of the fp32 value otherwise;
* bitwise-identical results across calls and graph replays (the partial
  sums are added in one fixed order, no atomics).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _rand(shape, seed, scale=1.0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(*shape, generator=g, device="cuda") * scale).bfloat16()


def _partials(x):
    M, N = x.shape
    return (x.float() ** 2).view(M, N // 16, 16).sum(-1).T.contiguous()


@pytest.mark.parametrize("T,H", [(1, 896), (37, 896), (160, 896), (5, 64), (64, 1024)])
def test_row_sumsq_matches_fp32(T, H):
    from nanosglang_amd import kernels
    print(f"case: row_sumsq T={T} H={H}", flush=True)
    x = _rand((T, H), seed=T + H, scale=3.0)
    ss = kernels.row_sumsq(x)
    torch.cuda.synchronize()
    assert ss.shape == (H // 16, T)
    ref = _partials(x)
    assert torch.allclose(ss, ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("M", [1, 17, 32, 100, 160])
@pytest.mark.parametrize("N,K", [(896, 896), (896, 4864), (1024, 512)])
def test_producer_adds_residual_and_writes_partials(M, N, K):
    from nanosglang_amd import kernels
    print(f"case: fold producer M={M} N={N} K={K}", flush=True)
    x = _rand((M, K), seed=M * 3 + K)
    w = _rand((N, K), seed=N + 1, scale=K ** -0.5)
    res0 = _rand((M, N), seed=M + 7, scale=2.0)
    res = res0.clone()
    ss = torch.full((N // 16, M), -1.0, device="cuda")
    y = kernels.linear(x, w, residual=res, sumsq_out=ss)
    torch.cuda.synchronize()
    assert y.data_ptr() == res.data_ptr()
    proj = x.float() @ w.float().T
    ref = (res0.float() + proj.bfloat16().float()).bfloat16().float()
    err = (res.float() - ref).abs()
    print(f"  max err {err.max().item():.3e}", flush=True)
    # the bf16 rounding of the projection may land on the other side of a
    # boundary (fp32 accumulation order): one ulp of the projection, then
    # one of the sum
    assert (err <= 2.0 ** -7 * (proj.abs() + ref.abs()) + 1e-3).all()
    assert torch.allclose(ss, _partials(res), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("M", [1, 16, 33, 96, 120, 150, 160])
def test_consumer_swiglu_scales_rows(M):
    from nanosglang_amd import kernels
    H, I = 896, 4864
    print(f"case: fold consumer swiglu M={M}", flush=True)
    x = _rand((M, H), seed=M + 11, scale=3.0)
    gamma = (torch.rand(H, generator=torch.Generator(device="cuda").manual_seed(5),
                        device="cuda") + 0.5).bfloat16()
    w = _rand((2 * I, H), seed=12, scale=H ** -0.5)
    wg = (w.float() * gamma.float()[None, :]).bfloat16()
    ss = kernels.row_sumsq(x)
    y = kernels.linear(x, wg, swiglu=True, sumsq_in=ss, norm_eps=EPS)
    torch.cuda.synchronize()
    r = torch.rsqrt((x.float() ** 2).mean(-1, keepdim=True) + EPS)
    a = r * (x.float() @ wg.float().T)
    ref = torch.nn.functional.silu(a[:, :I]) * a[:, I:]
    err = (y.float() - ref).abs()
    print(f"  max err {err.max().item():.3e}", flush=True)
    assert (err <= 2.0 ** -6 * ref.abs() + 2e-3).all()


def _power_of_two_rows(M, K, seed):
    """Rows of +-s_m with s_m in {1/2, 1, 2, 4}: with eps = 0 the row scale
    rsqrt(mean(x^2)) = 1 / s_m is exact, and so is x * scale = +-1, so the
    folded kernel and the plain kernel on the normalised rows must agree bit
    for bit (a wrong row's scale is off by a power of two)."""
    g = torch.Generator().manual_seed(seed)
    s = 2.0 ** torch.randint(-1, 3, (M, 1), generator=g).float()
    sign = torch.randint(0, 2, (M, K), generator=g).float() * 2 - 1
    return (s * sign).bfloat16().cuda(), sign.bfloat16().cuda()


@pytest.mark.parametrize("M", [1, 16, 33, 96, 120, 150, 160])
def test_consumer_swiglu_exact_rows(M):
    from nanosglang_amd import kernels
    H, I = 896, 4864
    print(f"case: fold consumer swiglu exact M={M}", flush=True)
    x, h = _power_of_two_rows(M, H, seed=M)
    g = torch.Generator().manual_seed(M + 1)
    w = torch.randint(-1, 2, (2 * I, H), generator=g).bfloat16().cuda()
    y = kernels.linear(x, w, swiglu=True, sumsq_in=kernels.row_sumsq(x), norm_eps=0.0)
    y2 = kernels.linear(h, w, swiglu=True, force=True)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)


@pytest.mark.parametrize("M", [1, 5, 17, 32, 100, 160])
@pytest.mark.parametrize("Hq,Hkv,D,K", [(14, 2, 64, 896), (4, 2, 128, 512)])
def test_consumer_rope_exact_rows(M, Hq, Hkv, D, K):
    """q/k/v + RoPE + KV write with the folded norm against the same fused
    kernel on the normalised rows, bit for bit (see _power_of_two_rows)."""
    from nanosglang_amd import kernels
    from nanosglang_amd.model.causal_lm import ModelConfig, rope_tables
    print(f"case: fold consumer rope exact M={M} Hq={Hq} Hkv={Hkv} D={D} K={K}", flush=True)
    N = (Hq + 2 * Hkv) * D
    x, h = _power_of_two_rows(M, K, seed=M + D)
    g = torch.Generator().manual_seed(M + 2)
    w = torch.randint(-1, 2, (N, K), generator=g).bfloat16().cuda()
    b = torch.randint(-8, 9, (N,), generator=g).bfloat16().cuda()
    cfg = ModelConfig(vocab_size=1000, hidden_size=Hq * D, intermediate_size=512,
                      num_hidden_layers=1, num_attention_heads=Hq, num_key_value_heads=Hkv,
                      max_position_embeddings=2048)
    cos, sin = rope_tables(cfg, "cuda")
    pos = torch.randint(0, 2048, (M,), generator=g).cuda()
    slots = torch.randperm(40 * 16, generator=g)[:M].cuda()
    kc = torch.zeros((40, 16, Hkv, D), dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    q = kernels.linear_rope_kv(x, w, b, Hq, Hkv, D, pos, cos, sin, slots, kc, vc,
                               sumsq_in=kernels.row_sumsq(x), norm_eps=0.0)
    q2 = kernels.linear_rope_kv(h, w, b, Hq, Hkv, D, pos, cos, sin, slots, kc2, vc2, force=True)
    torch.cuda.synchronize()
    assert torch.equal(q, q2) and torch.equal(kc, kc2) and torch.equal(vc, vc2)


@pytest.mark.parametrize("M", [1, 17, 32, 100, 160])
@pytest.mark.parametrize("N", [1000, 151936])
def test_lm_head_fold_exact_rows(M, N):
    """Folded lm_head against the plain lm_head on the normalised rows, bit
    for bit, logits and greedy tokens (see _power_of_two_rows; the integer
    weights make many equal logits, so the tokens also check the tie rule:
    the lowest column wins)."""
    from nanosglang_amd import kernels
    K = 896
    print(f"case: lm_head fold exact M={M} N={N}", flush=True)
    x, h = _power_of_two_rows(M, K, seed=M + N)
    g = torch.Generator(device="cuda").manual_seed(M + 3)
    w = torch.randint(-1, 2, (N, K), generator=g, device="cuda").bfloat16()
    ss = kernels.row_sumsq(x)
    assert kernels.lm_head_fold_supported(M, N, K, ss.shape[0])
    y = kernels.lm_head_fold(x, w, ss, 0.0)
    y2 = kernels.linear(h, w, force=True)
    tok = torch.full((M, 3), -1, dtype=torch.int64, device="cuda")
    kernels.lm_head_fold(x, w, ss, 0.0, argmax_out=tok[:, 1])
    tok2 = kernels.linear_argmax(h, w)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    assert torch.equal(tok[:, 1], tok2)
    assert (tok[:, 0] == -1).all() and (tok[:, 2] == -1).all()
    first = (y2.float() == y2.float().max(1, keepdim=True).values).int().argmax(1)
    assert torch.equal(tok2, first)


@pytest.mark.parametrize("M", [1, 33, 160])
def test_lm_head_fold_scales_rows(M):
    """Random rows and a random norm weight: the logits within bf16 rounding
    of the fp32 value r_m * (x_m . bf16(w_norm * W_n)), and each greedy token
    the first column of its row's largest returned logit."""
    from nanosglang_amd import kernels
    K, N = 896, 151936
    print(f"case: lm_head fold M={M}", flush=True)
    x = _rand((M, K), seed=M + 41, scale=3.0)
    gamma = (torch.rand(K, generator=torch.Generator(device="cuda").manual_seed(6),
                        device="cuda") + 0.5).bfloat16()
    w = _rand((N, K), seed=42, scale=K ** -0.5)
    wg = (w.float() * gamma.float()[None, :]).bfloat16()
    ss = kernels.row_sumsq(x)
    y = kernels.lm_head_fold(x, wg, ss, EPS)
    tok = kernels.lm_head_fold(x, wg, ss, EPS,
                               argmax_out=torch.empty(M, dtype=torch.int64, device="cuda"))
    torch.cuda.synchronize()
    r = torch.rsqrt((x.float() ** 2).mean(-1, keepdim=True) + EPS)
    ref = r * (x.float() @ wg.float().T)
    err = (y.float() - ref).abs()
    print(f"  max err {err.max().item():.3e}", flush=True)
    assert (err <= 2.0 ** -7 * ref.abs() + 1e-3).all()
    yf = y.float()
    first = (yf == yf.max(1, keepdim=True).values).int().argmax(1)
    assert torch.equal(tok, first)


def test_lm_head_fold_rejects_what_does_not_fit():
    """Shapes outside the folded kernel: an error, no launch."""
    from nanosglang_amd import kernels
    print("case: lm_head fold unsupported shapes", flush=True)
    assert not kernels.lm_head_fold_supported(160, 1000, 1024, 64)   # partials > one ring slot
    assert not kernels.lm_head_fold_supported(161, 1000, 896, 56)    # more than 160 rows
    x = _rand((160, 1024), seed=7)
    w = _rand((1000, 1024), seed=8)
    with pytest.raises(RuntimeError):
        kernels.lm_head_fold(x, w, kernels.row_sumsq(x), EPS)


def test_lm_head_fold_is_deterministic_and_graph_safe():
    """The folded lm_head (logits and tokens) after a producer: the same bits
    across eager calls and graph replays with eager work in between."""
    from nanosglang_amd import kernels
    print("case: lm_head fold graph replay", flush=True)
    M, H, N = 160, 896, 151936
    x = _rand((M, H), seed=51)
    wo = _rand((H, H), seed=52, scale=H ** -0.5)
    wl = _rand((N, H), seed=53, scale=H ** -0.5)
    res0 = _rand((M, H), seed=54, scale=2.0)
    res, ss = res0.clone(), torch.empty(H // 16, M, device="cuda")
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    tok = torch.empty(M, dtype=torch.int64, device="cuda")

    def step():
        kernels.linear(x, wo, residual=res, sumsq_out=ss)
        kernels.lm_head_fold(res, wl, ss, EPS, out=out)
        kernels.lm_head_fold(res, wl, ss, EPS, argmax_out=tok)

    step()
    ref, ref_tok = out.clone(), tok.clone()
    graph = torch.cuda.CUDAGraph()
    res.copy_(res0)
    with torch.cuda.graph(graph):
        step()
    for _ in range(3):
        res.copy_(res0)
        out.zero_()
        tok.fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref) and torch.equal(tok, ref_tok)
        res.copy_(res0)
        step()
        torch.cuda.synchronize()
        assert torch.equal(out, ref) and torch.equal(tok, ref_tok)


def test_folded_linears_are_deterministic_and_graph_safe():
    """A producer / consumer pair: bitwise-identical results across eager
    calls and across graph replays with eager work in between."""
    from nanosglang_amd import kernels
    print("case: folded pair graph replay", flush=True)
    M, H, I = 160, 896, 4864
    x = _rand((M, H), seed=31)
    wo = _rand((H, H), seed=32, scale=H ** -0.5)
    wg = _rand((2 * I, H), seed=33, scale=H ** -0.5)
    res0 = _rand((M, H), seed=34, scale=2.0)

    def step(res, ss, out):
        kernels.linear(x, wo, residual=res, sumsq_out=ss)
        return kernels.linear(res, wg, swiglu=True, sumsq_in=ss, norm_eps=EPS, out=out)

    res, ss = res0.clone(), torch.empty(H // 16, M, device="cuda")
    out = torch.empty(M, I, dtype=torch.bfloat16, device="cuda")
    ref = step(res, ss, out).clone()
    ref_res = res.clone()
    res.copy_(res0)
    step(res, ss, out)
    torch.cuda.synchronize()
    assert torch.equal(out, ref) and torch.equal(res, ref_res)
    graph = torch.cuda.CUDAGraph()
    res.copy_(res0)
    with torch.cuda.graph(graph):
        step(res, ss, out)
    for _ in range(3):
        res.copy_(res0)
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref) and torch.equal(res, ref_res)
        res2 = res0.clone()
        again = step(res2, torch.empty_like(ss), torch.empty_like(out))
        torch.cuda.synchronize()
        assert torch.equal(again, ref)


@pytest.mark.parametrize("shape", [(1,), (37,), (32, 5), (8, 5)])
def test_embed_rows_equals_lookup_and_writes_partials(shape):
    """nsg_embed_rows: the rows of F.embedding on an index view of any
    strides (a column of a (B, k+1) buffer, its transpose), bit for bit, and
    the partial sums of squares row_sumsq writes for the same rows."""
    from nanosglang_amd import kernels
    print(f"case: embed_rows ids {shape}", flush=True)
    V, H = 151936, 896
    g = torch.Generator(device="cuda").manual_seed(len(shape) * 100 + shape[0])
    table = torch.randn(V, H, generator=g, device="cuda").bfloat16()
    base = torch.randint(0, V, (shape[0], 7), generator=g, device="cuda")
    ids = base[:, 3] if len(shape) == 1 else base[:, :shape[1]].t().contiguous().t()
    rows = ids.numel()
    ss = torch.full((H // 16, rows), -1.0, device="cuda")
    out = kernels.embed_rows(ids, table, sumsq_out=ss)
    ref = torch.nn.functional.embedding(ids.reshape(-1), table)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert torch.equal(ss, kernels.row_sumsq(ref))
    # ids out of range read the nearest valid row
    bad = torch.tensor([-5, V + 3], device="cuda")
    got = kernels.embed_rows(bad, table)
    torch.cuda.synchronize()
    assert torch.equal(got[0], table[0]) and torch.equal(got[1], table[V - 1])
