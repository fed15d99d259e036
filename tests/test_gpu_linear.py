"""GPU numerics of the weight-streaming linear kernel (nsg_linear) against a
plain PyTorch fp32 reference of the same op:

* bias epilogue: y = bf16(x @ w.T + b), so |y - ref| is one bf16 rounding
  (<= 2^-8 |ref|) plus fp32 accumulation-order noise;
* SwiGLU epilogue: y = bf16(bf16(silu(bf16(g))) * bf16(u)), checked against
  the same formula on fp32 g, u (a rounding of g or u may land on the other
  side of a bf16 boundary, so two roundings of slack);
* every tile configuration (row counts 1 .. 160), strided x rows, a column
  count that is not a multiple of the workgroup's columns, and the library
  fallback above 160 rows.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _data(M, N, K, seed, ldx=None, rows=None):
    g = torch.Generator(device="cuda").manual_seed(seed)
    ldx = ldx or K
    xb = torch.randn(M, ldx, generator=g, device="cuda").bfloat16()
    x = xb[:, :K]
    w = (torch.randn(rows or N, K, generator=g, device="cuda") * K ** -0.5).bfloat16()
    b = torch.randn(N, generator=g, device="cuda").bfloat16()
    return x, w, b


def _check_bias(y, x, w, b):
    ref = x.float() @ w.float().T + (b.float() if b is not None else 0.0)
    err = (y.float() - ref).abs()
    # one bf16 rounding, plus fp32 accumulation-order noise (K <= 4864 terms
    # of size ~1/sqrt(K) each)
    bound = 2.0 ** -8 * ref.abs() + 2e-3
    print(f"  max err {err.max().item():.3e}  max |ref| {ref.abs().max().item():.3e}", flush=True)
    assert torch.isfinite(y.float()).all()
    assert (err <= bound).all()


@pytest.mark.parametrize("M", [1, 7, 16, 32, 33, 48, 80, 96, 100, 128, 129, 160])
@pytest.mark.parametrize("N,K", [(1152, 896), (896, 4864), (1000, 896)])
def test_linear_bias_matches_fp32_reference(M, N, K):
    from nanosglang_amd import kernels
    print(f"case: linear M={M} N={N} K={K}", flush=True)
    x, w, b = _data(M, N, K, seed=M * 7 + N)
    y = kernels.linear(x, w, b, force=True)
    torch.cuda.synchronize()
    _check_bias(y, x, w, b)
    y0 = kernels.linear(x, w, None, force=True)
    torch.cuda.synchronize()
    _check_bias(y0, x, w, None)


@pytest.mark.parametrize("M", [1, 2, 16, 17, 32])
def test_linear_wide_output_matches_fp32_reference(M):
    """Very wide outputs (lm_head: N >= 65536 columns) take their own tile
    shapes; N is not a multiple of any workgroup's columns."""
    from nanosglang_amd import kernels
    print(f"case: linear wide M={M}", flush=True)
    x, w, b = _data(M, 65540, 256, seed=40 + M)
    y = kernels.linear(x, w, b, force=True)
    torch.cuda.synchronize()
    _check_bias(y, x, w, b)


@pytest.mark.parametrize("M", [1, 32, 70, 160])
def test_linear_strided_rows_and_out_buffer(M):
    from nanosglang_amd import kernels
    print(f"case: linear strided M={M}", flush=True)
    x, w, b = _data(M, 896, 896, seed=5, ldx=1152)     # x is a column slice of wider rows
    out = torch.full((M, 1024), 7.0, dtype=torch.bfloat16, device="cuda")[:, :896]
    y = kernels.linear(x, w, b, out=out, force=True)
    torch.cuda.synchronize()
    assert y.data_ptr() == out.data_ptr()
    _check_bias(y, x, w, b)
    base = out._base if out._base is not None else out
    assert (base[:, 896:] == 7.0).all()                  # nothing written past N


@pytest.mark.parametrize("M", [1, 16, 17, 32, 48, 64, 96, 100, 128, 129, 160])
def test_linear_swiglu_matches_fp32_reference(M):
    from nanosglang_amd import kernels
    I, K = 4864, 896
    print(f"case: linear swiglu M={M} I={I} K={K}", flush=True)
    x, w, _ = _data(M, I, K, seed=11 + M, rows=2 * I)
    y = kernels.linear(x, w, swiglu=True, force=True)
    torch.cuda.synchronize()
    gu = x.float() @ w.float().T
    g, u = gu[:, :I], gu[:, I:]
    ref = torch.nn.functional.silu(g) * u
    err = (y.float() - ref).abs()
    print(f"  max err {err.max().item():.3e}", flush=True)
    assert (err <= 2.0 ** -6 * ref.abs() + 2e-3).all()


def test_linear_large_m_uses_library_gemm_with_same_semantics():
    from nanosglang_amd import kernels
    from nanosglang_amd._native import load
    print("case: linear M=300 (library path)", flush=True)
    lib = load()
    assert lib.nsg_linear_preferred(32, 1152, 896) == 1
    assert lib.nsg_linear_preferred(300, 1152, 896) == 0
    assert lib.nsg_linear_preferred(32, 151936, 896) == 1
    assert lib.nsg_linear_preferred(33, 151936, 896) == 0
    x, w, b = _data(300, 1152, 896, seed=3)
    _check_bias(kernels.linear(x, w, b), x, w, b)
    xs, ws, _ = _data(300, 4864, 896, seed=4, rows=2 * 4864)
    y = kernels.linear(xs, ws, swiglu=True)
    gu = xs.float() @ ws.float().T
    ref = torch.nn.functional.silu(gu[:, :4864]) * gu[:, 4864:]
    assert ((y.float() - ref).abs() <= 2.0 ** -6 * ref.abs() + 2e-3).all()


def test_linear_is_deterministic_and_graph_safe():
    """Bitwise-identical results across calls and across graph replays with
    eager work in between."""
    from nanosglang_amd import kernels
    print("case: linear graph replay", flush=True)
    x, w, b = _data(160, 1152, 896, seed=9)
    y_eager = kernels.linear(x, w, b, force=True)
    out = torch.empty_like(y_eager)
    kernels.linear(x, w, b, out=out, force=True)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        kernels.linear(x, w, b, out=out, force=True)
    for _ in range(3):
        out.zero_()
        graph.replay()
        again = kernels.linear(x, w, b, force=True)
        torch.cuda.synchronize()
        assert torch.equal(out, y_eager) and torch.equal(again, y_eager)


def _rope_case(M, Hq, Hkv, D, K, seed, exact):
    """x, w, bias on the GPU; exact=True draws integers in [-1, 1] (and an
    integer bias) so that every fp32 accumulation order gives the same,
    exact projection and the fused result is fixed bit for bit."""
    g = torch.Generator().manual_seed(seed)
    N = (Hq + 2 * Hkv) * D
    if exact:
        x = torch.randint(-1, 2, (M, K), generator=g).float()
        w = torch.randint(-1, 2, (N, K), generator=g).float()
        b = torch.randint(-8, 9, (N,), generator=g).float()
    else:
        x = torch.randn(M, K, generator=g)
        w = torch.randn(N, K, generator=g) * K ** -0.5
        b = torch.randn(N, generator=g)
    return x.bfloat16(), w.bfloat16(), b.bfloat16()


@pytest.mark.parametrize("M", [1, 5, 16, 17, 32, 33, 64, 100, 160])
@pytest.mark.parametrize("Hq,Hkv,D,K", [(14, 2, 64, 896), (4, 2, 128, 512)])
def test_linear_rope_kv_bit_exact_on_exact_projection(M, Hq, Hkv, D, K):
    """Fused q/k/v projection + RoPE + KV-slot write against the oracle's
    apply_rope on the bf16 projection (CPU, the reference's rounding order)
    and the slot rule: negative slots are skipped, other cache rows untouched."""
    from nanosglang_amd import kernels
    from nanosglang_amd.model.causal_lm import ModelConfig, rope_tables
    from oracle.model import apply_rope as oracle_rope
    print(f"case: linear_rope_kv exact M={M} Hq={Hq} Hkv={Hkv} D={D} K={K}", flush=True)
    x, w, b = _rope_case(M, Hq, Hkv, D, K, seed=M + D, exact=True)
    cfg = ModelConfig(vocab_size=1000, hidden_size=Hq * D, intermediate_size=512,
                      num_hidden_layers=1, num_attention_heads=Hq, num_key_value_heads=Hkv,
                      max_position_embeddings=2048)
    cos, sin = rope_tables(cfg, "cpu")
    g = torch.Generator().manual_seed(M)
    pos = torch.randint(0, 2048, (M,), generator=g)
    NB, P = 40, 16
    slots = torch.randperm(NB * P, generator=g)[:M]
    slots[::7] = -1                                                # padding rows: no write
    kc = torch.full((NB, P, Hkv, D), 3.0, dtype=torch.bfloat16, device="cuda")
    vc = torch.full_like(kc, 5.0)
    q = kernels.linear_rope_kv(x.cuda(), w.cuda(), b.cuda(), Hq, Hkv, D, pos.cuda(), cos.cuda(),
                               sin.cuda(), slots.cuda(), kc, vc, force=True)
    torch.cuda.synchronize()
    qkv = (x.float() @ w.float().T + b.float()).bfloat16()         # exact sum, one rounding
    heads = qkv.view(M, Hq + 2 * Hkv, D).transpose(0, 1)[None]
    ref = oracle_rope(heads, cos, sin, pos[None])[0].transpose(0, 1)
    assert torch.equal(q.cpu(), ref[:, :Hq])
    live = slots >= 0
    fk, fv = kc.view(-1, Hkv, D).cpu(), vc.view(-1, Hkv, D).cpu()
    assert torch.equal(fk[slots[live]], ref[live, Hq:Hq + Hkv])
    assert torch.equal(fv[slots[live]], qkv.view(M, -1, D)[live, Hq + Hkv:])
    untouched = torch.ones(NB * P, dtype=torch.bool)
    untouched[slots[live]] = False
    assert (fk[untouched] == 3.0).all() and (fv[untouched] == 5.0).all()
    # the unfused pair (linear, then rope_kv_write) gives the same bits
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    q2 = kernels.rope_kv_write(kernels.linear(x.cuda(), w.cuda(), b.cuda(), force=True), Hq, Hkv,
                               D, pos.cuda(), cos.cuda(), sin.cuda(), slots.cuda(), kc2, vc2)
    torch.cuda.synchronize()
    assert torch.equal(q, q2)


@pytest.mark.parametrize("M", [1, 32, 160])
def test_linear_rope_kv_random_data_within_rounding(M):
    """Random data: within a few bf16 roundings of RoPE applied in fp32 to
    the fp32 projection (a wrong index, sign or head would be off by O(1))."""
    from nanosglang_amd import kernels
    from nanosglang_amd.model.causal_lm import ModelConfig, rope_tables
    Hq, Hkv, D, K = 14, 2, 64, 896
    print(f"case: linear_rope_kv random M={M}", flush=True)
    x, w, b = _rope_case(M, Hq, Hkv, D, K, seed=100 + M, exact=False)
    cfg = ModelConfig(vocab_size=1000, hidden_size=896, intermediate_size=512,
                      num_hidden_layers=1, num_attention_heads=Hq, num_key_value_heads=Hkv,
                      max_position_embeddings=4096)
    cos, sin = rope_tables(cfg, "cpu")
    pos = torch.arange(M) * 17 % 4096
    slots = torch.arange(M) * 3
    kc = torch.zeros(M * 3, 1, Hkv, D, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    q = kernels.linear_rope_kv(x.cuda(), w.cuda(), b.cuda(), Hq, Hkv, D, pos.cuda(), cos.cuda(),
                               sin.cuda(), slots.cuda(), kc, vc, force=True)
    torch.cuda.synchronize()
    p = (x.float() @ w.float().T + b.float()).view(M, -1, D)
    x1, x2 = p[..., :D // 2], p[..., D // 2:]
    c, s = cos[pos][:, None], sin[pos][:, None]
    rot = torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], -1)
    mag = torch.cat([x1.abs() + x2.abs()] * 2, -1)
    bound = 2.0 ** -6 * mag + 1e-2
    got = torch.cat([q.cpu().float(), kc.view(-1, Hkv, D)[slots].cpu().float(),
                     vc.view(-1, Hkv, D)[slots].cpu().float()], 1)
    want = torch.cat([rot[:, :Hq + Hkv], p[:, Hq + Hkv:]], 1)
    err = (got - want).abs()
    print(f"  max err {err.max().item():.3e}", flush=True)
    assert (err <= bound).all()


def test_linear_rope_kv_flags_bad_slot_and_position():
    """Slots past the pool and positions outside the table set bit 0 of
    flags; the other rows are still written."""
    from nanosglang_amd._native import load
    from nanosglang_amd.kernels import _stream_ptr
    Hq, Hkv, D, K, M = 14, 2, 64, 896, 4
    print("case: linear_rope_kv flags", flush=True)
    lib = load()
    x, w, b = (t.cuda() for t in _rope_case(M, Hq, Hkv, D, K, seed=1, exact=True))
    cos = torch.rand(64, D // 2, device="cuda")
    sin = torch.rand(64, D // 2, device="cuda")
    q = torch.empty(M, Hq, D, dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros(8, Hkv, D, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    flags = torch.zeros(1, dtype=torch.int32, device="cuda")
    for pos_l, slot_l, want in (([0, 1, 2, 3], [0, 1, 2, 3], 0), ([0, 1, 2, 3], [0, 1, 8, 3], 1),
                                ([0, 64, 2, 3], [0, 1, 2, 3], 1)):
        flags.zero_()
        pos = torch.tensor(pos_l, device="cuda")
        slots = torch.tensor(slot_l, device="cuda")
        rc = lib.nsg_linear_rope_kv(x.data_ptr(), K, w.data_ptr(), K, b.data_ptr(), M, K, Hq, Hkv,
                                    D, pos.data_ptr(), cos.data_ptr(), sin.data_ptr(), 64,
                                    slots.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                    8, flags.data_ptr(), _stream_ptr(x.device))
        assert rc == 0
        torch.cuda.synchronize()
        assert flags.item() == want
