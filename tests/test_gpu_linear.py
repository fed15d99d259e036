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


@pytest.mark.parametrize("M,K", [(1, 256), (2, 256), (8, 256), (9, 256), (16, 256), (17, 256),
                                 (32, 256), (16, 2048), (24, 2048), (32, 4096)])
def test_linear_wide_output_matches_fp32_reference(M, K):
    """Very wide outputs (lm_head: N >= 65536 columns) take their own tile
    shapes, by row count and row length; N is not a multiple of any
    workgroup's columns."""
    from nanosglang_amd import kernels
    print(f"case: linear wide M={M} K={K}", flush=True)
    x, w, b = _data(M, 65540, K, seed=40 + M)
    y = kernels.linear(x, w, b, force=True)
    torch.cuda.synchronize()
    _check_bias(y, x, w, b)


@pytest.mark.parametrize("M", [1, 5, 16, 32, 33, 40, 64, 100, 128, 160])
@pytest.mark.parametrize("N,K", [(151936, 896), (65540, 896), (65540, 4096)])
def test_lm_head_rows_match_fp32_reference(M, N, K):
    """lm_head without a bias (rows shorter than 2048 at any row count, longer
    rows above 32: the kernel that shares x over 128 output columns, a
    persistent grid, an LDS ring fed by DMA): within one bf16 rounding of the
    fp32 reference; N = 65540 leaves 4 columns in the last 128-column
    tile."""
    from nanosglang_amd import kernels
    print(f"case: lm_head M={M} N={N} K={K}", flush=True)
    x, w, _ = _data(M, N, K, seed=60 + M + K)
    y = kernels.linear(x, w, None, force=True)
    torch.cuda.synchronize()
    _check_bias(y, x, w, None)


def test_lm_head_rows_do_not_depend_on_the_row_count():
    """Each output's K sum runs in k order in one wave: a row's logits are the
    same bits whether 1, 33 or 160 rows run (a verify batch and its padded
    graph batch agree, and so do draft and verify rows)."""
    from nanosglang_amd import kernels
    print("case: lm_head row independence", flush=True)
    x, w, _ = _data(160, 151936, 896, seed=77)
    full = kernels.linear(x, w, None, force=True)
    for M in (1, 7, 32, 33, 100):
        part = kernels.linear(x[:M], w, None, force=True)
        torch.cuda.synchronize()
        assert torch.equal(part, full[:M]), M


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


@pytest.mark.parametrize("M,I", [(40, 52), (160, 100), (150, 4864), (33, 196)])
def test_ring_swiglu_ragged_columns_and_out_buffer(M, I):
    """gate/up + SwiGLU from 33 rows (lm_head.hip's ring kernel: 48-column
    workgroups, row groups of up to 80): a last column tile that is partly
    past N, strided x rows and an out view with a wider row stride -- the
    fp32 reference within bf16 rounding, nothing written past N."""
    from nanosglang_amd import kernels
    K = 896
    print(f"case: ring swiglu M={M} I={I}", flush=True)
    x, w, _ = _data(M, I, K, seed=M + I, ldx=1024, rows=2 * I)
    out = torch.full((M, I + 12), 7.0, dtype=torch.bfloat16, device="cuda")[:, :I]
    y = kernels.linear(x, w, swiglu=True, out=out, force=True)
    torch.cuda.synchronize()
    assert y.data_ptr() == out.data_ptr()
    gu = x.float() @ w.float().T
    ref = torch.nn.functional.silu(gu[:, :I]) * gu[:, I:]
    assert ((y.float() - ref).abs() <= 2.0 ** -6 * ref.abs() + 2e-3).all()
    assert (out._base[:, I:] == 7.0).all()


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
    assert lib.nsg_linear_preferred(160, 151936, 896) == 1     # 0.5B lm_head
    assert lib.nsg_linear_preferred(161, 151936, 896) == 0
    assert lib.nsg_linear_preferred(32, 128256, 4096) == 1     # 8B lm_head
    assert lib.nsg_linear_preferred(33, 128256, 4096) == 0
    assert lib.nsg_linear_preferred(160, 896, 4864) == 1       # 0.5B down_proj
    assert lib.nsg_linear_preferred(64, 14336, 4096) == 0      # 8B-class weights
    assert lib.nsg_linear_preferred(32, 14336, 4096) == 1
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


# ---- FP8 weights (nsg_linear_fp8 / nsg_linear_rope_kv_fp8) ----

def test_fp8_kernel_decodes_every_e4m3_code():
    """One-hot x against a W8 whose row n holds code n: y[n] is the kernel's
    dequantised weight, which must be the oracle's bf16(decode(n) * scale)
    for all 256 codes (the OCP E4M3FN format, NaN codes included)."""
    import numpy as np
    from nanosglang_amd import kernels
    from oracle.quantization import fp8_dequant_bf16
    print("case: fp8 decode of all codes", flush=True)
    K = 64
    codes = torch.arange(256, dtype=torch.uint8)
    w8 = torch.zeros(256, K, dtype=torch.uint8)
    w8[:, 0] = codes
    w8 = w8.view(torch.float8_e4m3fn).cuda()
    x = torch.zeros(1, K, dtype=torch.bfloat16, device="cuda")
    x[0, 0] = 1.0
    for s in (1.0, 0.375, 3.0517578125e-05):       # bf16-exact scales (as applied)
        scale = torch.full((256,), s, dtype=torch.float32, device="cuda")
        y = kernels.linear(x, w8, None, w_scale=scale, force=True)
        torch.cuda.synchronize()
        got = y.float().cpu().numpy()[0]
        want = fp8_dequant_bf16(codes.numpy(), np.float32(s))
        assert np.array_equal(np.isnan(got), np.isnan(want))
        assert np.array_equal(got[~np.isnan(got)], want[~np.isnan(want)])


def test_fp8_dequant_matches_torch_on_the_gpu():
    """FP8Linear.forward's w8.to(bf16) * scale (0-dim fp32 scale) computed by
    torch on the GPU, the oracle's GPU form bf16(float(w8) * bf16(scale)) and
    the kernels' dequantisation with applied_scale agree bit for bit; the
    CPU form (scale kept in fp32) differs for most scales, so the check has
    teeth."""
    import numpy as np
    from nanosglang_amd import kernels
    from nanosglang_amd.model.quantization import applied_scale, fp8_quantize
    from oracle.quantization import fp8_dequant_bf16
    g = torch.Generator(device="cuda").manual_seed(3)
    cpu_form_differs = 0
    for t in range(40):
        w = torch.randn(64, 128, generator=g, device="cuda") * (0.001 + 0.37 * t)
        w8, s = fp8_quantize(w)
        ref = (w8.to(torch.bfloat16) * s).float().cpu().numpy()
        codes = w8.view(torch.uint8).cpu().numpy()
        assert np.array_equal(ref, fp8_dequant_bf16(codes, s.item(), scale_in_bf16=True)), t
        cpu_form_differs += not np.array_equal(ref, fp8_dequant_bf16(codes, s.item(), False))
        mine = kernels.dequant_fp8(w8, applied_scale(s).expand(64).contiguous())
        assert np.array_equal(mine.float().cpu().numpy(), ref), t
    assert cpu_form_differs >= 20


def test_fp8_dequant_kernel_all_codes_tails_and_strides():
    """nsg_dequant_fp8 (one pass, 16 bytes per thread) = torch's
    (float(w8) * row_scale).to(bf16) bit for bit: every e4m3 code, per-row
    scales, a column count with a scalar tail and rows wider than the copy."""
    from nanosglang_amd import kernels
    g = torch.Generator(device="cuda").manual_seed(7)
    for rows, cols, ld in ((256, 256, 256), (37, 1000, 1000), (9, 77, 96)):
        codes = torch.randint(0, 256, (rows, ld), generator=g, device="cuda", dtype=torch.int32)
        codes[:, :256 if cols >= 256 else cols] = torch.arange(256 if cols >= 256 else cols,
                                                                 device="cuda", dtype=torch.int32)
        base = codes.to(torch.uint8).view(torch.float8_e4m3fn)
        w8 = base[:, :cols]
        sc = torch.rand(rows, generator=g, device="cuda") * 3e-3 + 1e-5
        ref = (w8.float() * sc[:, None]).to(torch.bfloat16)
        got = kernels.dequant_fp8(w8, sc)
        nan = torch.isnan(ref)
        assert torch.equal(torch.isnan(got), nan)
        assert torch.equal(got[~nan].view(torch.int16), ref[~nan].view(torch.int16)), (rows, cols)


# bf16 gate/up + SwiGLU runs lm_head.hip's ring kernel from this many rows on
# (another K order than the weight-streaming kernel the FP8 weights use)
RING_SWIGLU_MIN_ROWS = 33


def _check_same_swiglu(y8, yb, M):
    """FP8 SwiGLU against bf16 SwiGLU on the dequantised weights: bit for bit
    while both run the weight-streaming kernel, else within the bf16
    rounding of two fp32 sums in different orders."""
    if M < RING_SWIGLU_MIN_ROWS:
        assert torch.equal(y8, yb)
    else:
        assert ((y8.float() - yb.float()).abs() <= 2.0 ** -6 * yb.float().abs() + 2e-3).all()


def _fp8_weights(rows_blocks, K, seed):
    from nanosglang_amd.model.quantization import fp8_quantize_rows
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(sum(rows_blocks), K, generator=g, device="cuda") * K ** -0.5
    for i, n in enumerate(rows_blocks):           # blocks of different magnitude
        w[sum(rows_blocks[:i]):sum(rows_blocks[:i]) + n] *= (1 + 3 * i)
    return fp8_quantize_rows(w, rows_blocks)


@pytest.mark.parametrize("M", [1, 16, 17, 32, 33, 64, 100, 160])
def test_fp8_linear_bit_exact_vs_bf16_kernel_on_dequantized_weights(M):
    """The FP8 kernels compute exactly what the bf16 kernels compute on the
    dequantised weights (bias, SwiGLU and RoPE + KV-write epilogues; SwiGLU
    from 33 rows within rounding, see _check_same_swiglu), and stay within
    bf16 rounding of an fp32 product."""
    from nanosglang_amd import kernels
    print(f"case: fp8 linear M={M}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(M)
    x = torch.randn(M, 896, generator=g, device="cuda").bfloat16()
    b = torch.randn(1152, generator=g, device="cuda").bfloat16()
    w8, s = _fp8_weights([896, 128, 128], 896, seed=M)
    wd = kernels.dequant_fp8(w8, s)
    y8 = kernels.linear(x, w8, b, w_scale=s, force=True)
    yb = kernels.linear(x, wd, b, force=True)
    torch.cuda.synchronize()
    assert torch.equal(y8, yb)
    _check_bias(y8, x, wd, b)
    # SwiGLU with separate gate / up scales
    g8, gs = _fp8_weights([512, 512], 896, seed=M + 1)
    ys8 = kernels.linear(x, g8, swiglu=True, w_scale=gs, force=True)
    ysb = kernels.linear(x, kernels.dequant_fp8(g8, gs), swiglu=True, force=True)
    torch.cuda.synchronize()
    _check_same_swiglu(ys8, ysb, M)
    # RoPE + KV write (q, k, v blocks with their own scales)
    from nanosglang_amd.model.causal_lm import ModelConfig, rope_tables
    cfg = ModelConfig(vocab_size=1000, hidden_size=896, intermediate_size=512,
                      num_hidden_layers=1, num_attention_heads=14, num_key_value_heads=2,
                      max_position_embeddings=2048)
    cos, sin = (t.cuda() for t in rope_tables(cfg, "cpu"))
    pos = (torch.arange(M, device="cuda") * 13) % 2048
    slots = torch.arange(M, device="cuda") * 2
    kc = torch.zeros(2 * M, 1, 2, 64, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    q8 = kernels.linear_rope_kv(x, w8, b, 14, 2, 64, pos, cos, sin, slots, kc, vc, w_scale=s,
                                force=True)
    qb = kernels.linear_rope_kv(x, wd, b, 14, 2, 64, pos, cos, sin, slots, kc2, vc2, force=True)
    torch.cuda.synchronize()
    assert torch.equal(q8, qb) and torch.equal(kc, kc2) and torch.equal(vc, vc2)


@pytest.mark.parametrize("M", [1, 32, 64, 160])
def test_fp8_linear_8b_shapes(M):
    """FP8 weights at the large shape's decoder linears (hidden 4096, 32 / 8
    heads of 128, FFN 14336): q/k/v 6144 x 4096 with RoPE + KV write, o_proj
    4096 x 4096, gate_up 28672 x 4096 with SwiGLU, down 4096 x 14336.  Each
    is bit-exact against the bf16 kernel on the dequantised weights (the
    weight-streaming kernel's 8B-class tile shapes, bf16 and FP8 alike) and
    within bf16 rounding of an fp32 product."""
    from nanosglang_amd import kernels
    from nanosglang_amd.model.causal_lm import ModelConfig, rope_tables
    print(f"case: fp8 linear, 8B shapes, M={M}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(100 + M)
    H, I, Hq, Hkv, D = 4096, 14336, 32, 8, 128
    x = torch.randn(M, H, generator=g, device="cuda").bfloat16()
    # q/k/v: bias path (no bias, as Llama) and RoPE + KV write
    w8, s = _fp8_weights([Hq * D, Hkv * D, Hkv * D], H, seed=M + 7)
    wd = kernels.dequant_fp8(w8, s)
    y8 = kernels.linear(x, w8, w_scale=s, force=True)
    assert torch.equal(y8, kernels.linear(x, wd, force=True))
    _check_bias(y8, x, wd, None)
    cfg = ModelConfig(model_type="llama", vocab_size=1000, hidden_size=H, intermediate_size=I,
                      num_hidden_layers=1, num_attention_heads=Hq, num_key_value_heads=Hkv,
                      max_position_embeddings=8192, rope_theta=5e5, attention_bias=False)
    cos, sin = (t.cuda() for t in rope_tables(cfg, "cpu"))
    pos = (torch.arange(M, device="cuda") * 37 + 2048) % 8192
    slots = torch.arange(M, device="cuda") * 3
    caches = [torch.zeros(3 * M, 1, Hkv, D, dtype=torch.bfloat16, device="cuda")
              for _ in range(4)]
    q8 = kernels.linear_rope_kv(x, w8, None, Hq, Hkv, D, pos, cos, sin, slots, caches[0],
                                caches[1], w_scale=s, force=True)
    qb = kernels.linear_rope_kv(x, wd, None, Hq, Hkv, D, pos, cos, sin, slots, caches[2],
                                caches[3], force=True)
    torch.cuda.synchronize()
    assert torch.equal(q8, qb)
    assert torch.equal(caches[0], caches[2]) and torch.equal(caches[1], caches[3])
    # o_proj
    w8, s = _fp8_weights([H], H, seed=M + 8)
    wd = kernels.dequant_fp8(w8, s)
    y8 = kernels.linear(x, w8, w_scale=s, force=True)
    assert torch.equal(y8, kernels.linear(x, wd, force=True))
    _check_bias(y8, x, wd, None)
    # gate_up with SwiGLU (separate gate / up scales)
    w8, s = _fp8_weights([I, I], H, seed=M + 9)
    wd = kernels.dequant_fp8(w8, s)
    y8 = kernels.linear(x, w8, swiglu=True, w_scale=s, force=True)
    _check_same_swiglu(y8, kernels.linear(x, wd, swiglu=True, force=True), M)
    gu = x.float() @ wd.float().T
    ref = torch.nn.functional.silu(gu[:, :I]) * gu[:, I:]
    assert ((y8.float() - ref).abs() <= 2.0 ** -6 * ref.abs() + 2e-3).all()
    del w8, wd, gu
    # down
    xd = torch.randn(M, I, generator=g, device="cuda").bfloat16()
    w8, s = _fp8_weights([H], I, seed=M + 10)
    wd = kernels.dequant_fp8(w8, s)
    y8 = kernels.linear(xd, w8, w_scale=s, force=True)
    assert torch.equal(y8, kernels.linear(xd, wd, force=True))
    _check_bias(y8, xd, wd, None)


def test_fp8_linear_library_path_for_prefill_rows():
    from nanosglang_amd import kernels
    print("case: fp8 linear M=300 (library path)", flush=True)
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(300, 896, generator=g, device="cuda").bfloat16()
    w8, s = _fp8_weights([1152], 896, seed=5)
    y = kernels.linear(x, w8, None, w_scale=s)
    torch.cuda.synchronize()
    _check_bias(y, x, kernels.dequant_fp8(w8, s), None)


def test_fp8linear_module_matches_reference_arithmetic():
    """FP8Linear (the reference's module interface) on the GPU: from_linear,
    then forward == F.linear(x, w8.to(bf16) * scale, bias) within bf16 rounding,
    and quantize_model swaps every nn.Linear outside the skip list."""
    from nanosglang_amd.model.quantization import FP8Linear, quantize_model
    print("case: FP8Linear module", flush=True)
    torch.manual_seed(0)
    lin = torch.nn.Linear(896, 1152, bias=True).cuda().to(torch.bfloat16)
    m = FP8Linear.from_linear(lin)
    x = torch.randn(3, 7, 896, device="cuda").bfloat16()
    y = m(x)
    ref = torch.nn.functional.linear(x.float(), (m.weight_fp8.to(torch.bfloat16)
                                                 * m.weight_scale).float(), m.bias.float())
    torch.cuda.synchronize()
    assert y.shape == (3, 7, 1152)
    assert ((y.float() - ref).abs() <= 2.0 ** -8 * ref.abs() + 3e-3).all()
    net = torch.nn.ModuleDict({"mlp": torch.nn.Linear(64, 64), "lm_head": torch.nn.Linear(64, 10)})
    quantize_model(net)
    assert isinstance(net["mlp"], FP8Linear) and isinstance(net["lm_head"], torch.nn.Linear)


@pytest.mark.parametrize("M", [1, 5, 8, 16, 17, 32, 33, 100, 160])
@pytest.mark.parametrize("N,K,bias", [(151936, 896, False), (65540, 896, False),
                                      (4096, 512, True), (1000, 128, False)])
def test_linear_argmax_equals_argmax_of_linear(M, N, K, bias):
    """nsg_linear_argmax: the greedy token of each row is the first-index
    argmax of exactly the bf16 rows the HIP linear kernel writes (same tile
    shapes, same accumulation order), bit for bit."""
    from nanosglang_amd import kernels
    print(f"case: linear_argmax M={M} N={N} K={K} bias={bias}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(M * 7 + N)
    x = torch.randn(M, K, generator=g, device="cuda").bfloat16()
    w = (torch.randn(N, K, generator=g, device="cuda") * K ** -0.5).bfloat16()
    b = torch.randn(N, generator=g, device="cuda").bfloat16() if bias else None
    tok = kernels.linear_argmax(x, w, b)
    y = kernels.linear(x, w, b, force=True)
    torch.cuda.synchronize()
    assert torch.equal(tok, y.float().argmax(dim=1))


@pytest.mark.parametrize("M,zero_bias", [(6, True), (6, False), (40, False), (160, False)])
def test_linear_argmax_ties_take_the_lowest_column(M, zero_bias):
    """Equal maxima (duplicated weight rows, in one workgroup's columns and in
    different workgroups', and +0 against -0) resolve to the lowest column,
    as torch.argmax and the reference's greedy sample_token do (with a zero
    bias: the weight-streaming kernel; without: the lm_head kernel, whose
    keys meet across lanes, waves and workgroups)."""
    from nanosglang_amd import kernels
    print(f"case: linear_argmax ties M={M} zero_bias={zero_bias}", flush=True)
    N, K = 151936, 896
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(M, K, generator=g, device="cuda").bfloat16()
    w = (torch.randn(N, K, generator=g, device="cuda") * K ** -0.5).bfloat16()
    # rows 0-1: a large row duplicated at columns 70001 and 9 (other tiles);
    # rows 2-3: duplicated at 40 and 41 (one tile)
    big = (x[0].float() * 0.5).bfloat16()
    w[9] = big
    w[70001] = big
    w[41] = (x[2].float() * 0.5).bfloat16()
    w[40] = w[41]
    # rows 4-5: x = 0 -> every logit is +0 or -0: the first column wins
    x[4:6] = 0
    b = torch.zeros(N, dtype=torch.bfloat16, device="cuda") if zero_bias else None
    tok = kernels.linear_argmax(x, w, b).cpu().tolist()
    torch.cuda.synchronize()
    assert tok[0] == 9 and tok[2] == 40 and tok[4] == 0 and tok[5] == 0


def test_linear_argmax_writes_a_strided_column():
    """The tokens may go straight into a column of a (B, k+1) id buffer: the
    other columns stay untouched."""
    from nanosglang_amd import kernels
    print("case: linear_argmax strided out", flush=True)
    M, N, K = 32, 151936, 896
    g = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(M, K, generator=g, device="cuda").bfloat16()
    w = (torch.randn(N, K, generator=g, device="cuda") * K ** -0.5).bfloat16()
    buf = torch.full((M, 5), -7, dtype=torch.int64, device="cuda")
    kernels.linear_argmax(x, w, out=buf[:, 2])
    ref = kernels.linear_argmax(x, w)
    torch.cuda.synchronize()
    assert torch.equal(buf[:, 2], ref)
    assert (buf[:, [0, 1, 3, 4]] == -7).all()
