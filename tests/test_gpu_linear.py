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


@pytest.mark.parametrize("M", [1, 7, 16, 32, 33, 48, 80, 96, 100, 128, 160])
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


@pytest.mark.parametrize("M", [1, 32, 64, 96, 160])
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
    assert lib.nsg_linear_preferred(32, 151936, 896) == 0
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
