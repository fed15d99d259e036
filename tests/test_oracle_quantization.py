"""The FP8 (OCP E4M3FN) restatement against torch's own float8_e4m3fn casts
(torch is the reference's dependency for this arithmetic,
nano_sglang/decode/quantization.py:13,68), and the product's per-tensor
quantiser against the restatement."""
import numpy as np
import torch

from oracle.quantization import e4m3_decode, e4m3_encode, fp8_dequant_bf16, fp8_quantize


def _torch_decode(codes):
    return torch.from_numpy(np.asarray(codes, np.uint8)).view(torch.float8_e4m3fn).float().numpy()


def test_decode_every_code_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    t, o = _torch_decode(codes), e4m3_decode(codes)
    assert np.array_equal(np.isnan(t), np.isnan(o)) and np.isnan(o).sum() == 2
    assert np.array_equal(t[~np.isnan(t)], o[~np.isnan(o)])
    assert np.nanmax(o) == 448.0 and o[1] == 2.0 ** -9    # largest finite, smallest subnormal
    # power: the other 8-bit E4M3 encoding (exponent bias 8, no negative zero)
    # decodes differently, so a format mix-up cannot pass this test
    e, m = (codes.astype(int) >> 3) & 15, codes & 7
    fnuz = np.where(e == 0, m / 8 * 2.0 ** -7, (1 + m / 8) * 2.0 ** (e - 8.0))
    assert not np.array_equal(fnuz[1:127], o[1:127])


def _cases():
    b = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float()
    b = b[torch.isfinite(b) & (b.abs() <= 480)].numpy()
    g = np.random.default_rng(0)
    vals = e4m3_decode(np.arange(256, dtype=np.uint8))
    vals = np.sort(vals[np.isfinite(vals) & (vals >= 0)])
    ties = (vals[:-1] + vals[1:]) / 2                     # exact midpoints: ties to even
    return np.concatenate([b, g.standard_normal(50000).astype(np.float32) * 40,
                           (g.standard_normal(50000) * 1e-3).astype(np.float32),
                           ties.astype(np.float32), -ties.astype(np.float32),
                           np.array([463.9, 464.0, 470.0, 0.0, -0.0], np.float32)])


def test_encode_matches_torch_cast():
    x = _cases()
    tc = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    oc = e4m3_encode(x)
    both_nan = np.isnan(_torch_decode(tc)) & np.isnan(e4m3_decode(oc))
    assert ((tc == oc) | both_nan).all()


def test_product_quantizer_matches_restatement():
    from nanosglang_amd.model.quantization import fp8_quantize as product_quantize
    g = torch.Generator().manual_seed(1)
    for w in (torch.randn(96, 64, generator=g) * 0.02, torch.randn(7, 13, generator=g) * 5,
              torch.zeros(4, 8)):
        w8, s = product_quantize(w)
        codes, so = fp8_quantize(w.numpy())
        assert s.dtype == torch.float32 and s.item() == float(so)
        assert np.array_equal(w8.view(torch.uint8).numpy(), codes)
        # the reference's forward arithmetic, w8.to(bf16) * scale, on the CPU
        # (torch keeps a 0-dim fp32 operand in fp32 there)
        deq = (w8.to(torch.bfloat16) * s).float().numpy()
        assert np.array_equal(deq, fp8_dequant_bf16(codes, so, scale_in_bf16=False))
