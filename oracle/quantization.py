"""FP8 (OCP E4M3FN) weight quantisation, restated in numpy (oracle side).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows nano_sglang/decode/quantization.py:
  * ``FP8Linear.from_linear`` (:54-75): per-tensor ``scale = absmax / 448``
    (``scale = 1`` when the tensor is all zero), ``w8 = (w / scale)`` cast
    to float8_e4m3fn;
  * ``FP8Linear.forward`` (:49-52): ``w8.to(x.dtype) * scale`` then
    ``F.linear``.  With x in bf16 the product of the bf16 tensor and the 0-dim
    fp32 ``scale`` follows torch's type promotion, which differs by device:
    on the GPU (where the reference runs it) the 0-dim operand is cast to
    the common dtype first, ``bf16(float(w8) * float(bf16(scale)))``; on the
    CPU the scale stays fp32, ``bf16(float(w8) * scale)``.  Both are
    ``fp8_dequant_bf16``; ``scale_in_bf16`` picks the device (checked against
    torch on each: tests/test_oracle_quantization.py, tests/test_gpu_linear.py).

E4M3FN (the OCP 8-bit float torch.float8_e4m3fn names): 1 sign, 4 exponent
(bias 7), 3 mantissa bits; no infinities; S.1111.111 is NaN, so the largest
finite magnitude is 448 (S.1111.110); subnormals below 2^-6 in steps of 2^-9.
Encoding rounds to nearest, ties to even, at every exponent (subnormals
included); magnitudes that round above 448 (>= 464) become NaN, as
torch's conversion does.

Pinning: ``e4m3_decode`` against torch.float8_e4m3fn -> float32 on all 256
codes, and ``e4m3_encode`` against torch's float32 -> float8_e4m3fn cast on
every bf16-representable value in [-480, 480] plus seeded random floats,
including exact ties (tests/test_oracle_quantization.py).  Torch is the
reference's own dependency for this arithmetic (quantization.py:13,68).
"""
import numpy as np

E4M3_MAX = 448.0


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """uint8 codes -> float32 values (NaN for S.1111.111)."""
    c = np.asarray(codes, np.uint8).astype(np.int32)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * 2.0 ** (e - 7.0))
    val = np.where((e == 15) & (m == 7), np.nan, val)
    return (sign * val).astype(np.float32)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> uint8 codes, round to nearest even; |x| rounding past 448 -> NaN."""
    x = np.asarray(x, np.float32).astype(np.float64)
    sign = np.where(np.signbit(x), 0x80, 0).astype(np.int32)
    a = np.abs(x)
    # exponent of the target binade (subnormals share the 2^-6 binade's step)
    e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    e = np.clip(e, -6, 8)
    step = 2.0 ** (e - 3)                       # spacing of representable values
    q = a / step
    r = np.floor(q)
    frac = q - r
    r = r + ((frac > 0.5) | ((frac == 0.5) & (r % 2 == 1)))
    mag = r * step                              # rounded magnitude
    out = np.zeros(a.shape, np.int32)
    # re-derive exponent / mantissa of the rounded magnitude
    nz = mag > 0
    e2 = np.floor(np.log2(np.where(nz, mag, 1.0)))
    sub = nz & (e2 < -6)
    norm = nz & ~sub
    m_sub = np.round(mag / 2.0 ** -9).astype(np.int32)           # 1..7
    m_norm = np.round((mag / 2.0 ** e2 - 1.0) * 8).astype(np.int32)
    out = np.where(sub, m_sub, out)
    out = np.where(norm, ((e2 + 7).astype(np.int32) << 3) | m_norm, out)
    nan = np.isnan(x) | (mag > E4M3_MAX)
    out = np.where(nan, 0x7F, out)
    return (out | sign).astype(np.uint8)


def fp8_quantize(w: np.ndarray):
    """Per-tensor FP8Linear.from_linear (quantization.py:60-70) ->
    (codes uint8, scale float32)."""
    w = np.asarray(w, np.float32)
    amax = np.float32(np.abs(w).max()) if w.size else np.float32(0)
    scale = np.float32(amax / np.float32(E4M3_MAX))
    if scale == 0:
        scale = np.float32(1.0)
    return e4m3_encode((w / scale).astype(np.float32)), scale


def _bf16_round(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, np.float32)
    u = v.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return np.where(np.isnan(v), np.float32(np.nan), u.astype(np.uint32).view(np.float32))


def fp8_dequant_bf16(codes: np.ndarray, scale, scale_in_bf16: bool = True) -> np.ndarray:
    """FP8Linear.forward's dequantised bf16 weights as float32 values (:51):
    bf16(float(w8) * s) with s = bf16(scale) (GPU, default) or scale (CPU)."""
    s = _bf16_round(np.float32(scale)) if scale_in_bf16 else np.float32(scale)
    v = (e4m3_decode(codes) * np.float32(s)).astype(np.float32)
    u = v.view(np.uint32).astype(np.uint64)
    nan = np.isnan(v)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = u.astype(np.uint32).view(np.float32)
    return np.where(nan, np.float32(np.nan), out)
