"""FP8 weights for the decoder's linear layers on MI355X.

Mirrors nano_sglang/decode/quantization.py's FP8 path:

* ``fp8_quantize(w)`` -- ``FP8Linear.from_linear`` (:54-75): per-tensor
  ``scale = absmax / 448`` (1 for an all-zero tensor), weights cast to
  float8_e4m3fn (OCP E4M3, gfx950's native FP8 format);
* ``FP8Linear`` -- same constructor, buffers (``weight_fp8``,
  ``weight_scale``), ``bias`` and ``from_linear`` as the reference (:24-75);
  ``forward`` computes ``x @ (w8.to(bf16) * scale).T + bias`` (:49-52) with
  the HIP weight-streaming kernel reading the FP8 bytes directly
  (``kernels.linear``, C ABI ``nsg_linear_fp8``);
* ``quantize_model`` -- the reference's module walk (:202-243) for FP8
  (AWQ/INT4 is not implemented here).

``CausalLM.quantize_fp8()`` applies the same per-tensor rule to the packed
decoder weights (q, k and v, and gate and up, keep separate scales, as the
reference's separate ``nn.Linear`` modules do).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .. import kernels

E4M3_MAX = 448.0


def fp8_quantize(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-tensor FP8 quantisation -> (float8_e4m3fn weight, fp32 0-dim scale)."""
    w = weight.detach().float()
    scale = w.abs().max() / E4M3_MAX
    if scale == 0:
        scale = torch.ones((), device=w.device)
    return (w / scale).to(torch.float8_e4m3fn), scale.reshape(()).float()


def applied_scale(scale: torch.Tensor) -> torch.Tensor:
    """The scale FP8Linear.forward's ``w8.to(bf16) * scale`` applies on the
    GPU: torch casts the 0-dim fp32 operand to bf16 (the common dtype) before
    the product, so the kernels get float(bf16(scale))."""
    return scale.float().to(torch.bfloat16).float()


def fp8_quantize_rows(weight: torch.Tensor, row_blocks: list[int]) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantise stacked tensors (``row_blocks`` rows each) with one scale per
    tensor -> (float8_e4m3fn weight, fp32 per-row applied scale)."""
    assert sum(row_blocks) == weight.shape[0]
    w8s, scales = [], []
    r = 0
    for n in row_blocks:
        w8, s = fp8_quantize(weight[r:r + n])
        w8s.append(w8)
        scales.append(applied_scale(s).expand(n))
        r += n
    return torch.cat(w8s).contiguous(), torch.cat(scales).contiguous()


class FP8Linear(nn.Module):
    """Linear layer with FP8 weight storage (quantization.py:24-75)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.register_buffer("weight_fp8",
                             torch.zeros(out_features, in_features, dtype=torch.float8_e4m3fn))
        self.register_buffer("weight_scale", torch.ones(()))
        self.bias = nn.Parameter(torch.zeros(out_features)) if bias else None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.in_features)
        if x2.is_cuda and x2.dtype == torch.bfloat16 and (
                self.bias is None or self.bias.dtype == torch.bfloat16):
            rows = applied_scale(self.weight_scale.reshape(())).expand(self.out_features)
            rows = rows.contiguous()
            y = kernels.linear(x2.contiguous(), self.weight_fp8, self.bias, w_scale=rows)
        else:   # the reference's arithmetic on other devices / dtypes
            w = self.weight_fp8.to(x.dtype) * self.weight_scale
            y = torch.nn.functional.linear(x2, w, self.bias)
        return y.reshape(*lead, self.out_features)

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> "FP8Linear":
        has_bias = linear.bias is not None
        m = cls(linear.in_features, linear.out_features, bias=has_bias)
        w8, scale = fp8_quantize(linear.weight.data)
        m.weight_fp8 = w8
        m.weight_scale = scale.to(linear.weight.device)
        if has_bias:
            m.bias = nn.Parameter(linear.bias.data.clone())
        return m


def quantize_model(model: nn.Module, method: str = "fp8", group_size: int = 128,
                   skip_modules: list[str] | None = None) -> nn.Module:
    """Replace every nn.Linear of ``model`` with FP8Linear, in place
    (quantization.py:202-243; the same default skip list)."""
    if method != "fp8":
        raise NotImplementedError(f"quantization method {method!r}: only 'fp8' is built")
    if skip_modules is None:
        skip_modules = ["embed_tokens", "lm_head", "norm"]
    # A linear is skipped when any skip substring occurs in its dotted path
    # (a parent's name is a prefix of that path, so one test covers both
    # levels the reference checks).  Targets are collected first, then swapped.
    targets = [path for path, mod in model.named_modules()
               if isinstance(mod, nn.Linear) and not any(s in path for s in skip_modules)]
    for path in targets:
        parent_path, _, attr = path.rpartition(".")
        parent = model.get_submodule(parent_path) if parent_path else model
        setattr(parent, attr, FP8Linear.from_linear(getattr(parent, attr)))
    return model
