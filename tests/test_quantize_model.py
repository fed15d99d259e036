"""quantize_model's module walk (CPU): every nn.Linear whose dotted path
holds none of the skip substrings becomes an FP8Linear carrying the
per-tensor absmax / 448 scale; skipped ones -- by their own name or by a
parent's -- stay nn.Linear (nano_sglang/decode/quantization.py:202-243)."""
import torch
import torch.nn as nn

from nanosglang_amd.model.quantization import FP8Linear, quantize_model


def _net():
    torch.manual_seed(0)
    layer = nn.ModuleDict({"q_proj": nn.Linear(32, 32), "post_norm": nn.Linear(32, 32),
                           "mlp": nn.Sequential(nn.Linear(32, 64), nn.SiLU(), nn.Linear(64, 32))})
    return nn.ModuleDict({
        "embed_tokens": nn.Embedding(10, 32),
        "layers": nn.ModuleList([layer]),
        "norm": nn.ModuleDict({"inner": nn.Linear(32, 32)}),   # skipped through its parent
        "lm_head": nn.Linear(32, 10, bias=False),
    })


def test_quantize_model_replaces_exactly_the_unskipped_linears():
    net = _net()
    before = {n: m.weight.detach().clone() for n, m in net.named_modules()
              if isinstance(m, nn.Linear)}
    quantize_model(net)
    kinds = {n: type(m) for n, m in net.named_modules() if isinstance(m, (nn.Linear, FP8Linear))}
    assert kinds == {
        "layers.0.q_proj": FP8Linear, "layers.0.post_norm": nn.Linear,
        "layers.0.mlp.0": FP8Linear, "layers.0.mlp.2": FP8Linear,
        "norm.inner": nn.Linear, "lm_head": nn.Linear,
    }
    for name in ("layers.0.q_proj", "layers.0.mlp.0", "layers.0.mlp.2"):
        m = net.get_submodule(name)
        w = before[name].float()
        assert torch.equal(m.weight_scale, w.abs().max() / 448.0)
        assert torch.equal(m.weight_fp8, (w / m.weight_scale).to(torch.float8_e4m3fn))
        assert m.bias is not None


def test_quantize_model_custom_skip_list_and_forward_on_cpu():
    net = _net()
    quantize_model(net, skip_modules=["mlp"])
    assert isinstance(net["lm_head"], FP8Linear)
    assert isinstance(net.get_submodule("layers.0.mlp.0"), nn.Linear)
    x = torch.randn(3, 32)
    m = net["lm_head"]
    ref = torch.nn.functional.linear(x, m.weight_fp8.to(torch.float32) * m.weight_scale)
    assert torch.equal(m(x), ref)
