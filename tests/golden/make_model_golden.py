"""Writes tests/golden/model_forward_golden.npz: fp32 CPU logits of the
reference's own CausalLM.forward (nano_sglang/model/causal_lm.py:564-583) on a
tiny random-init Qwen2-style config, the vectors that pin the oracle's model
restatement (oracle/model.py) to the reference bit for bit.

Runs only where the reference sources are present (it imports them from
/root/reference); the tests read the committed .npz alone:

    python tests/golden/make_model_golden.py

Contents (numpy arrays, no pickles):
  cfg_*            the config fields;
  w_*              every weight (float32), drawn here from a seeded numpy
                   generator: linears / embedding ~ N(0, 0.05^2), q/k/v biases
                   ~ N(0, 0.05^2), RMSNorm weights 1 + N(0, 0.1^2); lm_head is the
                   embedding (tied, as Qwen2.5-0.5B);
  full_ids / full_logits
                   one forward over 2 x 7 tokens from position 0 with the
                   causal mask, through a zeroed contiguous cache;
  inc_ids_0 / inc_logits_0, inc_ids_1 / inc_logits_1
                   the same cache written incrementally: 5 prompt tokens, then
                   a 3-token verify-style call at position 5 with the
                   bottom-right causal mask (causal_lm.py:400-415).
"""
import os
import sys

import numpy as np
import torch

REF = "/root/reference"
sys.path.insert(0, REF)
from nano_sglang.model.causal_lm import CausalLM, ModelConfig  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "model_forward_golden.npz")

CFG = dict(model_type="qwen2", vocab_size=61, hidden_size=32, intermediate_size=48,
           num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
           max_position_embeddings=64, rms_norm_eps=1e-6, rope_theta=1e6,
           tie_word_embeddings=True, torch_dtype="float32", attention_bias=True)


def mask(seq, full):
    row = torch.arange(seq)[:, None]
    col = torch.arange(full)[None, :]
    return torch.where(col <= (full - seq) + row, 0.0, float("-inf"))[None, None]


def main():
    torch.manual_seed(0)
    cfg = ModelConfig(**CFG)
    model = CausalLM(cfg).float().eval()
    rng = np.random.default_rng(20261201)
    H, I = cfg.hidden_size, cfg.intermediate_size
    Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    w = {}

    def n(name, *shape, scale=0.05, base=0.0):
        w[name] = (base + rng.standard_normal(shape) * scale).astype(np.float32)
        return torch.from_numpy(w[name])

    with torch.no_grad():
        model.embed_tokens.weight.copy_(n("embed", cfg.vocab_size, H))
        model.lm_head.weight.copy_(model.embed_tokens.weight)
        for i, L in enumerate(model.layers):
            a = L.self_attn
            a.q_proj.weight.copy_(n(f"l{i}_q", Hq * D, H))
            a.q_proj.bias.copy_(n(f"l{i}_qb", Hq * D))
            a.k_proj.weight.copy_(n(f"l{i}_k", Hkv * D, H))
            a.k_proj.bias.copy_(n(f"l{i}_kb", Hkv * D))
            a.v_proj.weight.copy_(n(f"l{i}_v", Hkv * D, H))
            a.v_proj.bias.copy_(n(f"l{i}_vb", Hkv * D))
            a.o_proj.weight.copy_(n(f"l{i}_o", H, Hq * D))
            L.mlp.gate_proj.weight.copy_(n(f"l{i}_gate", I, H))
            L.mlp.up_proj.weight.copy_(n(f"l{i}_up", I, H))
            L.mlp.down_proj.weight.copy_(n(f"l{i}_down", H, I))
            L.input_layernorm.weight.copy_(n(f"l{i}_ln1", H, scale=0.1, base=1.0))
            L.post_attention_layernorm.weight.copy_(n(f"l{i}_ln2", H, scale=0.1, base=1.0))
        model.norm.weight.copy_(n("norm", H, scale=0.1, base=1.0))

        def cache(B, S):
            return [(torch.zeros(B, Hkv, S, D), torch.zeros(B, Hkv, S, D))
                    for _ in range(cfg.num_hidden_layers)]

        out = {f"cfg_{k}": np.asarray(v) for k, v in CFG.items() if k not in ("model_type",
                                                                           "torch_dtype")}
        out.update({f"w_{k}": v for k, v in w.items()})
        ids = torch.from_numpy(rng.integers(0, cfg.vocab_size, (2, 7)))
        pos = torch.arange(7)[None].expand(2, 7)
        out["full_ids"] = ids.numpy()
        out["full_logits"] = model(ids, pos, cache(2, 16), 0, mask(7, 7)).numpy()
        kv = cache(1, 16)
        ids0 = torch.from_numpy(rng.integers(0, cfg.vocab_size, (1, 5)))
        out["inc_ids_0"] = ids0.numpy()
        out["inc_logits_0"] = model(ids0, torch.arange(5)[None], kv, 0, mask(5, 5)).numpy()
        ids1 = torch.from_numpy(rng.integers(0, cfg.vocab_size, (1, 3)))
        out["inc_ids_1"] = ids1.numpy()
        out["inc_logits_1"] = model(ids1, torch.arange(5, 8)[None], kv, 5, mask(3, 8)).numpy()
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
