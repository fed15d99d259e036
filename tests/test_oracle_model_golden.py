"""Pins the oracle's model restatement (oracle/model.py) to the reference's
own CausalLM.forward (nano_sglang/model/causal_lm.py:564-583): the fp32 CPU
logits in tests/golden/model_forward_golden.npz were written by
tests/golden/make_model_golden.py from the reference itself, on a tiny
Qwen2-style config with every weight random (biases and norm weights too).
The oracle must reproduce them bit for bit: same ops in the same order."""
import os

import numpy as np
import torch

from oracle.model import CPUCausalLM, ModelConfig, causal_mask

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "model_forward_golden.npz")


def _model():
    z = np.load(GOLDEN)
    c = {k[4:]: z[k].item() for k in z.files if k.startswith("cfg_")}
    cfg = ModelConfig(vocab_size=c["vocab_size"], hidden_size=c["hidden_size"],
                      intermediate_size=c["intermediate_size"],
                      num_hidden_layers=c["num_hidden_layers"],
                      num_attention_heads=c["num_attention_heads"],
                      num_key_value_heads=c["num_key_value_heads"],
                      max_position_embeddings=c["max_position_embeddings"],
                      rms_norm_eps=c["rms_norm_eps"], rope_theta=c["rope_theta"],
                      attention_bias=c["attention_bias"],
                      tie_word_embeddings=c["tie_word_embeddings"])
    t = lambda k: torch.from_numpy(z[f"w_{k}"])
    w = {"embed": t("embed"), "norm": t("norm"), "layers": []}
    for i in range(cfg.num_hidden_layers):
        w["layers"].append({
            "q": t(f"l{i}_q"), "k": t(f"l{i}_k"), "v": t(f"l{i}_v"), "o": t(f"l{i}_o"),
            "qb": t(f"l{i}_qb"), "kb": t(f"l{i}_kb"), "vb": t(f"l{i}_vb"),
            "gate": t(f"l{i}_gate"), "up": t(f"l{i}_up"), "down": t(f"l{i}_down"),
            "ln1": t(f"l{i}_ln1"), "ln2": t(f"l{i}_ln2")})
    return z, cfg, CPUCausalLM(cfg, w)


def test_full_forward_is_bit_exact_with_the_reference():
    z, cfg, m = _model()
    ids = torch.from_numpy(z["full_ids"])
    B, S = ids.shape
    got = m.forward(ids, torch.arange(S)[None].expand(B, S), m.new_cache(B, 16), 0,
                    causal_mask(S, S))
    assert got.dtype == torch.float32
    np.testing.assert_array_equal(got.numpy(), z["full_logits"])


def test_incremental_forward_with_cache_is_bit_exact_with_the_reference():
    """Prefill, then a 3-token verify-style call at position 5 through the
    same cache, with the bottom-right causal mask."""
    z, cfg, m = _model()
    kv = m.new_cache(1, 16)
    got0 = m.forward(torch.from_numpy(z["inc_ids_0"]), torch.arange(5)[None], kv, 0,
                     causal_mask(5, 5))
    np.testing.assert_array_equal(got0.numpy(), z["inc_logits_0"])
    got1 = m.forward(torch.from_numpy(z["inc_ids_1"]), torch.arange(5, 8)[None], kv, 5,
                     causal_mask(3, 8))
    np.testing.assert_array_equal(got1.numpy(), z["inc_logits_1"])


def test_golden_vectors_have_teeth():
    """A plausible slip -- RoPE positions at the wrong spacing (a uniform
    shift would not show: RoPE scores depend only on relative positions), or
    the GQA head map swapped -- moves the logits far beyond fp32 rounding."""
    z, cfg, m = _model()
    ids = torch.from_numpy(z["full_ids"])
    B, S = ids.shape
    ref = z["full_logits"]
    shifted = m.forward(ids, 2 * torch.arange(S)[None].expand(B, S), m.new_cache(B, 16), 0,
                        causal_mask(S, S)).numpy()
    assert np.abs(shifted - ref).max() > 1e-4
    for L in m.w["layers"]:   # swap the two KV heads' rows
        D = cfg.head_dim
        L["k"] = torch.cat([L["k"][D:], L["k"][:D]])
        L["kb"] = torch.cat([L["kb"][D:], L["kb"][:D]])
    swapped = m.forward(ids, torch.arange(S)[None].expand(B, S), m.new_cache(B, 16), 0,
                        causal_mask(S, S)).numpy()
    assert np.abs(swapped - ref).max() > 1e-4
