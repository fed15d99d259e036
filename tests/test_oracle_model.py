"""Pins oracle/model.py by invariants: cached incremental decoding equals a
full-sequence forward, and greedy speculative decoding equals plain greedy
decoding of the target whatever the draft (with and without the draft-KV hole
fill)."""
import numpy as np
import pytest
import torch

from oracle.model import (CPUCausalLM, CPUSpeculativeDecoder, ModelConfig, causal_mask,
                          greedy_decode, init_weights)
from oracle.philox import philox_uniforms

TINY = ModelConfig(vocab_size=97, hidden_size=64, intermediate_size=96, num_hidden_layers=4,
                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256)


def _models(scale=1.0, draft_layers=2):
    w = init_weights(TINY, seed=0)
    if scale != 1.0:  # larger weights -> less trivial argmax behaviour
        for L in w["layers"]:
            for k in ("q", "k", "v", "o", "gate", "up", "down"):
                L[k] *= scale
    return CPUCausalLM(TINY, w), CPUCausalLM(TINY, w, num_layers=draft_layers)


def test_incremental_equals_full_forward():
    t, _ = _models(scale=20.0)
    ids = torch.tensor([[5, 17, 3, 88, 42, 9, 61, 2]])
    S = ids.shape[1]
    full = t.forward(ids, torch.arange(S)[None], t.new_cache(1, S), 0, causal_mask(S, S))
    cache = t.new_cache(1, S)
    t.forward(ids[:, :3], torch.arange(3)[None], cache, 0, causal_mask(3, 3))
    part = t.forward(ids[:, 3:], torch.arange(3, S)[None], cache, 3, causal_mask(S - 3, S))
    torch.testing.assert_close(part, full[:, 3:], rtol=1e-5, atol=1e-5)
    # a non-causal mask over the verify rows must change the result (mask is live)
    cache2 = t.new_cache(1, S)
    t.forward(ids[:, :3], torch.arange(3)[None], cache2, 0, causal_mask(3, 3))
    leak = t.forward(ids[:, 3:], torch.arange(3, S)[None], cache2, 3, None)
    assert (leak - full[:, 3:]).abs().max() > 1e-4


@pytest.mark.parametrize("fill", [True, False])
@pytest.mark.parametrize("scale", [1.0, 30.0])
def test_greedy_speculative_equals_greedy(fill, scale):
    t, d = _models(scale=scale)
    rng = np.random.default_rng(1)
    prompt = rng.integers(0, TINY.vocab_size, 12).tolist()
    ref = greedy_decode(t, prompt, 24)
    spec = CPUSpeculativeDecoder(d, t, num_speculative=4, temperature=0.0, fill_draft_hole=fill)
    assert spec.generate(prompt, 24) == ref
    assert spec.stats["steps"] >= 24 // 5


def test_stochastic_runs_with_supplied_uniforms():
    t, d = _models(scale=30.0)
    off = [0]

    def uni(n):
        u = philox_uniforms(7, 0, off[0], n)
        off[0] += n
        return u.tolist()

    spec = CPUSpeculativeDecoder(d, t, 4, temperature=1.0, uniform=uni)
    out = spec.generate([1, 2, 3, 4], 20)
    assert len(out) == 20 and all(0 <= x < TINY.vocab_size for x in out)
