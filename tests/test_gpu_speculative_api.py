"""The reference-compatible batch-1 API (decode/speculative.py) on the GPU:
models with the reference's forward signature and contiguous caches; the
acceptance runs in the HIP kernel.  Greedy speculative decoding must equal
plain greedy decoding of the target (the speculative-sampling invariant)."""
import numpy as np
import pytest
import torch

from oracle.model import CPUCausalLM, ModelConfig, init_weights

pytestmark = pytest.mark.gpu

TINY = ModelConfig(vocab_size=500, hidden_size=128, intermediate_size=256, num_hidden_layers=4,
                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512)


class _GPUModel:
    """The oracle's decoder restated on the GPU (reference forward signature)."""

    def __init__(self, num_layers, scale=6.0):
        w = init_weights(TINY, seed=5)
        for L in w["layers"]:
            for key in ("q", "k", "v", "o", "gate", "up", "down"):
                L[key] *= scale
        w = {"embed": w["embed"].cuda(), "norm": w["norm"].cuda(),
             "layers": [{k: v.cuda() for k, v in L.items()} for L in w["layers"]]}
        self.m = CPUCausalLM(TINY, w, num_layers=num_layers)
        self.m.cos, self.m.sin = self.m.cos.cuda(), self.m.sin.cuda()

    def __call__(self, input_ids, position_ids, kv_caches, cache_position, attention_mask):
        return self.m.forward(input_ids, position_ids, kv_caches, cache_position, attention_mask)

    def new_cache(self, n):
        return [(a.cuda(), b.cuda()) for a, b in self.m.new_cache(1, n)]


def _greedy(target, prompt, n_new):
    from nanosglang_amd.decode.speculative import causal_mask
    cache = target.new_cache(len(prompt) + n_new + 8)
    S = len(prompt)
    lg = target(torch.tensor([prompt], device="cuda"), torch.arange(S, device="cuda")[None],
                cache, 0, causal_mask(S, S))
    out = [int(lg[0, -1].argmax())]
    pos = S
    while len(out) < n_new:
        lg = target(torch.tensor([[out[-1]]], device="cuda"),
                    torch.tensor([[pos]], device="cuda"), cache, pos, causal_mask(1, pos + 1))
        out.append(int(lg[0, -1].argmax()))
        pos += 1
    return out


@pytest.mark.parametrize("fill", [True, False])
def test_speculative_step_greedy_equals_greedy(fill):
    from nanosglang_amd.decode.speculative import SpeculativeDecoder, causal_mask
    target, draft = _GPUModel(4), _GPUModel(2)
    prompt = np.random.default_rng(2).integers(0, 500, 11).tolist()
    n_new = 25
    ref = _greedy(target, prompt, n_new)
    spec = SpeculativeDecoder(draft, target, num_speculative=4, temperature=0.0,
                              fill_draft_hole=fill)
    tc, dc = target.new_cache(64), draft.new_cache(64)
    S = len(prompt)
    ids = torch.tensor([prompt], device="cuda")
    lg = target(ids, torch.arange(S, device="cuda")[None], tc, 0, causal_mask(S, S))
    draft(ids, torch.arange(S, device="cuda")[None], dc, 0, causal_mask(S, S))
    out = [int(lg[0, -1].argmax())]
    pos = S
    steps = 0
    while len(out) < n_new:
        acc = spec.speculative_step(torch.tensor([[out[-1]]], device="cuda"), pos, dc, tc,
                                    causal_mask)
        assert 1 <= len(acc) <= 5
        out += acc
        pos += len(acc)
        steps += 1
    assert out[:n_new] == ref
    print(f"  {steps} steps for {n_new} tokens (fill_draft_hole={fill})", flush=True)


def test_speculative_step_stochastic_runs():
    from nanosglang_amd.decode.speculative import SpeculativeDecoder, causal_mask
    target, draft = _GPUModel(4), _GPUModel(2)
    spec = SpeculativeDecoder(draft, target, num_speculative=3, temperature=0.9, seed=11)
    tc, dc = target.new_cache(64), draft.new_cache(64)
    ids = torch.tensor([[3, 1, 4, 1, 5]], device="cuda")
    target(ids, torch.arange(5, device="cuda")[None], tc, 0, causal_mask(5, 5))
    draft(ids, torch.arange(5, device="cuda")[None], dc, 0, causal_mask(5, 5))
    acc = spec.speculative_step(torch.tensor([[9]], device="cuda"), 5, dc, tc, causal_mask)
    assert 1 <= len(acc) <= 4 and all(0 <= t < 500 for t in acc)


def test_speculative_step_top_k_top_p():
    """top_k / top_p reach the draft and bonus draws (sample_token sites,
    speculative.py:95-100, 174-182); top_k = 1 makes each draft the argmax."""
    from nanosglang_amd.decode.speculative import SpeculativeDecoder, causal_mask
    target, draft = _GPUModel(4), _GPUModel(2)
    for top_k, top_p in ((5, 0.8), (0, 0.5), (1, 1.0)):
        spec = SpeculativeDecoder(draft, target, num_speculative=3, temperature=0.9, seed=3,
                                  top_k=top_k, top_p=top_p)
        tc, dc = target.new_cache(64), draft.new_cache(64)
        ids = torch.tensor([[3, 1, 4, 1, 5]], device="cuda")
        target(ids, torch.arange(5, device="cuda")[None], tc, 0, causal_mask(5, 5))
        draft(ids, torch.arange(5, device="cuda")[None], dc, 0, causal_mask(5, 5))
        acc = spec.speculative_step(torch.tensor([[9]], device="cuda"), 5, dc, tc, causal_mask)
        assert 1 <= len(acc) <= 4 and all(0 <= t < 500 for t in acc)
        row = torch.randn(1, 500, device="cuda")
        if top_k == 1:
            assert int(spec._sample(row)) == int(row.argmax())
    with pytest.raises(ValueError):
        SpeculativeDecoder(draft, target, top_p=0.0)
