"""The large shape end to end under test: a random-init Llama-3-8B-shape
target (32 layers, hidden 4096, 32 / 8 heads of 128, FFN 14336, vocab
128,256, RoPE theta 5e5) with FP8 E4M3 per-tensor-scaled decoder weights and
bf16 KV, a draft of its first 4 layers, k = 8, stochastic verification at
T = 1.0, contexts U[2048, 8192] (seeded pool noise in place of a prefill,
long KV ranges split over workgroups and merged) -- 16 requests, two
speculative steps, captured graph and eager.

Asserted for each step: the acceptance equals the float64 oracle evaluated
on the step's own verify logits, draft logits, drafts and Philox uniforms
(nano_sglang/decode/speculative.py:130-196), bit-exact except requests whose
decision margin is below 1e-5; block tables hold exactly the kept
positions' pages; graph and eager steps agree bit for bit."""
import numpy as np
import pytest
import torch

from oracle.acceptance import spec_accept as oracle_accept

pytestmark = pytest.mark.gpu


def test_large_shape_engine_two_stochastic_steps():
    from nanosglang_amd.engine.spec_engine import SpecEngine
    from nanosglang_amd.model.causal_lm import CausalLM, ModelConfig
    print("case: large shape engine, 16 requests, k=8, T=1, 2 steps", flush=True)
    dev = torch.device("cuda", 0)
    B, k, P, T = 16, 8, 16, 1.0
    rng = np.random.default_rng(3)
    ctx = rng.integers(2048, 8193, B)
    cfg = ModelConfig(model_type="llama", vocab_size=128256, hidden_size=4096,
                      intermediate_size=14336, num_hidden_layers=32, num_attention_heads=32,
                      num_key_value_heads=8, max_position_embeddings=8192 + 256,
                      rms_norm_eps=1e-5, rope_theta=5e5, tie_word_embeddings=False,
                      attention_bias=False)
    model = CausalLM(cfg, device=dev, seed=0).quantize_fp8(resident_dequant=True)
    torch.cuda.empty_cache()
    prompts = [[int(t)] * int(L) for t, L in zip(rng.integers(0, cfg.vocab_size, B), ctx)]
    blocks = int(sum((int(L) + 2 * (k + 1) + P - 1) // P for L in ctx)) + B + 8
    runs = []
    for graphs in (True, False):
        eng = SpecEngine(model, draft_layers=4, num_speculative=k, num_blocks=blocks,
                         block_size=P, temperature=T, seed=0, max_batch=B, kv_split=True,
                         use_graphs=graphs)
        if not graphs:
            # the captured engine's dummy page is the pool's first allocation:
            # take it here too, so that both engines place every request on
            # the same pages (the synthetic context is per-page noise)
            eng.bm.allocate()
        eng.trace = []
        first, tables = eng.prefill(prompts, synthetic_context=True)
        last, start, got = list(first), [len(p) for p in prompts], []
        for s in range(2):
            res = eng.speculative_step_batch(last, start, tables)
            got.append(res)
            last = [r[-1] for r in res]
            start = [a + len(r) for a, r in zip(start, res)]
            for t, a in zip(tables, start):
                assert len(t.block_indices) == (a + P - 1) // P
        acc = rej = exempt = 0
        for s, rec in enumerate(eng.trace):
            ref = oracle_accept(rec["verify_logits"].float().numpy(),
                                rec["draft_logits"].float().numpy(), rec["drafts"],
                                rec["uniforms"], T, rec["kv_indptr"], rec["kv_indices"],
                                rec["start"], P)
            n, em, rb = rec["num_emitted"], rec["emitted"], rec["rollback"]
            bad = np.nonzero((n != ref["num_emitted"]) | (em != ref["emitted"]).any(1)
                             | (rb != ref["rollback"]).any(1))[0]
            assert all(ref["margin"][b] < 1e-5 for b in bad), (s, bad, ref["margin"][bad])
            exempt += len(bad)
            acc += int((n - 1).sum())
            rej += int((n <= k).sum())
        print(f"  graphs={graphs}: accepted drafts {acc}, rejections {rej}, within-margin "
              f"mismatches {exempt}", flush=True)
        assert rej > 0 and exempt <= 1
        runs.append((first, got, eng.trace))
        del eng
        torch.cuda.empty_cache()
    assert runs[0][0] == runs[1][0] and runs[0][1] == runs[1][1]
    for x, y in zip(runs[0][2], runs[1][2]):
        assert torch.equal(x["verify_logits"], y["verify_logits"])
        assert torch.equal(x["draft_logits"], y["draft_logits"])
        for key in ("drafts", "num_emitted", "emitted", "uniforms"):
            assert np.array_equal(x[key], y[key]), key
