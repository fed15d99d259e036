"""End-to-end greedy parity of the speculative step at the reference's own
shapes, through the HIP path.

* The CPU plumbing workload: a random-init Qwen2.5-0.5B-shape target (the
  oracle's seed-0 N(0, 0.02) weights, 24 layers, hidden 896, 14 / 2 heads,
  FFN 4864, vocab 151,936, RoPE theta 1e6) with a draft made of its first 2
  layers plus the shared embedding, norm and lm_head; batch 1, a prompt of
  64 uniform-random ids, k = 4, greedy, 32 output tokens
  (nano_sglang/decode/speculative.py:51-184).
* The end-to-end shape: the same target with a 4-layer draft, 32 requests
  with prompts U[100, 512], paged KV 8000 x 16, three speculative steps.

Asserted for every step: the verify rows' greedy tokens (taken straight from
the lm_head kernel) are the first argmax of the logits that kernel writes for
the same rows; the emitted tokens, counts and rollback slots equal
the greedy closed form (oracle.acceptance.spec_accept: drafts accepted while
each equals the first argmax of its target row, then that argmax; the
rejected positions' slots) evaluated on the verify logits the step actually
produced; and the captured-graph step and the eager step produce
bit-identical verify logits and outputs.

Reported (not asserted): the first divergence from plain greedy decoding on
the GPU (k = 0: one verify token per step, whose lm_head and attention run at
other row counts and so round differently) and from the CPU fp32 oracle's
speculative loop (sampling.py:44-45, speculative.py:174-182).
"""
import numpy as np
import pytest
import torch

from oracle.acceptance import spec_accept as oracle_accept
from oracle.model import CPUCausalLM, CPUSpeculativeDecoder, ModelConfig as OCfg, init_weights

pytestmark = pytest.mark.gpu


def _check_trace(trace, label):
    """Every recorded step's outputs equal the greedy closed form on its own
    verify logits."""
    assert trace, label
    for s, rec in enumerate(trace):
        tl = rec["verify_logits"].float().numpy()
        if rec["target_tokens"] is not None:
            # greedy verify from the lm_head kernel's tokens: each is the
            # first argmax of its verify row
            assert np.array_equal(rec["target_tokens"], tl.argmax(-1)), (label, s)
        ref = oracle_accept(tl, None, rec["drafts"], None, 0.0, rec["kv_indptr"],
                            rec["kv_indices"], rec["start"], rec["page_size"])
        assert np.array_equal(rec["num_emitted"], ref["num_emitted"]), (label, s)
        assert np.array_equal(rec["emitted"], ref["emitted"]), (label, s)
        assert np.array_equal(rec["rollback"], ref["rollback"]), (label, s)
    n = np.concatenate([r["num_emitted"] for r in trace])
    print(f"  {label}: {len(trace)} steps closed-form exact, tokens per request-step "
          f"{n.mean():.3f}", flush=True)


def _same_traces(a, b):
    """Graph and eager steps: identical verify logits, drafts and outputs.
    Rollback slots are compared with each run's own closed form instead: the
    captured engine holds a dummy page for its padding rows, so its requests
    sit on other page ids."""
    assert len(a) == len(b)
    for s, (x, y) in enumerate(zip(a, b)):
        assert torch.equal(x["verify_logits"], y["verify_logits"]), s
        for key in ("drafts", "num_emitted", "emitted", "start"):
            assert np.array_equal(x[key], y[key]), (key, s)
        assert np.array_equal(x["rollback"] >= 0, y["rollback"] >= 0), s


def _first_diff(a, b):
    return next((i for i, (x, y) in enumerate(zip(a, b)) if x != y), min(len(a), len(b)))


def _gpu_model(w):
    from nanosglang_amd.model.causal_lm import CausalLM, ModelConfig
    return CausalLM(ModelConfig(), device=torch.device("cuda", 0), weights=w)


@pytest.fixture(scope="module")
def weights():
    return init_weights(OCfg(), seed=0)          # the oracle's seed-0 rule, fp32 on the host


def test_cpu_plumbing_workload_through_hip_path(weights):
    from nanosglang_amd.engine.spec_engine import SpecEngine
    print("case: B=1, 0.5B-shape target, 2-layer draft, prompt 64, k=4, greedy, 32 tokens",
          flush=True)
    prompt = np.random.default_rng(0).integers(0, 151936, 64).tolist()
    model = _gpu_model(weights)
    outs, traces = [], []
    for graphs in (True, False):
        eng = SpecEngine(model, draft_layers=2, num_speculative=4, num_blocks=64,
                         use_graphs=graphs, max_batch=1)
        eng.trace = []
        outs.append(eng.generate([prompt], [32])[0])
        traces.append(eng.trace)
        assert len(outs[-1]) == 32
        assert eng.bm.num_free_blocks == 64 - (1 if graphs else 0)
        _check_trace(eng.trace, f"graphs={graphs}")
    assert outs[0] == outs[1]
    _same_traces(*traces)
    plain = SpecEngine(model, draft_layers=2, num_speculative=0, num_blocks=64, max_batch=1)
    ref_plain = plain.generate([prompt], [32])[0]
    print(f"  first divergence from plain greedy (GPU, k=0): {_first_diff(outs[0], ref_plain)}/32",
          flush=True)
    cfg = OCfg()
    target = CPUCausalLM(cfg, weights, max_pos=256)
    draft = CPUCausalLM(cfg, weights, num_layers=2, max_pos=256)
    ref_cpu = CPUSpeculativeDecoder(draft, target, 4).generate(prompt, 32)
    print(f"  first divergence from the CPU fp32 oracle: {_first_diff(outs[0], ref_cpu)}/32",
          flush=True)


def test_end_to_end_shape_closed_form(weights):
    from nanosglang_amd.engine.spec_engine import SpecEngine
    print("case: 32 requests, 0.5B-shape target, 4-layer draft, k=4, 3 greedy steps", flush=True)
    rng = np.random.default_rng(0)
    prompts = [rng.integers(0, 151936, int(L)).tolist() for L in rng.integers(100, 513, 32)]
    model = _gpu_model(weights)
    runs = []
    for graphs in (True, False):
        eng = SpecEngine(model, draft_layers=4, num_speculative=4, num_blocks=8000,
                         use_graphs=graphs, max_batch=32)
        eng.trace = []
        first, tables = eng.prefill(prompts)
        last, start, got = list(first), [len(p) for p in prompts], []
        for _ in range(3):
            res = eng.speculative_step_batch(last, start, tables)
            assert all(1 <= len(r) <= 5 for r in res)
            got.append(res)
            last = [r[-1] for r in res]
            start = [s + len(r) for s, r in zip(start, res)]
        _check_trace(eng.trace, f"graphs={graphs}")
        runs.append((first, got, eng.trace))
        del eng
        torch.cuda.empty_cache()
    assert runs[0][0] == runs[1][0]
    assert runs[0][1] == runs[1][1]
    _same_traces(runs[0][2], runs[1][2])
    spec = [[f] + sum((step[b] for step in runs[0][1]), [])
            for b, f in enumerate(runs[0][0])]
    n_new = [len(s) for s in spec]
    plain = SpecEngine(model, draft_layers=4, num_speculative=0, num_blocks=8000, max_batch=32)
    ref_plain = plain.generate(prompts, n_new)
    div = [_first_diff(a, b) for a, b in zip(spec, ref_plain)]
    print(f"  requests identical to plain greedy (GPU, k=0): "
          f"{sum(d == n for d, n in zip(div, n_new))}/32; first divergences {div}", flush=True)
    cfg = OCfg()
    target = CPUCausalLM(cfg, weights, max_pos=640)
    draft = CPUCausalLM(cfg, weights, num_layers=4, max_pos=640)
    for b in np.argsort([len(p) for p in prompts])[:2]:
        ref_cpu = CPUSpeculativeDecoder(draft, target, 4).generate(prompts[b], n_new[b])
        print(f"  request {b} (prompt {len(prompts[b])}): first divergence from the CPU fp32 "
              f"oracle {_first_diff(spec[b], ref_cpu)}/{n_new[b]}", flush=True)
