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

At the end-to-end shape the random-init 4-layer draft is almost never
accepted, so two more full-size runs exercise the accepted-draft branches:
* greedy with the draft equal to the target (all 24 layers): drafts accepted,
  multi-token emission, the bonus, partial rollback and the pages
  ``truncate`` frees, each checked per step against the closed form, with a
  floor on the mean tokens per request-step;
* stochastic at T = 0.8 with the 4-layer draft: each step's acceptance
  equals the float64 oracle on the step's own verify logits, draft logits
  and Philox uniforms (bit-exact except where a decision lies within 1e-5
  of its threshold), and the captured step equals the eager one.

Reported: the first divergence from plain greedy decoding on the GPU (k = 0:
one verify token per step, whose lm_head and attention run at other row
counts and so round differently) and from the CPU fp32 oracle's speculative
loop (sampling.py:44-45, speculative.py:174-182).
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


def _prompts32():
    rng = np.random.default_rng(0)
    return [rng.integers(0, 151936, int(L)).tolist() for L in rng.integers(100, 513, 32)]


def _run_steps(eng, prompts, steps, P=16, check_pages=True):
    """Prefill, then `steps` batched speculative steps; after each step every
    request's block table holds exactly the pages of its kept positions (the
    pages past them went back to the pool) and the pool's free count adds
    up.  Returns (first tokens, per-step results)."""
    first, tables = eng.prefill(prompts)
    last, start, got = list(first), [len(p) for p in prompts], []
    reserved = eng.bm.num_blocks - eng.bm.num_free_blocks - sum(len(t.block_indices)
                                                                  for t in tables)
    for _ in range(steps):
        res = eng.speculative_step_batch(last, start, tables)
        assert all(1 <= len(r) <= eng.k + 1 for r in res)
        got.append(res)
        last = [r[-1] for r in res]
        start = [s + len(r) for s, r in zip(start, res)]
        if check_pages:
            for t, s in zip(tables, start):
                assert len(t.block_indices) == (s + P - 1) // P, (len(t.block_indices), s)
            assert eng.bm.num_free_blocks == eng.bm.num_blocks - reserved - sum(
                len(t.block_indices) for t in tables)
    return first, got


def test_end_to_end_shape_draft_equals_target_accepts(weights):
    """Greedy at the end-to-end shape with the draft equal to the target (all
    24 layers): the drafts are the target's own greedy tokens at one row
    per request, so most are accepted and every step emits several tokens.
    Asserted per step: outputs equal the greedy closed form on the step's
    verify logits, graph == eager, block tables hold exactly the kept
    positions' pages; and at least 4 tokens per request-step on average."""
    from nanosglang_amd.engine.spec_engine import SpecEngine
    print("case: 32 requests, draft = target (24 layers), k=4, 3 greedy steps", flush=True)
    prompts = _prompts32()
    model = _gpu_model(weights)
    runs = []
    for graphs in (True, False):
        eng = SpecEngine(model, draft_layers=24, num_speculative=4, num_blocks=8000,
                         use_graphs=graphs, max_batch=32)
        eng.trace = []
        first, got = _run_steps(eng, prompts, 3)
        _check_trace(eng.trace, f"graphs={graphs}")
        n = np.concatenate([r["num_emitted"] for r in eng.trace])
        rb = np.concatenate([r["rollback"] for r in eng.trace])
        print(f"  graphs={graphs}: tokens per request-step {n.mean():.3f}, all-accepted "
              f"{(n == 5).mean():.3f}, partial rollbacks {((n > 1) & (n < 5)).sum()}, "
              f"slots rolled back {(rb >= 0).sum()}", flush=True)
        assert n.mean() >= 4.0
        assert (n == 5).any()
        runs.append((first, got, eng.trace))
        del eng
        torch.cuda.empty_cache()
    assert runs[0][0] == runs[1][0] and runs[0][1] == runs[1][1]
    _same_traces(runs[0][2], runs[1][2])
    spec = [[f] + sum((step[b] for step in runs[0][1]), []) for b, f in enumerate(runs[0][0])]
    n_new = [len(x) for x in spec]
    plain = SpecEngine(model, draft_layers=24, num_speculative=0, num_blocks=8000, max_batch=32)
    ref_plain = plain.generate(prompts, n_new)
    div = [_first_diff(a, b) for a, b in zip(spec, ref_plain)]
    print(f"  requests identical to plain greedy (GPU, k=0): "
          f"{sum(d == n for d, n in zip(div, n_new))}/32; first divergences {div}", flush=True)


def test_end_to_end_shape_stochastic(weights):
    """Stochastic verification (T = 0.8) at the end-to-end shape with the
    4-layer draft: three steps of 32 requests, graph and eager.  Each step's
    acceptance equals the float64 oracle evaluated on the step's own verify
    logits, draft logits, drafts and uniforms: bit-exact except requests
    whose decision margin is below 1e-5.  The graph and eager runs draw the
    same Philox uniforms, so they agree bit for bit."""
    from nanosglang_amd.engine.spec_engine import SpecEngine
    print("case: 32 requests, 4-layer draft, k=4, T=0.8, 3 stochastic steps", flush=True)
    prompts = _prompts32()
    model = _gpu_model(weights)
    runs = []
    for graphs in (True, False):
        eng = SpecEngine(model, draft_layers=4, num_speculative=4, num_blocks=8000,
                         use_graphs=graphs, max_batch=32, temperature=0.8, seed=7)
        eng.trace = []
        first, got = _run_steps(eng, prompts, 3)
        acc = rej = exempt = 0
        for s, rec in enumerate(eng.trace):
            assert rec["draft_logits"] is not None and rec["uniforms"] is not None
            ref = oracle_accept(rec["verify_logits"].float().numpy(),
                                rec["draft_logits"].float().numpy(), rec["drafts"],
                                rec["uniforms"], 0.8, rec["kv_indptr"], rec["kv_indices"],
                                rec["start"], rec["page_size"])
            n, em, rb = rec["num_emitted"], rec["emitted"], rec["rollback"]
            bad = np.nonzero((n != ref["num_emitted"]) | (em != ref["emitted"]).any(1)
                             | (rb != ref["rollback"]).any(1))[0]
            assert all(ref["margin"][b] < 1e-5 for b in bad), (s, bad, ref["margin"][bad])
            exempt += len(bad)
            acc += int((n - 1).sum())
            rej += int((n <= 4).sum())
        print(f"  graphs={graphs}: accepted drafts {acc}, rejections {rej}, within-margin "
              f"mismatches {exempt}", flush=True)
        assert acc > 0 and rej > 0 and exempt <= 2
        runs.append((first, got, eng.trace))
        del eng
        torch.cuda.empty_cache()
    assert runs[0][0] == runs[1][0] and runs[0][1] == runs[1][1]
    _same_traces(runs[0][2], runs[1][2])
