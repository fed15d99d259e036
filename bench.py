"""Benchmark of the speculative-decoding verify step on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-cpu]

Prints ONE JSON line.  ``value`` is end-to-end speculative-decoding
throughput (emitted tokens / wall time, prefill included) of the workload
"0.5B-shape spec decode": a random-init Qwen2.5-0.5B-shape target (24 layers,
hidden 896, 14 q / 2 kv heads, head dim 64, FFN 4864, vocab 151936, RoPE
theta 1e6, bf16), a draft made of its first 4 layers with the shared
embedding / norm / lm_head, k = 4, greedy verification, 32 requests admitted
together with prompts of uniform-random ids and lengths U[100, 512], outputs
of U[64, 128] tokens (EOS ignored), paged KV of 8000 blocks x 16 tokens.
One step = one full pass of that workload.

``roofline`` is the verify-attention kernel at the verify shape of that
workload (batch 32, 5 query tokens, 14/2 heads, D 64, page 16, KV lengths
U[100, 640], pages scattered over an 8000-block pool): algorithmic bytes per
launch / mean launch time, timed with HIP events around replays of a HIP
graph of 160 launches on the launch stream, each launch on its own copy of
the pool: a replay touches 160 x 6.4 MB = 1 GB of distinct K/V pages, so the
256 MB Infinity Cache and the L2s cannot serve a launch from an earlier one.
``kernels`` adds the acceptance calls -- ratio tests or the greedy rule,
residual / bonus draw and rollback slots from a page table -- at batch 64,
k 4, vocab 151936, T 0.8 and at batch 64, k 8, vocab 128256, T 1.0 (rotated
buffer sets of >= 580 MB in all), and the large verify shape (Llama-3-8B
heads, k 8, batch 64, KV U[2048, 8192]).  ``cpu_baseline`` is the CPU plumbing workload
(batch 1, the seed-0 0.5B-shape target with a 2-layer draft, prompt of 64
uniform ids, k 4, greedy, 32 tokens) on the oracle's fp32 PyTorch-CPU
restatement of the reference's loop, every affinity core, median of 5 runs
after a warm-up, prefill also timed alone; its ``kernels`` time the oracle's
numpy restatements of both kernels on the same inputs as the GPU calls.

    python bench.py --workload large-shape [--steps K] [--warmup W]

measures the large shape end to end instead (not the default line): a
random-init Llama-3-8B-shape target (32 layers, hidden 4096, 32 q / 8 kv
heads, head dim 128, FFN 14336, vocab 128256, RoPE theta 5e5) with FP8 E4M3
per-tensor-scaled decoder weights and bf16 KV, a draft of its first 4
layers, k = 8, 64 requests with contexts U[2048, 8192], 32 output tokens
each, stochastic verification at T = 1.0 (Philox uniforms).  The contexts'
K/V are seeded pool noise instead of a prefill (decoding alone is timed);
long KV ranges are split over workgroups and merged inside the captured step.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
ROOT = os.path.dirname(os.path.abspath(__file__))


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def c4_workload(seed=0, n=32, vocab=151936):
    rng = np.random.default_rng(seed)
    plens = rng.integers(100, 513, n)
    prompts = [rng.integers(0, vocab, int(L)).tolist() for L in plens]
    outs = rng.integers(64, 129, n).tolist()
    return prompts, outs


def graph_time_us(torch, fn, n, reps=5):
    """Mean per-launch time of fn(0..n-1) captured in one HIP graph: HIP
    events on the replay stream bracket each replay (median of reps), so host
    launch latency is excluded and the time is the GPU's, including the
    dispatch gaps between the graph's kernels."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        g.replay()
        e.record()
        torch.cuda.synchronize()
        ts.append(s.elapsed_time(e) * 1e3 / n)
    del g
    return float(np.median(ts))


def bench_verify_attention(torch, w, dev, reps=160, pools=160, shape=None):
    from nanosglang_amd import workloads
    from nanosglang_amd.kernels import BatchPrefillWithPagedKVCacheWrapper
    shape = shape or {}
    c = workloads.verify_attention_batch(seed=0, **shape)
    Hq, Hkv, D = c["q"].shape[1], c["k"].shape[2], c["k"].shape[3]
    B = len(c["kv_lens"])
    k0 = torch.from_numpy(c["k"]).to(dev).bfloat16()
    v0 = torch.from_numpy(c["v"]).to(dev).bfloat16()
    ks = [k0] + [k0.clone() for _ in range(pools - 1)]
    vs = [v0] + [v0.clone() for _ in range(pools - 1)]
    q = torch.from_numpy(c["q"]).to(dev).bfloat16()
    ws = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    wr = BatchPrefillWithPagedKVCacheWrapper(ws)
    wr.plan(c["qo_indptr"], c["kv_indptr"], c["kv_indices"], c["kv_last_page_len"], Hq, Hkv, D,
            c["page_size"])
    out = torch.empty_like(q)
    for i in range(2 * pools):
        wr.run(q, (ks[i % pools], vs[i % pools]), out=out)
    t = graph_time_us(torch, lambda i: wr.run(q, (ks[i % pools], vs[i % pools]), out=out), reps)
    nbytes = workloads.algorithmic_bytes_verify_attention(
        c["kv_lens"], c["qo_indptr"][-1], Hq, Hkv, D, B, c["kv_indptr"][-1])
    pi = wr.plan_info
    flops = 0
    for b in range(B):
        ql, L = int(c["q_lens"][b]), int(c["kv_lens"][b])
        flops += 4 * Hq * D * sum(L - ql + r + 1 for r in range(ql))
    del ks, vs
    return {"us": t, "bytes": nbytes, "gbs": nbytes / t / 1e3, "flops": flops,
            "work_items": pi.num_work, "merge_items": pi.num_merge, "kv_groups": pi.kv_groups,
            "row_tiles": pi.row_tiles, "pools_rotated": pools, "inputs": c}


def acceptance_inputs(**kw):
    """Host inputs of one acceptance workload: logits, draft tokens and the
    page table of the rollback slots (workloads.acceptance_batch /
    acceptance_page_table, seed 0)."""
    from nanosglang_amd import workloads
    a = workloads.acceptance_batch(seed=0, **kw)
    B, k1, _ = a["target"].shape
    a["start"], a["kv_indptr"], a["kv_indices"] = workloads.acceptance_page_table(
        batch=B, k=k1 - 1, seed=0)
    return a


def bench_acceptance(torch, dev, a, greedy, sets=None, reps=60):
    """Mean time of one full acceptance call (ratio tests or greedy rule,
    residual / bonus draw, emitted tokens, counts and rollback slots from the
    page table) on `sets` rotated logit buffers, from replays of a HIP graph
    of `reps` calls; by default as many sets as make >= 580 MB of logits in
    all, so that no call reads what an earlier one left in the 256 MB
    Infinity Cache.  Fills a["uniforms"] (host copy of the Philox uniforms
    the calls used)."""
    from nanosglang_amd import workloads
    from nanosglang_amd.kernels import philox_uniform, spec_accept
    B, k1, V = a["target"].shape
    k = k1 - 1
    tl = torch.from_numpy(a["target"]).to(dev).bfloat16()
    dl = torch.from_numpy(a["draft"]).to(dev).bfloat16()
    dt = torch.from_numpy(a["draft_tokens"]).to(dev)
    u = philox_uniform(123, 0, 0, B * k1, dev).view(B, k1)
    a["uniforms"] = u.cpu().numpy()
    pt = [torch.from_numpy(a[n]).to(dev) for n in ("kv_indptr", "kv_indices", "start")]
    T = 0.0 if greedy else a["temperature"]
    if sets is None:
        sets = max(3, -(-580_000_000 // workloads.algorithmic_bytes_acceptance(B, k, V, greedy)))
    bufs = [(tl, dl)] + [(tl.clone(), dl.clone()) for _ in range(sets - 1)]
    out = (torch.empty(B, dtype=torch.int32, device=dev),
           torch.empty(B, k1, dtype=torch.int64, device=dev),
           torch.empty(B, k, dtype=torch.int64, device=dev))

    def call(i):
        t_, d_ = bufs[i % sets]
        spec_accept(t_, None if greedy else d_, dt, None if greedy else u, T, *pt,
                    page_size=16, out=out)

    for i in range(2 * sets):
        call(i)
    t = graph_time_us(torch, call, reps)
    nbytes = workloads.algorithmic_bytes_acceptance(B, k, V, greedy)
    del bufs
    return {"us": t, "bytes": nbytes, "gbs": nbytes / t / 1e3, "sets_rotated": sets,
            "bytes_rotated": sets * nbytes}


def bench_lm_head(torch, dev, rows, copies=2, reps=10):
    """Mean time of one greedy lm_head call (x @ W^T over the 151,936 x 896
    bf16 vocabulary projection, each row's greedy token; the logits are never
    stored) at `rows` rows: the draft step's shape at 32 rows, the verify
    step's at 160.  `copies` weight copies (272 MB each) alternate so that
    the caches serve no call; HIP graph of `reps` calls."""
    from nanosglang_amd.kernels import linear_argmax
    N, K = 151936, 896
    g = torch.Generator(device=dev).manual_seed(7)
    ws = [(torch.randn(N, K, generator=g, device=dev) * K ** -0.5).bfloat16()
          for _ in range(copies)]
    x = torch.randn(rows, K, generator=g, device=dev).bfloat16()
    out = torch.empty(rows, dtype=torch.int64, device=dev)

    def call(i):
        linear_argmax(x, ws[i % copies], out=out)

    for i in range(copies):
        call(i)
    t = graph_time_us(torch, call, reps)
    nbytes = N * K * 2 + rows * K * 2 + rows * 8    # W once, x, the tokens
    del ws
    return {"us": t, "bytes": nbytes, "gbs": nbytes / t / 1e3,
            "flops": 2 * rows * N * K}


def pmc_probe(torch):
    """Dispatches whose HBM counters calibrate and measure traffic: a plain
    copy of COPY_BYTES (read COPY_BYTES, write COPY_BYTES), then the
    verify-shape attention launches on rotated pools (as in the bench)."""
    from nanosglang_amd import workloads
    from nanosglang_amd.kernels import BatchPrefillWithPagedKVCacheWrapper
    dev = torch.device("cuda", 0)
    src = torch.ones(COPY_BYTES // 4, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    c = workloads.verify_attention_batch(seed=0)
    k0 = torch.from_numpy(c["k"]).to(dev).bfloat16()
    v0 = torch.from_numpy(c["v"]).to(dev).bfloat16()
    pools = 16
    ks = [k0] + [k0.clone() for _ in range(pools - 1)]
    vs = [v0] + [v0.clone() for _ in range(pools - 1)]
    q = torch.from_numpy(c["q"]).to(dev).bfloat16()
    ws = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    wr = BatchPrefillWithPagedKVCacheWrapper(ws)
    wr.plan(c["qo_indptr"], c["kv_indptr"], c["kv_indices"], c["kv_last_page_len"], 14, 2, 64,
            c["page_size"])
    out = torch.empty_like(q)
    torch.cuda.synchronize()
    for i in range(10):
        wr.run(q, (ks[i % pools], vs[i % pools]), out=out)
    torch.cuda.synchronize()
    nbytes = workloads.algorithmic_bytes_verify_attention(
        c["kv_lens"], c["qo_indptr"][-1], 14, 2, 64, len(c["kv_lens"]), c["kv_indptr"][-1])
    print(json.dumps({"copy_bytes": COPY_BYTES, "attention_launches": 10,
                      "attention_algorithmic_bytes": nbytes}), flush=True)


COPY_BYTES = 256 << 20

# the large verify shape: 8B-shape heads, k = 8, batch 64, contexts U[2048, 8192]
LARGE_SHAPE = dict(batch=64, q_len=9, num_qo_heads=32, num_kv_heads=8, head_dim=128,
                   min_len=2048, max_len=8192, num_pages=21000)


def pmc_probe_lm_head(torch, copies=2):
    """A 256 MiB device copy (3x, the counter calibration), then greedy
    lm_head calls (151,936 x 896) at 32 rows and at 160 rows, each on
    `copies` alternating weight copies, for rocprofv3 FETCH_SIZE / WRITE_SIZE
    passes."""
    from nanosglang_amd.kernels import linear_argmax
    dev = torch.device("cuda", 0)
    src = torch.ones(COPY_BYTES // 4, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    N, K = 151936, 896
    g = torch.Generator(device=dev).manual_seed(7)
    ws = [(torch.randn(N, K, generator=g, device=dev) * K ** -0.5).bfloat16()
          for _ in range(copies)]
    for rows in (32, 160):
        x = torch.randn(rows, K, generator=g, device=dev).bfloat16()
        out = torch.empty(rows, dtype=torch.int64, device=dev)
        for i in range(2 * copies):
            linear_argmax(x, ws[i % copies], out=out)
        torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "rows": [32, 160], "calls_per_shape": 2 * copies,
                      "algorithmic_bytes": {r: N * K * 2 + r * K * 2 + r * 8 for r in (32, 160)}}),
          flush=True)


def pmc_probe_accept(torch, sets=3):
    """A 256 MiB device copy (3x, the counter calibration), then one
    stochastic and one greedy acceptance call (rollback slots included) at
    the acceptance shape on each of `sets` rotated buffer sets, for rocprofv3
    FETCH_SIZE / WRITE_SIZE passes."""
    from nanosglang_amd import workloads
    from nanosglang_amd.kernels import philox_uniform, spec_accept
    dev = torch.device("cuda", 0)
    src = torch.ones(COPY_BYTES // 4, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    a = acceptance_inputs()
    B, k1, V = a["target"].shape
    tl = torch.from_numpy(a["target"]).to(dev).bfloat16()
    dl = torch.from_numpy(a["draft"]).to(dev).bfloat16()
    dt = torch.from_numpy(a["draft_tokens"]).to(dev)
    u = philox_uniform(123, 0, 0, B * k1, dev).view(B, k1)
    pt = [torch.from_numpy(a[n]).to(dev) for n in ("kv_indptr", "kv_indices", "start")]
    bufs = [(tl, dl)] + [(tl.clone(), dl.clone()) for _ in range(sets - 1)]
    torch.cuda.synchronize()
    for t_, d_ in bufs:
        spec_accept(t_, d_, dt, u, a["temperature"], *pt, page_size=16)
    for t_, d_ in bufs:
        spec_accept(t_, None, dt, None, 0.0, *pt, page_size=16)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "calls": sets,
                      "stochastic_algorithmic_bytes":
                          workloads.algorithmic_bytes_acceptance(B, k1 - 1, V, False),
                      "greedy_algorithmic_bytes":
                          workloads.algorithmic_bytes_acceptance(B, k1 - 1, V, True)}),
          flush=True)


def pmc_probe_large(torch, launches=3):
    """A 256 MiB device copy (3x, the counter calibration), then
    verify-attention launches at the large shape (plus their merge launches),
    for rocprofv3 --pmc passes (MfmaUtil / MfmaFlopsBF16, FETCH_SIZE /
    WRITE_SIZE)."""
    from nanosglang_amd import workloads
    from nanosglang_amd.kernels import BatchPrefillWithPagedKVCacheWrapper
    dev = torch.device("cuda", 0)
    src = torch.ones(COPY_BYTES // 4, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    c = workloads.verify_attention_batch(seed=0, **LARGE_SHAPE)
    Hq, Hkv, D = c["q"].shape[1], c["k"].shape[2], c["k"].shape[3]
    k = torch.from_numpy(c["k"]).to(dev).bfloat16()
    v = torch.from_numpy(c["v"]).to(dev).bfloat16()
    q = torch.from_numpy(c["q"]).to(dev).bfloat16()
    ws = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    wr = BatchPrefillWithPagedKVCacheWrapper(ws)
    wr.plan(c["qo_indptr"], c["kv_indptr"], c["kv_indices"], c["kv_last_page_len"], Hq, Hkv, D,
            c["page_size"])
    out = torch.empty_like(q)
    torch.cuda.synchronize()
    for _ in range(launches):
        wr.run(q, (k, v), out=out)
    torch.cuda.synchronize()
    flops = sum(4 * Hq * D * sum(int(L) - int(ql) + r + 1 for r in range(int(ql)))
                for ql, L in zip(c["q_lens"], c["kv_lens"]))
    nbytes = workloads.algorithmic_bytes_verify_attention(
        c["kv_lens"], c["qo_indptr"][-1], Hq, Hkv, D, len(c["kv_lens"]), c["kv_indptr"][-1])
    print(json.dumps({"copy_bytes": COPY_BYTES, "attention_launches": launches,
                      "attention_flops": flops, "attention_algorithmic_bytes": nbytes}),
          flush=True)


def traffic_bytes():
    """HBM bytes per verify-attention launch at the verify shape, from the
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes recorded in
    profiles/verify_attention_traffic.json (each scaled by a plain copy kernel
    of known size); None when that record is absent."""
    p = os.path.join(ROOT, "profiles", "verify_attention_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("traffic_bytes_per_launch")


def _cpu_model_name() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(runs=5, n_tokens=32, prompt_len=64):
    """The CPU plumbing workload on the oracle's fp32 PyTorch-CPU restatement
    of the reference's speculative loop (speculative.py:51-184): the seed-0
    random-init 0.5B-shape target, a draft of its first 2 layers plus the
    shared embedding / norm / lm_head, batch 1, a prompt of 64 uniform-random
    ids, k = 4, greedy, 32 output tokens.  Every affinity core; 1 warm-up run,
    then the median of `runs`; the prompt's prefill (target + draft forward
    over the prompt) is also timed on its own."""
    import torch
    sys.path.insert(0, ROOT)
    from oracle.model import (CPUCausalLM, CPUSpeculativeDecoder, ModelConfig, causal_mask,
                              init_weights)
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cfg = ModelConfig()
    w = init_weights(cfg, seed=0)
    target = CPUCausalLM(cfg, w, max_pos=256)
    draft = CPUCausalLM(cfg, w, num_layers=2, max_pos=256)
    prompt = np.random.default_rng(0).integers(0, cfg.vocab_size, prompt_len).tolist()
    spec = CPUSpeculativeDecoder(draft, target, 4, temperature=0.0)
    spec.generate(prompt, n_tokens)                         # warm-up
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        out = spec.generate(prompt, n_tokens)
        times.append(time.perf_counter() - t0)
    assert len(out) == n_tokens
    ids, pos, mask = torch.tensor([prompt]), torch.arange(prompt_len)[None], \
        causal_mask(prompt_len, prompt_len)
    pre = []
    for _ in range(3):
        tc, dc = target.new_cache(1, prompt_len), draft.new_cache(1, prompt_len)
        t0 = time.perf_counter()
        target.forward(ids, pos, tc, 0, mask)
        draft.forward(ids, pos, dc, 0, mask)
        pre.append(time.perf_counter() - t0)
    med, prefill = float(np.median(times)), float(np.median(pre))
    return {"value": round(n_tokens / med, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"the whole CPU plumbing workload per run: batch 1, prompt {prompt_len} "
                      f"uniform ids, {n_tokens} output tokens (prefill included), fp32, "
                      f"0.5B-shape target / 2-layer draft, k=4, greedy; median of {runs} runs "
                      f"after 1 warm-up",
            "median_s": round(med, 3), "runs_s": [round(t, 3) for t in times],
            "prefill_s": round(prefill, 4),
            "decode_tok_per_s": round((n_tokens - 1) / max(1e-9, med - prefill), 3),
            "acceptance_rate": round(spec.stats["accepted"] / max(1, spec.stats["proposed"]), 4),
            "cpu_model": _cpu_model_name(), "torch": torch.__version__}


def cpu_restatements(c2, c3, c5, big, runs=3, big_requests=8):
    """The oracle's numpy restatements of the two kernels timed on the same
    inputs as the GPU calls (median of `runs`): verify attention at the
    verify shape (all 32 requests) and at the large shape (the first
    `big_requests` of 64, one run), acceptance at the
    acceptance shape and the large shape (stochastic and greedy, rollback
    slots included).  float64 numpy on the host: one thread for the
    elementwise work, the BLAS threads numpy was given for the einsums."""
    sys.path.insert(0, ROOT)
    from nanosglang_amd import workloads
    from oracle.acceptance import spec_accept as oracle_accept
    from oracle.verify_attention import verify_attention

    def med(fn, runs=runs):
        ts = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))

    def attn_entry(c, n_req, n_runs):
        kvl = np.asarray(c["kv_lens"][:n_req])
        qo = c["qo_indptr"][:n_req + 1]
        kvp = c["kv_indptr"][:n_req + 1]
        t = med(lambda: verify_attention(c["q"][:qo[-1]], c["k"], c["v"], qo, kvp,
                                         c["kv_indices"], c["kv_last_page_len"][:n_req],
                                         c["sm_scale"]), n_runs)
        nb = workloads.algorithmic_bytes_verify_attention(
            kvl, qo[-1], c["q"].shape[1], c["k"].shape[2], c["k"].shape[3], n_req, kvp[-1])
        return {"ms": round(t * 1e3, 2), "algorithmic_bytes": int(nb),
                "gbs": round(nb / t / 1e9, 3), "requests": int(n_req)}

    def acc_entry(a, greedy):
        B, k1, V = a["target"].shape
        t = med(lambda: oracle_accept(a["target"], None if greedy else a["draft"],
                                      a["draft_tokens"], None if greedy else a["uniforms"],
                                      0.0 if greedy else a["temperature"], a["kv_indptr"],
                                      a["kv_indices"], a["start"], 16))
        nb = workloads.algorithmic_bytes_acceptance(B, k1 - 1, V, greedy)
        return {"ms": round(t * 1e3, 2), "algorithmic_bytes": int(nb),
                "gbs": round(nb / t / 1e9, 3)}

    out = {"verify_attention_verify_shape": attn_entry(c2, len(c2["kv_lens"]), runs)}
    if big is not None:   # about 5 s per run: one run
        out["verify_attention_large_shape_sample"] = attn_entry(big, big_requests, 1)
    out["acceptance_stochastic_b64_k4_v151936"] = acc_entry(c3, False)
    out["acceptance_greedy_b64_k4_v151936"] = acc_entry(c3, True)
    if c5 is not None:
        out["acceptance_stochastic_b64_k8_v128256"] = acc_entry(c5, False)
        out["acceptance_greedy_b64_k8_v128256"] = acc_entry(c5, True)
    return out


def large_shape(args, torch):
    """The large shape end to end (decoding only): 8B-shape FP8 target, k 8,
    batch 64, contexts U[2048, 8192], T 1.0."""
    from nanosglang_amd.engine.spec_engine import SpecEngine
    from nanosglang_amd.model.causal_lm import CausalLM, ModelConfig
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B, k, n_out, P = 64, 8, 32, 16
    rng = np.random.default_rng(0)
    ctx = rng.integers(2048, 8193, B)
    cfg = ModelConfig(model_type="llama", vocab_size=128256, hidden_size=4096,
                      intermediate_size=14336, num_hidden_layers=32, num_attention_heads=32,
                      num_key_value_heads=8, max_position_embeddings=8192 + 256,
                      rms_norm_eps=1e-5, rope_theta=5e5, tie_word_embeddings=False,
                      attention_bias=False)
    t0 = time.perf_counter()
    model = CausalLM(cfg, device=dev, seed=0).quantize_fp8(resident_dequant=True)
    torch.cuda.empty_cache()
    log(f"8B-shape FP8 model built in {time.perf_counter() - t0:.1f} s")
    blocks = int(sum((int(L) + n_out + k + 1 + P - 1) // P for L in ctx)) + B + 8
    engine = SpecEngine(model, draft_layers=4, num_speculative=k, num_blocks=blocks,
                        block_size=P, temperature=1.0, seed=0, max_batch=B, kv_split=True)
    prompts = [[int(t)] * int(L) for t, L in zip(rng.integers(0, cfg.vocab_size, B), ctx)]
    outs = [n_out] * B
    t_cap = time.perf_counter()
    sizes = engine.capture()
    log(f"captured spec-step graphs for batch sizes {sizes} in "
        f"{time.perf_counter() - t_cap:.1f} s")
    for w in range(args.warmup):
        engine.generate(prompts, outs, synthetic_context=True)
        log(f"warmup {w}: {engine.stats}")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n_tok, steps, stats = 0, 0, []
    for s in range(args.steps):
        res = engine.generate(prompts, outs, synthetic_context=True)
        n_tok += sum(len(r) - 1 for r in res)       # the first token is the prompt's last
        stats.append(dict(engine.stats))
        steps += engine.stats["steps"]
        log(f"step {s}: {engine.stats}")
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    result = {
        "metric": "spec-decode tok/s, decoding only (8B-shape FP8, k=8, bs=64, ctx 2-8K, T=1)",
        "value": round(n_tok / elapsed, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(elapsed / args.steps * 1e3, 2),
        "ms_per_spec_step": round(elapsed / max(1, steps) * 1e3, 2),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8 weights / bf16", "data": "synthetic (random-init weights, noise KV context)",
        "config": {"workload": "8B-shape spec decode: 32-layer FP8 target / 4-layer draft, k=8, "
                               "64 requests, contexts U[2048,8192], 32 outputs, T=1.0",
                   "batch": B, "k": k, "page_size": P, "num_blocks": blocks},
        "acceptance_rate": round(float(np.mean([s["acceptance_rate"] for s in stats])), 4),
        "tokens_per_step": round(float(np.mean([s["tokens_per_step"] for s in stats])), 3),
        "tune_gemms": bool(args.tune_gemms),
    }
    print(json.dumps(result), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-kernels", action="store_true")
    ap.add_argument("--workload", default="0.5b", choices=["0.5b", "large-shape"],
                    help="large-shape: the 8B-shape FP8 end-to-end line instead of the default")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="only a 256 MiB device copy (3x) and 10 verify-attention launches at "
                         "the verify shape, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes")
    ap.add_argument("--tune-gemms", action="store_true",
                    help="large-shape: let PyTorch's TunableOp pick the library GEMM algorithm "
                         "per shape during the warm-up (results in a temporary file)")
    ap.add_argument("--pmc-probe-accept", action="store_true",
                    help="only a 256 MiB device copy (3x) and 3 stochastic + 3 greedy acceptance "
                         "calls at the acceptance shape, for rocprofv3 --pmc FETCH_SIZE / "
                         "WRITE_SIZE passes")
    ap.add_argument("--pmc-probe-lm-head", action="store_true",
                    help="only a 256 MiB device copy (3x) and 4 greedy lm_head calls at 32 and "
                         "at 160 rows, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes")
    ap.add_argument("--pmc-probe-large", action="store_true",
                    help="only a 256 MiB device copy (3x) and 3 verify-attention launches at "
                         "the large shape, for rocprofv3 --pmc passes (MFMA, HBM traffic)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the verify "
              f"step runs on a single MI355X.", file=sys.stderr)
        sys.exit(2)

    import torch
    sys.path.insert(0, ROOT)
    if args.pmc_probe:
        pmc_probe(torch)
        return
    if args.pmc_probe_accept:
        pmc_probe_accept(torch)
        return
    if args.pmc_probe_large:
        pmc_probe_large(torch)
        return
    if args.pmc_probe_lm_head:
        pmc_probe_lm_head(torch)
        return
    if args.tune_gemms and args.workload != "large-shape":
        print("--tune-gemms applies to --workload large-shape only (the default line runs "
              "no tuned library GEMM)", file=sys.stderr)
        sys.exit(2)
    if args.workload == "large-shape":
        if not args.tune_gemms:
            large_shape(args, torch)
            return
        import tempfile
        with tempfile.TemporaryDirectory() as tmp:
            torch.cuda.tunable.enable(True)
            torch.cuda.tunable.tuning_enable(True)
            torch.cuda.tunable.set_filename(os.path.join(tmp, "tunableop.csv"))
            torch.cuda.tunable.set_max_tuning_duration(30)
            torch.cuda.tunable.set_max_tuning_iterations(20)
            large_shape(args, torch)
        return
    from nanosglang_amd.engine.spec_engine import SpecEngine
    from nanosglang_amd.model.causal_lm import CausalLM, ModelConfig

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    prompts, outs = c4_workload()
    log(f"workload: {len(prompts)} requests, prompt tokens {sum(map(len, prompts))}, "
        f"output tokens {sum(outs)}")
    model = CausalLM(ModelConfig(), device=dev, seed=0)
    engine = SpecEngine(model, draft_layers=4, num_speculative=4, num_blocks=8000,
                        block_size=16, temperature=0.0, max_batch=len(prompts))
    t_cap = time.perf_counter()
    sizes = engine.capture()        # engine start-up, as the reference captures at start()
    log(f"captured spec-step graphs for batch sizes {sizes} in "
        f"{time.perf_counter() - t_cap:.1f} s")
    for w in range(args.warmup):
        engine.generate(prompts, outs)
        log(f"warmup {w}: {engine.stats}")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n_tok = 0
    stats = []
    for s in range(args.steps):
        res = engine.generate(prompts, outs)
        n_tok += sum(len(r) for r in res)
        stats.append(dict(engine.stats))
        log(f"step {s}: {engine.stats}")
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    value = n_tok / elapsed

    result = {
        "metric": "spec-decode tok/s (0.5B-shape, k=4, bs=32); verify-attn & accept % HBM peak",
        "value": round(value, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(elapsed / args.steps * 1e3, 2),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init weights, uniform-random prompt ids)",
        "config": {"workload": "0.5B-shape spec decode: 24-layer target / 4-layer draft, k=4, "
                               "32 requests, prompts U[100,512], outputs U[64,128], greedy, "
                               "paged KV 8000x16",
                   "batch": 32, "k": 4, "page_size": 16, "num_blocks": 8000},
        "decode_tok_per_s": round(float(np.mean([s["decode_tok_per_s"] for s in stats])), 1),
        "acceptance_rate": round(float(np.mean([s["acceptance_rate"] for s in stats])), 4),
        "tokens_per_step": round(float(np.mean([s["tokens_per_step"] for s in stats])), 3),
        "prefill_s": round(float(np.mean([s["prefill_s"] for s in stats])), 4),
    }
    del engine, model
    torch.cuda.empty_cache()

    inputs = {}
    if not args.skip_kernels:
        va = bench_verify_attention(torch, None, dev)
        inputs["c2"] = va.pop("inputs")
        log(f"verify attention (verify shape): {va}")
        launches = ("verify_attn_kernel" + (" + verify_merge_kernel" if va["merge_items"] else ""))
        result["roofline"] = {
            "bound": "hbm", "achieved": round(va["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(va["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic_bytes(),
            "kernel": f"verify attention ({launches}; {va['work_items']} work items x 2 KV heads, "
                      f"{va['kv_groups']} KV groups of {va['row_tiles']} waves per workgroup), "
                      f"batch 32, 5 query tokens, 14/2 heads, D 64",
            "us_per_launch": round(va["us"], 2), "algorithmic_bytes": va["bytes"]}
        entries = {"verify_attention_verify_shape": va}
        for name, kw in (("b64_k4_v151936", {}),
                         ("b64_k8_v128256", dict(k=8, vocab=128256, temperature=1.0))):
            a = acceptance_inputs(**kw)
            for greedy in (False, True):
                mode = "greedy" if greedy else "stochastic"
                d = bench_acceptance(torch, dev, a, greedy)
                log(f"acceptance {mode} {name}: {d}")
                entries[f"acceptance_{mode}_{name}"] = d
            inputs[name] = a
            torch.cuda.empty_cache()
        for rows in (32, 160):
            d = bench_lm_head(torch, dev, rows)
            log(f"lm_head greedy {rows} rows: {d}")
            entries[f"lm_head_greedy_{rows}_rows_v151936"] = d
            torch.cuda.empty_cache()
        big = bench_verify_attention(torch, None, dev, reps=20, pools=1, shape=LARGE_SHAPE)
        inputs["large"] = big.pop("inputs")
        log(f"verify attention (large shape): {big}")
        entries["verify_attention_large_shape"] = big

        def k_entry(d):
            e = {"us": round(d["us"], 2), "algorithmic_bytes": d["bytes"],
                 "achieved_gbs": round(d["gbs"], 1), "frac_hbm": round(d["gbs"] / HBM_PEAK_GBS, 4)}
            if "flops" in d:
                e["tflops"] = round(d["flops"] / d["us"] / 1e6, 2)
            return e

        result["kernels"] = {n: k_entry(d) for n, d in entries.items()}

    if not args.skip_cpu:
        cb = cpu_baseline()
        log(f"cpu baseline: {cb}")
        result["cpu_baseline"] = cb
        if inputs:
            rs = cpu_restatements(inputs["c2"], inputs["b64_k4_v151936"],
                                  inputs["b64_k8_v128256"], inputs["large"])
            log(f"cpu restatements: {rs}")
            result["cpu_baseline"]["kernels"] = rs
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
