"""Batched speculative decoding over the paged KV cache on one GPU.

The reference's ``SpeculativeDecoder.speculative_step``
(nano_sglang/decode/speculative.py:50-184) is batch-1 and runs on the
contiguous cache; its paged multi-query attention lives only in the engine's
FlashInfer path (nano_sglang/engine/engine.py:419-472).  This module joins
the two for a batch of requests:

1. admission: a block table per request (paged_kv_cache.py:113-120);
2. prefill of every prompt in one ragged packed forward (engine.py:298-472);
3. per step, for the active requests at positions ``start`` (the last
   emitted token, not yet in the cache):
   * reserve pages for positions ``< start + k + 1``
     (scheduler.py:221-232 applied to the verify window);
   * k draft forwards of one token each (speculative.py:76-107) -- the draft
     is the target's first ``draft_layers`` layers with the shared
     embedding, final norm and lm_head, so it reads and writes the target's
     own pool for those layers: the verify forward rewrites positions
     ``start .. start+k`` in every layer, which leaves no draft-cache hole
     after full acceptance (the reference's hole, speculative.py:76-107);
   * one verify forward of k+1 tokens per request (speculative.py:109-128)
     through the HIP verify-attention kernel;
   * the fused acceptance kernel (speculative.py:130-184) -> emitted tokens,
     counts and rollback slots;
   * rollback: pages wholly past the kept positions go back to the pool.
4. a request finishes after ``max_new_tokens`` tokens (EOS ignored, as the
   reference's benchmark asks for, bench_throughput.py:67-72).

Sampling: greedy when ``temperature < 1e-6`` (sampling.py:44); otherwise
draft tokens, ratio tests and resamples use Philox uniforms from
``kernels.philox_uniform`` (stream 0: acceptance, stream 1: draft sampling).
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import numpy as np
import torch

from .. import kernels
from ..kernels import BatchPrefillWithPagedKVCacheWrapper
from .paged_kv_cache import BlockManager, BlockTable, PagedKVCache


@dataclass
class _Req:
    rid: int
    prompt: list[int]
    max_new: int
    table: BlockTable = field(default_factory=BlockTable)
    out: list[int] = field(default_factory=list)
    start: int = 0          # position of out[-1]; KV holds positions < start


class SpecEngine:
    def __init__(self, model, draft_layers: int, num_speculative: int, num_blocks: int,
                 block_size: int = 16, temperature: float = 0.0, seed: int = 0,
                 workspace_bytes: int = 256 << 20):
        c = model.config
        self.model = model
        self.k = num_speculative
        self.draft_layers = draft_layers
        self.temperature = float(temperature)
        self.greedy = self.temperature < 1e-6
        self.seed = seed
        self.device = model.device
        self.bm = BlockManager(num_blocks, block_size, model.num_layers, c.num_key_value_heads,
                               c.head_dim, dtype=torch.bfloat16, device=self.device)
        self.kv = PagedKVCache(self.bm)
        self.P = block_size
        ws = torch.empty(workspace_bytes, dtype=torch.uint8, device=self.device)
        self.attn = BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
        self._rng_offset = [0, 0]
        self.stats = {}

    # ---- helpers ----
    def _uniforms(self, stream: int, n: int) -> torch.Tensor:
        u = kernels.philox_uniform(self.seed, stream, self._rng_offset[stream], n, self.device)
        self._rng_offset[stream] += n
        return u

    def _plan(self, reqs, q_lens, kv_lens):
        P = self.P
        c = self.model.config
        qo = np.zeros(len(reqs) + 1, np.int32)
        qo[1:] = np.cumsum(q_lens)
        kvp = np.zeros(len(reqs) + 1, np.int32)
        idx = []
        last = np.empty(len(reqs), np.int32)
        for i, (r, L) in enumerate(zip(reqs, kv_lens)):
            npg = (L + P - 1) // P
            idx.extend(r.table.block_indices[:npg])
            kvp[i + 1] = kvp[i] + npg
            last[i] = L - (npg - 1) * P
        idx = np.asarray(idx, np.int32)
        self.attn.plan(qo, kvp, idx, last, c.num_attention_heads, c.num_key_value_heads,
                       c.head_dim, P, causal=True)
        return kvp, idx

    def _slots(self, reqs, starts, counts) -> np.ndarray:
        P = self.P
        out = np.empty(int(sum(counts)), np.int64)
        o = 0
        for r, s, n in zip(reqs, starts, counts):
            bt = r.table.block_indices
            for t in range(n):
                pos = s + t
                out[o] = bt[pos // P] * P + pos % P
                o += 1
        return out

    def _to_dev(self, a, dtype=None):
        t = torch.from_numpy(np.ascontiguousarray(a))
        return t.to(self.device, non_blocking=False) if dtype is None else \
            t.to(self.device, dtype, non_blocking=False)

    def _pool(self):
        return (self.bm.k_cache, self.bm.v_cache)

    def _sample_rows(self, logits: torch.Tensor) -> torch.Tensor:
        """One token per row: argmax if greedy, else inverse CDF of
        softmax(logits / T) with Philox stream 1 (spec_accept with k = 0)."""
        B = logits.shape[0]
        u = None if self.greedy else self._uniforms(1, B).view(B, 1)
        _, em, _ = kernels.spec_accept(logits.view(B, 1, -1), None, None, u, self.temperature)
        return em[:, 0]

    # ---- main entry ----
    @torch.inference_mode()
    def generate(self, prompts: list[list[int]], max_new_tokens: list[int]):
        k, dev = self.k, self.device
        reqs = [_Req(i, list(p), int(m)) for i, (p, m) in enumerate(zip(prompts, max_new_tokens))]
        t0 = time.perf_counter()
        # 1. admission
        for r in reqs:
            r.table = self.kv.allocate_for_request(len(r.prompt))
        # 2. prefill (one ragged packed forward)
        lens = [len(r.prompt) for r in reqs]
        self._plan(reqs, lens, lens)
        ids = self._to_dev(np.concatenate([np.asarray(r.prompt, np.int64) for r in reqs]))
        pos = self._to_dev(np.concatenate([np.arange(n, dtype=np.int64) for n in lens]))
        slots = self._to_dev(self._slots(reqs, [0] * len(reqs), lens))
        last_idx = self._to_dev(np.cumsum(lens) - 1)
        logits = self.model.forward_packed(ids, pos, self._pool(), self.attn, slots, last_idx)
        first = self._sample_rows(logits).cpu().tolist()
        for r, f in zip(reqs, first):
            r.out.append(f)
            r.start = len(r.prompt)
        t_prefill = time.perf_counter() - t0
        steps = proposed = accepted = req_steps = 0
        active = [r for r in reqs if len(r.out) < r.max_new]
        for r in reqs:
            if r not in active:
                self.kv.free_request(r.table)
        # 3. speculative steps
        while active:
            B = len(active)
            starts = [r.start for r in active]
            for r in active:
                self.kv.reserve(r.table, r.start + k + 1)
            start_pos = np.asarray(starts, np.int64)
            tok = self._to_dev(np.asarray([r.out[-1] for r in active], np.int64))
            ones = [1] * B
            drafts = torch.empty(B, k, dtype=torch.int64, device=dev)
            dlog = None
            for i in range(k):
                self._plan(active, ones, [s + i + 1 for s in starts])
                sl = self._to_dev(self._slots(active, [s + i for s in starts], ones))
                lg = self.model.forward_packed(tok, self._to_dev(start_pos + i), self._pool(),
                                               self.attn, sl, None, self.draft_layers)
                if not self.greedy:
                    if dlog is None:
                        dlog = torch.empty(B, k, lg.shape[-1], dtype=lg.dtype, device=dev)
                    dlog[:, i] = lg
                tok = self._sample_rows(lg)
                drafts[:, i] = tok
            # verify: [last, d_0 .. d_{k-1}] at start .. start+k
            kvp, idx = self._plan(active, [k + 1] * B, [s + k + 1 for s in starts])
            vids = torch.empty(B, k + 1, dtype=torch.int64, device=dev)
            vids[:, 0] = self._to_dev(np.asarray([r.out[-1] for r in active], np.int64))
            vids[:, 1:] = drafts
            vpos = self._to_dev((start_pos[:, None] + np.arange(k + 1)[None]).reshape(-1))
            sl = self._to_dev(self._slots(active, starts, [k + 1] * B))
            tl = self.model.forward_packed(vids.view(-1), vpos, self._pool(), self.attn, sl)
            u = None if self.greedy else self._uniforms(0, B * (k + 1)).view(B, k + 1)
            n_out, emitted, rollback = kernels.spec_accept(
                tl.view(B, k + 1, -1), dlog, drafts, u, self.temperature,
                self._to_dev(kvp), self._to_dev(idx), self._to_dev(start_pos, torch.int32),
                page_size=self.P)
            n_h = n_out.cpu().numpy()
            em_h = emitted.cpu().numpy()
            steps += 1
            req_steps += B
            proposed += B * k
            accepted += int(n_h.sum()) - B
            still = []
            for j, r in enumerate(active):
                n = int(n_h[j])
                r.out.extend(em_h[j, :n].tolist())
                r.start += n
                self.kv.truncate(r.table, r.start)        # rollback of rejected pages
                if len(r.out) >= r.max_new:
                    del r.out[r.max_new:]
                    self.kv.free_request(r.table)
                else:
                    still.append(r)
            active = still
        torch.cuda.synchronize(dev)
        t_total = time.perf_counter() - t0
        n_tok = sum(len(r.out) for r in reqs)
        self.stats = {
            "elapsed_s": t_total, "prefill_s": t_prefill, "output_tokens": n_tok,
            "prompt_tokens": sum(lens), "steps": steps,
            "acceptance_rate": accepted / proposed if proposed else 0.0,
            "tokens_per_step": (accepted + req_steps) / max(1, req_steps),
            "tok_per_s": n_tok / t_total,
            "decode_tok_per_s": (n_tok - len(reqs)) / max(1e-9, t_total - t_prefill),
        }
        return [r.out for r in reqs]
