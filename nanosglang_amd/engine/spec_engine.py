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

Graph mode (default): as the reference's engine captures one CUDA graph of
the decode forward per batch size in ``[1, 2, 4] + range(8, max_bs + 1, 8)``
(engine.py:110-214) and pads a batch to the next captured size with rows on a
dummy page (engine.py:357-394), this engine captures one HIP graph of the
WHOLE speculative step per such size -- the k draft forwards and their
samplers, the verify forward and the acceptance kernels.  Before each replay
the host plans all k + 1 attention calls (fixed-size work lists) and writes
every per-step input (tokens, positions, KV slots, page tables, work lists)
into one pinned staging buffer, uploaded with a single copy; after the replay
it reads back the counts and tokens (the reference's ``.item()`` sites).

Sampling: greedy when ``temperature < 1e-6`` (sampling.py:44); otherwise
draft tokens, ratio tests and resamples use Philox uniforms from
``kernels.philox_uniform`` (stream 0: acceptance, stream 1: draft sampling).
"""

from __future__ import annotations

import time
import weakref
from dataclasses import dataclass, field

import numpy as np
import torch

from .. import _native, kernels
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
    row: int = -1           # row of the engine's page-table mirror (graph mode)
    synced: int = 0         # pages of `table` mirrored into that row


def _free_gate(flag: int) -> None:
    lib = _native._lib
    if lib is not None:
        lib.nsg_host_gate_free(flag)


def graph_batch_sizes(max_bs: int) -> list[int]:
    """The reference's captured decode sizes (engine.py:117-119), plus max_bs."""
    return sorted(set([b for b in (1, 2, 4) if b <= max_bs] + list(range(8, max_bs + 1, 8))
                      + [max_bs]))


class _Arena:
    """Named int/float arrays that live in one pinned host buffer and one
    device buffer at the same offsets: the host fills the pinned views, one
    ``upload`` copies them all (the device views have fixed addresses, so a
    captured graph reads them)."""

    def __init__(self, specs, device):
        offs, o = {}, 0
        for name, dt, n in specs:
            o = (o + 255) // 256 * 256
            es = torch.empty(0, dtype=dt).element_size()
            offs[name] = (o, dt, n, es)
            o += n * es
        self.nbytes = max(256, (o + 255) // 256 * 256)
        self.off = {name: v[0] for name, v in offs.items()}   # byte offset of each array
        self.host = torch.zeros(self.nbytes, dtype=torch.uint8, pin_memory=True)
        self.dev = torch.zeros(self.nbytes, dtype=torch.uint8, device=device)
        self.h, self.d = {}, {}
        for name, (o, dt, n, es) in offs.items():
            self.d[name] = self.dev[o:o + n * es].view(dt)
            self.h[name] = self.host[o:o + n * es].view(dt).numpy()

    def upload(self):
        self.dev.copy_(self.host, non_blocking=True)


def _round_up(n: int, m: int = 64) -> int:
    return (n + m - 1) // m * m


class _StepGraph:
    """Static buffers, attention wrappers and the captured graph of one
    speculative step at padded batch size ``bs``.

    Staging layout (one pinned host buffer, one device buffer, same offsets):
    token0 / start [bs]; draft positions and slots [k][bs]; verify positions
    and slots [bs][k+1]; then, per attention call a (k drafts, then the
    verify call), a block of qo / kv indptr and last-page lengths, page ids
    and the fixed-size work list, each block at a 256-byte aligned stride."""

    def __init__(self, eng: "SpecEngine", bs: int, max_page_ids: int):
        c = eng.model.config
        k, dev = eng.k, eng.device
        Hq, Hkv = c.num_attention_heads, c.num_key_value_heads
        self.bs = bs
        lib = kernels._lib()
        nw = 0
        for a in range(k + 1):                       # attention calls: k drafts, 1 verify
            ql = 1 if a < k else k + 1
            mw, mm = kernels.C.c_int32(0), kernels.C.c_int32(0)
            kernels.check(lib.nsg_attn_fixed_capacity(bs, ql, Hq, Hkv, kernels.MI355X_CUS,
                                                      eng.max_kv_len, kernels.C.byref(mw),
                                                      kernels.C.byref(mm)),
                          "nsg_attn_fixed_capacity")
            nw = max(nw, (mw.value + mm.value) * kernels.NSG_ATTN_WORK_INTS)
        si, sx, sw = _round_up(bs + 1), _round_up(max_page_ids), _round_up(nw)
        self.strides = (si, sx, sw)
        # "tok0": the step's token ids position-major, (k + 1) x bs: row 0
        # the requests' last tokens (the step fill writes it), row i + 1
        # draft i's tokens (written on the device during the step)
        specs = [("tok0", torch.int64, (k + 1) * bs), ("start", torch.int32, bs),
                 ("pos", torch.int64, k * bs), ("slot", torch.int64, k * bs),
                 ("vpos", torch.int64, bs * (k + 1)), ("vslot", torch.int64, bs * (k + 1)),
                 ("qo", torch.int32, (k + 1) * si), ("kvp", torch.int32, (k + 1) * si),
                 ("last", torch.int32, (k + 1) * si), ("work", torch.int32, (k + 1) * sw),
                 ("idx", torch.int32, (k + 1) * sx)]
        self.arena = A = _Arena(specs, dev)
        H = A.h
        self.bufs = _native.StepBufs(
            *[H[n].ctypes.data for n in ("tok0", "start", "pos", "slot", "vpos", "vslot", "qo",
                                         "kvp", "last", "idx", "work")], si, sx, sw)
        self.plans = (_native.AttnPlan * (k + 1))()
        D = A.d
        self.pos = [D["pos"][i * bs:(i + 1) * bs] for i in range(k)]
        self.slot = [D["slot"][i * bs:(i + 1) * bs] for i in range(k)]
        self.kvp = [D["kvp"][a * si:a * si + bs + 1] for a in range(k + 1)]
        self.idx = [D["idx"][a * sx:(a + 1) * sx] for a in range(k + 1)]
        self.attn = []
        for a in range(k + 1):
            self.attn.append(BatchPrefillWithPagedKVCacheWrapper(
                eng.attn_ws, "NHD", use_cuda_graph=True,
                qo_indptr_buf=D["qo"][a * si:a * si + bs + 1], paged_kv_indptr_buf=self.kvp[a],
                paged_kv_indices_buf=self.idx[a],
                paged_kv_last_page_len_buf=D["last"][a * si:a * si + bs],
                work_buf=D["work"][a * sw:(a + 1) * sw],
                max_q_len=1 if a < k else k + 1, max_kv_len=eng.max_kv_len))
        V = c.vocab_size
        self.drafts = torch.zeros(bs, k, dtype=torch.int64, device=dev)
        self.ids = D["tok0"].view(k + 1, bs)
        self.vids = self.ids.t()             # (bs, k + 1) verify ids, request-major
        self.n_out = torch.zeros(bs, dtype=torch.int32, device=dev)
        self.emitted = torch.zeros(bs, k + 1, dtype=torch.int64, device=dev)
        self.rollback = torch.zeros(bs, k, dtype=torch.int64, device=dev)
        self.n1 = torch.zeros(bs, dtype=torch.int32, device=dev)
        self.bonus = torch.zeros(bs, dtype=torch.int64, device=dev)
        # greedy verify straight from the lm_head kernel: each verify row's
        # token (the logits too, only when the engine records a trace)
        self.ttok = torch.zeros(bs * (k + 1), dtype=torch.int64, device=dev)
        self.tlog = (torch.zeros(bs * (k + 1), V, dtype=torch.bfloat16, device=dev)
                     if eng.trace is not None and eng._argmax_verify(bs) else None)
        self.em1 = torch.zeros(bs, 1, dtype=torch.int64, device=dev)
        self.rb1 = torch.zeros(bs, 0, dtype=torch.int64, device=dev)
        if not eng.greedy:
            self.u = torch.zeros(bs, k + 1, dtype=torch.float32, device=dev)
            self.ud = torch.zeros(k, bs, dtype=torch.float32, device=dev)
            self.dlog = torch.zeros(bs, k, V, dtype=eng.model.dtype, device=dev)
        else:
            self.u = self.ud = self.dlog = None
        self.n_h = torch.zeros(bs, dtype=torch.int32, pin_memory=True)
        self.em_h = torch.zeros(bs, k + 1, dtype=torch.int64, pin_memory=True)
        # coherent pinned word the step's export kernel sets once n_h / em_h
        # hold the step's results (the host polls it, then clears it)
        p = kernels.C.c_void_p()
        kernels.check(lib.nsg_host_gate_alloc(kernels.C.byref(p)), "nsg_host_gate_alloc")
        self.done_ptr = p.value
        self.done = kernels.C.c_int32.from_address(p.value)
        weakref.finalize(self, _free_gate, p.value)
        self.graph = None


class SpecEngine:
    def __init__(self, model, draft_layers: int, num_speculative: int, num_blocks: int,
                 block_size: int = 16, temperature: float = 0.0, seed: int = 0,
                 workspace_bytes: int = 256 << 20, use_graphs: bool = True,
                 max_batch: int = 32, top_k: int = 0, top_p: float = 1.0,
                 kv_split: bool = False, pipeline: bool = True):
        c = model.config
        self.model = model
        self.k = num_speculative
        self.draft_layers = draft_layers
        self.temperature = float(temperature)
        self.greedy = self.temperature < 1e-6
        if not 0.0 < top_p or top_p != top_p:
            raise ValueError(f"top_p {top_p} must be in (0, 1] (1 = off)")
        self.top_k, self.top_p = int(top_k), float(top_p)
        # top-k / top-p at the reference's sample_token sites: drafts and bonus
        self.filtered = not self.greedy and (self.top_k > 0 or self.top_p < 1.0)
        self.seed = seed
        self.device = model.device
        self.bm = BlockManager(num_blocks, block_size, model.num_layers, c.num_key_value_heads,
                               c.head_dim, dtype=torch.bfloat16, device=self.device)
        self.kv = PagedKVCache(self.bm)
        self.P = block_size
        self.attn_ws = torch.empty(workspace_bytes, dtype=torch.uint8, device=self.device)
        self.attn = BatchPrefillWithPagedKVCacheWrapper(self.attn_ws, "NHD")
        self._rng_offset = [0, 0]
        self.stats = {}
        self.use_graphs = use_graphs
        self.max_batch = max_batch
        self._graphs: dict[int, _StepGraph] = {}
        self._accept_ws = kernels.AcceptWorkspace(self.device)
        self._sample_ws = kernels.AcceptWorkspace(self.device)   # the sampler's own
        # greedy drafts: lm_head + argmax in one pass (kernels.linear_argmax),
        # the draft logits are never stored; its workspace is written before
        # it is read, so every call may share it
        self._argmax_ws = kernels.AcceptWorkspace(self.device)
        self._dummy_block = None
        self._tab = np.zeros((0, 0), np.int32)     # page-table mirror of graph mode
        # decode / verify contexts never exceed the position table: the
        # captured attention plans need no KV split (and no merge launch).
        # kv_split: long contexts (thousands of tokens) are split over more
        # workgroups instead, with the merge launch captured as well.
        self.max_kv_len = 0 if kv_split else min(c.max_position_embeddings, 1022 * block_size)
        self._noise = False
        # trace: a list to receive, after every speculative step, the step's
        # verify logits and acceptance inputs / outputs (numpy / CPU tensors),
        # so that a caller can check the acceptance on exactly the logits the
        # step produced; None (default) records nothing.
        self.trace: list | None = None
        # pipeline: in graph mode, generate() queues step s + 1 (behind a host
        # gate) while step s runs, so that the graph launch and input upload
        # overlap the GPU's work (see _decode_pipelined)
        self.pipeline = pipeline
        self._gate_flag = None          # coherent pinned host word (nsg_host_gate_alloc)
        self._gate_seq = 0              # the last gated step's release target
        self._gate_err = torch.zeros(1, dtype=torch.int32, device=self.device)

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
        softmax(logits / T) -- after top-k / top-p when set -- with Philox
        stream 1 (spec_accept with k = 0, or the sampler)."""
        B = logits.shape[0]
        u = None if self.greedy else self._uniforms(1, B).view(B, 1)
        if self.filtered:
            return kernels.sample(logits.view(B, -1), self.temperature, self.top_k, self.top_p,
                                  u.view(B))
        _, em, _ = kernels.spec_accept(logits.view(B, 1, -1), None, None, u, self.temperature)
        return em[:, 0]

    def _argmax_drafts(self, rows: int) -> bool:
        """Greedy draft tokens straight from the lm_head kernel (the argmax of
        the same bf16 logits spec_accept's k = 0 call would take)."""
        return (self.greedy and self.model.dtype == torch.bfloat16
                and rows <= kernels._lib().nsg_linear_max_rows())

    def _argmax_verify(self, batch: int) -> bool:
        """Greedy verify tokens straight from the lm_head kernel, accepted by
        kernels.spec_accept_greedy_tokens: the verify logits (48.6 MB at 160
        rows of vocabulary 151,936) are never written nor read back."""
        return self._argmax_drafts(batch * (self.k + 1))

    def _keys_mode(self, batch: int) -> bool:
        """Greedy drafts and verify hand their tokens on as the lm_head's
        argmax keys: each draft token is reduced by the next forward's
        embedding lookup (which also writes it into the step's ids), the
        verify tokens by the acceptance kernel -- no reduction launches."""
        return (self.k >= 1 and self._argmax_drafts(batch) and self._argmax_verify(batch)
                and self.model.keys_supported(batch)
                and self.model.keys_supported(batch * (self.k + 1)))

    def _bonus(self, tl: torch.Tensor, u: torch.Tensor | None, workspace=None, out=None):
        """speculative.py:174-182: the bonus after k accepted drafts is
        sample_token(target row k) with top-k / top-p; None without filters
        (the acceptance kernel draws it itself)."""
        if not self.filtered:
            return None
        return kernels.sample(tl[:, self.k], self.temperature, self.top_k, self.top_p,
                              u[:, self.k], workspace=workspace, out=out)

    # ---- graph mode ----
    def _max_pages(self) -> int:
        c = self.model.config
        return (c.max_position_embeddings + self.P - 1) // self.P

    def capture(self, max_batch: int | None = None) -> list[int]:
        """Capture one graph per padded batch size up to ``max_batch`` (the
        reference captures at engine start, engine.py:153-156, 164-216).  The
        KV pool contents are untouched except for the dummy page."""
        c = self.model.config
        if max_batch is not None:
            self.max_batch = max_batch
        if self._dummy_block is None:
            self._dummy_block = self.bm.allocate()       # engine.py:139-140
        if self.k + 1 > self._max_pages() * self.P:
            raise ValueError("verify window exceeds the position range")
        V = c.vocab_size
        # every accept call of every graph shares one workspace, every sampler
        # call another, each sized once
        lib = kernels._lib()
        self._accept_ws.get(max(lib.nsg_spec_accept_workspace_bytes(self.max_batch, self.k, V),
                                lib.nsg_spec_accept_workspace_bytes(self.max_batch, 0, V)))
        self._sample_ws.get(lib.nsg_sample_workspace_bytes(self.max_batch, V))
        # draft calls take max_batch rows, greedy verify calls k + 1 per request
        self._argmax_ws.get(lib.nsg_linear_argmax_workspace_bytes(
            self.max_batch * (self.k + 1), V))
        pool = torch.cuda.graph_pool_handle()
        for bs in graph_batch_sizes(self.max_batch):
            if bs in self._graphs:
                continue
            # page ids per attention call: every pool page at most once (no
            # table shares a page) plus the padding rows' dummy pages
            ids = min(bs * self._max_pages(),
                      self.bm.num_blocks + bs * ((self.k + self.P) // self.P))
            g = _StepGraph(self, bs, ids)
            self._fill_step(g, [])                       # all rows on the dummy page
            for a, w in enumerate(g.attn):
                ql = 1 if a < self.k else self.k + 1
                w.adopt_plan(g.plans[a], bs * ql, c.num_attention_heads,
                             c.num_key_value_heads, c.head_dim, self.P, causal=True)
            g.arena.upload()
            for _ in range(2):                           # warm-up (allocator, GEMM heuristics)
                self._graph_body(g)
            torch.cuda.synchronize(self.device)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=pool):
                self._graph_body(g)
            torch.cuda.synchronize(self.device)
            g.graph = graph
            self._graphs[bs] = g
        return sorted(self._graphs)

    def _graph_body(self, g: _StepGraph) -> None:
        """The captured step: k drafts, verify, acceptance (all on device)."""
        m, k, A = self.model, self.k, g.arena.d
        bs = g.bs
        pool = self._pool()
        tok = g.ids[0]
        direct = self._argmax_drafts(bs)
        if self._keys_mode(bs):
            V = m.config.vocab_size
            keys = self._argmax_ws.get(kernels._lib().nsg_linear_argmax_workspace_bytes(
                self.max_batch * (k + 1), V))
            kc = 0
            for i in range(k):
                # draft i's token column is written by draft i + 1's lookup
                # (the last one's by the verify's), from draft i's keys
                kc = m.forward_packed(g.ids[i], g.pos[i], pool, g.attn[i], g.slot[i], None,
                                      self.draft_layers, argmax_keys_out=keys,
                                      ids_keys=None if i == 0 else (keys, kc, 0))
            kcv = m.forward_packed(g.vids, A["vpos"], pool, g.attn[k], A["vslot"],
                                   argmax_keys_out=keys, argmax_logits=g.tlog,
                                   ids_keys=(keys, kc, k))
            g.tl = g.tlog
            kernels.spec_accept_greedy_keys(keys, kcv, bs, k, g.vids[:, 1:], V, g.kvp[k],
                                            g.idx[k], A["start"], page_size=self.P,
                                            workspace=self._accept_ws,
                                            out=(g.n_out, g.emitted, g.rollback),
                                            target_tokens_out=g.ttok)
            self._export(g)
            return
        for i in range(k):
            if direct:
                # the token lands in its row of the step's ids: the next
                # draft's input and a column of the verify ids
                m.forward_packed(g.ids[i], g.pos[i], pool, g.attn[i], g.slot[i], None,
                                 self.draft_layers, argmax_out=g.ids[i + 1],
                                 argmax_ws=self._argmax_ws)
                continue
            lg = m.forward_packed(tok, g.pos[i], pool, g.attn[i], g.slot[i], None,
                                  self.draft_layers)
            if g.dlog is not None:
                g.dlog[:, i].copy_(lg)
            u = None if g.ud is None else g.ud[i].view(bs, 1)
            if self.filtered:
                kernels.sample(lg.view(bs, -1), self.temperature, self.top_k, self.top_p,
                               u.view(bs), workspace=self._sample_ws, out=g.em1[:, 0])
            else:
                kernels.spec_accept(lg.view(bs, 1, -1), None, None, u, self.temperature,
                                    workspace=self._accept_ws, out=(g.n1, g.em1, g.rb1))
            g.drafts[:, i].copy_(g.em1[:, 0])
            tok = g.em1[:, 0]
        if not direct:
            g.ids[1:].copy_(g.drafts.t())
        if self._argmax_verify(bs):
            m.forward_packed(g.vids, A["vpos"], pool, g.attn[k], A["vslot"],
                             argmax_out=g.ttok, argmax_ws=self._argmax_ws, argmax_logits=g.tlog)
            g.tl = g.tlog
            kernels.spec_accept_greedy_tokens(g.ttok.view(bs, k + 1), g.vids[:, 1:],
                                              m.config.vocab_size, g.kvp[k], g.idx[k],
                                              A["start"], page_size=self.P,
                                              workspace=self._accept_ws,
                                              out=(g.n_out, g.emitted, g.rollback))
            self._export(g)
            return
        tl = m.forward_packed(g.vids, A["vpos"], pool, g.attn[k], A["vslot"])
        g.tl = tl        # allocated from the graph's pool: every replay rewrites it
        bonus = self._bonus(tl.view(bs, k + 1, -1), g.u, workspace=self._sample_ws,
                            out=g.bonus)
        kernels.spec_accept(tl.view(bs, k + 1, -1), g.dlog, g.drafts, g.u, self.temperature,
                            g.kvp[k], g.idx[k], A["start"], page_size=self.P,
                            workspace=self._accept_ws, out=(g.n_out, g.emitted, g.rollback),
                            bonus_tokens=bonus)
        self._export(g)

    def _export(self, g: _StepGraph) -> None:
        """The step's emitted counts and tokens into the graph's pinned host
        buffers (g.n_h, g.em_h), by a kernel captured at the end of the step."""
        kernels.check(kernels._lib().nsg_export_step(
            g.n_out.data_ptr(), g.emitted.data_ptr(), g.bs, self.k + 1, g.n_h.data_ptr(),
            g.em_h.data_ptr(), g.done_ptr, kernels._stream_ptr(self.device)), "nsg_export_step")

    def _fill_step(self, g: _StepGraph, active: list) -> None:
        """Host side of one step, one native call (``nsg_spec_step_fill``):
        tokens, positions, KV slots, the k + 1 page tables and attention plans,
        written into the graph's pinned staging buffer.  Request rows come
        from the engine's page-table mirror (``_sync_table``)."""
        B = len(active)
        self._fill_arrays(g, np.fromiter((r.row for r in active), np.int32, B),
                          np.fromiter((r.synced for r in active), np.int32, B),
                          np.fromiter((r.start for r in active), np.int64, B),
                          np.fromiter((r.out[-1] for r in active), np.int64, B))

    def _fill_next_args(self, nxt: _StepGraph, g: _StepGraph, cur: list) -> tuple:
        """Arguments of nsg_spec_step_fill_next: the inputs of step s + 1
        (graph nxt) from the results of step s (graph g's pinned n_out /
        emitted copies) for the requests `cur` of step s.  The arrays are
        kept alive in the returned tuple."""
        c, B = self.model.config, len(cur)
        arrs = (np.fromiter((r.row for r in cur), np.int32, B),
                np.fromiter((r.synced for r in cur), np.int32, B),
                np.fromiter((r.start for r in cur), np.int64, B),
                np.fromiter((r.max_new - len(r.out) for r in cur), np.int64, B))
        nb = kernels.C.c_int32(0)
        args = (self._tab.ctypes.data, self._tab.shape[1], *(a.ctypes.data for a in arrs),
                g.n_h.data_ptr(), g.em_h.data_ptr(), B, nxt.bs, self.k, self.P,
                self._dummy_block, c.num_attention_heads, c.num_key_value_heads, c.head_dim,
                kernels.MI355X_CUS, self.max_kv_len, kernels.C.byref(nxt.bufs), nxt.plans,
                kernels.C.byref(nb))
        return args, arrs, nb

    def _run_fill_next(self, fill_next: tuple) -> int:
        args, _, nb = fill_next
        kernels.check(kernels._lib().nsg_spec_step_fill_next(*args), "nsg_spec_step_fill_next")
        return nb.value

    def _fill_arrays(self, g: _StepGraph, rows, npg, starts, last) -> None:
        """_fill_step on per-request arrays: page-table mirror rows (int32),
        mirrored page counts (int32), start positions and last tokens (int64),
        all C-contiguous."""
        c = self.model.config
        B = len(rows)
        if B:
            ptrs = (self._tab.ctypes.data, self._tab.shape[1], rows.ctypes.data,
                    npg.ctypes.data, starts.ctypes.data, last.ctypes.data)
        else:
            ptrs = (None, 0, None, None, None, None)
        kernels.check(kernels._lib().nsg_spec_step_fill(
            *ptrs, B, g.bs, self.k, self.P, self._dummy_block, c.num_attention_heads,
            c.num_key_value_heads, c.head_dim, kernels.MI355X_CUS, self.max_kv_len,
            kernels.C.byref(g.bufs), g.plans), "nsg_spec_step_fill")

    def _sync_table(self, r: _Req) -> None:
        """Mirror request r's block table into its row of the int32 page table
        the native step fill reads (only pages added since the last sync are
        copied; a rollback only shortens the row)."""
        bt = r.table.block_indices
        n = len(bt)
        if n > r.synced:
            self._tab[r.row, r.synced:n] = bt[r.synced:]
        r.synced = n

    # the host gate gives up after this long (a host that never raises the
    # flag, e.g. after an exception, costs this much and sets the gate's error word)
    GATE_TIMEOUT_US = 2_000_000

    def _graph_for(self, n: int) -> _StepGraph:
        return self._graphs[min(b for b in self._graphs if b >= n)]

    def _gate(self) -> int:
        """The host gate's flag word (allocated once per engine)."""
        if self._gate_flag is None:
            p = kernels.C.c_void_p()
            kernels.check(kernels._lib().nsg_host_gate_alloc(kernels.C.byref(p)),
                          "nsg_host_gate_alloc")
            self._gate_flag = p.value
            weakref.finalize(self, _free_gate, p.value)
        return self._gate_flag

    def _raise_gate(self) -> None:
        """Releases the queued gated step (the flag word counts up to each
        gated launch's target; it is never reset)."""
        kernels.C.c_int32.from_address(self._gate_flag).value = self._gate_seq

    # a step that has not finished after this long is reported as hung
    STEP_TIMEOUT_S = 60.0

    def _wait_done(self, g: _StepGraph) -> None:
        """Waits (polling the pinned done word the step's export kernel sets)
        until the step queued on graph g has finished; its results are then
        in g.n_h / g.em_h."""
        done = g.done
        if done.value:
            return
        t0 = time.perf_counter()
        while not done.value:
            if time.perf_counter() - t0 > self.STEP_TIMEOUT_S:
                raise RuntimeError(f"speculative step (graph of {g.bs} rows) did not finish "
                                   f"within {self.STEP_TIMEOUT_S} s")

    def _gate_segments(self, g: _StepGraph, pages: int):
        """The byte ranges of g's staging a step uses when its attention calls
        hold at most ``pages`` page ids each: every array before the page
        ids (the ids are the arena's last array) and the first ``pages`` ids of
        each call's block."""
        A, sx = g.arena, g.strides[1]
        base = A.off["idx"]
        n = min(sx, pages) * 4
        n = (n + 15) // 16 * 16
        offs = [0] + [base + a * sx * 4 for a in range(self.k + 1)]
        lens = [base] + [min(n, A.nbytes - o) for o in offs[1:]]
        return ((kernels.C.c_int64 * len(offs))(*offs),
                (kernels.C.c_int64 * len(lens))(*lens), len(offs))

    def _launch(self, g: _StepGraph, gated: bool, pages: int | None = None) -> None:
        """Queues one speculative step of graph g on the current stream: the
        host gate (gated: the step waits until _raise_gate), the upload of
        its staging buffer, the Philox uniforms (sampling), the replay, whose
        last kernel exports the results to pinned memory and sets g's done
        word (cleared here for an ungated step; the gated step's owner clears
        it before raising the gate)."""
        bs, k = g.bs, self.k
        lib = kernels._lib()
        sp = kernels._stream_ptr(self.device)
        if not gated:
            g.done.value = 0
        if gated:    # the gate also uploads the staging buffer once released
            A = g.arena
            if pages is None:
                offs, lens, n = ((kernels.C.c_int64 * 1)(0), (kernels.C.c_int64 * 1)(A.nbytes),
                                 1)
            else:    # only the arrays' used prefixes: the pull over PCIe is slow
                offs, lens, n = self._gate_segments(g, pages)
            flag = self._gate()
            self._gate_seq += 1
            kernels.check(lib.nsg_host_gate_wait_segments(
                flag, self._gate_seq, self._gate_err.data_ptr(), self.GATE_TIMEOUT_US,
                A.host.data_ptr(), A.dev.data_ptr(), A.nbytes, offs, lens, n, sp),
                "nsg_host_gate_wait_segments")
        else:
            g.arena.upload()
        if not self.greedy:
            o0, o1 = self._rng_offset
            kernels.check(lib.nsg_philox_uniform(self.seed, 0, o0, bs * (k + 1), g.u.data_ptr(),
                                                 sp), "nsg_philox_uniform")
            kernels.check(lib.nsg_philox_uniform(self.seed, 1, o1, bs * k, g.ud.data_ptr(), sp),
                          "nsg_philox_uniform")
            self._rng_offset = [o0 + bs * (k + 1), o1 + bs * k]
        g.graph.replay()       # ends with the export of its results to g.n_h / g.em_h

    def _step_graph(self, active: list, rows: int = 0):
        B = len(active)
        g = self._graph_for(max(B, rows))
        self._fill_step(g, active)
        self._launch(g, gated=False)
        self._wait_done(g)
        if self.trace is not None:
            k, (si, sx, _) = self.k, g.strides
            kvp = g.arena.h["kvp"][k * si:k * si + B + 1].copy()
            if g.tl is None:
                raise RuntimeError("trace set after the step graphs were captured")
            ttok = g.ttok.view(g.bs, k + 1)[:B] if self._argmax_verify(g.bs) else None
            drafts = g.vids[:B, 1:] if self._argmax_drafts(g.bs) else g.drafts[:B]
            self._record(g.tl.view(g.bs, k + 1, -1)[:B], drafts,
                         g.arena.h["start"][:B], kvp,
                         g.arena.h["idx"][k * sx:k * sx + int(kvp[-1])],
                         g.n_out[:B], g.emitted[:B], g.rollback[:B], ttok,
                         None if g.dlog is None else g.dlog[:B],
                         None if g.u is None else g.u[:B])
        return g.n_h.numpy()[:B], g.em_h.numpy()[:B]

    def _record(self, tl, drafts, start, kv_indptr, kv_indices, n_out, emitted, rollback,
                target_tokens=None, draft_logits=None, uniforms=None):
        """Append one step's verify logits, acceptance inputs and outputs to
        ``self.trace`` (host copies); ``target_tokens``: the verify rows'
        tokens of the greedy lm_head kernel, when the step accepted from
        those; ``draft_logits`` / ``uniforms``: the stochastic acceptance's
        other inputs."""
        self.trace.append({
            "target_tokens": None if target_tokens is None else target_tokens.cpu().numpy(),
            "draft_logits": None if draft_logits is None else draft_logits.detach().cpu(),
            "uniforms": None if uniforms is None else uniforms.cpu().numpy(),
            "verify_logits": tl.detach().cpu(), "drafts": drafts.cpu().numpy(),
            "start": np.asarray(start, np.int64).copy(),
            "kv_indptr": np.asarray(kv_indptr, np.int32).copy(),
            "kv_indices": np.asarray(kv_indices, np.int32).copy(),
            "num_emitted": n_out.cpu().numpy(), "emitted": emitted.cpu().numpy(),
            "rollback": rollback.cpu().numpy(), "page_size": self.P,
            "temperature": self.temperature})

    # ---- eager mode ----
    def _step_eager(self, active: list):
        k, dev = self.k, self.device
        B = len(active)
        starts = [r.start for r in active]
        start_pos = np.asarray(starts, np.int64)
        tok = self._to_dev(np.asarray([r.out[-1] for r in active], np.int64))
        ones = [1] * B
        drafts = torch.empty(B, k, dtype=torch.int64, device=dev)
        vids = torch.empty(B, k + 1, dtype=torch.int64, device=dev)
        direct = self._argmax_drafts(B)
        dlog = None
        for i in range(k):
            self._plan(active, ones, [s + i + 1 for s in starts])
            sl = self._to_dev(self._slots(active, [s + i for s in starts], ones))
            if direct:
                tok = self.model.forward_packed(tok, self._to_dev(start_pos + i), self._pool(),
                                                self.attn, sl, None, self.draft_layers,
                                                argmax_out=vids[:, i + 1],
                                                argmax_ws=self._argmax_ws)
                continue
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
        vids[:, 0] = self._to_dev(np.asarray([r.out[-1] for r in active], np.int64))
        if direct:
            drafts = vids[:, 1:].contiguous()
        else:
            vids[:, 1:] = drafts
        vpos = self._to_dev((start_pos[:, None] + np.arange(k + 1)[None]).reshape(-1))
        sl = self._to_dev(self._slots(active, starts, [k + 1] * B))
        if self._argmax_verify(B):
            V = self.model.config.vocab_size
            ttok = torch.empty(B * (k + 1), dtype=torch.int64, device=dev)
            tl = (torch.empty(B * (k + 1), V, dtype=torch.bfloat16, device=dev)
                  if self.trace is not None else None)
            self.model.forward_packed(vids.view(-1), vpos, self._pool(), self.attn, sl,
                                      argmax_out=ttok, argmax_ws=self._argmax_ws,
                                      argmax_logits=tl)
            n_out, emitted, rollback = kernels.spec_accept_greedy_tokens(
                ttok.view(B, k + 1), drafts, V, self._to_dev(kvp), self._to_dev(idx),
                self._to_dev(start_pos, torch.int32), page_size=self.P,
                workspace=self._accept_ws)
            if self.trace is not None:
                self._record(tl.view(B, k + 1, -1), drafts, start_pos, kvp, idx, n_out, emitted,
                             rollback, ttok.view(B, k + 1))
            return n_out.cpu().numpy(), emitted.cpu().numpy()
        tl = self.model.forward_packed(vids.view(-1), vpos, self._pool(), self.attn, sl)
        u = None if self.greedy else self._uniforms(0, B * (k + 1)).view(B, k + 1)
        n_out, emitted, rollback = kernels.spec_accept(
            tl.view(B, k + 1, -1), dlog, drafts, u, self.temperature,
            self._to_dev(kvp), self._to_dev(idx), self._to_dev(start_pos, torch.int32),
            page_size=self.P, bonus_tokens=self._bonus(tl.view(B, k + 1, -1), u))
        if self.trace is not None:
            self._record(tl.view(B, k + 1, -1), drafts, start_pos, kvp, idx, n_out, emitted,
                         rollback, None, dlog, u)
        return n_out.cpu().numpy(), emitted.cpu().numpy()

    # ---- main entry ----
    def _admit(self, reqs: list, synthetic_context: bool = False) -> None:
        """Admission and prefill: a block table per request
        (paged_kv_cache.py:113-120), one ragged packed forward over every
        prompt (engine.py:298-472), the first token of each request.
        ``synthetic_context``: the prompt positions' K/V are the pool's seeded
        noise instead (decoding measured alone); the first token is then the
        prompt's last id."""
        for r in reqs:
            r.table = self.kv.allocate_for_request(len(r.prompt))
        if self.use_graphs:
            self._tab = np.zeros((len(reqs), self._max_pages()), np.int32)
            for i, r in enumerate(reqs):
                r.row = i
        lens = [len(r.prompt) for r in reqs]
        if synthetic_context:
            if not self._noise:
                g = torch.Generator(device=self.device).manual_seed(self.seed)
                for pool in self._pool():
                    for layer in pool:
                        layer.normal_(generator=g)
                self._noise = True
            first = [r.prompt[-1] for r in reqs]
        else:
            self._plan(reqs, lens, lens)
            ids = self._to_dev(np.concatenate([np.asarray(r.prompt, np.int64) for r in reqs]))
            pos = self._to_dev(np.concatenate([np.arange(n, dtype=np.int64) for n in lens]))
            slots = self._to_dev(self._slots(reqs, [0] * len(reqs), lens))
            last_idx = self._to_dev(np.cumsum(lens) - 1)
            logits = self.model.forward_packed(ids, pos, self._pool(), self.attn, slots,
                                               last_idx)
            first = self._sample_rows(logits).cpu().tolist()
        for r, f in zip(reqs, first):
            r.out.append(f)
            r.start = len(r.prompt)

    def _step(self, active: list, rows: int = 0):
        """One speculative step for the active requests: reserve the verify
        window's pages (scheduler.py:221-232 applied to k + 1 positions),
        draft, verify and accept (graph or eager), append the emitted tokens,
        advance the positions and roll back pages past them.  Returns the
        per-request emitted counts.  Graph mode runs the graph for at least
        ``rows`` rows (generate passes the previous step's batch)."""
        k = self.k
        for r in active:
            self.kv.reserve(r.table, r.start + k + 1)
            if self.use_graphs:
                self._sync_table(r)
        if self.use_graphs:
            n_h, em_h = self._step_graph(active, rows)
        else:
            n_h, em_h = self._step_eager(active)
        for j, r in enumerate(active):
            n = int(n_h[j])
            r.out.extend(em_h[j, :n].tolist())
            r.start += n
            self.kv.truncate(r.table, r.start)        # rollback of rejected pages
            r.synced = min(r.synced, len(r.table.block_indices))
        return n_h

    def _decode_pipelined(self, active: list, count) -> None:
        """The speculative steps of generate() in graph mode, pipelined: while
        step s runs on the GPU, step s + 1 is already queued behind the host
        gate (nsg_host_gate_wait), with pages reserved for its verify window
        whatever step s accepts.  Once step s's results are read, the host
        appends them, writes step s + 1's inputs (requests that finished at s
        become padding rows) and raises the gate; page rollback and frees
        follow while step s + 1 runs.  In both loops step s + 1 runs the
        graph sized for step s's batch (requests that finish at s are padding
        rows for one step), so its graph does not depend on step s's outcome;
        step s + 1 is queued early when some request surely outlives step s
        (more than k + 1 tokens to go).  Every step therefore runs the graph,
        inputs and Philox offsets of the unpipelined loop, and the tokens are
        identical.  ``count(B, n)`` receives each step's batch size and
        emitted counts."""
        k = self.k
        for r in active:
            self.kv.reserve(r.table, r.start + k + 1)
            self._sync_table(r)
        g = self._graph_for(len(active))
        self._fill_step(g, active)
        self._launch(g, gated=False)
        cur = active
        cap = self._max_pages() * self.P     # positions the page-table mirror holds
        pending = False                  # a gated step is queued and not yet released
        try:
            while cur:
                nxt = None
                if (any(r.max_new - len(r.out) > k + 1 for r in cur) and
                        all(r.start + 2 * (k + 1) <= cap for r in cur)):
                    for r in cur:        # step s + 1's window, whatever step s accepts
                        self.kv.reserve(r.table, r.start + 2 * (k + 1))
                        self._sync_table(r)
                    nxt = self._graph_for(len(cur))
                    # page ids per attention call of step s + 1: at most every
                    # page reserved now, plus the padding rows' dummy pages
                    pages = (sum(len(r.table.block_indices) for r in cur)
                             + (nxt.bs - len(cur)) * ((k + self.P) // self.P))
                    pending = True
                    self._launch(nxt, gated=True, pages=pages)
                    # step s + 1's fill, but for step s's results (n_out,
                    # emitted), prepared while step s runs
                    fill_next = self._fill_next_args(nxt, g, cur)
                self._wait_done(g)
                if nxt is not None:    # release step s + 1 first, bookkeeping after
                    self._run_fill_next(fill_next)
                    nxt.done.value = 0
                    self._raise_gate()
                    pending = False
                    si = nxt.strides[0]
                    kvp = nxt.arena.h["kvp"]
                    if max(int(kvp[a * si + nxt.bs]) for a in range(k + 1)) > pages:
                        raise RuntimeError("step fill wrote more page ids than the gate "
                                           f"copied ({pages}): that step ran on stale page ids")
                B = len(cur)
                n_h = g.n_h.numpy()[:B].copy()
                em_h = g.em_h.numpy()[:B].copy()
                count(B, n_h)
                still = []
                for j, r in enumerate(cur):
                    n = int(n_h[j])
                    r.out.extend(em_h[j, :n].tolist())
                    r.start += n
                    if len(r.out) < r.max_new:
                        still.append(r)
                # rollback and frees, off the GPU's path: keep step s + 1's
                # window when it is already queued
                keep = k + 1 if nxt is not None else 0
                for r in cur:
                    if len(r.out) >= r.max_new:
                        del r.out[r.max_new:]
                        self.kv.free_request(r.table)
                    else:
                        self.kv.truncate(r.table, r.start + keep)
                        r.synced = min(r.synced, len(r.table.block_indices))
                if nxt is not None:
                    g = nxt
                elif still:
                    for r in still:
                        self.kv.reserve(r.table, r.start + k + 1)
                        self._sync_table(r)
                    g = self._graph_for(len(cur))
                    self._fill_step(g, still)
                    self._launch(g, gated=False)
                cur = still
        finally:
            if pending:                  # an exception left a queued step held: release it
                self._raise_gate()
                torch.cuda.current_stream(self.device).synchronize()

    # device error bits of the attention and acceptance kernels (their
    # workspaces' flag words), by kernel
    _ATTN_FLAGS = {1: "a KV page id outside the pool (attention)"}
    _ACCEPT_FLAGS = {2: "a rolled-back position past its request's pages (acceptance)",
                     4: "a draft token outside the vocabulary (acceptance)",
                     8: "an acceptance hand-off wait gave up; its outputs are undefined "
                        "(the workspace was cleared)"}

    def check_device_flags(self) -> None:
        """Reads and clears the error flags the attention and acceptance
        kernels raise on the device, and raises RuntimeError naming every
        condition found, as the reference raises RuntimeError on bad KV state
        (paged_kv_cache.py:88-89,116-119).  Synchronises the stream."""
        found = []
        a = self.attn.check_flags()
        found += [msg for bit, msg in self._ATTN_FLAGS.items() if a & bit]
        c = self._accept_ws.check_flags()
        found += [msg for bit, msg in self._ACCEPT_FLAGS.items() if c & bit]
        if int(self._gate_err.item()):
            self._gate_err.zero_()
            found.append("the host gate timed out (a pipelined step ran on stale inputs)")
        if a & ~1 or c & ~14:
            found.append(f"unknown flag bits (attention {a:#x}, acceptance {c:#x})")
        if found:
            raise RuntimeError("device error flags: " + "; ".join(found))

    def _check_batch(self, n: int) -> None:
        if self.use_graphs and n > self.max_batch:
            raise ValueError(f"{n} requests > max_batch {self.max_batch} of the graphs")
        if self.use_graphs and not self._graphs:
            self.capture()

    @torch.inference_mode()
    def prefill(self, prompts: list[list[int]], synthetic_context: bool = False):
        """Admit and prefill ``prompts`` (additive API, with
        :meth:`speculative_step_batch`).  Returns (first tokens, block
        tables): request b's KV cache holds positions < len(prompts[b]) in
        block_tables[b]; its first token sits at position len(prompts[b]).
        ``synthetic_context``: as in :meth:`generate`, the prompt positions'
        K/V are the pool's seeded noise and the first token is the prompt's
        last id."""
        self._check_batch(len(prompts))
        reqs = [_Req(i, list(p), 1) for i, p in enumerate(prompts)]
        self._admit(reqs, synthetic_context)
        self.check_device_flags()
        return [r.out[0] for r in reqs], [r.table for r in reqs]

    @torch.inference_mode()
    def speculative_step_batch(self, last_tokens: list[int], start_pos: list[int],
                               block_tables: list[BlockTable]) -> list[list[int]]:
        """One batched speculative step on the paged cache (additive API: the
        reference's ``speculative_step``, speculative.py:50-184, is batch-1).

        Request b's last emitted token ``last_tokens[b]`` sits at position
        ``start_pos[b]``; its KV cache holds positions < start_pos[b] in
        ``block_tables[b]``.  Drafts k tokens, verifies them in one target
        forward, accepts, and returns the 1..k+1 emitted tokens per request.
        The tables are grown for the verify window and rolled back past the
        kept positions (the next call's start is start_pos[b] + len(result[b]),
        its last token result[b][-1])."""
        B = len(last_tokens)
        if len(start_pos) != B or len(block_tables) != B:
            raise ValueError("last_tokens, start_pos and block_tables disagree on the batch")
        if B == 0:
            return []
        self._check_batch(B)
        reqs = []
        for i, (t, s, bt) in enumerate(zip(last_tokens, start_pos, block_tables)):
            r = _Req(i, [], 1 << 30, table=bt, out=[int(t)], start=int(s))
            if r.start < 0 or len(bt.block_indices) * self.P < r.start:
                raise ValueError(f"request {i}: start {r.start} beyond its block table")
            reqs.append(r)
        if self.use_graphs:
            self._tab = np.zeros((B, self._max_pages()), np.int32)
            for i, r in enumerate(reqs):
                r.row = i
        self._step(reqs)
        self.check_device_flags()
        return [r.out[1:] for r in reqs]

    @torch.inference_mode()
    def generate(self, prompts: list[list[int]], max_new_tokens: list[int],
                 synthetic_context: bool = False):
        """Serve ``prompts`` to ``max_new_tokens`` tokens each (EOS ignored).

        ``synthetic_context``: measure decoding alone -- the prompt positions'
        K/V are the pool's seeded noise instead of a prefill forward, and the
        first output token is the prompt's last id."""
        k = self.k
        reqs = [_Req(i, list(p), int(m)) for i, (p, m) in enumerate(zip(prompts, max_new_tokens))]
        self._check_batch(len(reqs))
        t0 = time.perf_counter()
        # 1-2. admission and prefill
        self._admit(reqs, synthetic_context)
        lens = [len(r.prompt) for r in reqs]
        t_prefill = time.perf_counter() - t0
        active = [r for r in reqs if len(r.out) < r.max_new]
        for r in reqs:
            if r not in active:
                self.kv.free_request(r.table)
        # 3. speculative steps
        tally = [0, 0, 0, 0]                # steps, request-steps, proposed, accepted

        def count(B, n_h):
            tally[0] += 1
            tally[1] += B
            tally[2] += B * k
            tally[3] += int(n_h.sum()) - B

        if active and self.use_graphs and self.pipeline and self.trace is None:
            self._decode_pipelined(active, count)
            active = []
        prev = 0
        while active:
            B = len(active)
            n_h = self._step(active, prev)
            prev = B
            count(B, n_h)
            still = []
            for r in active:
                if len(r.out) >= r.max_new:
                    del r.out[r.max_new:]
                    self.kv.free_request(r.table)
                else:
                    still.append(r)
            active = still
        steps, req_steps, proposed, accepted = tally
        self.check_device_flags()           # synchronises the stream
        t_total = time.perf_counter() - t0
        n_tok = sum(len(r.out) for r in reqs)
        self.stats = {
            "elapsed_s": t_total, "prefill_s": t_prefill, "output_tokens": n_tok,
            "prompt_tokens": sum(lens), "steps": steps,
            "acceptance_rate": accepted / proposed if proposed else 0.0,
            "tokens_per_step": (accepted + req_steps) / max(1, req_steps),
            "tok_per_s": n_tok / t_total,
            "decode_tok_per_s": (n_tok - len(reqs)) / max(1e-9, t_total - t_prefill),
            "graphs": sorted(self._graphs),
        }
        return [r.out for r in reqs]
