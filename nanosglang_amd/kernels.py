"""PyTorch-facing wrappers of the verify-step C ABI (include/nsg_spec.h).

torch supplies device memory and the current HIP stream only; every
computation runs in the HIP kernels of libnsg_spec.so.  Nothing here falls
back to PyTorch or the CPU: a missing library or a non-GPU tensor raises.

* :class:`BatchPrefillWithPagedKVCacheWrapper` -- drop-in for the FlashInfer
  wrapper the reference uses for paged attention (constructed at
  nano_sglang/engine/engine.py:106-108, planned at engine.py:451-462, run at
  nano_sglang/model/causal_lm.py:340).
* :func:`spec_accept` -- fused acceptance / resample / bonus / rollback slots,
  replacing the loop at nano_sglang/decode/speculative.py:130-184.
* :func:`kv_write` -- replaces the index_put scatter at causal_lm.py:335-338.
* :func:`kv_clear_slots`, :func:`philox_uniform`.
"""

from __future__ import annotations

import ctypes as C
import math
import threading

import numpy as np
import torch

from . import _native
from ._native import NSG_ATTN_WORK_INTS, AttnPlan, check

MI355X_CUS = 256


def _lib():
    return _native.load()


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_gpu(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (no CPU path exists)")


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _host_i32(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        t = t.detach().to("cpu", torch.int32)
        return np.ascontiguousarray(t.numpy())
    return np.ascontiguousarray(np.asarray(t, dtype=np.int32))


def _dev_i32(t, device) -> torch.Tensor:
    if isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.int32 and t.is_contiguous():
        return t
    if isinstance(t, np.ndarray):
        t = torch.from_numpy(np.ascontiguousarray(t, dtype=np.int32))
    return torch.as_tensor(t, dtype=torch.int32).contiguous().to(device, non_blocking=True)


def attn_work_bound(qo_h: np.ndarray, kvp_h: np.ndarray, last_h: np.ndarray,
                    num_qo_heads: int, num_kv_heads: int, page_size: int) -> int:
    """Upper bound on the work (plus merge) items of a dynamic attention plan:
    every query tile split into every 32-token KV step, plus one merge item
    (tiles of the smallest size a plan takes: 16 rows when G <= 16)."""
    bound = 0
    G = max(1, num_qo_heads // max(1, num_kv_heads))
    T = max(1, min((16 if G <= 16 else 64) // G, int(np.diff(qo_h).max(initial=1))))
    for b in range(len(qo_h) - 1):
        ql = int(qo_h[b + 1] - qo_h[b])
        npg = int(kvp_h[b + 1] - kvp_h[b])
        L = (npg - 1) * page_size + int(last_h[b]) if npg else 0
        bound += math.ceil(ql / T) * (1 + max(1, math.ceil(L / 32)))
    return bound


class BatchPrefillWithPagedKVCacheWrapper:
    """Ragged multi-query attention over an NHD paged KV cache.

    Same constructor / plan / run shape as the FlashInfer wrapper the
    reference calls (engine.py:106-108, 451-462; causal_lm.py:340):

    >>> w = BatchPrefillWithPagedKVCacheWrapper(workspace_u8, kv_layout="NHD")
    >>> w.plan(qo_indptr, kv_indptr, kv_indices, kv_last_page_len,
    ...        num_qo_heads, num_kv_heads, head_dim, page_size, causal=True)
    >>> out = w.run(q, (k_cache[layer], v_cache[layer]))

    ``plan`` reads the CSR metadata on the host once per step; ``run`` enqueues
    one kernel per layer on the current stream and never syncs the host.
    The workspace is zero-filled here once; the kernel leaves it reusable.
    """

    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD",
                 use_cuda_graph: bool = False, qo_indptr_buf: torch.Tensor | None = None,
                 paged_kv_indptr_buf: torch.Tensor | None = None,
                 paged_kv_indices_buf: torch.Tensor | None = None,
                 paged_kv_last_page_len_buf: torch.Tensor | None = None,
                 num_cus: int = MI355X_CUS, work_buf: torch.Tensor | None = None,
                 host_bufs: dict | None = None, max_q_len: int | None = None,
                 max_kv_len: int = 0):
        """``use_cuda_graph=True`` with the four ``*_buf`` int32 device tensors
        is the reference's graph mode (engine.py:121-133): ``plan`` rewrites
        those fixed-address buffers and a fixed-size work list (``work_buf``,
        allocated at the first plan if not given), so a graph captured around
        ``run`` replays correctly after each re-plan.  The batch is
        ``len(qo_indptr_buf) - 1``; the tile shape follows ``max_q_len``
        (default: the first plan's longest query); ``max_kv_len`` > 0 bounds every
        request's KV length so that plans never split it (no merge launch).
        With ``host_bufs`` (numpy
        mirrors keyed qo_indptr / kv_indptr / kv_indices / kv_last / work),
        ``plan`` writes only the mirrors and the caller uploads them."""
        if kv_layout != "NHD":
            raise ValueError(f"kv_layout {kv_layout!r}: only 'NHD' (the reference's layout)")
        _require_gpu(float_workspace_buffer, "workspace")
        self._ws = float_workspace_buffer
        self._ws.zero_()
        self._device = float_workspace_buffer.device
        self._num_cus = num_cus
        self._work_cap = 0
        self._work_d: torch.Tensor | None = None
        self._work_h = np.zeros(0, np.int32)
        self._plan: AttnPlan | None = None
        self._graph = bool(use_cuda_graph)
        if self._graph:
            bufs = {"qo_indptr": qo_indptr_buf, "kv_indptr": paged_kv_indptr_buf,
                    "kv_indices": paged_kv_indices_buf, "kv_last": paged_kv_last_page_len_buf}
            for name, t in bufs.items():
                if t is None:
                    raise ValueError(f"use_cuda_graph=True needs the {name} buffer")
                _require_gpu(t, name)
                if t.dtype != torch.int32 or not t.is_contiguous():
                    raise ValueError(f"{name} buffer must be contiguous int32")
            self._batch = qo_indptr_buf.numel() - 1
            if (paged_kv_indptr_buf.numel() != self._batch + 1
                    or paged_kv_last_page_len_buf.numel() != self._batch):
                raise ValueError("graph buffers disagree on the batch size")
            if host_bufs is not None:
                for name, t in bufs.items():
                    if host_bufs[name].shape != (t.numel(),) or host_bufs[name].dtype != np.int32:
                        raise ValueError(f"host mirror {name} must be int32 ({t.numel()},)")
            self._gbufs = bufs
            self._host_bufs = host_bufs
            self._fixed_q = max_q_len
            self._fixed_kv = int(max_kv_len)
            self._fixed = None          # (max_q_len, max_work, max_merge) from the first plan
            self._work_d = work_buf

    def _plan_fixed(self, lib, qo_h, kvp_h, last_h, B, num_qo_heads, num_kv_heads, head_dim_qk,
                    page_size, causal, kv_indices) -> AttnPlan:
        if B != self._batch:
            raise ValueError(f"graph-mode wrapper holds batch {self._batch}, plan has {B}")
        if self._fixed is None:
            mq = self._fixed_q or max(1, int(np.diff(qo_h).max(initial=1)))
            mw, mm = C.c_int32(0), C.c_int32(0)
            check(lib.nsg_attn_fixed_capacity(B, mq, num_qo_heads, num_kv_heads, self._num_cus,
                                              self._fixed_kv, C.byref(mw), C.byref(mm)),
                  "nsg_attn_fixed_capacity")
            need = (mw.value + mm.value) * NSG_ATTN_WORK_INTS
            if self._work_d is None:
                self._work_d = torch.zeros(need, dtype=torch.int32, device=self._device)
            elif self._work_d.numel() < need or self._work_d.dtype != torch.int32:
                raise ValueError(f"work_buf must hold {need} int32")
            if self._host_bufs is not None:
                self._work_h = self._host_bufs["work"]
                if self._work_h.dtype != np.int32 or self._work_h.shape[0] < need:
                    raise ValueError(f"host work mirror must hold {need} int32")
            else:
                self._work_h = np.zeros(need, np.int32)
            self._fixed = (mq, mw.value, mm.value)
        mq, mw, mm = self._fixed
        pl = AttnPlan()
        check(lib.nsg_attn_plan_fixed(qo_h.ctypes.data, kvp_h.ctypes.data, last_h.ctypes.data, B,
                                      num_qo_heads, num_kv_heads, head_dim_qk, page_size,
                                      1 if causal else 0, self._num_cus, mq, self._fixed_kv,
                                      mw, mm,
                                      self._work_h.ctypes.data, self._work_h.shape[0],
                                      C.byref(pl)), "nsg_attn_plan_fixed")
        nnz = int(kvp_h[-1])
        idx_buf = self._gbufs["kv_indices"]
        if nnz > idx_buf.numel():
            raise ValueError(f"{nnz} page ids exceed the kv_indices buffer ({idx_buf.numel()})")
        idx_h = _host_i32(kv_indices)[:nnz]
        if self._host_bufs is not None:
            hb = self._host_bufs
            hb["qo_indptr"][:] = qo_h
            hb["kv_indptr"][:] = kvp_h
            hb["kv_last"][:] = last_h
            hb["kv_indices"][:nnz] = idx_h
        else:
            n = (pl.num_work + pl.num_merge) * NSG_ATTN_WORK_INTS
            for name, h in (("qo_indptr", qo_h), ("kv_indptr", kvp_h), ("kv_last", last_h),
                            ("kv_indices", idx_h)):
                self._gbufs[name][:h.shape[0]].copy_(torch.from_numpy(h))
            self._work_d[:n].copy_(torch.from_numpy(self._work_h[:n]))
        return pl

    def plan(self, qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len,
             num_qo_heads: int, num_kv_heads: int, head_dim_qk: int, page_size: int,
             causal: bool = True, q_data_type=torch.bfloat16, sm_scale: float | None = None):
        if q_data_type not in (torch.bfloat16, "bfloat16"):
            raise NotImplementedError(f"q_data_type {q_data_type}: the kernel is bf16")
        qo_h = _host_i32(qo_indptr)
        kvp_h = _host_i32(paged_kv_indptr)
        last_h = _host_i32(paged_kv_last_page_len)
        B = len(qo_h) - 1
        if len(kvp_h) != B + 1 or len(last_h) != B:
            raise ValueError("qo_indptr, paged_kv_indptr and last_page_len disagree on batch")
        lib = _lib()
        if self._graph:
            pl = self._plan_fixed(lib, qo_h, kvp_h, last_h, B, num_qo_heads, num_kv_heads,
                                  head_dim_qk, page_size, causal, paged_kv_indices)
        else:
            pl = self._plan_dynamic(lib, qo_h, kvp_h, last_h, B, num_qo_heads, num_kv_heads,
                                    head_dim_qk, page_size, causal)
        if not self._graph:
            self._qo_indptr = _dev_i32(qo_indptr, self._device)
            self._kv_indptr = _dev_i32(paged_kv_indptr, self._device)
            self._kv_indices = _dev_i32(paged_kv_indices, self._device)
            self._kv_last = _dev_i32(paged_kv_last_page_len, self._device)
        self._set_plan(pl, int(qo_h[-1]), num_qo_heads, num_kv_heads, head_dim_qk, page_size,
                       causal, sm_scale)

    def _set_plan(self, pl, total_q, num_qo_heads, num_kv_heads, head_dim_qk, page_size,
                  causal, sm_scale):
        if pl.workspace_bytes > self._ws.numel() * self._ws.element_size():
            raise RuntimeError(
                f"attention workspace too small: plan needs {pl.workspace_bytes} bytes, "
                f"buffer has {self._ws.numel() * self._ws.element_size()}")
        self._plan = pl
        if self._graph:
            g = self._gbufs
            self._qo_indptr, self._kv_indptr = g["qo_indptr"], g["kv_indptr"]
            self._kv_indices, self._kv_last = g["kv_indices"], g["kv_last"]
        self._total_q = int(total_q)
        self._page_size = page_size
        self._causal = causal
        self._sm_scale = (1.0 / math.sqrt(head_dim_qk)) if sm_scale is None else float(sm_scale)
        self._dims = (num_qo_heads, num_kv_heads, head_dim_qk)

    def adopt_plan(self, plan: AttnPlan, total_q: int, num_qo_heads: int, num_kv_heads: int,
                   head_dim_qk: int, page_size: int, causal: bool = True,
                   sm_scale: float | None = None) -> None:
        """Graph mode: take a plan whose metadata and work list a host routine
        (``nsg_spec_step_fill``) already wrote into this wrapper's buffers --
        the state ``plan`` leaves, without re-planning.  The plan must have the
        fixed shape of this wrapper's graph buffers (``max_q_len``,
        ``max_kv_len``), so that a graph captured around ``run`` replays it."""
        if not self._graph:
            raise ValueError("adopt_plan is for use_cuda_graph=True wrappers")
        if self._fixed is None:
            if not self._fixed_q:
                raise ValueError("adopt_plan needs a wrapper built with max_q_len")
            lib = _lib()
            mq = self._fixed_q
            mw, mm = C.c_int32(0), C.c_int32(0)
            check(lib.nsg_attn_fixed_capacity(self._batch, mq, num_qo_heads, num_kv_heads,
                                              self._num_cus, self._fixed_kv, C.byref(mw),
                                              C.byref(mm)), "nsg_attn_fixed_capacity")
            if self._work_d is None or self._work_d.numel() < (mw.value + mm.value) * \
                    NSG_ATTN_WORK_INTS:
                raise ValueError("adopt_plan needs a work_buf of the fixed capacity")
            self._fixed = (mq, mw.value, mm.value)
        mq, mw, mm = self._fixed
        if (plan.num_work, plan.num_merge) != (mw, mm):
            raise ValueError(f"plan holds {plan.num_work} + {plan.num_merge} work items, the "
                             f"fixed list {mw} + {mm}")
        self._set_plan(plan, total_q, num_qo_heads, num_kv_heads, head_dim_qk, page_size, causal,
                       sm_scale)

    def _plan_dynamic(self, lib, qo_h, kvp_h, last_h, B, num_qo_heads, num_kv_heads,
                      head_dim_qk, page_size, causal) -> AttnPlan:
        bound = attn_work_bound(qo_h, kvp_h, last_h, num_qo_heads, num_kv_heads, page_size)
        if bound > self._work_cap:
            self._work_cap = max(bound, 2 * self._work_cap, 64)
            self._work_h = np.zeros(self._work_cap * NSG_ATTN_WORK_INTS, np.int32)
            self._work_d = torch.empty(self._work_cap * NSG_ATTN_WORK_INTS, dtype=torch.int32,
                                       device=self._device)
        pl = AttnPlan()
        rc = lib.nsg_attn_plan(qo_h.ctypes.data, kvp_h.ctypes.data, last_h.ctypes.data, B,
                               num_qo_heads, num_kv_heads, head_dim_qk, page_size,
                               1 if causal else 0, self._num_cus, self._work_h.ctypes.data,
                               self._work_cap, C.byref(pl))
        check(rc, "nsg_attn_plan")
        n = (pl.num_work + pl.num_merge) * NSG_ATTN_WORK_INTS
        if n:
            self._work_d[:n].copy_(torch.from_numpy(self._work_h[:n]), non_blocking=False)
        return pl

    @property
    def plan_info(self) -> AttnPlan:
        return self._plan

    def run(self, q: torch.Tensor, paged_kv_cache, out: torch.Tensor | None = None) -> torch.Tensor:
        if self._plan is None:
            raise RuntimeError("run() before plan()")
        k_cache, v_cache = paged_kv_cache
        Hq, Hkv, D = self._dims
        for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
            _require_gpu(t, name)
            if t.dtype != torch.bfloat16:
                raise TypeError(f"{name} must be bfloat16, got {t.dtype}")
            if not t.is_contiguous():
                raise ValueError(f"{name} must be contiguous")
        if tuple(q.shape) != (self._total_q, Hq, D):
            raise ValueError(f"q shape {tuple(q.shape)} != planned {(self._total_q, Hq, D)}")
        if (k_cache.dim() != 4 or k_cache.shape[1] != self._page_size or k_cache.shape[2] != Hkv
                or k_cache.shape[3] != D or v_cache.shape != k_cache.shape):
            raise ValueError(f"KV cache shape {tuple(k_cache.shape)} is not "
                             f"[pages, {self._page_size}, {Hkv}, {D}]")
        if out is None:
            out = torch.empty_like(q)
        rc = _lib().nsg_attn_run(
            C.byref(self._plan), self._work_d.data_ptr(), q.data_ptr(), k_cache.data_ptr(),
            v_cache.data_ptr(), out.data_ptr(), self._qo_indptr.data_ptr(),
            self._kv_indptr.data_ptr(), self._kv_indices.data_ptr(), self._kv_last.data_ptr(),
            self._page_size, k_cache.shape[0], self._sm_scale, 1 if self._causal else 0,
            self._ws.data_ptr(), self._ws.numel() * self._ws.element_size(),
            _stream_ptr(q.device))
        check(rc, "nsg_attn_run")
        return out

    def check_flags(self) -> int:
        """Synchronises and returns (then clears) the kernel's error flags."""
        f = C.c_int32(0)
        check(_lib().nsg_attn_check_flags(self._ws.data_ptr(), C.byref(f),
                                          _stream_ptr(self._device)), "nsg_attn_check_flags")
        return f.value


class AcceptWorkspace:
    """Device scratch of :func:`spec_accept` (zero-filled once, grown on
    demand), or of :func:`sample` -- never both: the acceptance kernels pass
    records between workgroups through slots that must read zero between
    calls, and they leave them so.  Calls that share one workspace must not
    overlap on different streams."""

    def __init__(self, device):
        self.device = torch.device(device)
        self.buf = torch.zeros(0, dtype=torch.uint8, device=self.device)
        # buffers replaced by a larger one stay allocated: a HIP graph
        # captured while one of them was current keeps writing to it
        self._retired: list[torch.Tensor] = []

    def get(self, nbytes: int) -> torch.Tensor:
        if self.buf.numel() < nbytes:
            if self.buf.numel():
                self._retired.append(self.buf)
            self.buf = torch.zeros(max(nbytes, 2 * self.buf.numel()), dtype=torch.uint8,
                                   device=self.device)
        return self.buf

    def check_flags(self) -> int:
        """Synchronises and returns (then clears) the acceptance kernels'
        error flags: bit 1, a rolled-back position past its request's pages;
        bit 2, a draft token outside [0, vocab); bit 3, a hand-off between
        workgroups gave up waiting (the outputs of that call are undefined and
        the whole workspace is zeroed again here)."""
        if self.buf.numel() == 0:
            return 0
        f = C.c_int32(0)
        check(_lib().nsg_spec_accept_check_flags(self.buf.data_ptr(), self.buf.numel(),
                                                 C.byref(f), _stream_ptr(self.device)),
              "nsg_spec_accept_check_flags")
        return f.value


_default_ws: dict[tuple, AcceptWorkspace] = {}
_default_ws_lock = threading.Lock()


def _accept_ws(device, kind: str = "accept") -> AcceptWorkspace:
    """The default ``kind`` ("accept" or "sample") workspace of the current
    stream on ``device``: calls on one stream run in order, so they may share
    it; calls on different streams (or threads using different streams) get
    their own."""
    device = torch.device(device)
    key = (device, _stream_ptr(device), kind)
    ws = _default_ws.get(key)
    if ws is None:
        with _default_ws_lock:
            ws = _default_ws.setdefault(key, AcceptWorkspace(device))
    return ws


def spec_accept(target_logits: torch.Tensor, draft_logits: torch.Tensor | None,
                draft_tokens: torch.Tensor | None, uniforms: torch.Tensor | None,
                temperature: float, kv_indptr: torch.Tensor | None = None,
                kv_indices: torch.Tensor | None = None, start_pos: torch.Tensor | None = None,
                page_size: int = 16, workspace: AcceptWorkspace | None = None,
                out: tuple | None = None, bonus_tokens: torch.Tensor | None = None):
    """Fused verify-step acceptance for B requests (C ABI: nsg_spec_accept).

    target_logits (B, k+1, V) and draft_logits (B, k, V) in bf16 or fp32 with a
    unit stride along V; draft_tokens int64 (B, k); uniforms fp32 (B, k+1).
    Greedy when ``temperature < 1e-6`` (draft_logits / uniforms may be None).
    ``bonus_tokens`` int64 (B,) (stochastic only): the token emitted after k
    accepted drafts, e.g. a top-k / top-p draw from target row k
    (:func:`sample`); without it that bonus is drawn from softmax(row k / T).
    Returns (num_emitted int32 (B,), emitted int64 (B, k+1) padded -1,
    rollback_slots int64 (B, k) padded -1).
    """
    _require_gpu(target_logits, "target_logits")
    dev = target_logits.device
    if target_logits.dim() != 3:
        raise ValueError("target_logits must be (B, k+1, V)")
    B, k1, V = target_logits.shape
    k = k1 - 1
    dt = {torch.bfloat16: 0, torch.float32: 1}.get(target_logits.dtype)
    if dt is None:
        raise TypeError(f"logits dtype {target_logits.dtype}: bf16 or fp32")
    if target_logits.stride(2) != 1:
        raise ValueError("target_logits must be contiguous along the vocabulary")
    greedy = temperature < 1e-6
    if not greedy and k > 0:
        if draft_logits is None:
            raise ValueError("draft_logits required when temperature > 0")
        _require_gpu(draft_logits, "draft_logits")
        if draft_logits.dtype != target_logits.dtype or tuple(draft_logits.shape) != (B, k, V):
            raise ValueError("draft_logits must match target_logits' dtype with shape (B, k, V)")
        if draft_logits.stride(2) != 1:
            raise ValueError("draft_logits must be contiguous along the vocabulary")
        d_req, d_row = draft_logits.stride(0), draft_logits.stride(1)
    else:
        draft_logits, d_req, d_row = None, 0, 0
    if k > 0:
        if draft_tokens is None or tuple(draft_tokens.shape) != (B, k):
            raise ValueError("draft_tokens must be (B, k)")
        _require_gpu(draft_tokens, "draft_tokens")
        draft_tokens = draft_tokens.to(torch.int64).contiguous()
    if not greedy:
        if uniforms is None or tuple(uniforms.shape) != (B, k + 1):
            raise ValueError("uniforms must be (B, k+1) float32")
        _require_gpu(uniforms, "uniforms")
        uniforms = uniforms.to(torch.float32).contiguous()
    if bonus_tokens is not None and not greedy:
        _require_gpu(bonus_tokens, "bonus_tokens")
        if tuple(bonus_tokens.shape) != (B,) or bonus_tokens.dtype != torch.int64 \
                or not bonus_tokens.is_contiguous():
            raise ValueError("bonus_tokens must be contiguous int64 (B,)")
    else:
        bonus_tokens = None
    rb_ok = kv_indptr is not None and k > 0
    if rb_ok:
        for name, t in (("kv_indptr", kv_indptr), ("kv_indices", kv_indices),
                        ("start_pos", start_pos)):
            if t is None:
                raise ValueError(f"{name} required for rollback slots")
            _require_gpu(t, name)
        kv_indptr = kv_indptr.to(torch.int32).contiguous()
        kv_indices = kv_indices.to(torch.int32).contiguous()
        start_pos = start_pos.to(torch.int32).contiguous()
    if out is None:
        n_out = torch.empty(B, dtype=torch.int32, device=dev)
        emitted = torch.empty(B, k + 1, dtype=torch.int64, device=dev)
        rollback = torch.full((B, k), -1, dtype=torch.int64, device=dev)
    else:
        n_out, emitted, rollback = out
    lib = _lib()
    need = lib.nsg_spec_accept_workspace_bytes(B, k, V)
    ws = (workspace or _accept_ws(dev)).get(need)
    rc = lib.nsg_spec_accept(
        target_logits.data_ptr(), target_logits.stride(0), target_logits.stride(1),
        _ptr(draft_logits), d_req, d_row, dt, _ptr(draft_tokens) if k > 0 else None,
        _ptr(uniforms) if not greedy else None, _ptr(bonus_tokens), B, k, V, float(temperature),
        _ptr(kv_indptr) if rb_ok else None, _ptr(kv_indices) if rb_ok else None,
        _ptr(start_pos) if rb_ok else None, page_size, n_out.data_ptr(), emitted.data_ptr(),
        rollback.data_ptr() if rb_ok else None, ws.data_ptr(), ws.numel(), _stream_ptr(dev))
    check(rc, "nsg_spec_accept")
    return n_out, emitted, rollback


def _greedy_args(B, k, dev, draft_tokens, kv_indptr, kv_indices, start_pos, out):
    ds = (0, 0)
    if k > 0:
        if draft_tokens is None or tuple(draft_tokens.shape) != (B, k):
            raise ValueError("draft_tokens must be (B, k)")
        _require_gpu(draft_tokens, "draft_tokens")
        if draft_tokens.dtype != torch.int64:
            draft_tokens = draft_tokens.to(torch.int64)
        ds = (draft_tokens.stride(0), draft_tokens.stride(1))   # any strides
    rb_ok = kv_indptr is not None and k > 0
    if rb_ok:
        for name, t in (("kv_indptr", kv_indptr), ("kv_indices", kv_indices),
                        ("start_pos", start_pos)):
            if t is None:
                raise ValueError(f"{name} required for rollback slots")
            _require_gpu(t, name)
        kv_indptr = kv_indptr.to(torch.int32).contiguous()
        kv_indices = kv_indices.to(torch.int32).contiguous()
        start_pos = start_pos.to(torch.int32).contiguous()
    if out is None:
        n_out = torch.empty(B, dtype=torch.int32, device=dev)
        emitted = torch.empty(B, k + 1, dtype=torch.int64, device=dev)
        rollback = torch.full((B, k), -1, dtype=torch.int64, device=dev)
    else:
        n_out, emitted, rollback = out
    tail = (_ptr(kv_indptr) if rb_ok else None, _ptr(kv_indices) if rb_ok else None,
            _ptr(start_pos) if rb_ok else None)
    return (draft_tokens, ds, tail, rb_ok, (n_out, emitted, rollback))


def spec_accept_greedy_tokens(target_tokens: torch.Tensor, draft_tokens: torch.Tensor | None,
                              vocab: int, kv_indptr: torch.Tensor | None = None,
                              kv_indices: torch.Tensor | None = None,
                              start_pos: torch.Tensor | None = None, page_size: int = 16,
                              workspace: AcceptWorkspace | None = None, out: tuple | None = None):
    """Greedy acceptance from each target row's greedy token (C ABI:
    nsg_spec_accept_greedy_tokens): :func:`spec_accept` at temperature 0 with
    ``target_tokens`` int64 (B, k+1) = the first argmax of each target row
    (e.g. :func:`linear_argmax` of the verify forward), so the verify logits
    are never stored; ``draft_tokens`` (B, k) may have any strides.  Same
    outputs and rollback slots; draft tokens outside [0, vocab) set the error
    flag in ``workspace``'s header (read with its ``check_flags``)."""
    _require_gpu(target_tokens, "target_tokens")
    dev = target_tokens.device
    if target_tokens.dim() != 2 or target_tokens.dtype != torch.int64 \
            or not target_tokens.is_contiguous():
        raise ValueError("target_tokens must be contiguous int64 (B, k+1)")
    B, k1 = target_tokens.shape
    k = k1 - 1
    draft_tokens, ds, tail, rb_ok, (n_out, emitted, rollback) = _greedy_args(
        B, k, dev, draft_tokens, kv_indptr, kv_indices, start_pos, out)
    flags = (workspace or _accept_ws(dev)).get(256)
    rc = _lib().nsg_spec_accept_greedy_tokens(
        target_tokens.data_ptr(), _ptr(draft_tokens) if k > 0 else None, ds[0], ds[1], B, k,
        int(vocab), *tail, page_size, n_out.data_ptr(), emitted.data_ptr(),
        rollback.data_ptr() if rb_ok else None, flags.data_ptr(), _stream_ptr(dev))
    check(rc, "nsg_spec_accept_greedy_tokens")
    return n_out, emitted, rollback


def spec_accept_greedy_keys(target_keys: torch.Tensor, key_cols: int, B: int, k: int,
                            draft_tokens: torch.Tensor | None, vocab: int,
                            kv_indptr: torch.Tensor | None = None,
                            kv_indices: torch.Tensor | None = None,
                            start_pos: torch.Tensor | None = None, page_size: int = 16,
                            workspace: AcceptWorkspace | None = None, out: tuple | None = None,
                            target_tokens_out: torch.Tensor | None = None):
    """:func:`spec_accept_greedy_tokens` with each target row's token reduced
    in the same launch from the verify lm_head's argmax keys (C ABI:
    nsg_spec_accept_greedy_keys): ``target_keys`` holds B * (k + 1) rows of
    ``key_cols`` keys (:func:`lm_head_fold` with ``keys_out``);
    ``target_tokens_out`` (contiguous int64, B * (k + 1)) receives the tokens
    when given."""
    _require_gpu(target_keys, "target_keys")
    dev = target_keys.device
    if target_keys.numel() * target_keys.element_size() < B * (k + 1) * key_cols * 8:
        raise ValueError("target_keys holds fewer than B * (k + 1) * key_cols keys")
    if target_tokens_out is not None and (target_tokens_out.dtype != torch.int64
                                          or not target_tokens_out.is_contiguous()
                                          or target_tokens_out.numel() != B * (k + 1)):
        raise ValueError("target_tokens_out must be contiguous int64 (B * (k + 1),)")
    draft_tokens, ds, tail, rb_ok, (n_out, emitted, rollback) = _greedy_args(
        B, k, dev, draft_tokens, kv_indptr, kv_indices, start_pos, out)
    flags = (workspace or _accept_ws(dev)).get(256)
    rc = _lib().nsg_spec_accept_greedy_keys(
        target_keys.data_ptr(), int(key_cols), _ptr(target_tokens_out),
        _ptr(draft_tokens) if k > 0 else None, ds[0], ds[1], B, k, int(vocab), *tail,
        page_size, n_out.data_ptr(), emitted.data_ptr(),
        rollback.data_ptr() if rb_ok else None, flags.data_ptr(), _stream_ptr(dev))
    check(rc, "nsg_spec_accept_greedy_keys")
    return n_out, emitted, rollback


def sample(logits: torch.Tensor, temperature: float, top_k: int = 0, top_p: float = 1.0,
           uniforms: torch.Tensor | None = None, workspace: AcceptWorkspace | None = None,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """One token per row of ``logits`` (R, V) -- the reference's
    ``sample_token(logits, temperature, top_p, top_k)`` (engine/sampling.py:
    25-50, 71-88) with the draw taken by inverse CDF from ``uniforms`` (R,)
    (C ABI: nsg_sample).  Argmax when ``temperature < 1e-6``.  Rows may be a
    strided view with unit stride along V; bf16 or fp32.  Returns int64 (R,)."""
    _require_gpu(logits, "logits")
    if logits.dim() != 2:
        raise ValueError("logits must be (rows, V)")
    R, V = logits.shape
    dt = {torch.bfloat16: 0, torch.float32: 1}.get(logits.dtype)
    if dt is None:
        raise TypeError(f"logits dtype {logits.dtype}: bf16 or fp32")
    if logits.stride(1) != 1 and R > 0:
        raise ValueError("logits must be contiguous along the vocabulary")
    greedy = temperature < 1e-6
    if not greedy:
        if uniforms is None or uniforms.numel() != R:
            raise ValueError("uniforms (R,) float32 required when temperature > 0")
        _require_gpu(uniforms, "uniforms")
        uniforms = uniforms.reshape(R).to(torch.float32).contiguous()
    dev = logits.device
    if out is None:
        out = torch.empty(R, dtype=torch.int64, device=dev)
    elif out.dtype != torch.int64 or out.numel() != R or (R > 1 and out.stride(0) != 1):
        raise ValueError("out must be a contiguous int64 (R,) tensor")
    lib = _lib()
    need = lib.nsg_sample_workspace_bytes(R, V)
    ws = (workspace or _accept_ws(dev, "sample")).get(need)
    check(lib.nsg_sample(logits.data_ptr(), logits.stride(0) if R > 1 else V, dt, R, V,
                         float(temperature), int(top_k), float(top_p),
                         _ptr(uniforms) if not greedy else None, 1, out.data_ptr(),
                         ws.data_ptr(), ws.numel(), _stream_ptr(dev)), "nsg_sample")
    return out


def kv_write(k: torch.Tensor, v: torch.Tensor, slots: torch.Tensor, k_cache: torch.Tensor,
             v_cache: torch.Tensor) -> None:
    """k, v: (T, Hkv, D) bf16 (rows may be strided views); slots int64 (T,);
    caches: one layer's (N, P, Hkv, D) pool."""
    for name, t in (("k", k), ("v", v), ("slots", slots), ("k_cache", k_cache),
                    ("v_cache", v_cache)):
        _require_gpu(t, name)
    T, Hkv, D = k.shape
    if v.shape != k.shape or v.stride() != k.stride():
        raise ValueError("k and v must have the same shape and strides")
    if k.stride(2) != 1 or k.stride(1) != D:
        raise ValueError("each K/V row must be a contiguous (Hkv, D) block")
    if k_cache.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
        raise TypeError("K/V and caches must be bfloat16")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("caches must be contiguous")
    if k_cache.shape[-2:] != (Hkv, D):
        raise ValueError("cache head layout does not match K/V")
    slots = slots.to(torch.int64).contiguous()
    num_slots = k_cache.numel() // (Hkv * D)
    check(_lib().nsg_kv_write(k.data_ptr(), v.data_ptr(), k.stride(0), slots.data_ptr(), T,
                              k_cache.data_ptr(), v_cache.data_ptr(), Hkv, D, num_slots,
                              _stream_ptr(k.device)), "nsg_kv_write")


def kv_clear_slots(slots: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
    """Zero flat slots in every layer of (L, N, P, Hkv, D) pools."""
    _require_gpu(slots, "slots")
    L, N, P, Hkv, D = k_cache.shape
    slots = slots.reshape(-1).to(torch.int64).contiguous()
    check(_lib().nsg_kv_clear_slots(slots.data_ptr(), slots.numel(), k_cache.data_ptr(),
                                    v_cache.data_ptr(), L, N * P * Hkv * D, Hkv, D, N * P,
                                    _stream_ptr(k_cache.device)), "nsg_kv_clear_slots")


def rope_kv_write(qkv: torch.Tensor, num_qo_heads: int, num_kv_heads: int, head_dim: int,
                  positions: torch.Tensor, cos_table: torch.Tensor, sin_table: torch.Tensor,
                  slots: torch.Tensor | None, k_cache: torch.Tensor | None,
                  v_cache: torch.Tensor | None, q_out: torch.Tensor | None = None) -> torch.Tensor:
    """Fused RoPE of q, k plus the KV slot write (C ABI: nsg_rope_kv_write).

    qkv: (T, (Hq + 2 Hkv) * D) bf16 rows of the fused projection (unit inner
    stride); positions int64 (T,); cos/sin fp32 (max_pos, D/2); caches: one
    layer's (N, P, Hkv, D) pool.  Returns rotated q (T, Hq, D)."""
    _require_gpu(qkv, "qkv")
    T = qkv.shape[0]
    if qkv.dtype != torch.bfloat16 or qkv.stride(-1) != 1:
        raise ValueError("qkv must be bfloat16 with unit inner stride")
    if q_out is None:
        q_out = torch.empty(T, num_qo_heads, head_dim, dtype=torch.bfloat16, device=qkv.device)
    positions = positions.to(torch.int64).contiguous()
    if slots is not None:
        slots = slots.to(torch.int64).contiguous()
        num_slots = k_cache.numel() // (num_kv_heads * head_dim)
    else:
        num_slots = 0
    check(_lib().nsg_rope_kv_write(
        qkv.data_ptr(), qkv.stride(0), positions.data_ptr(), cos_table.data_ptr(),
        sin_table.data_ptr(), cos_table.shape[0], _ptr(slots), T, num_qo_heads, num_kv_heads,
        head_dim, q_out.data_ptr(), _ptr(k_cache), _ptr(v_cache), num_slots, None,
        _stream_ptr(qkv.device)), "nsg_rope_kv_write")
    return q_out


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float,
            residual: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """RMSNorm of (T, H) bf16 rows; with ``residual`` first residual += x in
    place and normalise the sum (C ABI: nsg_rmsnorm)."""
    _require_gpu(x, "x")
    T, H = x.shape
    for name, t in (("x", x), ("weight", weight), ("residual", residual)):
        if t is not None and (t.dtype != torch.bfloat16 or not t.is_contiguous()):
            raise ValueError(f"{name} must be contiguous bfloat16")
    if out is None:
        out = torch.empty_like(x)
    check(_lib().nsg_rmsnorm(x.data_ptr(), _ptr(residual), weight.data_ptr(), out.data_ptr(),
                             T, H, float(eps), _stream_ptr(x.device)), "nsg_rmsnorm")
    return out


def row_sumsq(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Partial sums of squares of (T, H) bf16 rows for a folded-RMSNorm
    consumer: out[g, t] = sum of x[t, 16 g : 16 g + 16]^2, float32 (H / 16, T)
    (C ABI: nsg_row_sumsq; the layout a producing ``linear(..., residual=,
    sumsq_out=)`` writes)."""
    _require_gpu(x, "x")
    T, H = x.shape
    if x.dtype != torch.bfloat16 or x.stride(1) != 1:
        raise ValueError("x must be bf16 rows with unit inner stride")
    if out is None:
        out = torch.empty(H // 16, T, dtype=torch.float32, device=x.device)
    check(_lib().nsg_row_sumsq(x.data_ptr(), x.stride(0), T, H, out.data_ptr(),
                               _stream_ptr(x.device)), "nsg_row_sumsq")
    return out


def linear_argmax(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
                  out: torch.Tensor | None = None,
                  workspace: AcceptWorkspace | None = None) -> torch.Tensor:
    """Greedy token of each row of the bf16 logits x @ weight.T (+ bias),
    never stored: the lowest column of the row's largest bf16 value -- the
    argmax of exactly the rows :func:`linear` would return (C ABI:
    nsg_linear_argmax).  (M,) int64; M up to nsg_linear_max_rows()."""
    _require_gpu(x, "x")
    M, K = x.shape
    N = weight.shape[0]
    lib = _lib()
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16 or x.stride(1) != 1 \
            or weight.stride(1) != 1 or weight.shape[1] != K:
        raise ValueError("x (M, K) and weight (N, K) must be bf16 rows with unit inner stride")
    if bias is not None and (bias.dtype != torch.bfloat16 or not bias.is_contiguous()):
        raise ValueError("bias must be contiguous bf16")
    if out is None:
        out = torch.empty(M, dtype=torch.int64, device=x.device)
    if out.dtype != torch.int64 or out.dim() != 1 or out.numel() != M or out.stride(0) < 1:
        raise ValueError("out must be int64 (M,) with a positive stride")
    ws = (workspace or _accept_ws(x.device, "argmax")).get(
        lib.nsg_linear_argmax_workspace_bytes(M, N))
    check(lib.nsg_linear_argmax(x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0),
                                _ptr(bias), M, N, K, ws.data_ptr(), ws.numel(), out.data_ptr(),
                                out.stride(0), _stream_ptr(x.device)), "nsg_linear_argmax")
    return out


def lm_head_fold_supported(M: int, N: int, K: int, parts: int) -> bool:
    """Whether :func:`lm_head_fold` takes M rows of K against N vocabulary
    rows with ``parts`` partial sums of squares per row."""
    return bool(_lib().nsg_lm_head_fold_supported(M, N, K, parts))


def lm_head_fold(x: torch.Tensor, weight: torch.Tensor, sumsq_in: torch.Tensor, eps: float,
                 out: torch.Tensor | None = None, argmax_out: torch.Tensor | None = None,
                 workspace: AcceptWorkspace | None = None,
                 keys_out: torch.Tensor | None = None):
    """The lm_head after the final RMSNorm with that norm folded in (C ABI:
    nsg_lm_head_fold / nsg_lm_head_fold_argmax): ``x`` (M, K) holds the
    un-normalised rows, ``weight`` (N, K) the norm weight folded into its
    columns, ``sumsq_in`` (K / 16, M) float32 the rows' partial sums of
    squares (the last layer's down_proj writes them); row m of x @ weight.T
    is scaled by rsqrt(mean(x_m^2) + eps) before its bf16 rounding.  Returns
    the (M, N) bf16 logits, or with ``argmax_out`` (int64 (M,), any positive
    stride) each row's greedy token (the lowest column of its largest
    logit), written there and returned; or with ``keys_out`` (a device
    buffer of at least nsg_linear_argmax_workspace_bytes(M, N) bytes) only
    the argmax keys, for a consumer that reduces them (:func:`embed_rows`,
    :func:`spec_accept_greedy_keys`), returning the keys per row."""
    _require_gpu(x, "x")
    M, K = x.shape
    N = weight.shape[0]
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16 or x.stride(1) != 1 \
            or weight.stride(1) != 1 or weight.shape[1] != K:
        raise ValueError("x (M, K) and weight (N, K) must be bf16 rows with unit inner stride")
    if sumsq_in.dtype != torch.float32 or sumsq_in.dim() != 2 or sumsq_in.shape[1] != M \
            or not sumsq_in.is_contiguous():
        raise ValueError("sumsq_in must be contiguous float32 (parts, M)")
    parts = sumsq_in.shape[0]
    lib = _lib()
    stream = _stream_ptr(x.device)
    if keys_out is not None:
        _require_gpu(keys_out, "keys_out")
        kc = C.c_int32(0)
        check(lib.nsg_lm_head_fold_keys(x.data_ptr(), x.stride(0), weight.data_ptr(),
                                        weight.stride(0), M, N, K, sumsq_in.data_ptr(), parts,
                                        K, float(eps), keys_out.data_ptr(),
                                        keys_out.numel() * keys_out.element_size(),
                                        C.byref(kc), stream), "nsg_lm_head_fold_keys")
        return kc.value
    if argmax_out is None:
        if out is None:
            out = torch.empty(M, N, dtype=torch.bfloat16, device=x.device)
        if out.dtype != torch.bfloat16 or out.shape != (M, N) or out.stride(1) != 1:
            raise ValueError("out must be bf16 (M, N) rows with unit inner stride")
        check(lib.nsg_lm_head_fold(x.data_ptr(), x.stride(0), weight.data_ptr(),
                                   weight.stride(0), out.data_ptr(), out.stride(0), M, N, K,
                                   sumsq_in.data_ptr(), parts, K, float(eps), stream),
              "nsg_lm_head_fold")
        return out
    if argmax_out.dtype != torch.int64 or argmax_out.dim() != 1 or argmax_out.numel() != M \
            or argmax_out.stride(0) < 1:
        raise ValueError("argmax_out must be int64 (M,) with a positive stride")
    ws = (workspace or _accept_ws(x.device, "argmax")).get(
        lib.nsg_linear_argmax_workspace_bytes(M, N))
    check(lib.nsg_lm_head_fold_argmax(x.data_ptr(), x.stride(0), weight.data_ptr(),
                                      weight.stride(0), M, N, K, sumsq_in.data_ptr(), parts, K,
                                      float(eps), ws.data_ptr(), ws.numel(),
                                      argmax_out.data_ptr(), argmax_out.stride(0), stream),
          "nsg_lm_head_fold_argmax")
    return argmax_out


def embed_rows(ids: torch.Tensor, table: torch.Tensor, out: torch.Tensor | None = None,
               sumsq_out: torch.Tensor | None = None, keys: tuple | None = None) -> torch.Tensor:
    """table[ids] for int64 ids of shape (T,) or (B, J), any strides, as
    (T or B * J, H) rows (C ABI: nsg_embed_rows); with ``sumsq_out``
    ((H / 16, rows) float32) also the rows' partial sums of squares, the
    layout :func:`row_sumsq` writes.  Ids outside [0, vocab) read the
    nearest valid row.  With ``keys`` = (key tensor, key_cols, key_j)
    (C ABI: nsg_embed_rows_keys), column key_j of ``ids`` first receives the
    greedy token of each key row b (the previous :func:`lm_head_fold` call's
    ``keys_out``), which is then looked up."""
    _require_gpu(table, "table")
    _require_gpu(ids, "ids")
    if ids.dtype != torch.int64 or ids.dim() not in (1, 2):
        raise ValueError("ids must be int64 (T,) or (B, J)")
    B, J = (ids.shape[0], 1) if ids.dim() == 1 else tuple(ids.shape)
    sb = ids.stride(0)
    sj = ids.stride(1) if ids.dim() == 2 else 0
    V, H = table.shape
    if table.dtype != torch.bfloat16 or table.stride(1) != 1:
        raise ValueError("table must be bf16 rows with unit inner stride")
    rows = B * J
    if out is None:
        out = torch.empty(rows, H, dtype=table.dtype, device=table.device)
    if sumsq_out is not None and (sumsq_out.dtype != torch.float32 or not sumsq_out.is_contiguous()
                                  or tuple(sumsq_out.shape) != (H // 16, rows)):
        raise ValueError("sumsq_out must be contiguous float32 (H / 16, rows)")
    if keys is not None:
        kt, key_cols, key_j = keys
        _require_gpu(kt, "keys")
        if kt.numel() * kt.element_size() < B * int(key_cols) * 8:
            raise ValueError("keys holds fewer than batch * key_cols keys")
        check(_lib().nsg_embed_rows_keys(ids.data_ptr(), sb, sj, B, J, int(key_j), kt.data_ptr(),
                                         int(key_cols), table.data_ptr(), table.stride(0), V, H,
                                         out.data_ptr(), out.stride(0), _ptr(sumsq_out),
                                         _stream_ptr(table.device)), "nsg_embed_rows_keys")
        return out
    check(_lib().nsg_embed_rows(ids.data_ptr(), sb, sj, B, J, table.data_ptr(), table.stride(0), V,
                                H, out.data_ptr(), out.stride(0), _ptr(sumsq_out),
                                _stream_ptr(table.device)), "nsg_embed_rows")
    return out


MAX_SUMSQ_PARTS = 64     # partial sums per row a folded-norm consumer reads (nsg_linear_fold)


def _fold_args(x, sumsq_in, norm_eps, residual, sumsq_out, n_out=None):
    """C-ABI arguments of the folded RMSNorm (see nsg_linear_fold).  The C
    ABI takes no sizes for ``residual`` / ``sumsq_out``: their shapes are
    checked here, against M = x rows and the N = ``n_out`` columns written."""
    M = x.shape[0]
    if sumsq_in is not None and (sumsq_in.dtype != torch.float32 or not sumsq_in.is_contiguous()
                                 or sumsq_in.dim() != 2 or sumsq_in.shape[1] != M
                                 or not 1 <= sumsq_in.shape[0] <= MAX_SUMSQ_PARTS):
        raise ValueError(f"sumsq_in must be contiguous float32 (parts <= {MAX_SUMSQ_PARTS}, "
                         f"M = {M})")
    if residual is not None and (residual.dtype != torch.bfloat16 or residual.dim() != 2
                                 or residual.stride(1) != 1 or residual.shape[0] < M
                                 or (n_out is not None and residual.shape[1] != n_out)):
        raise ValueError(f"residual must be bf16 (>= {M}, {n_out}) rows with unit inner stride")
    if sumsq_out is not None and (sumsq_out.dtype != torch.float32
                                  or not sumsq_out.is_contiguous()
                                  or (n_out is not None
                                      and tuple(sumsq_out.shape) != (n_out // 16, M))):
        raise ValueError(f"sumsq_out must be contiguous float32 ({n_out} // 16, {M})")
    return (_ptr(sumsq_in), 0 if sumsq_in is None else sumsq_in.shape[0], x.shape[1],
            float(norm_eps), _ptr(residual), 0 if residual is None else residual.stride(0),
            _ptr(sumsq_out))


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """(T, 2I) bf16 [gate | up] -> (T, I) silu(gate) * up (C ABI: nsg_silu_mul)."""
    _require_gpu(gate_up, "gate_up")
    T, I2 = gate_up.shape
    if gate_up.dtype != torch.bfloat16 or not gate_up.is_contiguous():
        raise ValueError("gate_up must be contiguous bfloat16")
    if out is None:
        out = torch.empty(T, I2 // 2, dtype=torch.bfloat16, device=gate_up.device)
    check(_lib().nsg_silu_mul(gate_up.data_ptr(), out.data_ptr(), T, I2 // 2,
                              _stream_ptr(gate_up.device)), "nsg_silu_mul")
    return out


LINEAR_BIAS, LINEAR_SILU_MUL = 0, 1
FP8 = torch.float8_e4m3fn


def dequant_fp8(w8: torch.Tensor, w_scale: torch.Tensor) -> torch.Tensor:
    """bf16(float(w8) * w_scale[row]): the weights the FP8 kernels multiply
    (FP8Linear.forward's ``w8.to(bf16) * scale``, quantization.py:49-52), in
    one HIP pass (C ABI: nsg_dequant_fp8)."""
    _require_gpu(w8, "w8")
    if w8.dtype != FP8 or w8.dim() != 2 or w8.stride(1) != 1:
        raise ValueError("w8 must be float8_e4m3fn (rows, cols) with unit inner stride")
    rows, cols = w8.shape
    w_scale = w_scale.to(torch.float32).contiguous()
    if w_scale.numel() != rows:
        raise ValueError(f"w_scale must hold one f32 per row ({rows})")
    out = torch.empty(rows, cols, dtype=torch.bfloat16, device=w8.device)
    check(_lib().nsg_dequant_fp8(w8.data_ptr(), w8.stride(0), w_scale.data_ptr(), out.data_ptr(),
                                 cols, rows, cols, _stream_ptr(w8.device)), "nsg_dequant_fp8")
    return out


def _check_fp8(weight, w_scale, K):
    if weight.dtype != FP8:
        if w_scale is not None:
            raise ValueError("w_scale is only for float8_e4m3fn weights")
        return False
    if w_scale is None or w_scale.dtype != torch.float32 or not w_scale.is_contiguous() or \
            w_scale.numel() != weight.shape[0] or w_scale.device != weight.device:
        raise ValueError("float8_e4m3fn weights need an fp32 w_scale with one entry per row")
    if weight.stride(1) != 1 or weight.shape[1] != K or weight.stride(0) % 8 or \
            weight.data_ptr() % 8:
        raise ValueError("fp8 weight must be (N, K) with unit inner stride, rows 8-byte aligned")
    return True


def _check_dequant(w_dequant: torch.Tensor, weight: torch.Tensor) -> None:
    """A resident dequantised copy must be the bf16 twin of ``weight``: same
    shape, same device (a stale copy of another tensor would go unnoticed)."""
    if (w_dequant.dtype != torch.bfloat16 or tuple(w_dequant.shape) != tuple(weight.shape)
            or w_dequant.device != weight.device):
        raise ValueError(f"w_dequant must be bfloat16 {tuple(weight.shape)} on {weight.device}, "
                         f"got {w_dequant.dtype} {tuple(w_dequant.shape)} on {w_dequant.device}")


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
           swiglu: bool = False, out: torch.Tensor | None = None,
           force: bool = False, w_scale: torch.Tensor | None = None,
           w_dequant: torch.Tensor | None = None, sumsq_in: torch.Tensor | None = None,
           norm_eps: float = 1e-6, residual: torch.Tensor | None = None,
           sumsq_out: torch.Tensor | None = None) -> torch.Tensor:
    """y = x @ weight.T (+ bias) for bf16 (M, K) rows (C ABI: nsg_linear).

    ``swiglu``: weight holds the fused [gate; up] rows (2I, K) and the
    result is bf16(silu(gate)) * up, (M, I).  ``weight`` may be
    float8_e4m3fn with fp32 per-row ``w_scale`` (C ABI: nsg_linear_fp8):
    the weights are then ``dequant_fp8(weight, w_scale)``.  Shapes where the
    library is faster (``nsg_linear_preferred``: many rows, prefill) go to
    hipBLASLt via F.linear (on the dequantised weights), plus the SwiGLU
    kernel; ``force`` runs the HIP kernel whenever it supports the shape
    (tests).

    Folded RMSNorm (C ABI: nsg_linear_fold; bf16 weights, the HIP kernel
    only): ``sumsq_in`` (parts, M) float32 makes this the consumer -- x holds
    un-normalised rows and ``weight`` the norm weight folded into its
    columns; ``residual`` and ``sumsq_out`` (N / 16, M) make it the producer
    -- the result is added to ``residual`` in bf16 and written there (when
    ``out`` is None) with the rows' partial sums of squares."""
    _require_gpu(x, "x")
    M, K = x.shape
    rows = weight.shape[0]
    N = rows // 2 if swiglu else rows
    lib = _lib()
    fp8 = _check_fp8(weight, w_scale, K)
    if sumsq_in is not None or residual is not None:
        if fp8 or weight.dtype != torch.bfloat16 or M > lib.nsg_linear_max_rows():
            raise ValueError("the folded RMSNorm takes bf16 weights and at most "
                             f"{lib.nsg_linear_max_rows()} rows")
        if out is None:
            out = residual if residual is not None else torch.empty(
                M, N, dtype=torch.bfloat16, device=x.device)
        check(lib.nsg_linear_fold(x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0),
                                  _ptr(bias), out.data_ptr(), out.stride(0), M, N, K,
                                  LINEAR_SILU_MUL if swiglu else LINEAR_BIAS,
                                  *_fold_args(x, sumsq_in, norm_eps, residual, sumsq_out, N),
                                  _stream_ptr(x.device)), "nsg_linear_fold")
        return out
    fits = (M <= lib.nsg_linear_max_rows() and K % 64 == 0 and N % 4 == 0 and x.stride(1) == 1
            and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0 and x.dtype == torch.bfloat16)
    # FP8 weights stay on the kernel whenever it fits: the library path would
    # first write the dequantised bf16 weights (three times the FP8 bytes)
    if not fits or not (force or fp8 or lib.nsg_linear_preferred(M, N, K)):
        if fp8:   # ``w_dequant``: a resident copy of exactly dequant_fp8(weight, w_scale)
            if w_dequant is not None:
                _check_dequant(w_dequant, weight)
                w = w_dequant
            else:
                w = dequant_fp8(weight, w_scale)
        else:
            w = weight
        y = torch.nn.functional.linear(x, w, bias)
        if swiglu:
            return silu_mul(y, out)
        if out is not None:
            out.copy_(y)
            return out
        return y
    if not fp8 and (weight.dtype != torch.bfloat16 or weight.stride(1) != 1
                    or weight.shape[1] != K):
        raise ValueError("weight must be bf16 (N, K) with unit inner stride")
    if bias is not None and (bias.dtype != torch.bfloat16 or not bias.is_contiguous()):
        raise ValueError("bias must be contiguous bf16")
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=x.device)
    epi = LINEAR_SILU_MUL if swiglu else LINEAR_BIAS
    if fp8:
        check(lib.nsg_linear_fp8(x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0),
                                 w_scale.data_ptr(), _ptr(bias), out.data_ptr(), out.stride(0),
                                 M, N, K, epi, _stream_ptr(x.device)), "nsg_linear_fp8")
    else:
        check(lib.nsg_linear(x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0),
                             _ptr(bias), out.data_ptr(), out.stride(0), M, N, K, epi,
                             _stream_ptr(x.device)), "nsg_linear")
    return out


def linear_rope_kv(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
                   num_qo_heads: int, num_kv_heads: int, head_dim: int,
                   positions: torch.Tensor, cos_table: torch.Tensor, sin_table: torch.Tensor,
                   slots: torch.Tensor | None, k_cache: torch.Tensor | None,
                   v_cache: torch.Tensor | None, q_out: torch.Tensor | None = None,
                   force: bool = False, w_scale: torch.Tensor | None = None,
                   w_dequant: torch.Tensor | None = None,
                   sumsq_in: torch.Tensor | None = None,
                   norm_eps: float = 1e-6) -> torch.Tensor:
    """q/k/v projection + RoPE + KV-slot write (C ABI: nsg_linear_rope_kv, or
    nsg_linear_rope_kv_fp8 for float8_e4m3fn weights with per-row w_scale).

    Same result as ``rope_kv_write(linear(x, weight, bias), ...)``; at row
    counts where the library GEMM is the faster projection (prefill), or for
    shapes the fused kernel does not take, it runs exactly that pair.
    ``sumsq_in``: the folded RMSNorm's consumer side (nsg_linear_rope_kv_fold,
    see ``linear``; the fused kernel only).  Returns rotated q (M, Hq, D)."""
    _require_gpu(x, "x")
    M, K = x.shape
    lib = _lib()
    N = weight.shape[0]
    fp8 = _check_fp8(weight, w_scale, K)
    if sumsq_in is not None and (fp8 or M > lib.nsg_linear_max_rows()):
        raise ValueError("the folded RMSNorm takes bf16 weights and at most "
                         f"{lib.nsg_linear_max_rows()} rows")
    fits = (M <= lib.nsg_linear_max_rows() and K % 64 == 0 and head_dim in (64, 128)
            and N == (num_qo_heads + 2 * num_kv_heads) * head_dim and x.stride(1) == 1
            and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0 and x.dtype == torch.bfloat16)
    if sumsq_in is not None and not fits:
        raise ValueError("the folded RMSNorm needs the fused kernel's shapes")
    if not fits or not (force or fp8 or sumsq_in is not None
                        or lib.nsg_linear_preferred(M, N, K)):
        qkv = linear(x, weight, bias, w_scale=w_scale, w_dequant=w_dequant)
        return rope_kv_write(qkv, num_qo_heads, num_kv_heads, head_dim, positions, cos_table,
                             sin_table, slots, k_cache, v_cache, q_out)
    if not fp8 and (weight.dtype != torch.bfloat16 or weight.stride(1) != 1
                    or weight.shape[1] != K):
        raise ValueError("weight must be bf16 (N, K) with unit inner stride")
    if bias is not None and (bias.dtype != torch.bfloat16 or not bias.is_contiguous()):
        raise ValueError("bias must be contiguous bf16")
    if q_out is None:
        q_out = torch.empty(M, num_qo_heads, head_dim, dtype=torch.bfloat16, device=x.device)
    positions = positions.to(torch.int64).contiguous()
    if slots is not None:
        slots = slots.to(torch.int64).contiguous()
        num_slots = k_cache.numel() // (num_kv_heads * head_dim)
    else:
        num_slots = 0
    tail = (num_qo_heads, num_kv_heads, head_dim, positions.data_ptr(), cos_table.data_ptr(),
            sin_table.data_ptr(), cos_table.shape[0], _ptr(slots), q_out.data_ptr(),
            _ptr(k_cache), _ptr(v_cache), num_slots, None, _stream_ptr(x.device))
    if sumsq_in is not None:
        check(lib.nsg_linear_rope_kv_fold(x.data_ptr(), x.stride(0), weight.data_ptr(),
                                          weight.stride(0), _ptr(bias), M, K, *tail[:-1],
                                          *_fold_args(x, sumsq_in, norm_eps, None, None)[:4],
                                          tail[-1]), "nsg_linear_rope_kv_fold")
    elif fp8:
        check(lib.nsg_linear_rope_kv_fp8(x.data_ptr(), x.stride(0), weight.data_ptr(),
                                         weight.stride(0), w_scale.data_ptr(), _ptr(bias), M, K,
                                         *tail), "nsg_linear_rope_kv_fp8")
    else:
        check(lib.nsg_linear_rope_kv(x.data_ptr(), x.stride(0), weight.data_ptr(),
                                     weight.stride(0), _ptr(bias), M, K, *tail),
              "nsg_linear_rope_kv")
    return q_out


def philox_uniform(seed: int, stream_id: int, offset: int, n: int, device) -> torch.Tensor:
    """n float32 uniforms of Philox4x32-10 stream ``stream_id`` (see nsg_spec.h)."""
    out = torch.empty(n, dtype=torch.float32, device=device)
    _require_gpu(out, "out")
    check(_lib().nsg_philox_uniform(seed, stream_id, offset, n, out.data_ptr(),
                                    _stream_ptr(out.device)), "nsg_philox_uniform")
    return out
