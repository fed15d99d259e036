"""PyTorch operators over the C ABI: ``torch.ops.nsg.*``.

The reference reaches this path through Python calls: FlashInfer's
``BatchPrefillWithPagedKVCacheWrapper.plan`` / ``.run``
(nano_sglang/engine/engine.py:451-462, nano_sglang/model/causal_lm.py:340),
the KV ``index_put`` (causal_lm.py:335-338) and the per-position loop of
``SpeculativeDecoder.speculative_step`` (nano_sglang/decode/speculative.py:
130-196) with ``sample_token`` (nano_sglang/engine/sampling.py:25-50).  The
same kernels are registered here as torch operators, with schemas and fake
(shape-only) implementations, so that traced or compiled code can hold them:

``nsg::verify_attention``
    plan + run in one call.  The planner reads the index arrays on the host,
    so the call synchronises; use the pair below (or the wrapper class's
    graph mode) inside a captured graph.
``nsg::verify_attention_plan``
    the planner alone: host int32 CSR arrays in; a plan record (int32
    [RECORD_INTS]: the bytes of ``nsg_attn_plan_t``, then the query-row count,
    the page-id count and the batch it was made for) and the work list out.
``nsg::verify_attention_run``
    one layer from a plan: allocates nothing and never synchronises (the
    caller owns the device work list, the workspace and ``out``).
``nsg::spec_accept``
    acceptance / residual resample / bonus / rollback slots.
``nsg::sample``
    temperature / top-k / top-p sampling, one token per row.
``nsg::kv_write``, ``nsg::rope_kv_write``
    K/V rows (after RoPE, for the second) into their flat KV slots.

Every operator runs the HIP kernels (CUDA dispatch on ROCm); there is no CPU
implementation.
"""

from __future__ import annotations

import ctypes as C
import threading
from typing import Optional

import numpy as np
import torch
from torch import Tensor

from . import kernels
from ._native import NSG_ATTN_WORK_INTS, AttnPlan, check

PLAN_INTS = C.sizeof(AttnPlan) // 4
RECORD_INTS = PLAN_INTS + 3          # + total query rows, page ids, batch

_lock = threading.Lock()
_attn: dict = {}


def _attn_wrapper(device: torch.device) -> kernels.BatchPrefillWithPagedKVCacheWrapper:
    """One dynamic-plan wrapper per device with the reference's 128 MiB
    workspace (engine.py:103-108)."""
    if device not in _attn:
        ws = torch.empty(128 << 20, dtype=torch.uint8, device=device)
        _attn[device] = kernels.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    return _attn[device]


def plan_record(plan: AttnPlan, total_q: int, num_page_ids: int, batch: int) -> Tensor:
    """The plan operator's output: nsg_attn_plan_t's bytes, then the shape it
    was made for (query rows, page ids, batch), as an int32 host tensor."""
    head = np.frombuffer(bytes(plan), dtype=np.int32)
    return torch.from_numpy(np.concatenate([head, np.asarray([total_q, num_page_ids, batch],
                                                             np.int32)]))


def plan_from_record(record: Tensor) -> tuple[AttnPlan, int, int, int]:
    """(plan, total query rows, page ids, batch) of a plan record."""
    if record.dtype != torch.int32 or record.numel() != RECORD_INTS or record.is_cuda:
        raise ValueError(f"plan record must be a host int32 tensor of {RECORD_INTS}")
    r = record.contiguous().numpy()
    return (AttnPlan.from_buffer_copy(r[:PLAN_INTS].tobytes()), int(r[PLAN_INTS]),
            int(r[PLAN_INTS + 1]), int(r[PLAN_INTS + 2]))


# ---- verify attention ----

@torch.library.custom_op("nsg::verify_attention", mutates_args=())
def verify_attention(q: Tensor, k_cache: Tensor, v_cache: Tensor, qo_indptr: Tensor,
                     paged_kv_indptr: Tensor, paged_kv_indices: Tensor,
                     paged_kv_last_page_len: Tensor, causal: bool = True,
                     sm_scale: Optional[float] = None) -> Tensor:
    """Ragged multi-query attention of q (total_q, Hq, D) over one layer's
    (pages, P, Hkv, D) caches: plan + run of the wrapper (engine.py:451-462,
    causal_lm.py:340).  ``sm_scale`` defaults to 1 / sqrt(D)."""
    _, Hq, D = q.shape
    P, Hkv = k_cache.shape[1], k_cache.shape[2]
    with _lock:
        w = _attn_wrapper(q.device)
        w.plan(qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len, Hq, Hkv,
               D, P, causal=causal, sm_scale=sm_scale)
        return w.run(q, (k_cache, v_cache))


@verify_attention.register_fake
def _(q, k_cache, v_cache, qo_indptr, paged_kv_indptr, paged_kv_indices,
      paged_kv_last_page_len, causal=True, sm_scale=None):
    return torch.empty_like(q)


@torch.library.custom_op("nsg::verify_attention_plan", mutates_args=())
def verify_attention_plan(qo_indptr: Tensor, paged_kv_indptr: Tensor,
                          paged_kv_last_page_len: Tensor, num_qo_heads: int, num_kv_heads: int,
                          head_dim: int, page_size: int, causal: bool = True,
                          num_cus: int = kernels.MI355X_CUS) -> tuple[Tensor, Tensor]:
    """The planner (nsg_attn_plan) on host int32 CSR arrays.  Returns the plan
    record (int32 [RECORD_INTS]; its workspace size via
    :func:`plan_workspace_bytes`) and the work list (int32, host) that
    :func:`verify_attention_run` reads from device memory."""
    qo_h = kernels._host_i32(qo_indptr)
    kvp_h = kernels._host_i32(paged_kv_indptr)
    last_h = kernels._host_i32(paged_kv_last_page_len)
    B = len(qo_h) - 1
    if len(kvp_h) != B + 1 or len(last_h) != B:
        raise ValueError("qo_indptr, paged_kv_indptr and last_page_len disagree on batch")
    cap = max(1, kernels.attn_work_bound(qo_h, kvp_h, last_h, num_qo_heads, num_kv_heads,
                                         page_size))
    work = np.zeros(cap * NSG_ATTN_WORK_INTS, np.int32)
    pl = AttnPlan()
    check(kernels._lib().nsg_attn_plan(qo_h.ctypes.data, kvp_h.ctypes.data, last_h.ctypes.data,
                                       B, num_qo_heads, num_kv_heads, head_dim, page_size,
                                       1 if causal else 0, num_cus, work.ctypes.data, cap,
                                       C.byref(pl)), "nsg_attn_plan")
    n = (pl.num_work + pl.num_merge) * NSG_ATTN_WORK_INTS
    return (plan_record(pl, int(qo_h[-1]), int(kvp_h[-1]), B),
            torch.from_numpy(work[:n].copy()))


@verify_attention_plan.register_fake
def _(qo_indptr, paged_kv_indptr, paged_kv_last_page_len, num_qo_heads, num_kv_heads,
      head_dim, page_size, causal=True, num_cus=kernels.MI355X_CUS):
    n = torch.library.get_ctx().new_dynamic_size()
    return (torch.empty(RECORD_INTS, dtype=torch.int32),
            torch.empty(n * NSG_ATTN_WORK_INTS, dtype=torch.int32))


def plan_workspace_bytes(record: Tensor) -> int:
    """Device workspace bytes a plan needs (zero-filled before first use)."""
    return int(plan_from_record(record)[0].workspace_bytes)


@torch.library.custom_op("nsg::verify_attention_run", mutates_args=("workspace", "out"))
def verify_attention_run(plan: Tensor, work: Tensor, q: Tensor, k_cache: Tensor,
                         v_cache: Tensor, qo_indptr: Tensor, paged_kv_indptr: Tensor,
                         paged_kv_indices: Tensor, paged_kv_last_page_len: Tensor,
                         sm_scale: float, causal: bool, workspace: Tensor, out: Tensor) -> None:
    """One layer (nsg_attn_run) from a plan record and its work list copied to
    the device; the CSR arrays are device copies of the arrays the plan was
    made from (their sizes and q's rows are checked against the record).
    Enqueues on the current stream; no allocation, no host sync."""
    pl, total_q, nnz, B = plan_from_record(plan)
    Hq, Hkv, D = pl.num_qo_heads, pl.num_kv_heads, pl.head_dim
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache), ("out", out)):
        kernels._require_gpu(t, name)
        if t.dtype != torch.bfloat16 or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous bfloat16")
    for name, t in (("work", work), ("qo_indptr", qo_indptr),
                    ("paged_kv_indptr", paged_kv_indptr), ("paged_kv_indices", paged_kv_indices),
                    ("paged_kv_last_page_len", paged_kv_last_page_len)):
        kernels._require_gpu(t, name)
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous int32 on the device")
    if q.dim() != 3 or tuple(q.shape) != (total_q, Hq, D) or out.shape != q.shape:
        raise ValueError(f"q / out must be ({total_q}, {Hq}, {D}) as planned")
    if (qo_indptr.numel() != B + 1 or paged_kv_indptr.numel() != B + 1
            or paged_kv_last_page_len.numel() != B or paged_kv_indices.numel() < nnz):
        raise ValueError(f"CSR arrays do not match the planned batch {B} / {nnz} page ids")
    if (k_cache.dim() != 4 or tuple(k_cache.shape[2:]) != (Hkv, D)
            or v_cache.shape != k_cache.shape):
        raise ValueError(f"caches must be (pages, P, {Hkv}, {D})")
    if work.numel() < (pl.num_work + pl.num_merge) * NSG_ATTN_WORK_INTS:
        raise ValueError("work list shorter than the plan")
    wsb = workspace.numel() * workspace.element_size()
    if wsb < pl.workspace_bytes:
        raise ValueError(f"workspace has {wsb} bytes, the plan needs {pl.workspace_bytes}")
    check(kernels._lib().nsg_attn_run(
        C.byref(pl), work.data_ptr(), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        out.data_ptr(), qo_indptr.data_ptr(), paged_kv_indptr.data_ptr(),
        paged_kv_indices.data_ptr(), paged_kv_last_page_len.data_ptr(), k_cache.shape[1],
        k_cache.shape[0], float(sm_scale), 1 if causal else 0, workspace.data_ptr(), wsb,
        kernels._stream_ptr(q.device)), "nsg_attn_run")


@verify_attention_run.register_fake
def _(plan, work, q, k_cache, v_cache, qo_indptr, paged_kv_indptr, paged_kv_indices,
      paged_kv_last_page_len, sm_scale, causal, workspace, out):
    return None


# ---- acceptance and sampling ----

@torch.library.custom_op("nsg::spec_accept", mutates_args=())
def spec_accept(target_logits: Tensor, draft_logits: Optional[Tensor],
                draft_tokens: Optional[Tensor], uniforms: Optional[Tensor], temperature: float,
                kv_indptr: Optional[Tensor] = None, kv_indices: Optional[Tensor] = None,
                start_pos: Optional[Tensor] = None, page_size: int = 16,
                bonus_tokens: Optional[Tensor] = None) -> tuple[Tensor, Tensor, Tensor]:
    """Fused acceptance of B requests (speculative.py:130-196): returns
    (num_emitted int32 (B,), emitted int64 (B, k+1) padded -1, rollback_slots
    int64 (B, k) padded -1); see ``kernels.spec_accept``."""
    return kernels.spec_accept(target_logits, draft_logits, draft_tokens, uniforms, temperature,
                               kv_indptr, kv_indices, start_pos, page_size=page_size,
                               bonus_tokens=bonus_tokens)


@spec_accept.register_fake
def _(target_logits, draft_logits, draft_tokens, uniforms, temperature, kv_indptr=None,
      kv_indices=None, start_pos=None, page_size=16, bonus_tokens=None):
    B, k1, _ = target_logits.shape
    return (target_logits.new_empty((B,), dtype=torch.int32),
            target_logits.new_empty((B, k1), dtype=torch.int64),
            target_logits.new_empty((B, k1 - 1), dtype=torch.int64))


@torch.library.custom_op("nsg::sample", mutates_args=())
def sample(logits: Tensor, temperature: float, top_k: int = 0, top_p: float = 1.0,
           uniforms: Optional[Tensor] = None) -> Tensor:
    """sample_token (sampling.py:25-50, 71-88) for every row of (R, V) logits:
    int64 (R,); see ``kernels.sample``."""
    return kernels.sample(logits, temperature, top_k, top_p, uniforms)


@sample.register_fake
def _(logits, temperature, top_k=0, top_p=1.0, uniforms=None):
    return logits.new_empty((logits.shape[0],), dtype=torch.int64)


# ---- KV writes ----

@torch.library.custom_op("nsg::kv_write", mutates_args=("k_cache", "v_cache"))
def kv_write(k: Tensor, v: Tensor, slots: Tensor, k_cache: Tensor, v_cache: Tensor) -> None:
    """k, v (T, Hkv, D) into flat slots of one layer's (N, P, Hkv, D) caches
    (the index_put of causal_lm.py:335-338)."""
    kernels.kv_write(k, v, slots, k_cache, v_cache)


@kv_write.register_fake
def _(k, v, slots, k_cache, v_cache):
    return None


@torch.library.custom_op("nsg::rope_kv_write", mutates_args=("k_cache", "v_cache"))
def rope_kv_write(qkv: Tensor, num_qo_heads: int, num_kv_heads: int, head_dim: int,
                  positions: Tensor, cos_table: Tensor, sin_table: Tensor, slots: Tensor,
                  k_cache: Tensor, v_cache: Tensor) -> Tensor:
    """RoPE of q and k from fused qkv rows (causal_lm.py:181-206), k / v into
    their flat KV slots; returns rotated q (T, Hq, D)."""
    return kernels.rope_kv_write(qkv, num_qo_heads, num_kv_heads, head_dim, positions,
                                 cos_table, sin_table, slots, k_cache, v_cache)


@rope_kv_write.register_fake
def _(qkv, num_qo_heads, num_kv_heads, head_dim, positions, cos_table, sin_table, slots,
      k_cache, v_cache):
    return qkv.new_empty((qkv.shape[0], num_qo_heads, head_dim))


__all__ = ["verify_attention", "verify_attention_plan", "verify_attention_run", "spec_accept",
           "sample", "kv_write", "rope_kv_write", "plan_record", "plan_from_record",
           "plan_workspace_bytes", "RECORD_INTS"]
