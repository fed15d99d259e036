"""PyTorch operators of the verify step: ``torch.ops.nsg.*``.

The operators are registered from C++ (``csrc/torch_ops.cpp``, built into
``libnsg_torch.so`` by ``python -m nanosglang_amd.build``): TORCH_LIBRARY
schemas, CUDA-key implementations that call the C ABI of ``libnsg_spec.so``
on the current HIP stream, and CPU-key implementations that reject host
tensors (the host planner excepted).  The reference reaches this path
through Python calls: FlashInfer's ``BatchPrefillWithPagedKVCacheWrapper.plan``
/ ``.run`` (nano_sglang/engine/engine.py:451-462,
nano_sglang/model/causal_lm.py:340), the KV ``index_put`` (causal_lm.py:
335-338) and the per-position loop of ``SpeculativeDecoder.speculative_step``
(nano_sglang/decode/speculative.py:130-196) with ``sample_token``
(nano_sglang/engine/sampling.py:25-50).

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

This module loads the operator library and registers the shape-only (fake)
implementations that tracing and compilation use.
"""

from __future__ import annotations

import ctypes as C
import os

import numpy as np
import torch
from torch import Tensor

from . import _native
from ._native import NSG_ATTN_WORK_INTS, AttnPlan

PLAN_INTS = C.sizeof(AttnPlan) // 4
RECORD_INTS = PLAN_INTS + 3          # + total query rows, page ids, batch
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libnsg_torch.so")


def _load() -> None:
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} not found: build it first (python -m nanosglang_amd.build)")
    _native.load()                   # the C-ABI library it links to, ABI-checked
    torch.ops.load_library(LIB_PATH)


_load()


def plan_record(plan: AttnPlan, total_q: int, num_page_ids: int, batch: int) -> Tensor:
    """A plan record: nsg_attn_plan_t's bytes, then the shape it was made for
    (query rows, page ids, batch), as an int32 host tensor."""
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


def plan_workspace_bytes(record: Tensor) -> int:
    """Device workspace bytes a plan needs (zero-filled before first use)."""
    return int(plan_from_record(record)[0].workspace_bytes)


# ---- shape-only implementations ----

@torch.library.register_fake("nsg::verify_attention")
def _(q, k_cache, v_cache, qo_indptr, paged_kv_indptr, paged_kv_indices,
      paged_kv_last_page_len, causal=True, sm_scale=None):
    return torch.empty_like(q)


@torch.library.register_fake("nsg::verify_attention_plan")
def _(qo_indptr, paged_kv_indptr, paged_kv_last_page_len, num_qo_heads, num_kv_heads,
      head_dim, page_size, causal=True, num_cus=256):
    n = torch.library.get_ctx().new_dynamic_size()
    return (torch.empty(RECORD_INTS, dtype=torch.int32),
            torch.empty(n * NSG_ATTN_WORK_INTS, dtype=torch.int32))


@torch.library.register_fake("nsg::verify_attention_run")
def _(plan, work, q, k_cache, v_cache, qo_indptr, paged_kv_indptr, paged_kv_indices,
      paged_kv_last_page_len, sm_scale, causal, workspace, out):
    return None


@torch.library.register_fake("nsg::spec_accept")
def _(target_logits, draft_logits, draft_tokens, uniforms, temperature, kv_indptr=None,
      kv_indices=None, start_pos=None, page_size=16, bonus_tokens=None):
    B, k1, _ = target_logits.shape
    return (target_logits.new_empty((B,), dtype=torch.int32),
            target_logits.new_empty((B, k1), dtype=torch.int64),
            target_logits.new_empty((B, k1 - 1), dtype=torch.int64))


@torch.library.register_fake("nsg::sample")
def _(logits, temperature, top_k=0, top_p=1.0, uniforms=None):
    return logits.new_empty((logits.shape[0],), dtype=torch.int64)


@torch.library.register_fake("nsg::kv_write")
def _(k, v, slots, k_cache, v_cache):
    return None


@torch.library.register_fake("nsg::rope_kv_write")
def _(qkv, num_qo_heads, num_kv_heads, head_dim, positions, cos_table, sin_table, slots,
      k_cache, v_cache):
    return qkv.new_empty((qkv.shape[0], num_qo_heads, head_dim))


__all__ = ["plan_record", "plan_from_record", "plan_workspace_bytes", "RECORD_INTS", "LIB_PATH"]
