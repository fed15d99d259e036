"""The torch operators (torch.ops.nsg.*) on a CPU-only host: registered with
the reference-shaped schemas; the planner operator returns exactly what the C
planner does (tests/test_capi.py pins that planner's coverage); the fake
implementations give the output shapes; the device operators reject host
tensors before any GPU call."""
import ctypes as C

import numpy as np
import pytest
import torch

from nanosglang_amd import ops
from nanosglang_amd._native import NSG_ATTN_WORK_INTS, AttnPlan


def test_operators_are_registered_with_their_arguments():
    want = {
        "verify_attention": ["q", "k_cache", "v_cache", "qo_indptr", "paged_kv_indptr",
                             "paged_kv_indices", "paged_kv_last_page_len", "causal", "sm_scale"],
        "verify_attention_plan": ["qo_indptr", "paged_kv_indptr", "paged_kv_last_page_len",
                                  "num_qo_heads", "num_kv_heads", "head_dim", "page_size",
                                  "causal", "num_cus"],
        "verify_attention_run": ["plan", "work", "q", "k_cache", "v_cache", "qo_indptr",
                                 "paged_kv_indptr", "paged_kv_indices", "paged_kv_last_page_len",
                                 "sm_scale", "causal", "workspace", "out"],
        "spec_accept": ["target_logits", "draft_logits", "draft_tokens", "uniforms",
                        "temperature", "kv_indptr", "kv_indices", "start_pos", "page_size",
                        "bonus_tokens"],
        "sample": ["logits", "temperature", "top_k", "top_p", "uniforms"],
        "kv_write": ["k", "v", "slots", "k_cache", "v_cache"],
        "rope_kv_write": ["qkv", "num_qo_heads", "num_kv_heads", "head_dim", "positions",
                          "cos_table", "sin_table", "slots", "k_cache", "v_cache"],
    }
    for name, args in want.items():
        schema = getattr(torch.ops.nsg, name).default._schema
        assert [a.name for a in schema.arguments] == args, name
    mutated = {a.name for a in torch.ops.nsg.verify_attention_run.default._schema.arguments
               if a.alias_info is not None and a.alias_info.is_write}
    assert mutated == {"workspace", "out"}


def test_plan_operator_matches_the_c_planner(lib):
    rng = np.random.default_rng(3)
    B, P = 12, 16
    q_lens = rng.integers(1, 9, B)
    kv_lens = q_lens + rng.integers(50, 900, B)
    qo = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    npg = (kv_lens + P - 1) // P
    kvp = np.concatenate([[0], np.cumsum(npg)]).astype(np.int32)
    last = (kv_lens - (npg - 1) * P).astype(np.int32)
    rec, work = torch.ops.nsg.verify_attention_plan(torch.from_numpy(qo), torch.from_numpy(kvp),
                                                    torch.from_numpy(last), 14, 2, 64, P)
    cap = 100000
    ref_work = np.zeros(cap * NSG_ATTN_WORK_INTS, np.int32)
    pl = AttnPlan()
    assert lib.nsg_attn_plan(qo.ctypes.data, kvp.ctypes.data, last.ctypes.data, B, 14, 2, 64, P,
                             1, 256, ref_work.ctypes.data, cap, C.byref(pl)) == 0
    got, total_q, nnz, batch = ops.plan_from_record(rec)
    assert bytes(got) == bytes(pl)
    assert (total_q, nnz, batch) == (int(qo[-1]), int(kvp[-1]), B)
    n = (pl.num_work + pl.num_merge) * NSG_ATTN_WORK_INTS
    np.testing.assert_array_equal(work.numpy(), ref_work[:n])
    assert ops.plan_workspace_bytes(rec) == pl.workspace_bytes


def test_plan_operator_rejects_bad_csr():
    with pytest.raises(ValueError):
        torch.ops.nsg.verify_attention_plan(torch.tensor([0, 5], dtype=torch.int32),
                                            torch.tensor([0, 1, 2], dtype=torch.int32),
                                            torch.tensor([3], dtype=torch.int32), 14, 2, 64, 16)
    with pytest.raises(RuntimeError):   # head_dim the kernel does not take
        torch.ops.nsg.verify_attention_plan(torch.tensor([0, 5], dtype=torch.int32),
                                            torch.tensor([0, 1], dtype=torch.int32),
                                            torch.tensor([8], dtype=torch.int32), 14, 2, 96, 16)


def _m(*shape, dtype=torch.bfloat16):
    return torch.empty(*shape, device="meta", dtype=dtype)


def test_fake_implementations_give_output_shapes():
    n, em, rb = torch.ops.nsg.spec_accept(_m(6, 5, 300), _m(6, 4, 300),
                                          _m(6, 4, dtype=torch.int64),
                                          _m(6, 5, dtype=torch.float32), 0.8)
    assert (n.shape, n.dtype) == ((6,), torch.int32)
    assert (em.shape, em.dtype, rb.shape) == ((6, 5), torch.int64, (6, 4))
    t = torch.ops.nsg.sample(_m(3, 1000), 0.7, 20, 0.9, _m(3, dtype=torch.float32))
    assert (t.shape, t.dtype) == ((3,), torch.int64)
    i32 = torch.int32
    o = torch.ops.nsg.verify_attention(_m(10, 14, 64), _m(8, 16, 2, 64), _m(8, 16, 2, 64),
                                       _m(3, dtype=i32), _m(3, dtype=i32), _m(7, dtype=i32),
                                       _m(2, dtype=i32))
    assert o.shape == (10, 14, 64) and o.dtype == torch.bfloat16
    q = torch.ops.nsg.rope_kv_write(_m(4, (14 + 4) * 64), 14, 2, 64, _m(4, dtype=torch.int64),
                                    _m(64, 32, dtype=torch.float32),
                                    _m(64, 32, dtype=torch.float32), _m(4, dtype=torch.int64),
                                    _m(8, 16, 2, 64), _m(8, 16, 2, 64))
    assert q.shape == (4, 14, 64)


def test_device_operators_reject_host_tensors_before_any_gpu_call():
    qo = torch.tensor([0, 5], dtype=torch.int32)
    kvp = torch.tensor([0, 1], dtype=torch.int32)
    last = torch.tensor([8], dtype=torch.int32)
    rec, work = torch.ops.nsg.verify_attention_plan(qo, kvp, last, 14, 2, 64, 16)
    q = torch.zeros(5, 14, 64, dtype=torch.bfloat16)
    kc = torch.zeros(4, 16, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        torch.ops.nsg.verify_attention_run(rec, work, q, kc, kc.clone(), qo, kvp,
                                           torch.zeros(1, dtype=torch.int32), last, 0.125, True,
                                           torch.zeros(ops.plan_workspace_bytes(rec),
                                                       dtype=torch.uint8), q.clone())
    with pytest.raises(RuntimeError, match="GPU tensor"):
        torch.ops.nsg.spec_accept(torch.zeros(2, 5, 100, dtype=torch.bfloat16), None,
                                  torch.zeros(2, 4, dtype=torch.int64), None, 0.0)
    with pytest.raises(ValueError):
        ops.plan_from_record(torch.zeros(3, dtype=torch.int32))


def test_operators_come_from_the_compiled_library():
    """torch.ops.nsg.* are the C++ TORCH_LIBRARY registrations of
    libnsg_torch.so (CUDA and CPU kernels), not Python custom ops."""
    import os
    maps = open(f"/proc/{os.getpid()}/maps").read()
    assert ops.LIB_PATH in maps or os.path.realpath(ops.LIB_PATH) in maps
    for name in ("verify_attention", "verify_attention_plan", "verify_attention_run",
                 "spec_accept", "sample", "kv_write", "rope_kv_write"):
        for key in ("CUDA", "CPU"):
            assert torch._C._dispatch_has_kernel_for_dispatch_key(f"nsg::{name}", key), (name, key)
