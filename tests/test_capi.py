"""The C-ABI library loads on a CPU-only host and exports every function
include/nsg_spec.h declares; its host-only entry points (the attention
planner, workspace sizing, argument checks) run without a GPU."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from nanosglang_amd import _native
from nanosglang_amd._native import NSG_ATTN_WORK_INTS, AttnPlan

HDR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                   "nsg_spec.h")


def _declared():
    text = open(HDR).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nsg_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_typed(lib):
    names = _declared()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
        assert n in _native.SIGNATURES, f"{n} has no ctypes signature"
    assert lib.nsg_abi_version() == _native.ABI_VERSION


def _plan(lib, q_lens, kv_lens, Hq=14, Hkv=2, D=64, P=16, causal=1, cus=256):
    B = len(q_lens)
    qo = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    npg = [(L + P - 1) // P for L in kv_lens]
    kvp = np.concatenate([[0], np.cumsum(npg)]).astype(np.int32)
    last = np.asarray([(L % P) or P for L in kv_lens], np.int32)
    cap = 100000
    work = np.zeros(cap * NSG_ATTN_WORK_INTS, np.int32)
    pl = AttnPlan()
    rc = lib.nsg_attn_plan(qo.ctypes.data, kvp.ctypes.data, last.ctypes.data, B, Hq, Hkv, D, P,
                           causal, cus, work.ctypes.data, cap, C.byref(pl))
    return rc, pl, work.reshape(cap, NSG_ATTN_WORK_INTS), qo, kvp


def _check_cover(pl, items, merges, q_lens, kv_lens, qo, kvp, G=7):
    """Every query row in exactly one tile; each tile's KV range [0, end)
    tiled exactly by its splits; merge items point at their splits."""
    T = pl.q_tile_tokens
    assert pl.row_tiles == (T * G + 15) // 16 and T * G <= 64
    seen_q = np.zeros(qo[-1], int)
    for b in range(len(q_lens)):
        L, ql = kv_lens[b], q_lens[b]
        for qb in range(0, ql, T):
            qn = min(T, ql - qb)
            qs = qo[b] + qb
            its = items[(items[:, 0] == qs) & (items[:, 1] == qn)]
            assert len(its) >= 1
            seen_q[qs:qs + qn] += 1
            kv_end = L - ql + qb + qn
            # KV ranges tile [0, kv_end) exactly, splits numbered consistently
            rngs = sorted((int(r[4]), int(r[5])) for r in its)
            assert rngs[0][0] == 0 and rngs[-1][1] == kv_end
            assert all(a[1] == b_[0] for a, b_ in zip(rngs, rngs[1:]))
            assert all(r[6] == len(its) for r in its)
            assert all(r[2] == L - ql + qb and r[3] == kvp[b] for r in its)
            if len(its) > 1:
                m = merges[(merges[:, 0] == qs) & (merges[:, 1] == qn)]
                assert len(m) == 1 and m[0, 3] == len(its)
                first = m[0, 2]
                assert (items[first:first + len(its), 0] == qs).all()
    assert (seen_q == 1).all()


@pytest.mark.parametrize("cus", [1, 256])
def test_planner_covers_every_query_row_and_kv_token_once(lib, cus):
    rng = np.random.default_rng(0)
    q_lens = [5] * 20 + [1, 300, 17]
    kv_lens = list(rng.integers(100, 641, 20)) + [50, 300, 17]
    rc, pl, work, qo, kvp = _plan(lib, q_lens, kv_lens, cus=cus)
    assert rc == 0
    _check_cover(pl, work[:pl.num_work], work[pl.num_work:pl.num_work + pl.num_merge], q_lens,
                 kv_lens, qo, kvp)
    assert pl.workspace_bytes >= 256 + pl.num_work * 2 * pl.row_tiles * 16 * (64 + 4) * 4


def test_planner_kv_groups_follow_the_work_size(lib):
    """Latency regime (few short items) -> several KV groups per workgroup;
    long contexts -> one, with more work items."""
    rc, small, _, _, _ = _plan(lib, [5] * 32, [370] * 32)
    rc2, big, _, _, _ = _plan(lib, [9] * 64, [5000] * 64, Hq=32, Hkv=8, D=128)
    assert rc == rc2 == 0
    assert small.kv_groups == 4 and small.num_merge == 0
    assert big.kv_groups == 1 and big.num_work >= 256


def _plan_fixed(lib, q_lens, kv_lens, batch_cap, max_q, Hq=14, Hkv=2, D=64, P=16, cus=256,
                max_kv=0):
    mw, mm = C.c_int32(0), C.c_int32(0)
    assert lib.nsg_attn_fixed_capacity(batch_cap, max_q, Hq, Hkv, cus, max_kv, C.byref(mw),
                                       C.byref(mm)) == 0
    B = len(q_lens)
    qo = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    npg = [(L + P - 1) // P for L in kv_lens]
    kvp = np.concatenate([[0], np.cumsum(npg)]).astype(np.int32)
    last = np.asarray([(L % P) or P for L in kv_lens], np.int32)
    cap = mw.value + mm.value
    work = np.full(cap * NSG_ATTN_WORK_INTS, 77, np.int32)    # garbage: padding must clear it
    pl = AttnPlan()
    rc = lib.nsg_attn_plan_fixed(qo.ctypes.data, kvp.ctypes.data, last.ctypes.data, B, Hq, Hkv,
                                 D, P, 1, cus, max_q, max_kv, mw.value, mm.value,
                                 work.ctypes.data, cap, C.byref(pl))
    return rc, pl, work.reshape(cap, NSG_ATTN_WORK_INTS), (mw.value, mm.value)


@pytest.mark.parametrize("q,B", [(1, 32), (5, 32), (5, 7), (9, 64)])
def test_fixed_plan_pads_to_a_constant_grid(lib, q, B):
    """The graph-mode plan without a KV bound: same grid and tile shape for
    every step, one KV group; on long contexts, where the dynamic planner
    takes that regime too, the real items are exactly the dynamic planner's;
    the rest are empty."""
    rng = np.random.default_rng(q * 100 + B)
    shapes = set()
    for step in range(6):
        kv_lens = list(rng.integers(2000, 2000 + 4000 * (step + 1), B))
        rc, pl, work, (mw, mm) = _plan_fixed(lib, [q] * B, kv_lens, B, q)
        assert rc == 0, lib.nsg_last_error()
        shapes.add((pl.num_work, pl.num_merge, pl.row_tiles, pl.q_tile_tokens,
                    pl.workspace_bytes))
        assert (pl.num_work, pl.num_merge) == (mw, mm)
        assert pl.kv_groups == 1
        qo = np.concatenate([[0], np.cumsum([q] * B)]).astype(np.int32)
        kvp = np.concatenate([[0], np.cumsum([(L + 15) // 16 for L in kv_lens])]).astype(np.int32)
        _check_cover(pl, work[:mw][work[:mw, 1] > 0], work[mw:][work[mw:, 3] > 1], [q] * B,
                     kv_lens, qo, kvp)
        rc2, pd, wd, _, _ = _plan(lib, [q] * B, kv_lens)
        assert rc2 == 0
        if pd.kv_groups != 1:      # the dynamic planner chose the latency regime
            continue
        n, m = pd.num_work, pd.num_merge
        assert np.array_equal(work[:n], wd[:n])                       # real work items
        assert (work[n:mw] == 0).all()                                # empty work items
        assert np.array_equal(work[mw:mw + m], wd[n:n + m])           # real merge items
        assert (work[mw + m:] == 0).all()                             # empty merge items
    assert len(shapes) == 1


def test_fixed_plan_covers_long_contexts(lib):
    rng = np.random.default_rng(3)
    kv_lens = list(rng.integers(2000, 8000, 16))
    rc, pl, work, (mw, mm) = _plan_fixed(lib, [5] * 16, kv_lens, 16, 5)
    assert rc == 0, lib.nsg_last_error()
    qo = np.concatenate([[0], np.cumsum([5] * 16)]).astype(np.int32)
    kvp = np.concatenate([[0], np.cumsum([(L + 15) // 16 for L in kv_lens])]).astype(np.int32)
    items = work[:mw][work[:mw, 1] > 0]
    merges = work[mw:][work[mw:, 3] > 1]
    _check_cover(pl, items, merges, [5] * 16, kv_lens, qo, kvp)


def test_fixed_plan_with_kv_bound_never_splits(lib):
    rng = np.random.default_rng(4)
    for kv_lens in ([5] * 32, list(rng.integers(100, 641, 32)), [4096] * 32):
        rc, pl, work, (mw, mm) = _plan_fixed(lib, [5] * 32, kv_lens, 32, 5, max_kv=4096)
        assert rc == 0, lib.nsg_last_error()
        # latency regime: query tiles of at most 16 rows (2 tokens x 7 heads):
        # three per request, one work item each, no split, no merge
        assert (pl.q_tile_tokens, pl.row_tiles) == (2, 1)
        assert (mw, mm) == (96, 0) and (pl.num_work, pl.num_merge) == (96, 0)
        assert pl.max_splits == 1 and pl.kv_groups == 4
        qo = np.concatenate([[0], np.cumsum([5] * 32)]).astype(np.int32)
        kvp = np.concatenate([[0], np.cumsum([(L + 15) // 16 for L in kv_lens])]).astype(np.int32)
        _check_cover(pl, work[:mw], work[mw:mw], [5] * 32, kv_lens, qo, kvp)
    assert _plan_fixed(lib, [5] * 2, [4097, 10], 2, 5, max_kv=4096)[0] == 1   # over the bound
    assert "bound" in lib.nsg_last_error().decode()


def test_fixed_plan_keeps_tile_shape_and_rejects_longer_queries(lib):
    # fewer query tokens than the graph's length: same tile shape as the full one
    rc, pl, _, _ = _plan_fixed(lib, [2] * 8, [100] * 8, 8, 5)
    rc5, pl5, _, _ = _plan_fixed(lib, [5] * 8, [100] * 8, 8, 5)
    assert rc == rc5 == 0
    assert (pl.row_tiles, pl.q_tile_tokens) == (pl5.row_tiles, pl5.q_tile_tokens)
    assert _plan_fixed(lib, [6] * 8, [100] * 8, 8, 5)[0] == 1       # longer than fixed
    assert "fixed plan" in lib.nsg_last_error().decode()
    # capacity for one request on one CU; three long requests need more merge items
    assert _plan_fixed(lib, [5] * 3, [2000] * 3, 1, 5, cus=1)[0] == 3


def test_planner_rejects_bad_input(lib):
    assert _plan(lib, [5], [3])[0] == 1                 # L < q_len under the causal rule
    assert _plan(lib, [5], [30], D=96)[0] == 2          # unsupported head dim
    assert _plan(lib, [5], [30], Hq=14, Hkv=3)[0] == 1  # Hq % Hkv
    assert _plan(lib, [5], [30], P=12)[0] == 1          # page size not a power of two
    assert "page_size" in lib.nsg_last_error().decode()


def test_accept_workspace_and_argument_checks(lib):
    assert lib.nsg_spec_accept_workspace_bytes(64, 4, 151936) > 64 * 9 * 4 * 8
    assert lib.nsg_spec_accept_workspace_bytes(-1, 4, 10) == -1
    # k beyond the kernel's limit is an argument error before any GPU work
    rc = lib.nsg_spec_accept(None, 0, 0, None, 0, 0, 0, None, None, None, 1, 99, 10, 0.0, None,
                             None, None, 16, None, None, None, None, 0, None)
    assert rc == 1 and "k 99" in lib.nsg_last_error().decode()


def test_sample_workspace_and_argument_checks(lib):
    assert lib.nsg_sample_workspace_bytes(64, 151936) > 64 * 8 * 256 * 12
    assert lib.nsg_sample_workspace_bytes(-1, 10) == -1
    # argument errors before any GPU work: top_p outside (0, 1], missing uniforms
    rc = lib.nsg_sample(None, 10, 0, 1, 10, 1.0, 0, 0.0, None, 1, None, None, 0, None)
    assert rc == 1 and "top_p" in lib.nsg_last_error().decode()
    rc = lib.nsg_sample(None, 10, 2, 1, 10, 1.0, 0, 1.0, None, 1, None, None, 0, None)
    assert rc == 1 and "logits_dtype" in lib.nsg_last_error().decode()
    assert lib.nsg_sample(None, 10, 0, 0, 10, 1.0, 5, 0.5, None, 1, None, None, 0, None) == 0


def test_lm_head_fold_shape_rule_and_argument_checks(lib):
    """nsg_lm_head_fold_supported is host logic: the partial sums of every
    row must fit one ring slot of the lm_head kernel (M * parts a multiple of
    4, whole 1 KB copies, one KB kept for the row scales)."""
    ok = lib.nsg_lm_head_fold_supported
    assert ok(160, 151936, 896, 56) == 1          # the 0.5B verify call
    assert ok(32, 151936, 896, 56) == 1           # a draft call
    assert ok(1, 1000, 896, 56) == 1
    assert ok(160, 151936, 1024, 64) == 0         # 40 KB of partials > the slot
    assert ok(128, 151936, 1024, 64) == 0         # 32 KB: no KB left for the scales
    assert ok(96, 151936, 1024, 64) == 1
    assert ok(161, 151936, 896, 56) == 0          # more rows than the kernel takes
    assert ok(7, 1000, 896, 57) == 0              # 7 * 57 not a multiple of 4
    assert ok(32, 1002, 896, 56) == 0             # N % 4
    assert ok(32, 1000, 800, 50) == 0             # K % 64
    # argument errors before any GPU work
    rc = lib.nsg_lm_head_fold(None, 896, None, 896, None, 1000, 32, 1000, 896, None, 56, 896,
                              1e-6, None)
    assert rc == 1 and "null" in lib.nsg_last_error().decode()
    rc = lib.nsg_lm_head_fold_argmax(16, 896, 16, 896, 161, 1000, 896, 16, 56, 896, 1e-6, None,
                                     0, None, 1, None)
    assert rc == 1 and "M 161" in lib.nsg_last_error().decode()


def test_argmax_key_consumers_check_arguments(lib):
    """The keyed entry points refuse missing keys before any GPU work."""
    rc = lib.nsg_embed_rows_keys(8, 1, 0, 4, 1, 0, None, 16, 16, 896, 1000, 896, 16, 896, None,
                                 None)
    assert rc == 1 and "keys" in lib.nsg_last_error().decode()
    rc = lib.nsg_embed_rows_keys(8, 1, 0, 4, 1, 1, 8, 16, 16, 896, 1000, 896, 16, 896, None,
                                 None)   # key_j outside [0, per_batch)
    assert rc == 1 and "key_j" in lib.nsg_last_error().decode()
    rc = lib.nsg_spec_accept_greedy_keys(8, 0, None, 8, 4, 1, 2, 4, 1000, None, None, None, 16,
                                         8, 8, None, None, None)
    assert rc == 1 and "key_cols" in lib.nsg_last_error().decode()
    rc = lib.nsg_lm_head_fold_keys(16, 896, 16, 896, 32, 1000, 896, 16, 56, 896, 1e-6, 16,
                                   1 << 20, None, None)
    assert rc == 1 and "key_cols" in lib.nsg_last_error().decode()


def test_host_gate_segments_check_arguments(lib):
    """Segment lists the gate cannot copy are refused before any GPU work."""
    I64 = C.c_int64 * 9
    offs, lens = I64(*([0] * 9)), I64(*([16] * 9))
    rc = lib.nsg_host_gate_wait_segments(8, 1, 8, 1000, 16, 16, 4096, offs, lens, 9, None)
    assert rc == 1 and "n_segs 9" in lib.nsg_last_error().decode()
    offs2, lens2 = (C.c_int64 * 2)(0, 8), (C.c_int64 * 2)(16, 16)
    rc = lib.nsg_host_gate_wait_segments(8, 1, 8, 1000, 16, 16, 4096, offs2, lens2, 2, None)
    assert rc == 1 and "segment 1" in lib.nsg_last_error().decode()
    offs3, lens3 = (C.c_int64 * 1)(4080,), (C.c_int64 * 1)(32,)
    rc = lib.nsg_host_gate_wait_segments(8, 1, 8, 1000, 16, 16, 4096, offs3, lens3, 1, None)
    assert rc == 1 and "within the 4096-byte" in lib.nsg_last_error().decode()
    rc = lib.nsg_host_gate_wait_segments(8, 0, 8, 1000, 16, 16, 4096, offs3, (C.c_int64 * 1)(16), 1,
                                         None)
    assert rc == 1 and "target 0" in lib.nsg_last_error().decode()
