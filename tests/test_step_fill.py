"""nsg_spec_step_fill (host only): one call writes a speculative step's
tokens, positions, KV slots, k + 1 CSR page tables and fixed-size attention
plans.  Checked against the page-table oracle (engine.py:357-394 rules:
CSR, last-page lengths, write slots, dummy-page padding rows) and against
nsg_attn_plan_fixed run on the oracle's CSR."""
import ctypes as C

import numpy as np
import pytest

from nanosglang_amd._native import NSG_ATTN_WORK_INTS, AttnPlan, StepBufs
from oracle import page_table as opt

Hq, Hkv, D, CUS = 14, 2, 64, 256


class _Staging:
    def __init__(self, lib, bs, k, max_kv_len, ids_stride):
        nw = 0
        for a in range(k + 1):
            ql = 1 if a < k else k + 1
            mw, mm = C.c_int32(0), C.c_int32(0)
            assert lib.nsg_attn_fixed_capacity(bs, ql, Hq, Hkv, CUS, max_kv_len, C.byref(mw),
                                               C.byref(mm)) == 0
            nw = max(nw, (mw.value + mm.value) * NSG_ATTN_WORK_INTS)
        self.si, self.sx, self.sw = bs + 3, ids_stride, nw + 8
        # canaries: every array starts at -7 so untouched entries show up
        f = lambda n, dt: np.full(n, -7, dt)
        self.tok0, self.start = f(bs, np.int64), f(bs, np.int32)
        self.pos, self.slot = f(k * bs, np.int64), f(k * bs, np.int64)
        self.vpos, self.vslot = f(bs * (k + 1), np.int64), f(bs * (k + 1), np.int64)
        self.qo, self.kvp = f((k + 1) * self.si, np.int32), f((k + 1) * self.si, np.int32)
        self.last = f((k + 1) * self.si, np.int32)
        self.idx, self.work = f((k + 1) * self.sx, np.int32), f((k + 1) * self.sw, np.int32)
        self.bufs = StepBufs(*[a.ctypes.data for a in (
            self.tok0, self.start, self.pos, self.slot, self.vpos, self.vslot, self.qo, self.kvp,
            self.last, self.idx, self.work)], self.si, self.sx, self.sw)
        self.plans = (AttnPlan * (k + 1))()


def _fill(lib, st, tab, rows, npg, starts, last, bs, k, P, dummy, max_kv_len):
    B = len(rows)
    arrs = [np.ascontiguousarray(rows, np.int32), np.ascontiguousarray(npg, np.int32),
            np.ascontiguousarray(starts, np.int64), np.ascontiguousarray(last, np.int64)]
    ptrs = [a.ctypes.data if B else None for a in arrs]
    return lib.nsg_spec_step_fill(tab.ctypes.data if B else None, tab.shape[1] if B else 0,
                                  *ptrs, B, bs, k, P, dummy, Hq, Hkv, D, CUS, max_kv_len,
                                  C.byref(st.bufs), st.plans)


def _case(seed, B, bs, k, P, n_pool=4000):
    rng = np.random.default_rng(seed)
    dummy = n_pool - 1
    perm = rng.permutation(n_pool - 1).astype(np.int32)
    starts = rng.integers(0, 300, B).astype(np.int64)
    starts[: min(B, 2)] = [P - 1, 0][: min(B, 2)]          # a page boundary and position 0
    tables, o = [], 0
    for s in starts:
        n = (s + k + 1 + P - 1) // P + int(rng.integers(0, 3))   # reserve may leave spare pages
        tables.append(perm[o:o + n])
        o += n
    width = max([len(t) for t in tables] + [1]) + 5
    tab = np.full((B + 3, width), -1, np.int32)
    rows = rng.permutation(B + 3)[:B].astype(np.int32)     # requests in arbitrary rows
    for t, r in zip(tables, rows):
        tab[r, :len(t)] = t
    last = rng.integers(0, 150000, B).astype(np.int64)
    npg = np.asarray([len(t) for t in tables], np.int32)
    return tab, rows, npg, starts, last, tables, dummy


@pytest.mark.parametrize("B,bs,k,P", [(0, 4, 4, 16), (5, 8, 4, 16), (32, 32, 4, 16),
                                      (3, 4, 1, 16), (7, 8, 6, 4), (6, 8, 3, 1),
                                      (9, 16, 8, 2), (5, 8, 0, 16)])
def test_step_fill_matches_the_page_table_oracle(lib, B, bs, k, P):
    tab, rows, npg, starts, last, tables, dummy = _case(B * 31 + k, B, bs, k, P)
    max_kv = 1022 * P if P >= 2 else 0
    st = _Staging(lib, bs, k, max_kv, ids_stride=4000 + bs * ((k + P) // P) + 7)
    assert _fill(lib, st, tab, rows, npg, starts, last, bs, k, P, dummy, max_kv) == 0, \
        lib.nsg_last_error()
    pad = bs - B
    full_tables = [list(t) for t in tables] + [[dummy] * ((k + P) // P + 1)] * pad
    full_starts = list(starts) + [0] * pad
    np.testing.assert_array_equal(st.tok0, list(last) + [0] * pad)
    np.testing.assert_array_equal(st.start, full_starts)
    for a in range(k):
        np.testing.assert_array_equal(st.pos[a * bs:(a + 1) * bs], np.add(full_starts, a))
        np.testing.assert_array_equal(st.slot[a * bs:(a + 1) * bs],
                                      opt.write_indices(full_tables, np.add(full_starts, a),
                                                        [1] * bs, P))
    np.testing.assert_array_equal(
        st.vpos, (np.asarray(full_starts)[:, None] + np.arange(k + 1)[None]).reshape(-1))
    np.testing.assert_array_equal(st.vslot,
                                  opt.write_indices(full_tables, full_starts, [k + 1] * bs, P))
    for a in range(k + 1):
        ql = 1 if a < k else k + 1
        kv_lens = [s + (a + 1 if a < k else k + 1) for s in full_starts]
        kvp, idx, lpl = opt.build_csr(full_tables, kv_lens, P)
        qo = (np.arange(bs + 1) * ql).astype(np.int32)
        si, sx, sw = st.si, st.sx, st.sw
        np.testing.assert_array_equal(st.qo[a * si:a * si + bs + 1], qo)
        np.testing.assert_array_equal(st.kvp[a * si:a * si + bs + 1], kvp)
        np.testing.assert_array_equal(st.last[a * si:a * si + bs], lpl)
        np.testing.assert_array_equal(st.idx[a * sx:a * sx + len(idx)], idx)
        assert (st.idx[a * sx + len(idx):(a + 1) * sx] == -7).all()
        # the plan and work list nsg_attn_plan_fixed gives for the oracle's CSR
        mw, mm = C.c_int32(0), C.c_int32(0)
        assert lib.nsg_attn_fixed_capacity(bs, ql, Hq, Hkv, CUS, max_kv, C.byref(mw),
                                           C.byref(mm)) == 0
        work = np.zeros(sw, np.int32)
        pl = AttnPlan()
        assert lib.nsg_attn_plan_fixed(qo.ctypes.data, kvp.ctypes.data, lpl.ctypes.data, bs, Hq,
                                       Hkv, D, P, 1, CUS, ql, max_kv, mw.value, mm.value,
                                       work.ctypes.data, sw // NSG_ATTN_WORK_INTS,
                                       C.byref(pl)) == 0
        n = (pl.num_work + pl.num_merge) * NSG_ATTN_WORK_INTS
        np.testing.assert_array_equal(st.work[a * sw:a * sw + n], work[:n])
        got = st.plans[a]
        for f, _ in AttnPlan._fields_:
            assert getattr(got, f) == getattr(pl, f), (a, f)


def test_step_fill_rejects_bad_input(lib):
    bs, k, P = 8, 4, 16
    tab, rows, npg, starts, last, tables, dummy = _case(3, 5, bs, k, P)
    st = _Staging(lib, bs, k, 1022 * P, ids_stride=4000 + bs * 2)
    ok = lambda **kw: _fill(lib, st, kw.get("tab", tab), kw.get("rows", rows),
                            kw.get("npg", npg), kw.get("starts", starts), last,
                            kw.get("bs", bs), kw.get("k", k), P, dummy, 1022 * P)
    assert ok() == 0
    short = npg.copy()
    short[2] = (starts[2] + k) // P              # one page fewer than the verify window needs
    assert ok(npg=short) == 1 and b"pages" in lib.nsg_last_error()
    assert ok(k=-1) == 1 and ok(k=33) == 1
    assert ok(bs=4) == 1                         # batch 5 > padded batch 4
    neg = starts.copy()
    neg[1] = -1
    assert ok(starts=neg) == 1
    far = starts.copy()
    far[0] = 1022 * P                            # past the fixed plans' KV bound
    wide = np.full((tab.shape[0], 1030), 0, np.int32)
    wide[:, :tab.shape[1]] = tab
    big = npg.copy()
    big[0] = 1030
    assert ok(starts=far, tab=wide, npg=big) == 1 and b"bound" in lib.nsg_last_error()
    small = _Staging(lib, bs, k, 1022 * P, ids_stride=8)
    assert _fill(lib, small, tab, rows, npg, starts, last, bs, k, P, dummy, 1022 * P) == 1
    assert b"indices_stride" in lib.nsg_last_error()


def test_step_fill_mirrors_into_a_persistent_page_table():
    """The engine's page-table mirror copies only pages added since the last
    sync; a rollback shortens the row (stale entries past it are never read)."""
    from nanosglang_amd.engine.spec_engine import SpecEngine, _Req

    class _Eng:
        _sync_table = SpecEngine._sync_table

    e = _Eng()
    e._tab = np.full((2, 8), -1, np.int32)
    r = _Req(0, [1, 2], 10)
    r.row = 1
    r.table.block_indices[:] = [5, 9]
    e._sync_table(r)
    assert r.synced == 2 and list(e._tab[1, :2]) == [5, 9]
    r.table.block_indices.append(4)
    e._sync_table(r)
    assert list(e._tab[1, :3]) == [5, 9, 4]
    del r.table.block_indices[1:]                  # rollback to one page
    r.synced = min(r.synced, 1)
    r.table.block_indices.append(7)                # re-grown with another page
    e._sync_table(r)
    assert list(e._tab[1, :2]) == [5, 7] and r.synced == 2
    assert (e._tab[0] == -1).all()


@pytest.mark.parametrize("B,bs,k,P", [(6, 8, 4, 16), (32, 32, 4, 16), (5, 8, 2, 4)])
def test_step_fill_next_equals_fill_on_the_continuing_requests(lib, B, bs, k, P):
    """nsg_spec_step_fill_next (the pipelined engine's fill from the previous
    step's results) writes exactly what nsg_spec_step_fill writes for the
    requests that continue: to_go > emitted count, at start + n with their
    last emitted token, in order; the others drop out."""
    tab, rows, npg, starts, _, _, dummy = _case(11 + B, B, bs, 2 * k + 1, P)   # pages for two windows
    rng = np.random.default_rng(B)
    n = rng.integers(1, k + 2, B).astype(np.int32)
    emitted = rng.integers(0, 150000, (B, k + 1)).astype(np.int64)
    to_go = rng.integers(1, 3 * (k + 1), B).astype(np.int64)
    to_go[0], to_go[-1] = n[0], n[-1] + 1            # one request ends, one just continues
    live = to_go > n
    max_kv_len = 1022 * P
    ref = _Staging(lib, bs, k, max_kv_len, 4096)
    assert _fill(lib, ref, tab, rows[live], npg[live], starts[live] + n[live],
                 emitted[live, n[live] - 1], bs, k, P, dummy, max_kv_len) == 0
    got = _Staging(lib, bs, k, max_kv_len, 4096)
    nb = C.c_int32(-1)
    arrs = [np.ascontiguousarray(a) for a in (rows, npg, starts, to_go, n, emitted)]
    rc = lib.nsg_spec_step_fill_next(tab.ctypes.data, tab.shape[1],
                                     *[a.ctypes.data for a in arrs], B, bs, k, P, dummy, Hq,
                                     Hkv, D, CUS, max_kv_len, C.byref(got.bufs), got.plans,
                                     C.byref(nb))
    assert rc == 0
    assert nb.value == int(live.sum())
    for name in ("tok0", "start", "pos", "slot", "vpos", "vslot", "qo", "kvp", "last", "idx",
                 "work"):
        np.testing.assert_array_equal(getattr(got, name), getattr(ref, name), err_msg=name)
    for a in range(k + 1):
        assert bytes(got.plans[a]) == bytes(ref.plans[a])
    # an emitted count outside [1, k + 1] is refused
    bad = n.copy()
    bad[1] = k + 2
    arrs[4] = bad
    assert lib.nsg_spec_step_fill_next(tab.ctypes.data, tab.shape[1],
                                       *[a.ctypes.data for a in arrs], B, bs, k, P, dummy, Hq,
                                       Hkv, D, CUS, max_kv_len, C.byref(got.bufs), got.plans,
                                       C.byref(nb)) == 1
