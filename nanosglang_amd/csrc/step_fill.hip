// Host-side inputs of one captured speculative step, in one call.
//
// The reference's graph decode path builds the page-table CSR, last-page
// lengths and write slots of every request in Python, pads the batch with
// rows on a dummy page and re-plans the attention wrapper before each replay
// (nano_sglang/engine/engine.py:357-410).  A speculative step repeats that for
// k one-token draft calls and one (k+1)-token verify call
// (nano_sglang/decode/speculative.py:76-128), so here the whole step's inputs
// -- tokens, positions, KV slots, k + 1 CSR page tables and k + 1 fixed-size
// work lists -- are written straight into the caller's pinned staging buffer
// (one upload, then the graph replay).  No GPU call is made.
//
// Rules (the reference's, applied per attention call):
//   kv length L = start + a + 1 (draft a) or start + k + 1 (verify);
//   pages ceil(L / P); last page length L - (pages - 1) * P (engine.py:367-371);
//   slot of position p: page_table[p / P] * P + p % P (engine.py:373-376);
//   padding rows: every page the dummy page, start 0, token 0 (engine.py:378-391).
#include <climits>
#include <cstring>
#include <vector>

#include "common.hpp"

namespace nsg {
namespace {

constexpr int kMaxDrafts = 32;

int32_t fill_impl(const int32_t* page_table, int64_t page_table_stride, const int32_t* rows,
                  const int32_t* num_pages, const int64_t* start_pos, const int64_t* last_token,
                  int32_t batch, int32_t padded_batch, int32_t k, int32_t page_size,
                  int32_t dummy_page, int32_t num_qo_heads, int32_t num_kv_heads,
                  int32_t head_dim, int32_t num_cus, int32_t max_kv_len,
                  const nsg_spec_step_bufs_t* bufs, nsg_attn_plan_t* plans);

}  // namespace
}  // namespace nsg

using namespace nsg;

extern "C" int32_t nsg_spec_step_fill(const int32_t* page_table, int64_t page_table_stride,
                                      const int32_t* rows, const int32_t* num_pages,
                                      const int64_t* start_pos, const int64_t* last_token,
                                      int32_t batch, int32_t padded_batch, int32_t k,
                                      int32_t page_size, int32_t dummy_page,
                                      int32_t num_qo_heads, int32_t num_kv_heads,
                                      int32_t head_dim, int32_t num_cus, int32_t max_kv_len,
                                      const nsg_spec_step_bufs_t* bufs, nsg_attn_plan_t* plans) {
  return fill_impl(page_table, page_table_stride, rows, num_pages, start_pos, last_token, batch,
                   padded_batch, k, page_size, dummy_page, num_qo_heads, num_kv_heads, head_dim,
                   num_cus, max_kv_len, bufs, plans);
}

extern "C" int32_t nsg_spec_step_fill_next(
    const int32_t* page_table, int64_t page_table_stride, const int32_t* rows,
    const int32_t* num_pages, const int64_t* start_pos, const int64_t* to_go,
    const int32_t* n_emitted, const int64_t* emitted, int32_t batch, int32_t padded_batch,
    int32_t k, int32_t page_size, int32_t dummy_page, int32_t num_qo_heads,
    int32_t num_kv_heads, int32_t head_dim, int32_t num_cus, int32_t max_kv_len,
    const nsg_spec_step_bufs_t* bufs, nsg_attn_plan_t* plans, int32_t* next_batch) {
  NSG_CHECK_ARG(next_batch != nullptr, "null next_batch");
  NSG_CHECK_ARG(batch >= 0 && batch <= padded_batch, "batch %d outside [0, padded_batch %d]",
                batch, padded_batch);
  NSG_CHECK_ARG(k >= 0 && k <= kMaxDrafts, "k %d outside [0, %d]", k, kMaxDrafts);
  NSG_CHECK_ARG(batch == 0 || (rows && num_pages && start_pos && to_go && n_emitted && emitted),
                "null request array");
  std::vector<int32_t> r2, np2;
  std::vector<int64_t> s2, t2;
  r2.reserve(batch);
  np2.reserve(batch);
  s2.reserve(batch);
  t2.reserve(batch);
  for (int j = 0; j < batch; ++j) {
    const int n = n_emitted[j];
    NSG_CHECK_ARG(n >= 1 && n <= k + 1, "request %d emitted %d tokens, outside [1, k + 1]", j,
                  n);
    if (to_go[j] <= n) continue;  // done after this step
    r2.push_back(rows[j]);
    np2.push_back(num_pages[j]);
    s2.push_back(start_pos[j] + n);
    t2.push_back(emitted[(int64_t)j * (k + 1) + n - 1]);
  }
  const int32_t nb = (int32_t)r2.size();
  const int32_t rc = fill_impl(page_table, page_table_stride, r2.data(), np2.data(), s2.data(),
                               t2.data(), nb, padded_batch, k, page_size, dummy_page,
                               num_qo_heads, num_kv_heads, head_dim, num_cus, max_kv_len, bufs,
                               plans);
  if (rc == NSG_OK) *next_batch = nb;
  return rc;
}

namespace nsg {
namespace {

int32_t fill_impl(const int32_t* page_table, int64_t page_table_stride, const int32_t* rows,
                  const int32_t* num_pages, const int64_t* start_pos, const int64_t* last_token,
                  int32_t batch, int32_t padded_batch, int32_t k, int32_t page_size,
                  int32_t dummy_page, int32_t num_qo_heads, int32_t num_kv_heads,
                  int32_t head_dim, int32_t num_cus, int32_t max_kv_len,
                  const nsg_spec_step_bufs_t* bufs, nsg_attn_plan_t* plans) {
  NSG_CHECK_ARG(bufs && plans, "null bufs or plans");
  NSG_CHECK_ARG(batch >= 0 && batch <= padded_batch, "batch %d outside [0, padded_batch %d]",
                batch, padded_batch);
  NSG_CHECK_ARG(k >= 0 && k <= kMaxDrafts, "k %d outside [0, %d]", k, kMaxDrafts);
  NSG_CHECK_ARG(page_size > 0 && (page_size & (page_size - 1)) == 0,
                "page_size %d must be a power of two", page_size);
  NSG_CHECK_ARG(dummy_page >= 0, "dummy_page %d < 0", dummy_page);
  NSG_CHECK_ARG(batch == 0 || (page_table && rows && num_pages && start_pos && last_token),
                "null request array");
  const nsg_spec_step_bufs_t& o = *bufs;
  NSG_CHECK_ARG(o.token0 && o.start && (k == 0 || (o.draft_pos && o.draft_slot)) && o.verify_pos &&
                    o.verify_slot && o.qo_indptr && o.kv_indptr && o.kv_last_page_len &&
                    o.kv_indices && o.work,
                "null staging pointer");
  NSG_CHECK_ARG(o.indptr_stride >= padded_batch + 1, "indptr_stride %d < padded_batch + 1",
                o.indptr_stride);
  const int P = page_size;
  const int S = padded_batch;

  // per-row view: page list, its length and the start position
  for (int j = 0; j < batch; ++j) {
    const int64_t s = start_pos[j];
    NSG_CHECK_ARG(s >= 0 && s <= INT32_MAX - k - 1, "request %d: start position %lld outside "
                  "[0, INT32_MAX - k - 1]", j, (long long)s);
    const int64_t need = (s + k + 1 + P - 1) / P;
    NSG_CHECK_ARG(num_pages[j] >= need, "request %d holds %d pages, the step needs %lld", j,
                  num_pages[j], (long long)need);
    NSG_CHECK_ARG(num_pages[j] <= page_table_stride, "request %d: %d pages exceed the page "
                  "table's row stride %lld", j, num_pages[j], (long long)page_table_stride);
    NSG_CHECK_ARG(rows[j] >= 0, "request %d: row %d < 0", j, rows[j]);
    o.token0[j] = last_token[j];
    o.start[j] = (int32_t)s;
  }
  for (int j = batch; j < S; ++j) {
    o.token0[j] = 0;
    o.start[j] = 0;
  }
  auto page_of = [&](int j, int64_t pg) -> int64_t {
    return j < batch ? page_table[(int64_t)rows[j] * page_table_stride + pg] : dummy_page;
  };
  auto slot_of = [&](int j, int64_t pos) -> int64_t {
    return page_of(j, pos / P) * P + pos % P;
  };

  // positions and KV slots of the k draft calls and of the verify call
  for (int a = 0; a < k; ++a) {
    int64_t* pos = o.draft_pos + (size_t)a * S;
    int64_t* slot = o.draft_slot + (size_t)a * S;
    for (int j = 0; j < S; ++j) {
      const int64_t p = (int64_t)o.start[j] + a;
      pos[j] = p;
      slot[j] = slot_of(j, p);
    }
  }
  for (int j = 0; j < S; ++j) {
    for (int t = 0; t <= k; ++t) {
      const int64_t p = (int64_t)o.start[j] + t;
      o.verify_pos[(size_t)j * (k + 1) + t] = p;
      o.verify_slot[(size_t)j * (k + 1) + t] = slot_of(j, p);
    }
  }

  // the k + 1 attention calls: CSR page tables and fixed-size plans
  for (int a = 0; a <= k; ++a) {
    const int ql = a < k ? 1 : k + 1;
    const int extra = a < k ? a + 1 : k + 1;
    int32_t* qo = o.qo_indptr + (size_t)a * o.indptr_stride;
    int32_t* kvp = o.kv_indptr + (size_t)a * o.indptr_stride;
    int32_t* last = o.kv_last_page_len + (size_t)a * o.indptr_stride;
    int32_t* idx = o.kv_indices + (size_t)a * o.indices_stride;
    qo[0] = 0;
    kvp[0] = 0;
    int64_t nnz = 0;
    for (int j = 0; j < S; ++j) {
      const int64_t L = (int64_t)o.start[j] + extra;
      const int64_t np = (L + P - 1) / P;
      NSG_CHECK_ARG(nnz + np <= o.indices_stride,
                    "attention call %d: %lld page ids exceed indices_stride %d", a,
                    (long long)(nnz + np), o.indices_stride);
      if (j < batch) {
        std::memcpy(idx + nnz, page_table + (int64_t)rows[j] * page_table_stride,
                    (size_t)np * sizeof(int32_t));
      } else {
        for (int64_t pg = 0; pg < np; ++pg) idx[nnz + pg] = dummy_page;
      }
      nnz += np;
      qo[j + 1] = (j + 1) * ql;
      kvp[j + 1] = (int32_t)nnz;
      last[j] = (int32_t)(L - (np - 1) * P);
    }
    int32_t* work = o.work + (size_t)a * o.work_stride;
    const nsg_attn_plan_t& p0 = plans[0];
    if (a >= 1 && a < k && p0.q_tile_tokens == 1 && p0.max_splits == 1 && p0.num_merge == 0 &&
        p0.num_work == S && p0.num_groups == S) {
      // a later draft call: one query token per row, so the plan of draft
      // call 0 with each row's KV range moved (its work item n is row n, one
      // KV split): the planner would write exactly this
      plans[a] = p0;
      for (int j = 0; j < S; ++j) {
        const int32_t L = (kvp[j + 1] - kvp[j] - 1) * P + last[j];
        int32_t* w = work + (size_t)j * NSG_ATTN_WORK_INTS;
        w[0] = j;
        w[1] = 1;
        w[2] = L - 1;
        w[3] = kvp[j];
        w[4] = 0;
        w[5] = L;
        w[6] = 1;
        w[7] = 0;
      }
      continue;
    }
    int32_t mw = 0, mm = 0;
    int32_t rc = nsg_attn_fixed_capacity(S, ql, num_qo_heads, num_kv_heads, num_cus, max_kv_len,
                                         &mw, &mm);
    if (rc != NSG_OK) return rc;
    rc = nsg_attn_plan_fixed(qo, kvp, last, S, num_qo_heads, num_kv_heads, head_dim, P,
                             /*causal=*/1, num_cus, ql, max_kv_len, mw, mm, work,
                             o.work_stride / NSG_ATTN_WORK_INTS, plans + a);
    if (rc != NSG_OK) return rc;
  }
  clear_error();
  return NSG_OK;
}

}  // namespace
}  // namespace nsg
