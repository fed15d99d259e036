/*
 * nsg_spec.h -- C ABI of the MI355X (gfx950) speculative-decoding verify step.
 *
 * One shared library, libnsg_spec.so, built from the HIP sources in nanosglang_amd/csrc/.
 * Every entry point:
 *   - takes plain device pointers, sizes and a hipStream_t (as void*);
 *   - enqueues on that stream and never synchronises the host;
 *   - returns 0 on success or an NSG_ERR_* code, with a message available from
 *     nsg_last_error() (thread-local).  No C++ exception crosses the ABI.
 * All tensors are borrowed; the library frees nothing it did not allocate and
 * keeps no global mutable state besides the per-thread error string and the
 * per-GPU static workspace of nsg_spec_accept_noalloc.
 *
 * Layouts follow the reference (xiehuanyi/nanoSGLang):
 *   KV pool per layer: [num_pages, page_size, num_kv_heads, head_dim] bf16
 *     ("NHD", nano_sglang/engine/paged_kv_cache.py:60-69);
 *   page table: CSR kv_indptr int32[B+1], kv_indices int32[nnz],
 *     kv_last_page_len int32[B] (nano_sglang/engine/engine.py:419-448);
 *   queries / outputs: [total_q, num_qo_heads, head_dim] bf16 with
 *     qo_indptr int32[B+1] (nano_sglang/engine/engine.py:340-342).
 */
#ifndef NSG_SPEC_H
#define NSG_SPEC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* nsg_stream_t; /* a hipStream_t; NULL = the null stream */

enum {
  NSG_OK = 0,
  NSG_ERR_ARG = 1,         /* bad shape, size, pointer or index argument */
  NSG_ERR_UNSUPPORTED = 2, /* valid input outside what the kernels implement */
  NSG_ERR_WORKSPACE = 3,   /* workspace or work-list buffer too small */
  NSG_ERR_HIP = 4          /* a HIP runtime call failed */
};

/* Message for the last failing call on this thread ("" after success). */
const char* nsg_last_error(void);
/* ABI version of this header (NSG_ABI_VERSION). */
int32_t nsg_abi_version(void);
#define NSG_ABI_VERSION 21

/* ------------------------------------------------------------------------
 * Verify attention: ragged multi-query attention over the paged KV cache
 * with GQA and the bottom-right causal rule (row r of a request with q_len
 * query tokens and L KV tokens sees KV positions <= L - q_len + r).
 *
 * Replaces FlashInfer's BatchPrefillWithPagedKVCacheWrapper as the reference
 * uses it: .plan(...) at nano_sglang/engine/engine.py:451-462 (host, once per
 * step) and .run(q, (k_cache[layer], v_cache[layer])) at
 * nano_sglang/model/causal_lm.py:340 (device, once per layer).
 * ---------------------------------------------------------------------- */

#define NSG_ATTN_WORK_INTS 8

typedef struct {
  int32_t num_work;        /* work items: (request, query tile, KV split)        */
  int32_t num_merge;       /* query tiles whose KV splits need a merge pass      */
  int32_t num_groups;      /* (request, query tile) pairs                        */
  int32_t row_tiles;       /* 16-row MFMA tiles per work item, 1..4              */
  int32_t q_tile_tokens;   /* query tokens per query tile                        */
  int32_t max_splits;      /* largest KV split count of any group                */
  int32_t head_dim;
  int32_t num_qo_heads;
  int32_t num_kv_heads;
  int32_t kv_groups;       /* KV groups per workgroup (1, or several in the latency regime) */
  int64_t workspace_bytes; /* device workspace nsg_attn_run needs for this plan  */
} nsg_attn_plan_t;

/* Host-side planner (replaces BatchPrefillWithPagedKVCacheWrapper.plan,
 * engine.py:451-462).  Reads HOST copies of the CSR metadata and writes the
 * work list ((num_work + num_merge) * NSG_ATTN_WORK_INTS int32) into work_h,
 * which the caller copies to device memory for nsg_attn_run.  num_cus sizes the KV
 * split (256 on MI355X).  head_dim must be 64 or 128; num_qo_heads a multiple
 * of num_kv_heads with a group of at most 64; page_size a power of two. */
int32_t nsg_attn_plan(const int32_t* qo_indptr_h, const int32_t* kv_indptr_h,
                      const int32_t* kv_last_page_len_h, int32_t batch,
                      int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                      int32_t page_size, int32_t causal, int32_t num_cus,
                      int32_t* work_h, int32_t work_capacity, nsg_attn_plan_t* plan);

/* Graph-capturable planning: the counterpart of the FlashInfer wrapper built
 * with use_cuda_graph=True and fixed-address buffers (engine.py:110-133,
 * planned before each replay at engine.py:396-410).
 *
 * nsg_attn_fixed_capacity gives the work-list size that every plan of at most
 * `batch` requests with at most `max_q_len` query tokens each fits.
 * nsg_attn_plan_fixed is nsg_attn_plan with that size fixed: the work list is
 * always max_work work items followed by max_merge merge items (unused ones
 * are empty and cost one early-exiting workgroup each), and the tile shape
 * follows max_q_len, so nsg_attn_run launches the same grid with the same
 * arguments for every such plan.  A plan that does not fit returns
 * NSG_ERR_WORKSPACE.  With max_kv_len > 0 (at most 1022 pages) no request's
 * KV range is split: the list holds one work item per query tile, no merge
 * items, and nsg_attn_run launches no merge pass; a longer request is an
 * argument error.  With max_kv_len <= 0 (long contexts) the plan always takes
 * the one-KV-group shape: KV ranges split over enough workgroups to fill the
 * GPU, merged by the second launch. */
int32_t nsg_attn_fixed_capacity(int32_t batch, int32_t max_q_len, int32_t num_qo_heads,
                                int32_t num_kv_heads, int32_t num_cus, int32_t max_kv_len,
                                int32_t* max_work, int32_t* max_merge);
int32_t nsg_attn_plan_fixed(const int32_t* qo_indptr_h, const int32_t* kv_indptr_h,
                            const int32_t* kv_last_page_len_h, int32_t batch,
                            int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                            int32_t page_size, int32_t causal, int32_t num_cus,
                            int32_t max_q_len, int32_t max_kv_len, int32_t max_work,
                            int32_t max_merge, int32_t* work_h, int32_t work_capacity,
                            nsg_attn_plan_t* plan);

/* Bytes of device workspace nsg_attn_run needs for this plan (split partials
 * and an error-flag word, which should start at zero). */
int64_t nsg_attn_workspace_bytes(const nsg_attn_plan_t* plan);

/* Runs one layer (replaces wrapper.run, causal_lm.py:340).
 * q/out: [total_q, Hq, D] bf16; k_cache/v_cache: [num_pages, P, Hkv, D] bf16;
 * work_d: device copy of the planner's work list.  sm_scale must be
 * positive (the kernel scales each row's maximum raw score).  Page ids
 * outside [0, num_pages) read other rows of the pool (the outputs of their
 * rows are undefined) and raise a flag returned by nsg_attn_check_flags.
 * page_size must be the plan's (plans with several KV groups need pages of
 * 16+ tokens: the planner picks one group for smaller pages). */
int32_t nsg_attn_run(const nsg_attn_plan_t* plan, const int32_t* work_d,
                     const void* q, const void* k_cache, const void* v_cache, void* out,
                     const int32_t* qo_indptr, const int32_t* kv_indptr,
                     const int32_t* kv_indices, const int32_t* kv_last_page_len,
                     int32_t page_size, int32_t num_pages, float sm_scale, int32_t causal,
                     void* workspace, int64_t workspace_bytes, nsg_stream_t stream);

/* Copies the workspace's error flags (bit 0: page id out of range) to
 * *flags_h after synchronising the stream, and clears them. */
int32_t nsg_attn_check_flags(void* workspace, int32_t* flags_h, nsg_stream_t stream);

/* ------------------------------------------------------------------------
 * Host-side inputs of one captured speculative step (host only; no GPU call).
 *
 * Replaces the per-step preparation of the reference's graph decode path
 * (engine.py:357-410: page-table CSR, last-page lengths, write slots, padding
 * rows on a dummy page, wrapper.plan before g.replay), widened to the k
 * one-token draft calls and the (k+1)-token verify call of a speculative step
 * (speculative.py:76-128).  Request j of `batch` owns row rows[j] of
 * page_table (num_pages[j] valid page ids; the step needs
 * ceil((start_pos[j] + k + 1) / page_size) of them) and its last emitted
 * token last_token[j] sits at position start_pos[j], not yet in the cache.
 * Rows batch .. padded_batch-1 are padding: start 0, token 0, every page
 * dummy_page.  Attention call a < k (draft a) has one query per row over
 * start + a + 1 keys; call k (verify) has k + 1 queries over start + k + 1
 * keys; each is planned by nsg_attn_plan_fixed with max_q_len = its query
 * count and the given max_kv_len, into plans[a].  k may be 0 (no draft
 * calls: plain decode).  Arrays with a stride hold
 * one block per attention call (k + 1 blocks). */
typedef struct {
  int64_t* token0;            /* [padded_batch] last emitted token            */
  int32_t* start;             /* [padded_batch] start position                */
  int64_t* draft_pos;         /* [k][padded_batch] position of draft call a   */
  int64_t* draft_slot;        /* [k][padded_batch] KV slot of draft call a
                                 (both may be NULL when k = 0)               */
  int64_t* verify_pos;        /* [padded_batch][k+1]                          */
  int64_t* verify_slot;       /* [padded_batch][k+1]                          */
  int32_t* qo_indptr;         /* [k+1][indptr_stride], padded_batch+1 used    */
  int32_t* kv_indptr;         /* [k+1][indptr_stride], padded_batch+1 used    */
  int32_t* kv_last_page_len;  /* [k+1][indptr_stride], padded_batch used      */
  int32_t* kv_indices;        /* [k+1][indices_stride]                        */
  int32_t* work;              /* [k+1][work_stride] work lists                */
  int32_t indptr_stride;
  int32_t indices_stride;
  int32_t work_stride;
} nsg_spec_step_bufs_t;

int32_t nsg_spec_step_fill(const int32_t* page_table, int64_t page_table_stride,
                           const int32_t* rows, const int32_t* num_pages,
                           const int64_t* start_pos, const int64_t* last_token, int32_t batch,
                           int32_t padded_batch, int32_t k, int32_t page_size,
                           int32_t dummy_page, int32_t num_qo_heads, int32_t num_kv_heads,
                           int32_t head_dim, int32_t num_cus, int32_t max_kv_len,
                           const nsg_spec_step_bufs_t* bufs, nsg_attn_plan_t* plans);

/* nsg_spec_step_fill for the step after one whose results just arrived, for
 * an engine that queued that next step before those results (see the host
 * gate below): request j of the finished step (rows[j], num_pages[j],
 * start_pos[j]) emitted n_emitted[j] tokens emitted[j * (k + 1) + 0 ..
 * n_emitted[j] - 1] and had to_go[j] tokens left to produce before it.  The
 * requests with to_go[j] > n_emitted[j] continue, in order, at start_pos[j] +
 * n_emitted[j] with their last emitted token; *next_batch receives their
 * count.  No separate reference line: it is the reference's per-request
 * bookkeeping (speculative.py:184-196, positions and last token) folded into
 * the next step's fill. */
int32_t nsg_spec_step_fill_next(const int32_t* page_table, int64_t page_table_stride,
                                const int32_t* rows, const int32_t* num_pages,
                                const int64_t* start_pos, const int64_t* to_go,
                                const int32_t* n_emitted, const int64_t* emitted, int32_t batch,
                                int32_t padded_batch, int32_t k, int32_t page_size,
                                int32_t dummy_page, int32_t num_qo_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t num_cus, int32_t max_kv_len,
                                const nsg_spec_step_bufs_t* bufs, nsg_attn_plan_t* plans,
                                int32_t* next_batch);

/* ------------------------------------------------------------------------
 * Fused acceptance: ratio test, residual resample, bonus token and rollback
 * slots for one verify step of B requests.
 *
 * Replaces nano_sglang/decode/speculative.py:130-184 (the per-position
 * Python loop) and gives the paged counterpart of reset_draft_cache
 * (speculative.py:186-196).
 *
 * target_logits: B x (k+1) rows of `vocab` logits; draft_logits: B x k rows
 *   (may be NULL when temperature < 1e-6, the greedy rule of
 *   nano_sglang/engine/sampling.py:44).  Row r of request b starts at
 *   element b*req_stride + r*row_stride; logits_dtype 0 = bf16, 1 = fp32.
 * draft_tokens int64 [B, k]; uniforms fp32 [B, k+1] (columns 0..k-1 for the
 *   ratio tests, column k for the residual / bonus draw).
 * bonus_tokens int64 [B] (may be NULL; ignored when greedy): when every draft
 *   of request b is accepted, emitted[b][k] = bonus_tokens[b] instead of a
 *   draw from target row k -- the reference's bonus is sample_token with
 *   top-k / top-p (speculative.py:174-182), which nsg_sample computes.
 * Page table (may be NULL, then no rollback slots): kv_indptr / kv_indices
 *   as in the attention entry points, start_pos int32 [B] = position of the
 *   first verify token (the cache length before verify).
 * Outputs: num_emitted int32 [B] in [1, k+1]; emitted int64 [B, k+1] padded
 *   with -1; rollback_slots int64 [B, k] padded with -1 = flat slots
 *   block*P + offset of positions start+n .. start+k.
 * k may be 0: the call then samples one token per request from row 0
 *   (argmax when greedy), which is the reference's sample_token
 *   (sampling.py:25-50) without top-k / top-p (nsg_sample has them).
 * Workspace: zero when first used, and for acceptance calls only (not shared
 *   with nsg_sample).  Past its 256-byte flag header it holds hand-off slots
 *   through which a request's workgroups pass records to the one that
 *   finishes the request; every slot is zero between calls (the readers clear
 *   what the writers published), so one workspace serves calls of any (B, k)
 *   in turn.  Calls sharing a workspace must not overlap.
 * Bad inputs found on the device leave well-defined outputs and set bits of
 *   an error-flag word at the start of the workspace (which should start at
 *   zero), read with nsg_spec_accept_check_flags: bit 1, a rolled-back
 *   position past the request's pages (its slot is -1); bit 2, a draft token
 *   outside [0, vocab) (rejected, as a draft the target never proposes);
 *   bit 3, a hand-off wait that ran out its bounded spin (a workspace that was
 *   not zero, or shared with an overlapping call; outputs then undefined, and
 *   nsg_spec_accept_check_flags zeroes the whole workspace).
 * ---------------------------------------------------------------------- */
int64_t nsg_spec_accept_workspace_bytes(int32_t batch, int32_t k, int32_t vocab);

int32_t nsg_spec_accept(const void* target_logits, int64_t target_req_stride,
                        int64_t target_row_stride, const void* draft_logits,
                        int64_t draft_req_stride, int64_t draft_row_stride,
                        int32_t logits_dtype, const int64_t* draft_tokens,
                        const float* uniforms, const int64_t* bonus_tokens, int32_t batch,
                        int32_t k, int32_t vocab,
                        float temperature, const int32_t* kv_indptr,
                        const int32_t* kv_indices, const int32_t* start_pos,
                        int32_t page_size, int32_t* num_emitted, int64_t* emitted,
                        int64_t* rollback_slots, void* workspace, int64_t workspace_bytes,
                        nsg_stream_t stream);

/* Greedy acceptance from the target rows' tokens: nsg_spec_accept at
 * temperature 0 with target_tokens[b * (k + 1) + i] = the first argmax of
 * target row i of request b (computed without storing the logits, e.g. by
 * nsg_linear_argmax in the verify forward's lm_head, causal_lm.py:643-645).
 * Same rule, outputs, rollback slots and error bits as nsg_spec_accept's
 * greedy form (speculative.py:130-141, 174-182, 186-196); the bits go to
 * *flags (a device int32, may be NULL), e.g. an acceptance workspace's
 * flag word.  Draft token i of request b at draft_tokens[b * draft_stride_b
 * + i * draft_stride_j] (k and 1 for a contiguous [B, k] array; any strides,
 * e.g. rows of a position-major id buffer).  No workspace. */
int32_t nsg_spec_accept_greedy_tokens(const int64_t* target_tokens,
                                      const int64_t* draft_tokens, int64_t draft_stride_b,
                                      int64_t draft_stride_j, int32_t batch, int32_t k,
                                      int32_t vocab, const int32_t* kv_indptr,
                                      const int32_t* kv_indices, const int32_t* start_pos,
                                      int32_t page_size, int32_t* num_emitted, int64_t* emitted,
                                      int64_t* rollback_slots, int32_t* flags,
                                      nsg_stream_t stream);

/* nsg_spec_accept_greedy_tokens with target token i of request b the greedy
 * token of keys row b * (k + 1) + i (key_cols keys per row, from
 * nsg_lm_head_fold_keys over the verify rows), reduced in the same launch;
 * target_tokens_out (may be NULL) receives those tokens. */
int32_t nsg_spec_accept_greedy_keys(const void* target_keys, int32_t key_cols,
                                    int64_t* target_tokens_out, const int64_t* draft_tokens,
                                    int64_t draft_stride_b, int64_t draft_stride_j,
                                    int32_t batch, int32_t k, int32_t vocab,
                                    const int32_t* kv_indptr, const int32_t* kv_indices,
                                    const int32_t* start_pos, int32_t page_size,
                                    int32_t* num_emitted, int64_t* emitted,
                                    int64_t* rollback_slots, int32_t* flags,
                                    nsg_stream_t stream);

/* Copies the acceptance workspace's error flags (bits as above) to *flags_h
 * after synchronising the stream, and clears them.  After bit 3 it zeroes
 * all workspace_bytes of the workspace (hand-off slots a call gave up on may
 * be left published anywhere in the body), so the next call starts clean.
 * Synchronises: not for use under graph capture. */
int32_t nsg_spec_accept_check_flags(void* workspace, int64_t workspace_bytes, int32_t* flags_h,
                                    nsg_stream_t stream);

/* nsg_spec_accept without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  It has no counterpart in the reference.
 * The workspace is a static device array of the library, one per GPU, of
 * nsg_spec_accept_noalloc_max_bytes() bytes (8 MiB), held until the process
 * ends; a call whose nsg_spec_accept_workspace_bytes(batch, k, vocab)
 * exceeds it returns NSG_ERR_WORKSPACE and launches nothing.  The call makes
 * no allocation of any kind.  Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (different streams or threads) race.
 * flags: a device int32 that receives the error bits nsg_spec_accept keeps in
 * its workspace (the caller zeroes it; NULL: not reported).  Every other
 * argument and all outputs are those of nsg_spec_accept, bit for bit. */
int64_t nsg_spec_accept_noalloc_max_bytes(void);
/* Zeroes the current device's static workspace of nsg_spec_accept_noalloc
 * with a fill kernel on `stream` (no allocation, no memset node): the
 * recovery after a call reported flag bit 3, whose hand-off slots may be
 * left published.  Must not overlap a nsg_spec_accept_noalloc call on the
 * same GPU. */
int32_t nsg_spec_accept_noalloc_reset(nsg_stream_t stream);
int32_t nsg_spec_accept_noalloc(const void* target_logits, int64_t target_req_stride,
                                int64_t target_row_stride, const void* draft_logits,
                                int64_t draft_req_stride, int64_t draft_row_stride,
                                int32_t logits_dtype, const int64_t* draft_tokens,
                                const float* uniforms, const int64_t* bonus_tokens,
                                int32_t batch, int32_t k, int32_t vocab, float temperature,
                                const int32_t* kv_indptr, const int32_t* kv_indices,
                                const int32_t* start_pos, int32_t page_size,
                                int32_t* num_emitted, int64_t* emitted, int64_t* rollback_slots,
                                int32_t* flags, nsg_stream_t stream);

/* ------------------------------------------------------------------------
 * Sampling with temperature, top-k and top-p: one token per logits row.
 *
 * Replaces sample_token (nano_sglang/engine/sampling.py:25-50) and its
 * filters (_sample_pytorch, :71-88): argmax (first index) when
 * temperature < 1e-6; otherwise logits / T, top-k keeps every logit >= the
 * k-th largest (top_k <= 0 or >= vocab: off), top-p drops a token when the
 * probability mass of the tokens before it in descending order reaches top_p
 * (top_p in (0, 1]; 1 = off; equal logits ordered by index), then an inverse-
 * CDF draw in vocabulary order with uniforms[r * uniform_stride].  Masses are
 * exact 2^-40 fixed-point sums, so the result does not depend on the order
 * of summation.  logits: rows of `vocab` values, row r at r * row_stride
 * elements; logits_dtype 0 = bf16, 1 = fp32 (no NaN).  tokens int64 [rows]
 * (-1 for a row of -inf).  The workspace needs no initialisation.
 * ---------------------------------------------------------------------- */
int64_t nsg_sample_workspace_bytes(int32_t rows, int32_t vocab);
int32_t nsg_sample(const void* logits, int64_t row_stride, int32_t logits_dtype, int32_t rows,
                   int32_t vocab, float temperature, int32_t top_k, float top_p,
                   const float* uniforms, int64_t uniform_stride, int64_t* tokens,
                   void* workspace, int64_t workspace_bytes, nsg_stream_t stream);

/* ------------------------------------------------------------------------
 * KV slot writes and rollback.
 * ---------------------------------------------------------------------- */

/* Scatter num_tokens rows of K and V ([num_kv_heads, head_dim] bf16 each,
 * consecutive rows src_token_stride elements apart) into flat slots of one
 * layer's pool ([num_slots, num_kv_heads, head_dim]); slot < 0 skips the
 * row.  Replaces `k_flat[write_indices] = k; v_flat[write_indices] = v`
 * (nano_sglang/model/causal_lm.py:335-338). */
int32_t nsg_kv_write(const void* k, const void* v, int64_t src_token_stride,
                     const int64_t* slots, int32_t num_tokens, void* k_cache,
                     void* v_cache, int32_t num_kv_heads, int32_t head_dim,
                     int64_t num_slots, nsg_stream_t stream);

/* Fused RoPE + KV slot write for one layer.  qkv: num_tokens rows of the
 * fused projection [q heads | k heads | v heads] x head_dim (bf16, rows
 * qkv_token_stride elements apart); positions int64; cos/sin tables fp32
 * [max_position, head_dim/2] (nano_sglang/model/causal_lm.py:157-164).
 * q and k are rotated with the half-split rule and bf16 rounding of
 * causal_lm.py:167-206; rotated q -> q_out [num_tokens, Hq, D]; rotated k and
 * v -> flat slot slots[t] of the layer's pool (slot < 0 skips; slots may be
 * NULL to skip the cache write).  Replaces apply_rope (causal_lm.py:300-301)
 * plus the scatter at causal_lm.py:335-338.  Positions outside
 * [0, max_position) or slots >= num_slots set bit 0 of *flags (if given). */
int32_t nsg_rope_kv_write(const void* qkv, int64_t qkv_token_stride, const int64_t* positions,
                          const float* cos_table, const float* sin_table,
                          int32_t max_position, const int64_t* slots, int32_t num_tokens,
                          int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                          void* q_out, void* k_cache, void* v_cache, int64_t num_slots,
                          int32_t* flags, nsg_stream_t stream);

/* Zero the K and V rows of `count` flat slots (negative slots are skipped)
 * in `num_layers` consecutive layer pools, layer_stride elements apart.
 * Used after nsg_spec_accept so rolled-back positions hold no stale data. */
int32_t nsg_kv_clear_slots(const int64_t* slots, int32_t count, void* k_cache, void* v_cache,
                           int32_t num_layers, int64_t layer_stride, int32_t num_kv_heads,
                           int32_t head_dim, int64_t num_slots, nsg_stream_t stream);

/* ------------------------------------------------------------------------
 * Fused per-token layer ops of the draft / verify forwards.
 * ---------------------------------------------------------------------- */

/* RMSNorm of num_tokens rows of `hidden` bf16 values (hidden % 8 == 0,
 * <= 8192): out = bf16(w * (x * rsqrt(mean(x^2) + eps))) in fp32
 * (nano_sglang/model/causal_lm.py:139-145).  With residual != NULL it first
 * does residual = bf16(residual + x) in place and normalises the sum
 * (forward_fused_residual, causal_lm.py:147-154). */
int32_t nsg_rmsnorm(const void* x, void* residual, const void* weight, void* out,
                    int32_t num_tokens, int32_t hidden, float eps, nsg_stream_t stream);

/* SwiGLU gate: gate_up rows hold [gate | up] (2 * intermediate bf16 each);
 * out[t, j] = bf16(bf16(silu(gate)) * up) (causal_lm.py:481-482). */
int32_t nsg_silu_mul(const void* gate_up, void* out, int64_t num_tokens,
                     int32_t intermediate, nsg_stream_t stream);

/* Linear layers at decode / verify row counts (M <= nsg_linear_max_rows(),
 * 160): y[m, n] = x[m, :] . w[n, :] for bf16 x (M x K, row stride ldx) and
 * w (row stride ldw), fp32 accumulation, one rounding to bf16.
 *   NSG_LINEAR_BIAS:     y = bf16(acc + bias[n]) (bias may be NULL) -- the
 *                        q/k/v, o_proj, down_proj and lm_head calls of
 *                        causal_lm.py:229-231, 261, 482, 643-645;
 *   NSG_LINEAR_SILU_MUL: w has 2N rows [gate; up] and
 *                        y = bf16(bf16(silu(bf16(g))) * bf16(u)), the gate_proj /
 *                        up_proj pair plus F.silu(gate) * up (causal_lm.py:481-482).
 * K must be a multiple of 64 and N of 4; x and w rows 16-byte aligned.  Larger
 * M returns NSG_ERR_UNSUPPORTED (a library GEMM serves prefill).  Wide
 * outputs (N >= 65536: lm_head) without a bias, 192 <= K < 2048 (any M) or
 * K >= 2048 (M > 32), run on a kernel that shares x across 128 output
 * columns; there every output's K sum runs in k order in one wave, so the
 * values do not depend on M or the grid. */
#define NSG_LINEAR_BIAS 0
#define NSG_LINEAR_SILU_MUL 1
int32_t nsg_linear_max_rows(void);
/* 1 if nsg_linear is the faster choice for this shape on MI355X (few rows;
 * measured against hipBLASLt), 0 if a library GEMM is. */
int32_t nsg_linear_preferred(int32_t M, int32_t N, int32_t K);
int32_t nsg_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias,
                   void* y, int64_t ldy, int32_t M, int32_t N, int32_t K, int32_t epilogue,
                   nsg_stream_t stream);

/* FP8 weights (FP8Linear, nano_sglang/decode/quantization.py:24-75): w8 holds
 * OCP e4m3fn bytes (row stride ldw8 bytes, rows 8-byte aligned) and w_scale
 * one f32 per weight row (a per-tensor scale repeated over the tensor's rows;
 * several tensors stacked -- q/k/v, gate/up -- keep their own scales).  Each
 * weight is dequantised to bf16(float(w8) * w_scale[row]), the arithmetic of
 * FP8Linear.forward's w8.to(bf16) * scale (:49-52), and the product then runs
 * exactly as nsg_linear / nsg_linear_rope_kv on those bf16 weights (bf16 MFMA,
 * fp32 accumulation), streaming half the weight bytes.  SwiGLU: w8 and
 * w_scale have 2N rows.  Other arguments as in the bf16 entry points. */
int32_t nsg_linear_fp8(const void* x, int64_t ldx, const void* w8, int64_t ldw8,
                       const float* w_scale, const void* bias, void* y, int64_t ldy, int32_t M,
                       int32_t N, int32_t K, int32_t epilogue, nsg_stream_t stream);
int32_t nsg_linear_rope_kv_fp8(const void* x, int64_t ldx, const void* w8, int64_t ldw8,
                               const float* w_scale, const void* bias, int32_t M, int32_t K,
                               int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                               const int64_t* positions, const float* cos_table,
                               const float* sin_table, int32_t max_position,
                               const int64_t* slots, void* q_out, void* k_cache,
                               void* v_cache, int64_t num_slots, int32_t* flags,
                               nsg_stream_t stream);

/* The q/k/v projection with RoPE and the KV-slot write as its epilogue:
 * nsg_linear (NSG_LINEAR_BIAS) of x (M x K) with the fused q/k/v weight w
 * ((Hq + 2 Hkv) * head_dim rows) and bias, immediately followed by
 * nsg_rope_kv_write on the bf16 result -- the same arithmetic (the
 * projection is rounded to bf16 after the bias, then rotated with the
 * bf16 rounding of causal_lm.py:167-206), without the projection ever
 * reaching HBM.  Replaces the q/k/v calls of causal_lm.py:229-231 plus
 * apply_rope (:300-301) and the KV scatter (:335-338).  head_dim 64 or 128;
 * M <= nsg_linear_max_rows(); K % 64 == 0.  Arguments after K mean what
 * they mean for nsg_rope_kv_write. */
/* bf16 copy of FP8 weights for a library GEMM (row counts past the
 * weight-streaming kernel, prefill): out[r][c] = bf16(float(w8[r][c]) *
 * w_scale[r]), the dequantisation of FP8Linear.forward (w8.to(bf16) * scale,
 * nano_sglang/decode/quantization.py:49-52) in one pass.  w8: rows x cols
 * float8_e4m3fn, rows ld8 bytes apart; out: bf16 rows ldo elements apart. */
int32_t nsg_dequant_fp8(const void* w8, int64_t ld8, const float* w_scale, void* out,
                        int64_t ldo, int32_t rows, int32_t cols, nsg_stream_t stream);

int32_t nsg_linear_rope_kv(const void* x, int64_t ldx, const void* w, int64_t ldw,
                           const void* bias, int32_t M, int32_t K, int32_t num_qo_heads,
                           int32_t num_kv_heads, int32_t head_dim, const int64_t* positions,
                           const float* cos_table, const float* sin_table,
                           int32_t max_position, const int64_t* slots, void* q_out,
                           void* k_cache, void* v_cache, int64_t num_slots, int32_t* flags,
                           nsg_stream_t stream);

/* RMSNorm folded into the linears around it (bf16 weights, M up to 160,
 * hidden up to 1024).  No counterpart entry in the reference, whose decoder
 * layer runs residual add + RMSNorm (causal_lm.py:133-154) between the
 * projections; here that norm costs no launch of its own:
 *  - the norm weight w_ln is folded into the columns of the next linear's
 *    weight once (W'[n, k] = bf16(w_ln[k] * W[n, k])), and that linear (the
 *    consumer: q/k/v with RoPE, or gate/up with SwiGLU) takes the
 *    un-normalised rows x and scales row m of x W'^T by
 *    rsqrt(S_m / norm_dim + eps) before its epilogue, where S_m, the sum of
 *    squares of x's row m, arrives as sumsq_parts (1 .. 64) partial sums
 *    sumsq_in[c * M + m] added in a fixed order;
 *  - the linear before it (the producer: o_proj, down_proj, bias epilogue)
 *    adds its result to the residual stream in bf16 (y = bf16(residual +
 *    bf16(x W^T + bias)), y may be the residual buffer itself) and writes
 *    sumsq_out[(n / 16) * M + m], the sum of squares of y's row m over
 *    columns n .. n + 15 (N / 16 partials per row, N % 16 == 0);
 *  - nsg_row_sumsq writes the same partials for the first layer's input.
 * Rounding differs from the reference's norm in two places: w_ln * W is
 * rounded to bf16 instead of w_ln * bf16(x * r), and x * r is not rounded.
 * nsg_linear_fold: the consumer side when sumsq_in is given, the producer
 * side when residual and sumsq_out are (NSG_LINEAR_BIAS only), else
 * nsg_linear. */
int32_t nsg_linear_fold(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias,
                        void* y, int64_t ldy, int32_t M, int32_t N, int32_t K, int32_t epilogue,
                        const float* sumsq_in, int32_t sumsq_parts, int32_t norm_dim, float eps,
                        const void* residual, int64_t ldr, float* sumsq_out,
                        nsg_stream_t stream);
int32_t nsg_linear_rope_kv_fold(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                const void* bias, int32_t M, int32_t K, int32_t num_qo_heads,
                                int32_t num_kv_heads, int32_t head_dim,
                                const int64_t* positions, const float* cos_table,
                                const float* sin_table, int32_t max_position,
                                const int64_t* slots, void* q_out, void* k_cache,
                                void* v_cache, int64_t num_slots, int32_t* flags,
                                const float* sumsq_in, int32_t sumsq_parts, int32_t norm_dim,
                                float eps, nsg_stream_t stream);
int32_t nsg_row_sumsq(const void* x, int64_t ldx, int32_t num_tokens, int32_t hidden,
                      float* sumsq_out, nsg_stream_t stream);

/* Greedy token of each row of the bf16 logits x W^T (+ bias) without
 * storing them: tokens[m * token_stride] = the lowest column n at which
 * bf16(x_m . W_n +
 * bias_n) is largest (-0 and +0 equal), the same value and rounding as the
 * row nsg_linear writes, the tie rule of sample_token's greedy branch
 * (torch.argmax, nano_sglang/engine/sampling.py:44-45).  It replaces
 * lm_head (causal_lm.py:643-645) + the argmax at the draft model's greedy
 * call site (speculative.py:95-100), whose logits nothing else reads.
 * M <= nsg_linear_max_rows(), K % 64 == 0, N % 4 == 0, bf16 weights; the
 * workspace (8-byte aligned, nsg_linear_argmax_workspace_bytes(M, N)) holds
 * one key per row and workgroup (or wave), written before it is read.  At
 * the verify forward's row counts this is also the target's greedy token
 * per verify row (speculative.py:130-141 at temperature 0), for
 * nsg_spec_accept_greedy_tokens. */
int64_t nsg_linear_argmax_workspace_bytes(int32_t M, int32_t N);
int32_t nsg_linear_argmax(const void* x, int64_t ldx, const void* w, int64_t ldw,
                          const void* bias, int32_t M, int32_t N, int32_t K, void* workspace,
                          int64_t workspace_bytes, int64_t* tokens, int64_t token_stride,
                          nsg_stream_t stream);

/* The lm_head after the final RMSNorm (causal_lm.py:643-645, logits =
 * lm_head(norm(h))) with that norm folded in, as nsg_linear_fold folds a
 * layer's norms: W' = bf16(w_norm[k] * W[n, k]) (w_norm folded into W's
 * columns), x the un-normalised rows (the last layer's residual stream), and
 * row m of x W'^T scaled by rsqrt(S_m / norm_dim + eps) before its single
 * bf16 rounding, S_m the sum of sumsq_in[c * M + m] over c < sumsq_parts in
 * order c = 0, 1, ... (the partials the last layer's down_proj epilogue
 * writes).  One launch fewer than nsg_rmsnorm + the lm_head; rounding differs
 * from the reference's norm as nsg_linear_fold's does.  1 <= M <= 160,
 * N % 4 == 0, K % 64 == 0, K >= 192, bf16 weights, x / w rows and sumsq_in
 * 16-byte aligned; nsg_lm_head_fold_supported(M, N, K, sumsq_parts) tells
 * whether a shape fits (M * sumsq_parts a multiple of 4, the partials within
 * one LDS ring slot, at most 64 partials: sumsq_parts <= 56 at 160 rows), else the calls return
 * NSG_ERR_UNSUPPORTED.
 * nsg_lm_head_fold: the logits, y (M x N, ldy elements apart, 8-byte aligned
 * rows); nsg_lm_head_fold_argmax: the greedy token of each row, as
 * nsg_linear_argmax (same workspace size and key rule), of those logits. */
int32_t nsg_lm_head_fold_supported(int32_t M, int32_t N, int32_t K, int32_t sumsq_parts);
int32_t nsg_lm_head_fold(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y,
                         int64_t ldy, int32_t M, int32_t N, int32_t K, const float* sumsq_in,
                         int32_t sumsq_parts, int32_t norm_dim, float eps, nsg_stream_t stream);
int32_t nsg_lm_head_fold_argmax(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                int32_t M, int32_t N, int32_t K, const float* sumsq_in,
                                int32_t sumsq_parts, int32_t norm_dim, float eps,
                                void* workspace, int64_t workspace_bytes, int64_t* tokens,
                                int64_t token_stride, nsg_stream_t stream);
/* nsg_lm_head_fold_argmax without the second launch: only the argmax keys
 * (M rows of *key_cols uint64 keys, written to keys, keys_bytes >=
 * nsg_linear_argmax_workspace_bytes(M, N)), for a consumer that reduces them
 * itself (nsg_embed_rows_keys, nsg_spec_accept_greedy_keys): the row's token
 * is the column of its largest key (0xffffffff - the key's low 32 bits),
 * the token nsg_lm_head_fold_argmax writes.  *key_cols (at most
 * 4 * ceil(N / 128)) depends only on M, N and the device. */
int32_t nsg_lm_head_fold_keys(const void* x, int64_t ldx, const void* w, int64_t ldw, int32_t M,
                              int32_t N, int32_t K, const float* sumsq_in, int32_t sumsq_parts,
                              int32_t norm_dim, float eps, void* keys, int64_t keys_bytes,
                              int32_t* key_cols, nsg_stream_t stream);

/* Embedding rows: out[r] = table[ids[b * id_stride_b + j * id_stride_j]] for
 * r = b * per_batch + j (embed_tokens(input_ids), causal_lm.py:613, on an index view
 * of any strides); ids outside [0, vocab) read the nearest valid row (the
 * reference's lookup would fault).  With sumsq_out, also the per-16-column
 * sums of squares of every row in nsg_row_sumsq's layout, for a folded
 * RMSNorm's first consumer. */
int32_t nsg_embed_rows(const int64_t* ids, int64_t id_stride_b, int64_t id_stride_j,
                       int32_t batch, int32_t per_batch, const void* table, int64_t ld_table,
                       int32_t vocab, int32_t hidden, void* out, int64_t ld_out,
                       float* sumsq_out, nsg_stream_t stream);
/* nsg_embed_rows where column key_j of the ids is the greedy token of the
 * previous lm_head call (its argmax keys, nsg_lm_head_fold_keys: keys row b,
 * key_cols keys): for every b, ids[b * id_stride_b + key_j * id_stride_j] =
 * that token is written, then its row looked up with the others.  The draft
 * model's next input (speculative.py:95-100, 104-109) without a launch of
 * its own. */
int32_t nsg_embed_rows_keys(int64_t* ids, int64_t id_stride_b, int64_t id_stride_j,
                            int32_t batch, int32_t per_batch, int32_t key_j, const void* keys,
                            int32_t key_cols, const void* table, int64_t ld_table, int32_t vocab,
                            int32_t hidden, void* out, int64_t ld_out, float* sumsq_out,
                            nsg_stream_t stream);

/* ------------------------------------------------------------------------
 * Philox4x32-10 uniforms: out[i] = u(seed, stream_id, offset + i) with
 * u = (word >> 8) * 2^-24 and word n of a stream = component n % 4 of
 * philox(ctr = [n/4 lo, n/4 hi, stream_id, 0], key = [seed lo, seed hi]).
 * Supplies the verify step's uniforms in place of torch.rand
 * (nano_sglang/decode/speculative.py:150).
 * ---------------------------------------------------------------------- */
int32_t nsg_philox_uniform(uint64_t seed, uint32_t stream_id, uint64_t offset, int64_t n,
                           float* out, nsg_stream_t stream);

/* ------------------------------------------------------------------------
 * Host gate.  No single reference line: the reference's step loop is
 * synchronous (read a step's results, build the next inputs, launch; its
 * engine around nano_sglang/decode/speculative.py:50-184).  These let an
 * engine queue step s + 1 while step s runs and release it once the host has
 * written step s + 1's inputs.
 *
 * nsg_host_gate_alloc: a 64-byte coherent pinned host word pair, zeroed;
 *   *flag is a host pointer the GPU can also read.  nsg_host_gate_free frees it.
 * nsg_host_gate_wait: enqueues one small kernel that waits until *flag != 0
 *   (system-scope reads), copies nbytes (a multiple of 16, both pointers
 *   16-byte aligned; 0 = no copy) from the pinned host buffer src_host to
 *   the device buffer dst, then writes *flag = 0.  After timeout_us (at most
 *   60 s) it stops waiting, sets bit 0 of the device word *err, copies and
 *   returns: the work queued after it then runs on whatever inputs are there.
 * The host raises the flag with a plain store of 1 after writing the inputs
 * (and not again before the gate has run).
 * ---------------------------------------------------------------------- */
/* nsg_export_step: n_host[i] = n_emitted[i] (i < rows) and emitted_host[i] =
 * emitted[i] (i < rows * cols), by one kernel (graph-capturable) writing
 * straight into pinned host memory: a step's emitted counts and tokens for
 * the host, without copy commands after the step.  Then, when done_host is
 * not NULL (a word from nsg_host_gate_alloc), *done_host = 1 once those
 * stores are visible to the host: the host may poll it instead of waiting
 * on an event, and clears it before the next use. */
int32_t nsg_export_step(const int32_t* n_emitted, const int64_t* emitted, int32_t rows,
                        int32_t cols, int32_t* n_host, int64_t* emitted_host, int32_t* done_host,
                        nsg_stream_t stream);
int32_t nsg_host_gate_alloc(int32_t** flag);
int32_t nsg_host_gate_free(int32_t* flag);
int32_t nsg_host_gate_wait(int32_t* flag, int32_t* err, int64_t timeout_us,
                           const void* src_host, void* dst, int64_t nbytes, nsg_stream_t stream);

/* A host gate that copies only n_segs (<= 8) byte ranges [seg_offsets[i],
 * + seg_bytes[i]) of the nbytes-byte staging buffer (16-byte multiples), in
 * place, with several workgroups: a step's staging holds fixed-capacity
 * arrays (page ids per attention call) of which a step uses a prefix, and one
 * workgroup pulls host memory at about 10 KB per microsecond.  The queued
 * work is held until *flag >= target (target >= 1): the host releases it by
 * writing target (or more) to the flag word, which this gate never resets,
 * so the host's targets must grow from call to call (a word used with
 * nsg_host_gate_wait, which waits for non-zero and resets, must not be
 * shared with it).  Timeout and error bit as nsg_host_gate_wait.  No
 * reference counterpart (the reference's loop is synchronous); it serves the
 * same pipelined loop. */
int32_t nsg_host_gate_wait_segments(int32_t* flag, int32_t target, int32_t* err,
                                    int64_t timeout_us, const void* src_host, void* dst,
                                    int64_t nbytes, const int64_t* seg_offsets,
                                    const int64_t* seg_bytes, int32_t n_segs,
                                    nsg_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NSG_SPEC_H */
