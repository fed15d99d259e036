// Verify attention for gfx950: ragged multi-query attention of the draft's
// k tokens plus the bonus token against the NHD paged KV cache, with GQA and
// the bottom-right causal rule.  The same kernel serves decode (q_len = 1),
// verify (q_len = k + 1) and chunked prefill (any q_len).
//
// Reference semantics: nano_sglang/model/causal_lm.py:359-471 (the PyTorch
// packed-attention fallbacks that define what the FlashInfer call at
// causal_lm.py:340 computes); KV layout nano_sglang/engine/paged_kv_cache.py:
// 60-69; page table nano_sglang/engine/engine.py:419-448.
//
// Work decomposition (planned on the host, nsg_attn_plan):
//   one workgroup = (request, query tile, KV split) x one KV head.
//   A query tile holds up to 64 query rows = q_tile_tokens x GQA group,
//   row rho -> (token rho / G, head-in-group rho % G), padded to 16-row MFMA
//   tiles.  Long KV ranges are split; split workgroups write partial
//   (O, m, l) rows and a second, small launch merges them.  No workgroup
//   waits on another inside a launch: on gfx950 a cross-workgroup handshake
//   needs agent-scope fences, which write back and invalidate the XCD's L2.
//
// Inside a workgroup wave w owns query rows [16w, 16w+16) of the tile.  The
// workgroup walks its KV range in 32-token steps; per step:
//   - all threads load the NEXT step's K and V rows (16-byte coalesced loads
//     of NHD page rows) into registers, overlapping this step's math;
//   - each wave computes S^T = K Q^T with v_mfma_f32_16x16x32_bf16
//     (M = 16 tokens, N = 16 query rows, K = head dim; K fragments read from
//     LDS with ds_read_b128), so each lane holds 4 tokens of ONE query row and
//     the row max / sum need two cross-lane steps;
//   - P^T, converted to bf16 in registers, is already the B operand of
//     O^T += V^T P^T (M = head dim, N = query rows, K = 32 tokens); V^T comes
//     from the LDS tile in the same token order;
//   - the prefetched registers go to the other LDS buffer; one barrier.
#include <algorithm>
#include <numeric>
#include <type_traits>
#include <cstdarg>
#include <vector>

#include "common.hpp"

namespace nsg {
namespace {

constexpr int kThreads = 256;         // merge kernel
constexpr int kMinSplitSteps = 4;     // 32-token steps per KV split, at least
// ... per KV group in the latency regime, where a split costs a merge launch
// (~4 us) and a step of a group ~0.35 us
constexpr int kMinGroupSteps = 8;
constexpr int kTokIt = 32;           // KV tokens per wave step
constexpr float kMaskVal = -1.0e30f; // finite "minus infinity" (no inf - inf)
constexpr int64_t kHeaderBytes = 256;  // flags word + padding
constexpr int kTargetWgPerCu = 8;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef short v8i16 __attribute__((ext_vector_type(8)));

struct AttnParams {
  const bf16* q;
  const bf16* kc;
  const bf16* vc;
  bf16* out;
  const int* qo_indptr;
  const int* kv_indptr;
  const int* kv_indices;
  const int* kv_last;
  const int* work;
  int num_work;
  int Hq, Hkv, G, log2P, num_pages, causal;
  float scale_log2;
  int* flags;
  float* partials;
};

__device__ __forceinline__ bf16x8 load_bf16x8(const bf16* p) {
  u32x4 v = *reinterpret_cast<const u32x4*>(p);
  return __builtin_bit_cast(bf16x8, v);
}

typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16 pair (v_cvt_pk_bf16_f32, round to nearest even).
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(floatx2{lo, hi}, bf16x2));
}

// Transposing LDS reads of the V^T fragments, in asm.  Written through the
// builtin, every such read after a global_load_lds gets a conservative
// vmcnt(0) from the compiler (it cannot tell the read from the ring slots
// still being filled), which stalls each step until every copy in flight has
// landed; the ring's own waits (vmcnt per step plus the barrier) already
// order these reads.  tr_issue starts the two reads of one d tile; tr_wait
// waits until at most N LDS operations are outstanding, after which the
// tile's registers (tied operands, so that the compiler reads them only
// after the wait) hold the data.  LDS operations complete in order, so the
// reads of tile dt are done once those of tile dt + 1 are the only ones left.
__device__ __forceinline__ void tr_issue(v4i16& lo, v4i16& hi, uint32_t a0, uint32_t a1) {
  asm volatile("ds_read_b64_tr_b16 %0, %2\n\tds_read_b64_tr_b16 %1, %3"
               : "=&v"(lo), "=&v"(hi)
               : "v"(a0), "v"(a1)
               : "memory");
}
template <int N>
__device__ __forceinline__ void tr_wait(v4i16& lo, v4i16& hi) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(lo), "+v"(hi) : "n"(N) : "memory");
}


// LDS tile swizzles: 16-byte chunk c of token row t is stored at physical
// chunk c ^ swz(t).  K fragments read one logical chunk of 16 consecutive
// tokens (needs distinct banks across t).  A V^T transposing read takes one
// 32-byte chunk pair from each of 16 rows t = 4g + j (g, j < 4): the pair
// index is XORed with a function of t that spreads those 16 rows over every
// 32-byte bank window (with 256-byte bank rows: 2 rows per window, the
// minimum).
template <int D>
__device__ __forceinline__ int swz_k(int t) {
  if constexpr (D == 64) return (t >> 1) & 7;  // 128-byte rows: two rows per bank cycle
  return t & 15;                               // 256-byte rows: one row per bank cycle
}
template <int D>
__device__ __forceinline__ int swz_v(int t) {
  if constexpr (D == 64) return 2 * ((t >> 1) & 3);  // odd rows sit in the other half-row
  return 2 * (t & 7);
}

constexpr float kLazyRescale = 8.f;  // rescale O only when a row max grows by > 2^8

// LDS ring depth.  With one KV group a shallower ring lets more workgroups
// (waves) share a CU, which hides more latency (measured: depth 3 beats 4 by
// ~8 % on the large shape); depth - 1 steps are in flight ahead of the math.
// With several KV groups (latency regime) the rings take all 160 KB of the
// CU's LDS, 5 slots per group, and a group issues all of its first 5 steps
// at once: up to 5 * 32 tokens per group, i.e. 640 tokens of an item at head
// dim 64, arrive in one memory round trip (a 4-deep ring with 3 steps ahead
// needed a second round trip, ~2 us, for items past 384 tokens).
constexpr int kRingOne = 3;
constexpr int kRingGroups = 5;
constexpr int ring_depth(int KS) { return KS == 1 ? kRingOne : kRingGroups; }
// KV groups per workgroup in the latency regime: as many 5-deep rings as fit
// 160 KB of LDS (8 KB per step at head_dim 64, 16 KB at 128).
constexpr int kv_groups_max(int D) { return D == 64 ? 4 : 2; }
constexpr int kLdsBytes = 160 * 1024;
constexpr int kMaxItemPages = 1024; // page ids one work item may span
// Pages of at least 16 tokens for several KV groups: a 32-token step then
// spans at most two pages, looked up with two scalar loads.
constexpr int kMinGroupPage = 16;

// One workgroup = one work item x one KV head.  Its KS * RT waves form KS
// groups of RT; group g takes the g-th contiguous share of the item's 32-token
// KV steps, and wave w of a group owns query rows [16w, 16w + 16) of the
// item's query tile.  KS > 1 is the latency regime (few, short items: the
// verify and draft steps of a decode batch): the groups run side by side and
// their partial results meet in LDS, so the item needs neither a second
// launch nor more sequential steps per wave.
// With one KV group the item's page ids are staged in LDS once; with
// several the rings fill the LDS, and each DMA instruction's page id (one
// page per instruction: its token rows are 8 (head dim 64) or 4 (128)
// consecutive tokens of a 32-aligned step) is a wave-uniform scalar load,
// issued for all first steps before any copy.  K and V rows of each step go
// straight from HBM to a ring slot of the group with global_load_lds_dwordx4
// (no staging registers) ahead of the math; an explicit vmcnt wait per step
// (plus a raw s_barrier when a group has several waves) keeps the ring full
// (__syncthreads would drain it).  Every group iterates the same number of
// steps (idle ones do nothing but the barrier), so the workgroup-wide barrier
// stays matched.
template <int D, int RT, int KS>
__global__ __launch_bounds__(RT * KS * 64) void verify_attn_kernel(AttnParams p) {
  constexpr int KC = D / 32;              // K-dim chunks of QK^T
  constexpr int DT = D / 16;              // d tiles of PV
  constexpr int ROWS = RT * 16;
  constexpr int CPR = D / 8;              // 16-byte chunks per token row
  constexpr int TILE = kTokIt * D;        // bf16 per K (or V) tile
  constexpr int NINST = 2 * TILE / 512;   // 1 KB DMA instructions per step (K + V)
  constexpr int TPI = 64 / CPR;           // token rows per DMA instruction
  constexpr int NI = (NINST + RT - 1) / RT;  // DMA instructions per wave per step
  constexpr int PSTRIDE = D + 4;          // partial row: O[D], m, l, 2 pad
  constexpr int NTHR = RT * KS * 64;
  constexpr int kNBuf = ring_depth(KS);
  // Cache policy of the K / V copies: non-temporal (the pool is streamed
  // once) for one or two KV groups -- measured 321 -> 301 us at the large
  // shape (one group), 30.7 -> 29.4 us for head dim 128 verify steps (two
  // groups) -- but the default policy for the four groups of head dim 64,
  // where non-temporal measured 9.8 -> 10.7 us at the verify shape.
  constexpr int kDmaPolicy = KS <= 2 ? 2 : 0;  // 2: the nt bit
  // steps issued before the first wait: all ring slots with several groups,
  // all but one with one group (that slot is filled at the first iteration)
  constexpr int PF = KS > 1 ? kNBuf : kNBuf - 1;
  constexpr int kRingBytes = KS * kNBuf * 2 * TILE * 2;
  constexpr int kPageBytes = KS == 1 ? kMaxItemPages * 4 : 0;
  static_assert(kRingBytes + kPageBytes <= kLdsBytes, "LDS budget");
  // One KV group: typed arrays.  Several: one 160 KB block (rings only, no
  // room for the 4-byte minimum of a second array).  With the block, the
  // compiler cannot tell the rings' reads from their pending copies and
  // waits for every copy before each transposing read; the typed rings of
  // one group keep it from doing so (measured: the one-group kernel at the
  // large shape 307 us typed, 351 us with the block), and the several-group
  // kernel reads V^T in asm instead.
  bf16 (*ring)[kNBuf][2][TILE];
  int* s_pages;
  if constexpr (KS == 1) {
    __shared__ __attribute__((aligned(16))) bf16 ring1[1][kNBuf][2][TILE];
    __shared__ int pages1[kMaxItemPages];
    ring = ring1;
    s_pages = pages1;
  } else {
    __shared__ __attribute__((aligned(16))) unsigned char ringg[kRingBytes];
    ring = reinterpret_cast<bf16 (*)[kNBuf][2][TILE]>(ringg);
    s_pages = nullptr;
  }

  // blockIdx.x = KV head (fastest), so the Hkv workgroups of one work item
  // are dispatched together and read the interleaved head slices of the same
  // NHD token rows close in time (DRAM row locality).
  const int wi = blockIdx.y;
  if (wi >= p.num_work) return;
  const int h = blockIdx.x;
  // Work item (host-precomputed, so the first loads need no index chase):
  // [first query token, query tokens, KV limit of the tile's first row,
  //  first page-table entry, KV begin, KV end, splits, -]
  const int* wk = p.work + (size_t)wi * NSG_ATTN_WORK_INTS;
  const int qs = wk[0], qn = wk[1], lim0 = wk[2], pb = wk[3], kvb = wk[4], kve = wk[5];
  const int nsplit = wk[6];
  if (qn == 0) return;  // padding item of a fixed-size (graph-captured) work list
  const int P = 1 << p.log2P;
  const int G = p.G;
  const int nrows = qn * G;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wid / RT;   // KV group
  const int wave = wid % RT;  // row tile inside the group
  const int r16 = lane & 15;
  const int g4 = lane >> 4;

  // ---- one KV group: stage the item's page ids in LDS ----
  const int page0 = kvb >> p.log2P;
  const int npages = kve > kvb ? ((kve - 1) >> p.log2P) - page0 + 1 : 0;
  if constexpr (KS == 1)
    for (int i = tid; i < npages; i += NTHR) s_pages[i] = p.kv_indices[pb + page0 + i];

  // ---- this group's share of the item's 32-token steps ----
  const int n_all = (kve - kvb + kTokIt - 1) / kTokIt;  // steps of the item
  const int per = (n_all + KS - 1) / KS;                // steps per group (loop count)
  const int n_it = max(0, min(per, n_all - grp * per)); // this group's real steps
  const int gkvb = kvb + grp * per * kTokIt;            // this group's first token
  const int last_tok = kve - 1;

  // ---- this lane's query row (B operand of S^T = K Q^T) and causal limit ----
  const int row = wave * 16 + r16;
  const bool row_ok = row < nrows;
  const int tau = row / G;
  const int gam = row - tau * G;
  const int lim = row_ok ? lim0 + (p.causal ? tau : 0) : -1;
  bf16x8 qf[KC];
  {
    // (padding rows load the tile's first row -- real data, their scores are
    // all masked: lim = -1 -- so that every lane loads unconditionally)
    const bf16* qrow = p.q + (row_ok ? ((size_t)(qs + tau) * p.Hq + h * G + gam) * D
                                     : ((size_t)qs * p.Hq + h * G) * D);
#pragma unroll
    for (int c = 0; c < KC; ++c) qf[c] = load_bf16x8(qrow + 32 * c + 8 * g4);
  }
  // Several KV groups: the page ids of the group's first 64 pages, one per
  // lane (lookups past the item's range read its last page), in one vector
  // load beside Q's; the copies take them with v_readlane.
  const int gpage0 = min(gkvb, last_tok) >> p.log2P;
  int vpages = 0;
  if constexpr (KS > 1) vpages = p.kv_indices[pb + min(gpage0 + lane, last_tok >> p.log2P)];
  // Q must have landed before the first copy is issued, and the compiler
  // must see it: an empty asm statement that reads Q makes it wait here (Q and
  // the page ids arrive in the same round trip).  Left to itself it keeps Q
  // pending and, since the copies issued after Q vary by path, waits for
  // every copy in flight (vmcnt 0) before each step's first MFMA -- which
  // turned the ring into one memory round trip per step.
#pragma unroll
  for (int c = 0; c < KC; ++c) asm volatile("" ::"v"(__builtin_bit_cast(u32x4, qf[c])));
  if constexpr (KS == 1) __syncthreads();  // page ids visible; nothing is in flight besides Q

  floatx4 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = kMaskVal, l_run = 0.f;  // m_run: exponent base (lazily raised)

  const size_t head_off = (size_t)h * D;
  const size_t tok_stride = (size_t)p.Hkv * D;
  bool bad_page = false;
  // Dummy source for lanes past the item's end or with a bad page id: the
  // item's first token row (real, finite data); its value is masked out.
  // (one KV group only; with several, lanes past the end copy the item's
  // last token row instead -- see issue_pages)
  const int pg_first = KS == 1 && npages > 0 ? s_pages[0] : 0;
  const bf16* dummy_k = p.kc + ((size_t)((unsigned)pg_first < (unsigned)p.num_pages ? pg_first : 0) * P +
                                (kvb & (P - 1))) * tok_stride + head_off;
  const bf16* dummy_v = p.vc + (dummy_k - p.kc);

  // Per-lane LDS read offsets (bf16 elements inside one K or V tile).
  //   K fragment c of sub-tile s: token 16 s + r16, logical chunk 4 c + g4.
  //   V^T fragment dt: rows 4 g4 + j (+16), column dt * 16 + r16.
  int koff[KC];
#pragma unroll
  for (int c = 0; c < KC; ++c) koff[c] = r16 * D + (((4 * c + g4) ^ swz_k<D>(r16)) * 8);
  // V^T fragments come from ds_read_b64_tr_b16: within each 16-lane group,
  // result element j of lane i is element i % 4 of the 8 bytes addressed by
  // lane 4 j + i / 4.  So lane (r16, g4) addresses token row
  // 4 g4 + r16 / 4 (+ 16 for elements 4..7), columns 16 dt + 4 (r16 % 4) ..
  // + 3, and receives V[4 g4 + j][16 dt + r16], j = 0..3 -- the token order
  // of the P^T operand.  Offsets are in bf16 elements, swizzle applied.
  int vtr[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int t = 16 * hh + 4 * g4 + (r16 >> 2);
      const int c = 16 * dt + 4 * (r16 & 3);
      vtr[dt][hh] = t * D + (((c >> 3) ^ swz_v<D>(t)) << 3) + (c & 7);
    }

  // Loop-invariant parts of this lane's DMA copies: token row inside the
  // step, source offset inside the token's head slice, and LDS destination.
  int d_t[NI];
  int d_off[NI];
  int d_lds[NI];
  bool d_v[NI];
  bool d_hi[NI];  // the copy's rows are tokens 16..31 of the step
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int j = (wave + RT * i) % NINST;      // padding repeats a real copy
    const int which = j / (NINST / 2);
    const int jj = j - which * (NINST / 2);
    const int t = jj * TPI + lane / CPR;        // token row inside the step
    const int pc = lane % CPR;                   // physical chunk written by this lane
    const int lc = pc ^ (which ? swz_v<D>(t) : swz_k<D>(t));  // logical chunk it carries
    d_t[i] = t;
    d_off[i] = lc * 8;
    d_lds[i] = which * TILE + jj * TPI * D;
    d_v[i] = which != 0;
    d_hi[i] = jj * TPI >= 16;  // (16 is a multiple of TPI: a copy never straddles)
  }
  // Pages of at least 16 tokens: a step (32 tokens from a multiple of 32)
  // spans at most two pages, and each copy's offset inside its page is fixed,
  // so a step needs two page ids and one multiply-add per copy.  Measured to
  // pay only for single-wave groups (one wave issues all of a step's copies);
  // with several waves per group the per-copy lookup is faster.
  const bool big_pages = RT == 1 && P >= 16;
  int d_pg[NI];          // which of the step's two pages (big pages)
  int64_t d_inpage[NI];  // element offset of the copy inside its page (big pages)
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    d_pg[i] = P < kTokIt ? (d_t[i] >> p.log2P) : 0;
    d_inpage[i] = (int64_t)(d_t[i] & (P - 1)) * (int64_t)tok_stride + (int64_t)head_off + d_off[i];
  }
  const int64_t page_elems = (int64_t)P * (int64_t)tok_stride;
  // Several KV groups (pages of 16+ tokens, which the planner requires for
  // them): a 32-token step spans at most two pages, the pages of its first
  // and second 16 tokens (equal for pages of 32+).  Past the group's first 64
  // pages (items over 4096 tokens at head dim 64, 2048 at 128: long
  // fixed-bound plans only) a wave-uniform scalar load reads them.
  auto page_at = [&](int t) {
    const int pg = min(t, last_tok) >> p.log2P;
    const int idx = pg - gpage0;
    if (idx < 64) return __builtin_amdgcn_readlane(vpages, idx);
    // an explicit scalar load: as a plain load the compiler would hoist it
    // above the branch and wait for it on every refill
    // (the address through readfirstlane: uniform by construction, which an
    // "s" operand needs even where the compiler cannot prove it)
    const uint64_t a = reinterpret_cast<uint64_t>(p.kv_indices + pb + pg);
    const uint64_t au = (uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)a) |
                        ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) << 32);
    int v;
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(au) : "memory");
    return v;
  };
  // ... and the copies themselves, given those page ids.  The page part of
  // each address is wave-uniform (scalar arithmetic, once per step); a lane
  // adds its fixed byte offset inside the step (row d_t & (P - 1) of its page:
  // the step starts at a multiple of 32, so rows 16..31 fall on the second
  // page exactly when pages hold 16 tokens).  A lane past the item's end
  // copies the step's first row instead: real, finite data, masked out (a
  // P = 0 weight on a non-finite V row would still give NaN).  A bad page id
  // copies from the pool's first page and raises the flag.
  uint32_t lo_row[NI], lo_end[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    lo_row[i] = (uint32_t)((((size_t)(d_t[i] & (P - 1))) * tok_stride + head_off + d_off[i]) * 2);
    lo_end[i] = (uint32_t)((head_off + d_off[i]) * 2);
  }
  const uint64_t page_bytes = (uint64_t)P * tok_stride * 2;
  auto issue_pages = [&](int it, int slot, int pga, int pgb) {
    const int t0 = gkvb + it * kTokIt;
    const bool oka = (unsigned)pga < (unsigned)p.num_pages;
    const bool okb = (unsigned)pgb < (unsigned)p.num_pages;
    bad_page |= !oka || !okb;  // both ids are of tokens in the range
    const uint32_t rowb = (uint32_t)(t0 & (P - 1)) * (uint32_t)(tok_stride * 2);  // < one page
    const uint64_t offa = oka ? (uint64_t)(uint32_t)pga * page_bytes : 0;
    const uint64_t offb = okb ? (uint64_t)(uint32_t)pgb * page_bytes : 0;
    if (t0 + kTokIt - 1 <= last_tok) {
      // a full step (every step but an item's last): the address is a
      // wave-uniform page base plus the lane's fixed 32-bit offset, so each
      // copy is one instruction with a scalar base
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const char* base =
            reinterpret_cast<const char*>(d_v[i] ? p.vc : p.kc) + (d_hi[i] ? offb : offa) + rowb;
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(base + lo_row[i]),
                                         static_cast<void*>(&ring[grp][slot][0][0] + d_lds[i]),
                                         16, 0, kDmaPolicy);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const char* base = reinterpret_cast<const char*>(d_v[i] ? p.vc : p.kc);
      const bool in = t0 + d_t[i] <= last_tok;
      const char* src =
          base + ((in && d_hi[i]) ? offb : offa) + ((in ? lo_row[i] : lo_end[i]) + rowb);
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(src),
                                       static_cast<void*>(&ring[grp][slot][0][0] + d_lds[i]), 16,
                                       0, kDmaPolicy);
    }
  };
  // One KV group: issue this wave's DMA instructions for step `it` into ring
  // slot `slot`, page ids from LDS.
  auto issue = [&](int it, int slot) {
    const int t0 = gkvb + it * kTokIt;
    const bool full = t0 + kTokIt <= kve;  // no token of the step past the range
    int pg0 = 0, pg1 = 0;
    int64_t shift = 0;
    if (big_pages && full) {
      const int pidx = (t0 >> p.log2P) - page0;
      pg0 = s_pages[pidx];
      pg1 = P < kTokIt ? s_pages[pidx + 1] : pg0;
      shift = P > kTokIt ? (int64_t)(t0 & (P - 1)) * (int64_t)tok_stride : 0;
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const bf16* src = d_v[i] ? dummy_v : dummy_k;
      if (big_pages && full) {
        const int page = d_pg[i] ? pg1 : pg0;
        if ((unsigned)page < (unsigned)p.num_pages) {
          src = (d_v[i] ? p.vc : p.kc) + (int64_t)page * page_elems + shift + d_inpage[i];
        } else {
          bad_page = true;
        }
      } else {
        const int tok = t0 + d_t[i];
        if (tok < kve) {
          const int page = s_pages[(tok >> p.log2P) - page0];
          if ((unsigned)page < (unsigned)p.num_pages) {
            src = (d_v[i] ? p.vc : p.kc) + ((size_t)page * P + (tok & (P - 1))) * tok_stride +
                  head_off + d_off[i];
          } else {
            bad_page = true;
          }
        }
      }
      // void* operands: with typed pointers the host pass silently drops the
      // kernel stubs of this template
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(src),
                                       static_cast<void*>(&ring[grp][slot][0][0] + d_lds[i]), 16,
                                       0, kDmaPolicy);
    }
  };

  if constexpr (KS > 1) {
    // the first PF steps lie within the first 64 pages (PF * 32 tokens in
    // pages of 16+)
    static_assert(PF * kTokIt / kMinGroupPage <= 64, "prefetched steps within the lane pages");
    // (all ids read before any copy: one wait for the page-id load on every path)
    int pga[PF], pgb[PF];
#pragma unroll
    for (int it = 0; it < PF; ++it) {
      const int t0 = gkvb + it * kTokIt;
      pga[it] = __builtin_amdgcn_readlane(vpages, (min(t0, last_tok) >> p.log2P) - gpage0);
      pgb[it] = __builtin_amdgcn_readlane(vpages, (min(t0 + 16, last_tok) >> p.log2P) - gpage0);
    }
#pragma unroll
    for (int it = 0; it < PF; ++it)
      if (it < n_it) issue_pages(it, it, pga[it], pgb[it]);
  } else {
#pragma unroll
    for (int it = 0; it < PF; ++it)
      if (it < n_it) issue(it, it);
  }

  // Groups of one wave have no barrier inside the loop and run only their
  // own steps; the waves of a larger group all run `per` iterations so that
  // their barriers stay matched.
  const int n_loop = RT == 1 ? n_it : per;
  for (int it0 = 0; it0 < n_loop; it0 += kNBuf) {
#pragma unroll
    for (int slot = 0; slot < kNBuf; ++slot) {  // unrolled: ring slot is a constant
      const int it = it0 + slot;
      if (it >= n_loop) break;
      const bool real = RT == 1 || it < n_it;
      if (real) {
        // Steps issued so far: min(n_it, max(PF, it + kNBuf - 1)); wait until
        // at most those after `it` are in flight.  With several groups (PF =
        // kNBuf) that is min(steps left, kNBuf - 2) past the first iteration,
        // which the common case settles with one compare.
        const int left = n_it - 1 - it;
        if (KS > 1 && (slot > 0 || it0 > 0))
          wait_steps<NI, kNBuf - 2>(min(left, kNBuf - 2));
        else
          wait_steps<NI, PF - 1>(min(n_it, max(PF, it + kNBuf - 1)) - 1 - it);
      }
      if constexpr (RT > 1) {
        // step `it` landed for every wave of the group and slot (it - 1) is
        // free; the empty asm statements keep the compiler from moving LDS
        // accesses across the raw barrier (which, unlike __syncthreads, does
        // not drain the ring)
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
      }
      // refill the slot consumed at iteration it - 1 (free after the barrier)
      if (it + kNBuf - 1 >= PF && it + kNBuf - 1 < n_it) {
        if constexpr (KS > 1) {
          const int t0 = gkvb + (it + kNBuf - 1) * kTokIt;
          issue_pages(it + kNBuf - 1, (slot + kNBuf - 1) % kNBuf, page_at(t0), page_at(t0 + 16));
        } else {
          issue(it + kNBuf - 1, (slot + kNBuf - 1) % kNBuf);
        }
      }
      if (!real) continue;

      const int t0 = gkvb + it * kTokIt;
      const bf16* Kt = ring[grp][slot][0];
      const bf16* Vt = ring[grp][slot][1];

      // ---- S^T = K Q^T: lane holds tokens 16s + 4*g4 + i of query row r16 ----
      floatx4 sacc[2];
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < KC; ++c) {
          const bf16x8 kf = *reinterpret_cast<const bf16x8*>(&Kt[16 * s2 * D + koff[c]]);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[c], acc, 0, 0, 0);
        }
        sacc[s2] = acc;
      }

      float pv[8];
      if constexpr (KS == 1) {
        // ---- online softmax (base 2) with lazy rescaling (one KV group: the
        //      plain form, which keeps the head-dim-128 kernel at 3 waves per
        //      SIMD; the form below needs more registers) ----
        float sv[8];
        if (t0 + kTokIt - 1 <= lim0 && t0 + kTokIt <= kve) {
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
            for (int i = 0; i < 4; ++i) sv[4 * s2 + i] = sacc[s2][i] * p.scale_log2;
        } else {
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int j = t0 + 16 * s2 + 4 * g4 + i;
              sv[4 * s2 + i] = (j <= lim && j < kve) ? sacc[s2][i] * p.scale_log2 : kMaskVal;
            }
          }
        }
        float mx = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                         fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const bool grow = mx > m_run + kLazyRescale;
        if (__builtin_amdgcn_ballot_w64(grow)) {
          const float mnew = grow ? mx : m_run;
          const float alpha = __builtin_amdgcn_exp2f(m_run - mnew);
          m_run = mnew;
          l_run *= alpha;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
        }
        float ps = 0.f;
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          pv[x] = __builtin_amdgcn_exp2f(sv[x] - m_run);
          ps += pv[x];
        }
        l_run += ps;
      } else {
        // ---- online softmax (base 2) with lazy rescaling.  The max is taken
        //      over the raw scores and scaled once (the scale is positive); the
        //      scale folds into the exponent's FMA.  Masked scores get P = 0
        //      outright, and a row with nothing visible leaves its max alone
        //      (an FMA of a sentinel against a rounded sentinel max could give
        //      exp2 of a huge residue) ----
        auto softmax = [&](auto masked) {
          constexpr bool MASKED = decltype(masked)::value;
          float sv[8];
          bool vis[8];
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int j = t0 + 16 * s2 + 4 * g4 + i;
              vis[4 * s2 + i] = !MASKED || (j <= lim && j < kve);
              sv[4 * s2 + i] = vis[4 * s2 + i] ? sacc[s2][i] : kMaskVal;
            }
          }
          float mx = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                           fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
          mx = max_xor16_32(mx);
          mx = (MASKED && mx == kMaskVal) ? kMaskVal : mx * p.scale_log2;
          // Raise the exponent base only when a row max exceeds it by > 2^8, and
          // skip the O rescale entirely when no row of the wave needs it.
          const bool grow = mx > m_run + kLazyRescale;
          if (__builtin_amdgcn_ballot_w64(grow)) {
            const float mnew = grow ? mx : m_run;
            const float alpha = __builtin_amdgcn_exp2f(m_run - mnew);
            m_run = mnew;
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
          }
          float ps = 0.f;
#pragma unroll
          for (int x = 0; x < 8; ++x) {
            const float e = __builtin_amdgcn_exp2f(fmaf(sv[x], p.scale_log2, -m_run));
            pv[x] = MASKED && !vis[x] ? 0.f : e;
            ps += pv[x];
          }
          l_run += ps;
        };
        if (t0 + kTokIt - 1 <= lim0 && t0 + kTokIt <= kve) {
          // every row of the tile sees every token of the step (lim0 is the
          // tile's smallest causal limit): no mask
          softmax(std::false_type{});
        } else {
          softmax(std::true_type{});
        }
      }
      const bf16x8 pf = __builtin_bit_cast(
          bf16x8, u32x4{cvt_pk_bf16(pv[0], pv[1]), cvt_pk_bf16(pv[2], pv[3]),
                        cvt_pk_bf16(pv[4], pv[5]), cvt_pk_bf16(pv[6], pv[7])});

      // ---- O^T += V^T P^T; element e of lane group g4 is token
      //      4*g4 + e (e < 4) or 16 + 4*g4 + (e - 4), matching pf ----
      if constexpr (KS == 1) {
        // (the builtin: with typed rings the compiler adds no wait, and
        // interleaves the reads with the MFMAs itself)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) v4i16*)(Vt + vtr[dt][0]));
          const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) v4i16*)(Vt + vtr[dt][1]));
          const v8i16 w = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          oacc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, w), pf,
                                                             oacc[dt], 0, 0, 0);
        }
        continue;
      }
      // (reads of tile dt + 1 in flight while tile dt's MFMA issues)
      const uint32_t vbase = lds_addr(Vt);
      v4i16 rl[DT], rh[DT];
      tr_issue(rl[0], rh[0], vbase + 2 * vtr[0][0], vbase + 2 * vtr[0][1]);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        if (dt + 1 < DT) {
          tr_issue(rl[dt + 1], rh[dt + 1], vbase + 2 * vtr[dt + 1][0], vbase + 2 * vtr[dt + 1][1]);
          tr_wait<2>(rl[dt], rh[dt]);
        } else {
          tr_wait<0>(rl[dt], rh[dt]);
        }
        const v8i16 w = __builtin_shufflevector(rl[dt], rh[dt], 0, 1, 2, 3, 4, 5, 6, 7);
        oacc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, w), pf,
                                                           oacc[dt], 0, 0, 0);
      }
    }
  }

  if (bad_page) atomicOr(p.flags, 1);
  // ---- the 4 lane groups sharing query row r16 hold partial sums ----
  float l = sum_xor16_32(l_run);
  if constexpr (KS == 1) {
    if (!row_ok) return;
    if (nsplit == 1) {
      const float inv = l > 0.f ? 1.f / l : 0.f;
      bf16* orow = p.out + ((size_t)(qs + tau) * p.Hq + h * G + gam) * D + 4 * g4;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const floatx4 o = oacc[dt];
        *reinterpret_cast<u32x2*>(orow + dt * 16) =
            u32x2{cvt_pk_bf16(o[0] * inv, o[1] * inv), cvt_pk_bf16(o[2] * inv, o[3] * inv)};
      }
    } else {
      float* prow = p.partials + ((size_t)wi * p.Hkv + h) * ROWS * PSTRIDE + (size_t)row * PSTRIDE;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        *reinterpret_cast<floatx4*>(prow + dt * 16 + 4 * g4) = oacc[dt];
      if (g4 == 0) {
        prow[D] = m_run;
        prow[D + 1] = l;
      }
    }
  } else {
    // ---- combine the KV groups through LDS.  Every group writes its
    //      partial (O, m, l); group g then finishes the d tiles g, g + KS, ...
    //      of its rows from all KS partials, so every wave shares the
    //      combine and the output stores.  No branch depends on the group:
    //      its tiles are addressed, not selected. ----
    constexpr int SROW = D + 4;   // O[D], m, l, 2 pad
    constexpr int OWN = DT / KS;  // d tiles each group finishes
    static_assert(DT % KS == 0, "d tiles split evenly over the KV groups");
    // Single-wave groups write into their own ring, idle once the wave's
    // last step is read (all of its copies landed before that step), so one
    // barrier suffices; the waves of a larger group share a ring and wait for
    // each other first.
    float* sc = reinterpret_cast<float*>(&ring[0][0][0][0]);
    auto part = [&](int g) {
      return RT == 1 ? reinterpret_cast<float*>(&ring[g][0][0][0]) + (size_t)row * SROW
                     : sc + ((size_t)g * ROWS + row) * SROW;
    };
    static_assert(RT == 1 ? (size_t)ROWS * SROW * 4 <= (size_t)kNBuf * 2 * TILE * 2
                          : (size_t)KS * ROWS * SROW * 4 <= (size_t)kRingBytes,
                  "combine partials fit the rings");
    if constexpr (RT > 1) __syncthreads();
    {
      float* mine = part(grp);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        *reinterpret_cast<floatx4*>(mine + dt * 16 + 4 * g4) = oacc[dt];
      // (the four lane groups of a row hold the same m and l)
      *reinterpret_cast<floatx2*>(mine + D) = floatx2{m_run, l};
    }
    __syncthreads();
    // every group's (m, l) and this group's d tiles of every partial, read
    // in one batch
    float mg[KS], lg[KS];
    floatx4 og[KS][OWN];
#pragma unroll
    for (int g = 0; g < KS; ++g) {
      const float* o = part(g);
      const floatx2 ml = *reinterpret_cast<const floatx2*>(o + D);
      mg[g] = ml[0];
      lg[g] = ml[1];
#pragma unroll
      for (int j = 0; j < OWN; ++j)
        og[g][j] = *reinterpret_cast<const floatx4*>(o + (grp + KS * j) * 16 + 4 * g4);
    }
    float M = mg[0];
#pragma unroll
    for (int g = 1; g < KS; ++g) M = fmaxf(M, mg[g]);
    float lsum = 0.f;
    floatx4 acc[OWN];
#pragma unroll
    for (int j = 0; j < OWN; ++j) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < KS; ++g) {
      const float w = __builtin_amdgcn_exp2f(mg[g] - M);
      lsum += w * lg[g];
#pragma unroll
      for (int j = 0; j < OWN; ++j) acc[j] += w * og[g][j];
    }
    if (!row_ok) return;
    if (nsplit == 1) {
      const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
      bf16* orow = p.out + ((size_t)(qs + tau) * p.Hq + h * G + gam) * D + 4 * g4;
#pragma unroll
      for (int j = 0; j < OWN; ++j) {
        const floatx4 o = acc[j];
        *reinterpret_cast<u32x2*>(orow + (grp + KS * j) * 16) =
            u32x2{cvt_pk_bf16(o[0] * inv, o[1] * inv), cvt_pk_bf16(o[2] * inv, o[3] * inv)};
      }
    } else {
      float* prow = p.partials + ((size_t)wi * p.Hkv + h) * ROWS * PSTRIDE + (size_t)row * PSTRIDE;
#pragma unroll
      for (int j = 0; j < OWN; ++j)
        *reinterpret_cast<floatx4*>(prow + (grp + KS * j) * 16 + 4 * g4) = acc[j];
      if (g4 == 0 && grp == 0) {
        prow[D] = M;
        prow[D + 1] = lsum;
      }
    }
  }
}

// Merge of the split partials of one (request, query tile) group x KV head.
// A separate launch: partials written by workgroups on other XCDs become
// visible at the kernel boundary, so no in-kernel cross-workgroup fence (an
// L2 write-back + invalidate on gfx950) is needed.  Each thread owns one
// (row, 8-column) piece (blockIdx.z picks the group's kThreads-piece
// slice) and issues the loads of up to kMergeBatch splits at once, then
// combines them in split order: one memory round trip per kMergeBatch
// splits (a 4-deep rolling loop over a strided item loop took 11 us at the
// large shape: 64 groups x 8 heads, up to 7 splits).
constexpr int kMergeBatch = 8;

template <int D, int RT>
__global__ __launch_bounds__(kThreads) void verify_merge_kernel(AttnParams p, const int* merge,
                                                               int num_merge) {
  constexpr int ROWS = RT * 16;
  constexpr int PSTRIDE = D + 4;
  constexpr int CH = D / 8;  // 8-column pieces per row
  const int mi = blockIdx.x;
  if (mi >= num_merge) return;
  const int h = blockIdx.y;
  // merge item: [first query token, query tokens, first work item, splits, -...]
  const int* mw = merge + (size_t)mi * NSG_ATTN_WORK_INTS;
  const int qs = mw[0], qn = mw[1], wi0 = mw[2], nsplit = mw[3];
  if (nsplit < 2) return;  // padding item of a fixed-size (graph-captured) work list
  const int G = p.G;
  const int nrows = qn * G;
  const int item = (int)blockIdx.z * kThreads + (int)threadIdx.x;
  if (item >= nrows * CH) return;
  const int row = item / CH;
  const int c0 = (item - row * CH) * 8;
  const float* base = p.partials + ((size_t)wi0 * p.Hkv + h) * ROWS * PSTRIDE +
                      (size_t)row * PSTRIDE;
  const size_t sstride = (size_t)p.Hkv * ROWS * PSTRIDE;
  float M = kMaskVal, lsum = 0.f;
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < nsplit; s0 += kMergeBatch) {
    floatx4 ml[kMergeBatch], a[kMergeBatch], b[kMergeBatch];
#pragma unroll
    for (int j = 0; j < kMergeBatch; ++j) {  // splits past nsplit re-read the last one
      const float* prow = base + min(s0 + j, nsplit - 1) * sstride;
      ml[j] = *reinterpret_cast<const floatx4*>(prow + D);  // m, l, pad, pad
      a[j] = *reinterpret_cast<const floatx4*>(prow + c0);
      b[j] = *reinterpret_cast<const floatx4*>(prow + c0 + 4);
    }
#pragma unroll
    for (int j = 0; j < kMergeBatch; ++j) {
      if (s0 + j >= nsplit) break;
      const float Mn = fmaxf(M, ml[j][0]);
      const float sc = __builtin_amdgcn_exp2f(M - Mn);
      const float wt = __builtin_amdgcn_exp2f(ml[j][0] - Mn);
      lsum = lsum * sc + wt * ml[j][1];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[i] = o[i] * sc + wt * a[j][i];
        o[4 + i] = o[4 + i] * sc + wt * b[j][i];
      }
      M = Mn;
    }
  }
  const int tau = row / G;
  const int gam = row - tau * G;
  bf16* orow = p.out + ((size_t)(qs + tau) * p.Hq + h * G + gam) * D + c0;
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  *reinterpret_cast<u32x4*>(orow) =
      u32x4{cvt_pk_bf16(o[0] * inv, o[1] * inv), cvt_pk_bf16(o[2] * inv, o[3] * inv),
            cvt_pk_bf16(o[4] * inv, o[5] * inv), cvt_pk_bf16(o[6] * inv, o[7] * inv)};
}

template <int D, int RT>
int32_t launch_rt(const nsg_attn_plan_t* plan, const AttnParams& prm, const int* merge,
                  hipStream_t stream) {
  const dim3 grid(plan->num_kv_heads, plan->num_work);
  constexpr int KSX = kv_groups_max(D);
  if (plan->kv_groups == KSX) {
    hipLaunchKernelGGL((verify_attn_kernel<D, RT, KSX>), grid, dim3(RT * KSX * 64), 0, stream, prm);
  } else if (plan->kv_groups == 1) {
    hipLaunchKernelGGL((verify_attn_kernel<D, RT, 1>), grid, dim3(RT * 64), 0, stream, prm);
  } else {
    set_error("kv_groups %d not supported for head_dim %d", plan->kv_groups, D);
    return NSG_ERR_ARG;
  }
  int32_t rc = launch_status("verify_attn_kernel");
  if (rc || plan->num_merge == 0) return rc;
  constexpr int kSlices = (RT * 16 * (D / 8) + kThreads - 1) / kThreads;  // a group's pieces
  hipLaunchKernelGGL((verify_merge_kernel<D, RT>),
                     dim3(plan->num_merge, plan->num_kv_heads, kSlices), dim3(kThreads), 0, stream,
                     prm, merge, plan->num_merge);
  return launch_status("verify_merge_kernel");
}

template <int D>
int32_t launch_d(const nsg_attn_plan_t* plan, const AttnParams& prm, const int* merge,
                 hipStream_t stream) {
  switch (plan->row_tiles) {
    case 1: return launch_rt<D, 1>(plan, prm, merge, stream);
    case 2: return launch_rt<D, 2>(plan, prm, merge, stream);
    case 3: return launch_rt<D, 3>(plan, prm, merge, stream);
    case 4: return launch_rt<D, 4>(plan, prm, merge, stream);
    default: set_error("row_tiles %d out of range", plan->row_tiles); return NSG_ERR_ARG;
  }
}

int ilog2_exact(int v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int r = 0;
  while ((1 << r) < v) ++r;
  return r;
}

}  // namespace
}  // namespace nsg

using namespace nsg;

extern "C" int64_t nsg_attn_workspace_bytes(const nsg_attn_plan_t* plan) {
  if (!plan) return -1;
  return plan->workspace_bytes;
}

namespace nsg {
namespace {

// Query-tile shape of a plan: T query tokens per tile (T * G <= 64 rows).  In
// the latency regime (several KV groups per workgroup: short contexts) tiles
// of at most 16 rows when the GQA group allows: one row-tile wave per KV
// group and, at the verify shape (5 tokens x 7 heads), three workgroups per
// request and KV head instead of one -- more of the idle CUs, and each group's
// math on one wave instead of three per SIMD (9.5 -> 8.6 us per launch); each
// tile reads the request's KV range (from L2 after the first).
int q_tile_tokens(int G, int max_ql, bool latency) {
  const int rows = latency && G <= 16 ? 16 : 64;
  return std::max(1, std::min(rows / G, max_ql));
}

// Work-list capacity that any plan with at most `batch` requests of at most
// `max_ql` query tokens fits: the split size is chosen so that the KV steps
// make at most target_items items, plus at most one rounding item per
// (request, query tile) group; every group needs at most one merge item.
// Work items the KV split aims for: with one KV group a workgroup is small
// (kTargetWgPerCu fit a CU); with several (latency regime) it holds 128 KB of
// LDS and a CU runs one.
long long target_items(int kv_groups, int num_cus, int num_kv_heads) {
  return std::max(1, (kv_groups > 1 ? num_cus : num_cus * kTargetWgPerCu) / num_kv_heads);
}

// Graph-captured plans keep one shape across re-plans.  With a KV-length
// bound (max_kv_len > 0: decode / verify steps over short contexts) they take
// the latency regime and never split a query tile's KV range: one work item
// per tile and no merge launch at all.  Without one (long contexts) they take
// the one-group regime, split to fill the GPU and merged by a second launch
// (at the large shape 456 us per call in the latency regime, 301 us here).
void fixed_capacity(int batch, int max_ql, int G, int num_kv_heads, int num_cus, int max_kv_len,
                    int* max_work, int* max_merge) {
  const int T = q_tile_tokens(G, max_ql, max_kv_len > 0);
  const int groups = batch * ((std::max(1, max_ql) + T - 1) / T);
  if (max_kv_len > 0) {
    *max_work = groups;
    *max_merge = 0;
    return;
  }
  *max_work = (int)target_items(1, num_cus, num_kv_heads) + groups;
  *max_merge = groups;
}

int max_splits_planned(const std::vector<int>& split_counts) {
  int mx = 1;
  for (int c : split_counts) mx = std::max(mx, c);
  return mx;
}

// Shared planner.  fixed_work < 0: the work list holds exactly the items the
// plan needs.  fixed_work >= 0: it holds exactly fixed_work work items (the
// tail padded with empty items, query tokens 0) followed by fixed_merge merge
// items (padded with split count 0), so that nsg_attn_run launches the same
// grid for every plan and a captured graph replays after re-planning.
int32_t plan_impl(const int32_t* qo_indptr_h, const int32_t* kv_indptr_h,
                  const int32_t* kv_last_page_len_h, int32_t batch, int32_t num_qo_heads,
                  int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int32_t causal,
                  int32_t num_cus, int32_t* work_h, int32_t work_capacity, int32_t fixed_work,
                  int32_t fixed_merge, int32_t fixed_q_len, int32_t fixed_kv_len,
                  nsg_attn_plan_t* plan) {
  NSG_CHECK_ARG(plan && qo_indptr_h && kv_indptr_h && kv_last_page_len_h, "null argument");
  NSG_CHECK_ARG(batch >= 0, "batch %d < 0", batch);
  NSG_CHECK_ARG(num_kv_heads > 0 && num_qo_heads > 0 && num_qo_heads % num_kv_heads == 0,
                "num_qo_heads %d must be a positive multiple of num_kv_heads %d",
                num_qo_heads, num_kv_heads);
  const int G = num_qo_heads / num_kv_heads;
  if (G > 64) {
    set_error("GQA group %d > 64 is not supported", G);
    return NSG_ERR_UNSUPPORTED;
  }
  if (head_dim != 64 && head_dim != 128) {
    set_error("head_dim %d not supported (64 or 128)", head_dim);
    return NSG_ERR_UNSUPPORTED;
  }
  NSG_CHECK_ARG(ilog2_exact(page_size) >= 0, "page_size %d must be a power of two", page_size);
  NSG_CHECK_ARG(qo_indptr_h[0] == 0 && kv_indptr_h[0] == 0, "indptr arrays must start at 0");
  if (num_cus <= 0) num_cus = 256;

  int max_ql = 0;
  for (int b = 0; b < batch; ++b) {
    const int ql = qo_indptr_h[b + 1] - qo_indptr_h[b];
    const int np = kv_indptr_h[b + 1] - kv_indptr_h[b];
    NSG_CHECK_ARG(ql >= 0 && np >= 0, "request %d: decreasing indptr", b);
    if (np > 0) {
      NSG_CHECK_ARG(kv_last_page_len_h[b] >= 1 && kv_last_page_len_h[b] <= page_size,
                    "request %d: last_page_len %d outside [1, %d]", b, kv_last_page_len_h[b],
                    page_size);
    }
    max_ql = std::max(max_ql, ql);
  }
  if (fixed_work >= 0) {
    // the tile shape (a kernel template parameter) must not change between
    // plans of one captured graph: it follows the graph's query length
    NSG_CHECK_ARG(max_ql <= fixed_q_len, "a request has %d query tokens, the fixed plan "
                  "allows %d", max_ql, fixed_q_len);
    max_ql = fixed_q_len;
  }
  struct Group { int b, qb, qn, kv_end, lim0; };
  std::vector<Group> groups;
  groups.reserve((size_t)batch * std::max(1, max_ql));
  long long total_it = 0;
  // query tiles of T tokens, each with its KV range (bottom-right causal)
  auto make_groups = [&](int T) -> int32_t {
    groups.clear();
    total_it = 0;
    for (int b = 0; b < batch; ++b) {
      const int ql = qo_indptr_h[b + 1] - qo_indptr_h[b];
      if (ql == 0) continue;
      const int np = kv_indptr_h[b + 1] - kv_indptr_h[b];
      const int L = np > 0 ? (np - 1) * page_size + kv_last_page_len_h[b] : 0;
      NSG_CHECK_ARG(L >= 1, "request %d has %d query tokens but an empty KV range", b, ql);
      NSG_CHECK_ARG(fixed_kv_len <= 0 || L <= fixed_kv_len,
                    "request %d: kv length %d exceeds the fixed plan's bound %d", b, L,
                    fixed_kv_len);
      NSG_CHECK_ARG(!causal || L >= ql, "request %d: kv length %d < query length %d", b, L, ql);
      for (int qb = 0; qb < ql; qb += T) {
        const int qn = std::min(T, ql - qb);
        const int kv_end = causal ? L - ql + qb + qn : L;
        groups.push_back({b, qb, qn, kv_end, causal ? L - ql + qb : L - 1});
        total_it += (kv_end + kTokIt - 1) / kTokIt;
      }
    }
    return NSG_OK;
  };
  // KV groups: several per workgroup when even minimum-length items cannot
  // fill the GPU (the latency regime), one otherwise; a graph-captured plan
  // takes the latency regime exactly when it has a KV-length bound (see
  // fixed_capacity), known before the tiles are made.  A split is at least
  // kMinSplitSteps steps per group: its partial rows cost about as much
  // traffic as one step of K and V.
  const long long t1 = target_items(1, num_cus, num_kv_heads);
  bool latency;
  int T;
  if (fixed_work >= 0) {
    latency = page_size >= kMinGroupPage && fixed_kv_len > 0;
    T = q_tile_tokens(G, max_ql, latency);
    if (int32_t rc = make_groups(T)) return rc;
  } else {
    T = q_tile_tokens(G, max_ql, false);
    if (int32_t rc = make_groups(T)) return rc;
    latency = page_size >= kMinGroupPage && (total_it + t1 - 1) / t1 <= kMinSplitSteps;
    if (latency && q_tile_tokens(G, max_ql, true) != T) {
      T = q_tile_tokens(G, max_ql, true);
      if (int32_t rc = make_groups(T)) return rc;
    }
  }
  const int RT = (T * G + 15) / 16;
  const int KS = latency ? kv_groups_max(head_dim) : 1;
  const long long tgt = target_items(KS, num_cus, num_kv_heads);
  long long chunk_it = std::max<long long>(
      (long long)(KS > 1 ? kMinGroupSteps : kMinSplitSteps) * KS, (total_it + tgt - 1) / tgt);
  // a work item's page ids must fit the kernel's LDS list (kMaxItemPages)
  const long long max_chunk_it =
      std::max<long long>(1, ((long long)(kMaxItemPages - 2) * page_size) / kTokIt);
  chunk_it = std::min(chunk_it, max_chunk_it);
  if (fixed_kv_len > 0) chunk_it = std::max<long long>(chunk_it, (fixed_kv_len + kTokIt - 1) / kTokIt);

  int n = 0, max_splits = 0, n_merge = 0;
  std::vector<int> split_counts(groups.size());
  for (size_t gi = 0; gi < groups.size(); ++gi) {
    const long long its = (groups[gi].kv_end + kTokIt - 1) / kTokIt;
    split_counts[gi] = (int)std::max<long long>(1, (its + chunk_it - 1) / chunk_it);
    n += split_counts[gi];
    n_merge += split_counts[gi] > 1;
  }
  if (fixed_work >= 0 && (n > fixed_work || n_merge > fixed_merge)) {
    set_error("plan needs %d work and %d merge items, the fixed list holds %d and %d", n,
              n_merge, fixed_work, fixed_merge);
    return NSG_ERR_WORKSPACE;
  }
  const int n_work = fixed_work >= 0 ? fixed_work : n;
  const int n_merge_slots = fixed_work >= 0 ? fixed_merge : n_merge;
  if (!work_h || n_work + n_merge_slots > work_capacity) {
    set_error("work list needs %d items, buffer holds %d", n_work + n_merge_slots,
              work_capacity);
    return NSG_ERR_WORKSPACE;
  }
  // Work-item order.  Workgroups go round-robin over the 8 XCDs (linear id
  // = item * KV heads + head), so items P = 8 / gcd(heads, 8) apart sit on
  // one XCD; with several query tiles per request and no split, a request's
  // tiles are placed P apart, and all but the first read the request's KV
  // range from that XCD's L2 instead of another XCD's.
  std::vector<int> order(groups.size());
  std::iota(order.begin(), order.end(), 0);
  const int P = 8 / std::gcd(num_kv_heads, 8);
  if (latency && P > 1 && max_splits_planned(split_counts) == 1) {
    std::vector<std::pair<int, int>> reqs;  // (first group, groups) per request
    reqs.reserve((size_t)batch);
    for (size_t gi = 0; gi < groups.size(); ++gi) {
      if (gi == 0 || groups[gi].b != groups[gi - 1].b) reqs.push_back({(int)gi, 0});
      ++reqs.back().second;
    }
    order.clear();
    for (size_t c0 = 0; c0 < reqs.size(); c0 += P) {
      const size_t c1 = std::min(reqs.size(), c0 + P);
      int tiles = 0;
      for (size_t r = c0; r < c1; ++r) tiles = std::max(tiles, reqs[r].second);
      for (int t = 0; t < tiles; ++t)
        for (size_t r = c0; r < c1; ++r)
          if (t < reqs[r].second) order.push_back(reqs[r].first + t);
    }
  }
  n = 0;
  int m = 0;
  for (size_t oi = 0; oi < groups.size(); ++oi) {
    const size_t gi = (size_t)order[oi];
    const Group& g = groups[gi];
    const int ns = split_counts[gi];
    max_splits = std::max(max_splits, ns);
    const int qs = qo_indptr_h[g.b] + g.qb;
    if (ns > 1) {  // merge item: (first query token, query tokens, first work item, splits)
      int32_t* w = work_h + (size_t)(n_work + m) * NSG_ATTN_WORK_INTS;
      w[0] = qs;
      w[1] = g.qn;
      w[2] = n;
      w[3] = ns;
      w[4] = w[5] = w[6] = w[7] = 0;
      ++m;
    }
    for (int s = 0; s < ns; ++s) {
      int32_t* w = work_h + (size_t)n * NSG_ATTN_WORK_INTS;
      w[0] = qs;
      w[1] = g.qn;
      w[2] = g.lim0;
      w[3] = kv_indptr_h[g.b];
      w[4] = (int)(s * chunk_it * kTokIt);
      w[5] = (int)std::min<long long>(g.kv_end, (s + 1) * chunk_it * kTokIt);
      w[6] = ns;
      w[7] = 0;
      ++n;
    }
  }
  // padding: empty work items (query tokens 0), merge items with 0 splits
  std::fill(work_h + (size_t)n * NSG_ATTN_WORK_INTS,
            work_h + (size_t)n_work * NSG_ATTN_WORK_INTS, 0);
  std::fill(work_h + (size_t)(n_work + m) * NSG_ATTN_WORK_INTS,
            work_h + (size_t)(n_work + n_merge_slots) * NSG_ATTN_WORK_INTS, 0);
  plan->num_work = n_work;
  plan->num_merge = n_merge_slots;
  plan->num_groups = (int)groups.size();
  plan->row_tiles = RT;
  plan->q_tile_tokens = T;
  plan->max_splits = max_splits;
  plan->head_dim = head_dim;
  plan->num_qo_heads = num_qo_heads;
  plan->num_kv_heads = num_kv_heads;
  plan->kv_groups = KS;
  plan->workspace_bytes =
      kHeaderBytes + (int64_t)n_work * num_kv_heads * RT * 16 * (head_dim + 4) * 4;
  clear_error();
  return NSG_OK;
}

}  // namespace
}  // namespace nsg

extern "C" int32_t nsg_attn_plan(const int32_t* qo_indptr_h, const int32_t* kv_indptr_h,
                                 const int32_t* kv_last_page_len_h, int32_t batch,
                                 int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                                 int32_t page_size, int32_t causal, int32_t num_cus,
                                 int32_t* work_h, int32_t work_capacity, nsg_attn_plan_t* plan) {
  return plan_impl(qo_indptr_h, kv_indptr_h, kv_last_page_len_h, batch, num_qo_heads,
                   num_kv_heads, head_dim, page_size, causal, num_cus, work_h, work_capacity,
                   -1, 0, 0, 0, plan);
}

extern "C" int32_t nsg_attn_fixed_capacity(int32_t batch, int32_t max_q_len,
                                           int32_t num_qo_heads, int32_t num_kv_heads,
                                           int32_t num_cus, int32_t max_kv_len,
                                           int32_t* max_work, int32_t* max_merge) {
  NSG_CHECK_ARG(max_work && max_merge, "null argument");
  NSG_CHECK_ARG(batch >= 1 && max_q_len >= 1, "batch %d and max_q_len %d must be >= 1", batch,
                max_q_len);
  NSG_CHECK_ARG(num_kv_heads > 0 && num_qo_heads > 0 && num_qo_heads % num_kv_heads == 0 &&
                    num_qo_heads / num_kv_heads <= 64,
                "num_qo_heads %d / num_kv_heads %d", num_qo_heads, num_kv_heads);
  if (num_cus <= 0) num_cus = 256;
  fixed_capacity(batch, max_q_len, num_qo_heads / num_kv_heads, num_kv_heads, num_cus,
                 max_kv_len, max_work, max_merge);
  clear_error();
  return NSG_OK;
}

extern "C" int32_t nsg_attn_plan_fixed(const int32_t* qo_indptr_h, const int32_t* kv_indptr_h,
                                       const int32_t* kv_last_page_len_h, int32_t batch,
                                       int32_t num_qo_heads, int32_t num_kv_heads,
                                       int32_t head_dim, int32_t page_size, int32_t causal,
                                       int32_t num_cus, int32_t max_q_len, int32_t max_kv_len,
                                       int32_t max_work, int32_t max_merge, int32_t* work_h,
                                       int32_t work_capacity, nsg_attn_plan_t* plan) {
  NSG_CHECK_ARG(max_q_len >= 1 && max_work >= 1 && max_merge >= 0,
                "max_q_len %d, max_work %d, max_merge %d", max_q_len, max_work, max_merge);
  NSG_CHECK_ARG(page_size > 0 && max_kv_len <= (kMaxItemPages - 2) * page_size,
                "max_kv_len %d exceeds one work item's page list (%d tokens)", max_kv_len,
                (kMaxItemPages - 2) * page_size);
  return plan_impl(qo_indptr_h, kv_indptr_h, kv_last_page_len_h, batch, num_qo_heads,
                   num_kv_heads, head_dim, page_size, causal, num_cus, work_h, work_capacity,
                   max_work, max_merge, max_q_len, max_kv_len, plan);
}

extern "C" int32_t nsg_attn_run(const nsg_attn_plan_t* plan, const int32_t* work_d,
                                const void* q, const void* k_cache, const void* v_cache,
                                void* out, const int32_t* qo_indptr, const int32_t* kv_indptr,
                                const int32_t* kv_indices, const int32_t* kv_last_page_len,
                                int32_t page_size, int32_t num_pages, float sm_scale,
                                int32_t causal, void* workspace, int64_t workspace_bytes,
                                nsg_stream_t stream) {
  NSG_CHECK_ARG(plan != nullptr, "null plan");
  if (plan->num_work == 0) {
    clear_error();
    return NSG_OK;
  }
  NSG_CHECK_ARG(work_d && q && k_cache && v_cache && out && qo_indptr && kv_indptr &&
                    kv_indices && kv_last_page_len && workspace,
                "null pointer argument");
  const int log2P = ilog2_exact(page_size);
  NSG_CHECK_ARG(log2P >= 0, "page_size %d must be a power of two", page_size);
  NSG_CHECK_ARG(num_pages > 0, "num_pages %d", num_pages);
  NSG_CHECK_ARG(sm_scale > 0.f, "sm_scale %g must be positive", (double)sm_scale);
  NSG_CHECK_ARG(plan->kv_groups == 1 || page_size >= kMinGroupPage,
                "page_size %d: the plan's %d KV groups need pages of %d+ tokens (plan and run "
                "with the same page size)", page_size, plan->kv_groups, kMinGroupPage);
  if (workspace_bytes < plan->workspace_bytes) {
    set_error("workspace has %lld bytes, plan needs %lld", (long long)workspace_bytes,
              (long long)plan->workspace_bytes);
    return NSG_ERR_WORKSPACE;
  }
  AttnParams prm{};
  prm.q = static_cast<const bf16*>(q);
  prm.kc = static_cast<const bf16*>(k_cache);
  prm.vc = static_cast<const bf16*>(v_cache);
  prm.out = static_cast<bf16*>(out);
  prm.qo_indptr = qo_indptr;
  prm.kv_indptr = kv_indptr;
  prm.kv_indices = kv_indices;
  prm.kv_last = kv_last_page_len;
  prm.work = work_d;
  prm.num_work = plan->num_work;
  prm.Hq = plan->num_qo_heads;
  prm.Hkv = plan->num_kv_heads;
  prm.G = plan->num_qo_heads / plan->num_kv_heads;
  prm.log2P = log2P;
  prm.num_pages = num_pages;
  prm.causal = causal ? 1 : 0;
  prm.scale_log2 = sm_scale * 1.4426950408889634f;
  char* ws = static_cast<char*>(workspace);
  prm.flags = reinterpret_cast<int*>(ws);
  prm.partials = reinterpret_cast<float*>(ws + kHeaderBytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int* merge = work_d + (size_t)plan->num_work * NSG_ATTN_WORK_INTS;
  if (plan->head_dim == 64) return launch_d<64>(plan, prm, merge, s);
  if (plan->head_dim == 128) return launch_d<128>(plan, prm, merge, s);
  set_error("head_dim %d not supported", plan->head_dim);
  return NSG_ERR_UNSUPPORTED;
}

extern "C" int32_t nsg_attn_check_flags(void* workspace, int32_t* flags_h, nsg_stream_t stream) {
  NSG_CHECK_ARG(workspace && flags_h, "null argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  NSG_CHECK_HIP(hipMemcpyAsync(flags_h, workspace, sizeof(int32_t), hipMemcpyDeviceToHost, s));
  NSG_CHECK_HIP(hipStreamSynchronize(s));
  NSG_CHECK_HIP(hipMemsetAsync(workspace, 0, sizeof(int32_t), s));
  clear_error();
  return NSG_OK;
}
