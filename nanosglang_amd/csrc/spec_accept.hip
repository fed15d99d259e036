// Fused acceptance for one speculative verify step on gfx950: greedy or
// stochastic ratio test, textbook residual resample, bonus token and
// rollback slots, for B requests at once.
//
// Reference: nano_sglang/decode/speculative.py:130-184 (per-position Python
// loop: softmax over the vocabulary, ratio test, resample, bonus) and
// speculative.py:186-196 (rollback, a no-op there).  Parity decisions:
//   greedy (T < 1e-6, nano_sglang/engine/sampling.py:44): T->0 limit of the
//     ratio test -- accept d_i iff d_i == argmax(target row i) (lowest index on
//     ties); the first mismatch emits that argmax; all-match emits
//     argmax(target row k);
//   stochastic: p = softmax(logits / T); accept iff u_i < min(1, pt/pd)
//     (pd == 0 accepts); on rejection sample max(0, pt - pd) (falls back to pt
//     if that sums to 0) by inverse CDF with u_k; else the bonus from pt_k,
//     or the caller's bonus token when one is given (a top-k / top-p draw
//     from target row k, speculative.py:174-182).
//
// Launches:
//   greedy: greedy_fused_kernel, grid (chunks, target rows): every target
//     row is cut into chunks; a workgroup reduces its chunk to (max, first
//     argmax) from batches of non-temporal 16-byte loads issued together, and
//     each request's last workgroup loads all of that request's chunk records
//     at once, compares with the drafts and writes tokens, counts and rollback
//     slots.  One launch, one read of every logit; a request's tail overlaps
//     later requests' streaming.
//   stochastic (V % 8 == 0): stoch_fused_kernel, one launch: chunk statistics
//     (max, sum 2^x with a lazily rescaled running sum; the chunk holding a
//     draft token publishes that logit) of every target and draft row; each
//     request's decision (k ratio tests, a ballot for the first rejection) by
//     its last statistics workgroup; then range workgroups that stream the
//     decided row pair into step sums, and the token pick by inverse CDF.
//   stochastic (other V): stats_kernel, then decide_kernel, sum_kernel
//     (chunk sums) and select_kernel (chunk prefix, block scan of one chunk).
// Workgroups hand words to each other inside a launch only through
// device-scope atomic exchanges and coherent loads of slots that read zero
// between calls (common.hpp; "hand-off slots" below).
#include <cfloat>
#include <climits>
#include <mutex>
#include <type_traits>

#include "common.hpp"

namespace nsg {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxK = 32;
constexpr int kMaxBatch = 1 << 14;
constexpr int kMaxChunks = 64;
constexpr int kTargetWgs = 4096;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kSlack = 16.f;  // lazy-rescale headroom of the running sums (log2 units)
constexpr int kSpinLimit = 1 << 20;  // polls of a hand-off slot before giving up (flag bit 3)
// Per-request decision record (three hand-off slots), one 128-byte line per
// request, so that the pollers of different requests use different lines.
constexpr int kDecStride = 32;       // floats per request

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct AccParams {
  const void* tl;
  int64_t t_req, t_row;
  const void* dl;
  int64_t d_req, d_row;
  const int64_t* dtok;
  const float* u;
  const int64_t* bonus;  // optional precomputed bonus tokens [B] (stochastic)
  int B, k, V;
  float c;  // log2(e) / T
  int greedy;
  int rpr;  // rows per request: k+1 (greedy) or 2k+1 (target rows, then draft rows)
  const int* kv_indptr;
  const int* kv_indices;
  const int* start_pos;
  int log2P;
  int* n_out;
  int64_t* emitted;
  int64_t* rollback;
  int nch, cs;    // stats chunks / chunk size
  int nch2, cs2;  // sample chunks / chunk size
  float2* stats;  // [B][rpr][nch] chunk records, request-major
  float* dec;     // [B][kDecStride]: decision slots
  float* psum;    // [B][nch2]
  float2* rsum;   // [B][kRsRanges][kRsMaxSteps] step sums (residual, target)
  float2* xlog;   // [B][rpr] (logit at the row's draft token, 1): marked hand-off slots
  int* flags;
};

template <typename T>
struct Logit;
template <>
struct Logit<bf16> {
  static __device__ __forceinline__ float at(const void* base, int64_t off) {
    return bf16_bits_to_float(reinterpret_cast<const uint16_t*>(base)[off]);
  }
  // 8 consecutive values from a 16-byte aligned element offset
  static __device__ __forceinline__ void load8(const void* base, int64_t off, float* x) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(base) + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(v[i] << 16);
      x[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
    }
  }
  static constexpr int kAlign = 8;
};
template <>
struct Logit<float> {
  static __device__ __forceinline__ float at(const void* base, int64_t off) {
    return reinterpret_cast<const float*>(base)[off];
  }
  static __device__ __forceinline__ void load8(const void* base, int64_t off, float* x) {
    const float* p = reinterpret_cast<const float*>(base) + off;
    const floatx4 a = *reinterpret_cast<const floatx4*>(p);
    const floatx4 b = *reinterpret_cast<const floatx4*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = a[i];
      x[4 + i] = b[i];
    }
  }
  static constexpr int kAlign = 4;
};

// Element e of 8 logits held as raw 16-byte words.
template <typename T>
__device__ __forceinline__ float raw_at(const u32x4* r, int e) {
  if constexpr (sizeof(T) == 2) {
    const uint32_t w = r[0][e >> 1];
    return __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
  } else {
    return __uint_as_float(r[e >> 2][e & 3]);
  }
}

// (max, sum 2^(x - max)) pair merge.
__device__ __forceinline__ void ms_merge(float& m, float& s, float m2, float s2) {
  const float M = fmaxf(m, m2);
  if (M == -INFINITY) {  // both empty (or all -inf): keep s = 0, no inf - inf
    s = 0.f;
    m = M;
    return;
  }
  s = s * exp2f(m - M) + s2 * exp2f(m2 - M);
  m = M;
}

// (value, index) argmax merge: larger value wins, ties -> lower index.
__device__ __forceinline__ void am_merge(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

__device__ __forceinline__ void wave_ms(float& m, float& s) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float m2 = __shfl_xor(m, o, 64);
    const float s2 = __shfl_xor(s, o, 64);
    ms_merge(m, s, m2, s2);
  }
}

__device__ __forceinline__ void wave_am(float& v, int& i) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float v2 = __shfl_xor(v, o, 64);
    const int i2 = __shfl_xor(i, o, 64);
    am_merge(v, i, v2, i2);
  }
}

// Greedy, bf16 logits: (value, column) of a chunk's best logit as one
// 32-bit key whose unsigned order is "larger value, then lower column": the
// bf16 bits made order-preserving (-0 ranks with +0), then the column's
// distance from the chunk end (columns inside a chunk of < 65,536).  0 = no
// column.
__device__ __forceinline__ uint32_t am_key(float v, int i, int v0) {
  if (i == INT_MAX) return 0u;
  uint32_t b = __float_as_uint(v) >> 16;   // v is a bf16 value
  b = b == 0x8000u ? 0u : b;
  const uint32_t ord = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
  return (ord << 16) | (0xffffu - (uint32_t)(i - v0));
}
__device__ __forceinline__ void am_unkey(uint32_t key, int v0, float& v, int& i) {
  const uint32_t ord = key >> 16;
  const uint32_t b = (ord & 0x8000u) ? (ord & 0x7fffu) : (~ord & 0xffffu);
  v = __uint_as_float(b << 16);
  i = v0 + (int)(0xffffu - (key & 0xffffu));
}
// Max of a 32-bit key over the wave in the VALU: DPP quad swaps and row
// mirrors inside each 16-lane row, then gfx950's row swaps (no LDS trips,
// unlike the shuffles of wave_am).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t k) {
  k = max(k, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0xb1, 0xf, 0xf, false));   // lane ^ 1
  k = max(k, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0x4e, 0xf, 0xf, false));   // lane ^ 2
  k = max(k, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0x141, 0xf, 0xf, false));  // 7 - lane in 8
  k = max(k, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0x140, 0xf, 0xf, false));  // 15 - lane in 16
  const auto a = __builtin_amdgcn_permlane16_swap(k, k, false, false);
  k = max((uint32_t)a[0], (uint32_t)a[1]);
  const auto c = __builtin_amdgcn_permlane32_swap(k, k, false, false);
  return max((uint32_t)c[0], (uint32_t)c[1]);
}

__device__ __forceinline__ int64_t trow(const AccParams& p, int b, int i) {
  return (int64_t)b * p.t_req + (int64_t)i * p.t_row;
}
__device__ __forceinline__ int64_t drow(const AccParams& p, int b, int i) {
  return (int64_t)b * p.d_req + (int64_t)i * p.d_row;
}

// Rollback slots in two halves, so that the page-table loads leave the
// finishing wave's critical path.  rollback_prefetch (lane i < k of one wave,
// issued before the request's outcome is known): the flat slot of verify
// position start + 1 + i, or -2 past the request's pages.  rollback_lanes,
// once n tokens are emitted: lane i writes the slot of rejected position
// start + n + i (-1 past start + k; past the pages -1 and flag bit 1).
__device__ int64_t rollback_prefetch(const AccParams& p, int b, int lane) {
  if (!p.rollback || lane >= p.k) return -1;
  const int pos = p.start_pos[b] + 1 + lane;
  const int pb = p.kv_indptr[b];
  const int np = p.kv_indptr[b + 1] - pb;
  const int pg = pos >> p.log2P;
  if (pos < 0 || pg >= np) return -2;
  return ((int64_t)p.kv_indices[pb + pg] << p.log2P) + (pos & ((1 << p.log2P) - 1));
}
__device__ void rollback_lanes(const AccParams& p, int b, int n, int lane, int64_t pre) {
  const int src = min(63, max(0, n - 1 + lane));
  const int64_t got = __shfl(pre, src, 64);   // every lane takes part
  if (!p.rollback || lane >= p.k) return;
  int64_t slot = -1;
  if (n + lane <= p.k) {
    slot = got;
    if (slot == -2) {
      slot = -1;
      if (p.flags) atomicOr(p.flags, 2);
    }
  }
  p.rollback[(int64_t)b * p.k + lane] = slot;
}

// ---- hand-off slots ----
// Every word the acceptance kernels write into the workspace body is zero
// again when the call ends (the reader of each word clears it), so the body
// is all zero between calls whatever layout (batch, k, vocabulary) the
// previous call used.  Chunk records and step sums pass between workgroups
// of one launch through slots that hold zero between calls.  A published value is never all-zero
// bits -- a greedy record is (max, ~index); a stochastic record (m, s) has
// s >= 1, or m = -FLT_MAX for an all -inf chunk; step sums carry their sign
// bit set (both sums are >= +0) -- so a reader polls a slot until it is
// non-zero, and the one reader of a slot clears it after use.  Each
// request's finishing workgroup is the last one dispatched among those it
// waits for (workgroups start in index order), so its polls end at once or
// after the stragglers' last stores; they are bounded all the same (flag
// bit 3).
__device__ __forceinline__ float2 poll_slot(const AccParams& p, float2* slot) {
  uint64_t bits = hand_get_bits(slot);
  for (int n = 0; bits == 0; ++n) {
    if (n == kSpinLimit) {
      atomicOr(p.flags, 8);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
    bits = hand_get_bits(slot);
  }
  return make_float2(__uint_as_float((uint32_t)bits), __uint_as_float((uint32_t)(bits >> 32)));
}

__device__ __forceinline__ void clear_slot(float2* slot) { hand_put(slot, make_float2(0.f, 0.f)); }

__device__ __forceinline__ float2 mark_sums(float a, float b) {
  return make_float2(__uint_as_float(__float_as_uint(a) | 0x80000000u),
                     __uint_as_float(__float_as_uint(b) | 0x80000000u));
}

__device__ __forceinline__ float2 unmark_sums(float2 v) {
  return make_float2(__uint_as_float(__float_as_uint(v.x) & 0x7fffffffu),
                     __uint_as_float(__float_as_uint(v.y) & 0x7fffffffu));
}

__device__ __forceinline__ void clear_slots(float2* base, int n) {
  for (int c = threadIdx.x & 63; c < n; c += 64) clear_slot(base + c);
}

constexpr int kRecCap = 128;  // chunk records per request: two per lane of one wave

// A request's n <= kRecCap chunk records, lane l holding records l and l + 64
// (both loads in flight together; each re-polled until published).
struct Recs {
  uint64_t r0, r1;
};
__device__ __forceinline__ uint64_t repoll(const AccParams& p, const float2* slot, uint64_t bits) {
  for (int n = 0; bits == 0; ++n) {
    if (n == kSpinLimit) {
      atomicOr(p.flags, 8);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
    bits = hand_get_bits(slot);
  }
  return bits;
}
__device__ __forceinline__ Recs poll_recs(const AccParams& p, const float2* base, int n) {
  const int lane = threadIdx.x & 63;
  Recs r;
  r.r0 = lane < n ? hand_get_bits(base + lane) : 1;
  r.r1 = lane + 64 < n ? hand_get_bits(base + lane + 64) : 1;
  r.r0 = repoll(p, base + lane, r.r0);
  r.r1 = repoll(p, base + lane + 64, r.r1);
  return r;
}
// Record idx (< kRecCap) of the request, fetched from the lane holding it
// (every lane of the wave takes part).
__device__ __forceinline__ float2 rec_at(const Recs& r, int idx) {
  const int src = idx & 63;
  const uint32_t a0 = __shfl((uint32_t)r.r0, src, 64), b0 = __shfl((uint32_t)(r.r0 >> 32), src, 64);
  const uint32_t a1 = __shfl((uint32_t)r.r1, src, 64), b1 = __shfl((uint32_t)(r.r1 >> 32), src, 64);
  return idx < 64 ? make_float2(__uint_as_float(a0), __uint_as_float(b0))
                  : make_float2(__uint_as_float(a1), __uint_as_float(b1));
}

// Chunk `chunk` of request b's row lr (target rows 0..k, then draft rows
// k+1..2k) reduced by the whole workgroup; thread 0 publishes the chunk record
// at record lr * nch + chunk of the request and, for a stochastic ratio-test
// row, the thread whose vector holds the draft token publishes that logit
// first (hand-off words, so that a workgroup on another XCD may read them
// inside the same launch).
template <typename T, bool GREEDY>
__device__ void row_chunk_stats(const AccParams& p, int b, int lr, int chunk) {
  __shared__ float sm_a[kThreads / 64];
  __shared__ float sm_b[kThreads / 64];
  const bool draft = lr > p.k;
  const int i = draft ? lr - p.k - 1 : lr;
  const int r = b * p.rpr + lr;
  const void* base = draft ? p.dl : p.tl;
  const int64_t roff = draft ? drow(p, b, i) : trow(p, b, i);
  const int v0 = chunk * p.cs;
  const int v1 = min(p.V, v0 + p.cs);
  const int tid = threadIdx.x;
  const bool vec = ((roff % Logit<T>::kAlign) == 0);
  // stochastic rows i < k: the chunk holding the draft token records that
  // logit, so the decision needs no second read of the logits
  int xt = -1;
  float xval = 0.f;
  bool xhit = false;
  if constexpr (!GREEDY) {
    if (i < p.k) {
      const int64_t x = p.dtok[(int64_t)b * p.k + i];
      if (x >= v0 && x < v1) xt = (int)x;
    }
  }

  // stochastic: running reference m and sum of 2^(x c - m).  m starts finite
  // (-FLT_MAX): an all -inf chunk then sums exact zeros instead of NaN.
  float m = -FLT_MAX, s = 0.f;
  float m_hi = -FLT_MAX;         // rescale threshold: m + kSlack
  float bv = -INFINITY;          // greedy, scalar elements: best value / index
  int bi = INT_MAX;
  // greedy, whole vectors (branch-free): the first vector holding this lane's
  // maximum (strict >), its start index and its raw words; the element is
  // found once, after the stream
  constexpr int W = sizeof(T) * 8 / 16;  // 16-byte words per 8 logits
  float vbest = -INFINITY;
  int vidx = INT_MAX;
  u32x4 vraw[W];
#pragma unroll
  for (int w = 0; w < W; ++w) vraw[w] = u32x4{0u, 0u, 0u, 0u};
  auto take = [&](float x, int v) {
    if constexpr (GREEDY) {
      am_merge(bv, bi, x, v);
    } else {
      if (v == xt) {
        xval = x;
        xhit = true;
      }
      const float y = x * p.c;
      if (y > m) {
        s = s * exp2f(m - y);
        m = y;
        m_hi = m + kSlack;
      }
      s += exp2f(y - m);
    }
  };
  int v = v0 + tid * 8;
  // Per 8 logits: greedy -- one max, and the (rare) index search only when the
  // vector beats the running best; stochastic -- max on the raw logits (c > 0),
  // then exp2(fma(x, c, -m)) with the bare v_exp_f32 (arguments <= 0).
  auto take8 = [&](const float* x, int vv, const u32x4* rw) {
    float mx = fmaxf(fmaxf(fmaxf(fmaxf(x[0], x[1]), x[2]), fmaxf(x[3], x[4])),
                     fmaxf(fmaxf(x[5], x[6]), x[7]));  // v_max3 x 3 + v_max
    if constexpr (GREEDY) {
      const bool better = mx > vbest || vidx == INT_MAX;   // selects, no branch
      vbest = better ? mx : vbest;
      vidx = better ? vv : vidx;
#pragma unroll
      for (int w = 0; w < W; ++w) vraw[w] = better ? rw[w] : vraw[w];
    } else {
      if (__builtin_expect(vv == (xt & ~7), 0)) {  // never for xt = -1
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (e == (xt & 7)) xval = x[e];
        xhit = true;
      }
      // lazy rescale: the reference m moves only when a logit exceeds it by
      // more than kSlack (terms stay <= 2^kSlack), so the common path is one
      // compare per 8 logits and fma + exp + add per logit
      mx *= p.c;
      if (__builtin_expect(mx > m_hi, 0)) {
        s = s * __builtin_amdgcn_exp2f(m - mx);  // argument < 0; 0 from the -FLT_MAX start
        m = mx;
        m_hi = m + kSlack;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) s += __builtin_amdgcn_exp2f(__builtin_fmaf(x[e], p.c, -m));
    }
  };
  // Full 8-vectors of the chunk (chunk starts are multiples of 8), read in
  // batches of U independent 16-byte loads per thread: every load of a batch
  // is issued before any is consumed, the batch's missing tail predicated
  // off, so a chunk costs one or two memory round trips, not one per vector.
  const int vfull = v0 + ((v1 - v0) & ~7);
  if (vec) {
    // (stochastic bf16: 12 loads, so that a chunk of up to 24,576 logits is
    // one round trip: 46.2 -> 45.2 us at batch 64, k 4, vocab 151,936 and
    // 58.6 -> 57.3 us at k 8, vocab 128,256 against 8)
    constexpr int U = !GREEDY && sizeof(T) == 2 ? 12 : 8;
    constexpr int STRIDE = kThreads * 8;
    auto batch = [&](int vb, auto full) {
      u32x4 raw[U][W];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int w = 0; w < W; ++w) {
          const u32x4* src = reinterpret_cast<const u32x4*>(
              reinterpret_cast<const char*>(base) + (roff + vb + u * STRIDE) * sizeof(T) + 16 * w);
          if constexpr (decltype(full)::value)
            raw[u][w] = __builtin_nontemporal_load(src);
          else
            raw[u][w] = vb + u * STRIDE < vfull ? __builtin_nontemporal_load(src)
                                                 : u32x4{0u, 0u, 0u, 0u};
        }
      // all U*W loads are issued before any is consumed (the compiler would
      // otherwise sink each load to its use and serialise them).  Non-temporal:
      // a streaming read of every logit once, which MI355X serves faster than
      // cached loads
      asm volatile("" ::: "memory");
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (!decltype(full)::value && vb + u * STRIDE >= vfull) break;
        float x[8];
        if constexpr (sizeof(T) == 2) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            x[2 * i] = __uint_as_float(raw[u][0][i] << 16);
            x[2 * i + 1] = __uint_as_float(raw[u][0][i] & 0xffff0000u);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) x[i] = __uint_as_float(raw[u][i >> 2][i & 3]);
        }
        take8(x, vb + u * STRIDE, raw[u]);
      }
    };
    int vb = v;
    for (; vb + (U - 1) * STRIDE < vfull; vb += U * STRIDE) batch(vb, std::true_type{});
    if (vb < vfull) batch(vb, std::false_type{});
  }
  // the chunk's partial last vector, or every element of an unaligned row:
  // scalar, in increasing index per thread
  for (int vv = (vec ? vfull : v0) + tid; vv < v1; vv += kThreads) take(Logit<T>::at(base, roff + vv), vv);

  if constexpr (!GREEDY) {
    // the draft token's logit, with a marker word (the slot is never all-zero
    // bits once published; the decision polls it beside the records)
    if (xhit) hand_put(p.xlog + r, make_float2(xval, __int_as_float(1)));
  }
  const int lane = tid & 63, wave = tid >> 6;
  if constexpr (GREEDY) {
    if (vidx != INT_MAX) {  // the first element of the best vector equal to its max
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = raw_at<T>(vraw, e);
      int e = 0;
      while (e < 7 && !(x[e] == vbest)) ++e;   // NaN-free rows
      am_merge(bv, bi, vbest, vidx + e);
    }
    if (sizeof(T) == 2 && p.cs < 65536) {   // workgroup-uniform
      const uint32_t key = wave_max_u32(am_key(bv, bi, v0));
      if (lane == 0) sm_a[wave] = __uint_as_float(key);
    } else {
      wave_am(bv, bi);
      if (lane == 0) {
        sm_a[wave] = bv;
        sm_b[wave] = __int_as_float(bi);
      }
    }
  } else {
    if (m == -INFINITY) s = 0.f;
    wave_ms(m, s);
    if (lane == 0) {
      sm_a[wave] = m;
      sm_b[wave] = s;
    }
  }
  __syncthreads();
  if (tid == 0) {
    float a = sm_a[0], c2 = sm_b[0];
    if (GREEDY && sizeof(T) == 2 && p.cs < 65536) {
      uint32_t key = __float_as_uint(sm_a[0]);
      for (int w = 1; w < kThreads / 64; ++w) key = max(key, __float_as_uint(sm_a[w]));
      int ia = INT_MAX;   // (an empty chunk: no column, as in the other form)
      a = -INFINITY;
      if (key != 0u) am_unkey(key, v0, a, ia);
      c2 = __int_as_float(ia);
    } else {
      for (int w = 1; w < kThreads / 64; ++w) {
        if constexpr (GREEDY) {
          int ia = __float_as_int(c2);
          am_merge(a, ia, sm_a[w], __float_as_int(sm_b[w]));
          c2 = __int_as_float(ia);
        } else {
          ms_merge(a, c2, sm_a[w], sm_b[w]);
        }
      }
    }
    if constexpr (GREEDY) c2 = __int_as_float(~__float_as_int(c2));  // never all-zero bits
    hand_put(p.stats + (int64_t)r * p.nch + chunk, make_float2(a, c2));
  }
}

template <typename T, bool GREEDY>
__global__ __launch_bounds__(kThreads) void stats_kernel(AccParams p) {
  const int b = blockIdx.y / p.rpr;
  row_chunk_stats<T, GREEDY>(p, b, blockIdx.y - b * p.rpr, blockIdx.x);
}

// Greedy: one wave combines the argmax chunk records of request b's k+1
// target rows (all loaded at once), compares them with the drafts and writes
// every output; then it clears the records.
__device__ void greedy_finalize(const AccParams& p, int b, int64_t pre) {
  const int lane = threadIdx.x & 63;
  const int k = p.k;
  const int n = (k + 1) * p.nch;
  int64_t x = -1;
  if (lane < k) x = p.dtok[(int64_t)b * k + lane];   // in flight with the records
  float2* recs = p.stats + (int64_t)b * n;
  const Recs rc = poll_recs(p, recs, n);
  float v = -INFINITY;   // lane i <= k: argmax of target row i (first index on ties)
  int ix = INT_MAX;
  for (int c = 0; c < p.nch; ++c) {
    const float2 st = rec_at(rc, min(lane, k) * p.nch + c);
    if (lane <= k) am_merge(v, ix, st.x, ~__float_as_int(st.y));
  }
  if (lane < k && (x < 0 || x >= p.V)) atomicOr(p.flags, 4);  // never matches; flag it
  const uint64_t miss = __builtin_amdgcn_ballot_w64(lane < k && x != (int64_t)ix);
  const int j = miss ? (int)__builtin_ctzll(miss) : k;           // first mismatch, or k
  int64_t* em = p.emitted + (int64_t)b * (k + 1);
  if (lane <= k) em[lane] = lane < j ? x : (lane == j ? (int64_t)ix : -1);
  if (lane == 0) p.n_out[b] = j + 1;
  rollback_lanes(p, b, j + 1, lane, pre);
  clear_slots(recs, n);
}

// Greedy in one launch: the argmax pass over every target row; request b's
// last workgroup (its last row's last chunk, the last of b's workgroups to
// start) finalises b while later requests still stream.
template <typename T>
__global__ __launch_bounds__(kThreads) void greedy_fused_kernel(AccParams p) {
  const int b = blockIdx.y / p.rpr;
  const int lr = blockIdx.y - b * p.rpr;
  const bool last = lr == p.k && (int)blockIdx.x == p.nch - 1 && threadIdx.x < 64;
  const int64_t pre = last ? rollback_prefetch(p, b, threadIdx.x) : -1;  // under the stream
  row_chunk_stats<T, true>(p, b, lr, blockIdx.x);
  if (last) greedy_finalize(p, b, pre);
}

struct Decision {
  int j;      // first rejected position; k = all accepted
  int mode;   // 0 = residual of row j, 1 = target row j alone (bonus)
  float Mt, iZt, Md, iZd;
};

// The decision record of request b: three hand-off slots, each never
// all-zero bits once published -- (j + 1, mode + 1), (Mt, 1/Zt) with 1/Zt > 0,
// (Md, 1/Zd) with 1/Zd > 0, or (0, 1) when mode = 1 -- cleared by the
// request's token pick.
__device__ __forceinline__ float2* dec_slots(const AccParams& p, int b) {
  return reinterpret_cast<float2*>(p.dec + (int64_t)b * kDecStride);
}
__device__ __forceinline__ void clear_slots3(float2* ds) {
  for (int i = 0; i < 3; ++i) clear_slot(ds + i);
}
__device__ __forceinline__ void publish_decision(const AccParams& p, int b, const Decision& d,
                                                 int lane) {
  float2* ds = dec_slots(p, b);
  if (lane == 0) hand_put(ds, make_float2(__int_as_float(d.j + 1), __int_as_float(d.mode + 1)));
  if (lane == 1) hand_put(ds + 1, make_float2(d.Mt, d.iZt));
  if (lane == 2) hand_put(ds + 2, d.mode == 0 ? make_float2(d.Md, d.iZd) : make_float2(0.f, 1.f));
}
// Every lane returns request b's decision (lanes 0..2 poll one slot each).
__device__ Decision read_decision(const AccParams& p, int b) {
  const int lane = threadIdx.x & 63;
  const float2* ds = dec_slots(p, b);
  uint64_t bits = lane < 3 ? hand_get_bits(ds + lane) : 1;
  bits = repoll(p, ds + min(lane, 2), bits);
  const uint32_t lo = (uint32_t)bits, hi = (uint32_t)(bits >> 32);
  Decision d;
  d.j = (int)__shfl(lo, 0, 64) - 1;
  d.mode = (int)__shfl(hi, 0, 64) - 1;
  d.Mt = __uint_as_float(__shfl(lo, 1, 64));
  d.iZt = __uint_as_float(__shfl(hi, 1, 64));
  d.Md = __uint_as_float(__shfl(lo, 2, 64));
  d.iZd = __uint_as_float(__shfl(hi, 2, 64));
  return d;
}

// Request b's decision in a later launch than the one that published it.
__device__ __forceinline__ Decision decision_of(const AccParams& p, int b) {
  const float2* ds = dec_slots(p, b);
  const float2 s0 = ds[0], s1 = ds[1], s2 = ds[2];
  Decision d;
  d.j = __float_as_int(s0.x) - 1;
  d.mode = __float_as_int(s0.y) - 1;
  d.Mt = s1.x;
  d.iZt = s1.y;
  d.Md = s2.x;
  d.iZd = s2.y;
  return d;
}

// Stochastic decision of request b by one wave: every chunk record of its 2k+1
// rows is loaded at once (lane l: records l and l + 64), then lane i merges
// target row i and draft row i and runs ratio test i with the draft-token
// logits the chunks published; a ballot finds the first rejection.  The wave
// writes the accepted prefix, num_emitted, the rollback slots and the caller's
// bonus (all accepted), publishes the decision and clears the records.
template <typename T>
__device__ Decision decide(const AccParams& p, int b, int64_t pre) {
  const int lane = threadIdx.x & 63;
  const int k = p.k;
  const int rpr = 2 * k + 1;
  const int n = rpr * p.nch;
  int64_t x = 0;
  float u = 0.f;
  if (lane < k) {                            // in flight with the records
    x = p.dtok[(int64_t)b * k + lane];
    u = p.u[(int64_t)b * (k + 1) + lane];
  }
  float2* recs = p.stats + (int64_t)b * n;
  // the draft-token logits of target row i and draft row i (lane i < k; an
  // out-of-vocabulary draft token has none), loaded in the same round as
  // the records and polled until published
  const bool xok = lane < k && x >= 0 && x < p.V;
  float2* xs_t = p.xlog + (int64_t)b * rpr + min(lane, k - 1);
  float2* xs_d = p.xlog + (int64_t)b * rpr + k + 1 + min(lane, k - 1);
  uint64_t bt = xok ? hand_get_bits(xs_t) : 1, bd = xok ? hand_get_bits(xs_d) : 1;
  const Recs rc = poll_recs(p, recs, n);
  float xt = 0.f, xd = 0.f;
  if (xok) {
    bt = repoll(p, xs_t, bt);
    bd = repoll(p, xs_d, bd);
    xt = __uint_as_float((uint32_t)bt);
    xd = __uint_as_float((uint32_t)bd);
    clear_slot(xs_t);                        // the workspace ends zero
    clear_slot(xs_d);
  }
  float mt = -INFINITY, zt = 0.f, md = -INFINITY, zd = 0.f;
  for (int c = 0; c < p.nch; ++c) {
    const float2 t = rec_at(rc, min(lane, k) * p.nch + c);
    const float2 dr = rec_at(rc, (k + 1 + min(lane, k - 1)) * p.nch + c);
    if (lane <= k) ms_merge(mt, zt, t.x, t.y);
    if (lane < k) ms_merge(md, zd, dr.x, dr.y);
  }
  bool reject = false;
  if (lane < k) {
    if (x < 0 || x >= p.V) {
      atomicOr(p.flags, 4);
      reject = true;
    } else {
      const float lt = xt * p.c;
      const float ld = xd * p.c;
      const float pt = exp2f(lt - mt) / zt;
      const float pd = exp2f(ld - md) / zd;
      reject = pd > 0.f && !(u < fminf(1.f, pt / pd));
    }
  }
  const uint64_t rej = __builtin_amdgcn_ballot_w64(reject);
  const int j = rej ? min(k, (int)__builtin_ctzll(rej)) : k;
  Decision d;
  d.j = j;
  d.mode = j < k ? 0 : 1;
  d.Mt = __shfl(mt, j, 64);
  d.iZt = 1.f / __shfl(zt, j, 64);
  d.Md = j < k ? __shfl(md, j, 64) : 0.f;
  d.iZd = j < k ? 1.f / __shfl(zd, j, 64) : 0.f;
  int64_t* em = p.emitted + (int64_t)b * (k + 1);
  if (lane < j) em[lane] = x;
  else if (lane > j && lane <= k) em[lane] = -1;   // em[j]: the token pick's alone
  if (lane == 0) {
    p.n_out[b] = j + 1;
    if (d.mode == 1 && p.bonus) em[k] = p.bonus[b];  // all accepted: the caller's bonus
  }
  rollback_lanes(p, b, j + 1, lane, pre);
  publish_decision(p, b, d, lane);
  clear_slots(recs, n);
  return d;
}

// Weight of vocabulary entry v for the decided row pair.
template <typename T>
__device__ __forceinline__ float weight(const AccParams& p, int64_t to, int64_t dof, int mode,
                                        float Mt, float iZt, float Md, float iZd, int v) {
  const float pt = __builtin_amdgcn_exp2f(__builtin_fmaf(Logit<T>::at(p.tl, to + v), p.c, -Mt)) * iZt;
  if (mode != 0) return pt;
  const float pd = __builtin_amdgcn_exp2f(__builtin_fmaf(Logit<T>::at(p.dl, dof + v), p.c, -Md)) * iZd;
  return fmaxf(0.f, pt - pd);
}

// Block-wide inclusive scan of one float per thread (fixed order).
__device__ float block_incl_scan(float x, float* sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) sh[wave] = x;
  __syncthreads();
  float pre = 0.f;
  for (int w = 0; w < wave; ++w) pre += sh[w];
  __syncthreads();
  return pre + x;
}

// One wave per request: the decision, the accepted prefix, counts and slots.
template <typename T>
__global__ __launch_bounds__(64) void decide_kernel(AccParams p) {
  decide<T>(p, blockIdx.x, rollback_prefetch(p, blockIdx.x, threadIdx.x));
}

// Chunk sums of the decided weights (residual of row j, or target row j).
template <typename T>
__global__ __launch_bounds__(kThreads) void sum_kernel(AccParams p) {
  __shared__ float sh[kThreads / 64];
  const int b = blockIdx.y;
  const int chunk = blockIdx.x;
  const int tid = threadIdx.x;
  const Decision d = decision_of(p, b);
  const int64_t to = trow(p, b, d.j);
  const int64_t dof = d.mode == 0 ? drow(p, b, d.j) : 0;
  const int v0 = chunk * p.cs2;
  const int v1 = min(p.V, v0 + p.cs2);
  float acc = 0.f;
  int v = v0 + tid * 8;
  if (((to | dof) % Logit<T>::kAlign) == 0) {
    for (; v + 8 <= v1; v += kThreads * 8) {
      float xt[8], xd[8];
      Logit<T>::load8(p.tl, to + v, xt);
      if (d.mode == 0) Logit<T>::load8(p.dl, dof + v, xd);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float pt = __builtin_amdgcn_exp2f(__builtin_fmaf(xt[e], p.c, -d.Mt)) * d.iZt;
        acc += d.mode == 0
                   ? fmaxf(0.f, pt - __builtin_amdgcn_exp2f(__builtin_fmaf(xd[e], p.c, -d.Md)) * d.iZd)
                   : pt;
      }
    }
  }
  for (; v < v1; v += kThreads * 8)
    for (int e = 0; e < 8 && v + e < v1; ++e)
      acc += weight<T>(p, to, dof, d.mode, d.Mt, d.iZt, d.Md, d.iZd, v + e);
  acc = wave_sum(acc);
  if ((tid & 63) == 0) sh[tid >> 6] = acc;
  __syncthreads();
  if (tid == 0) {
    float t = 0.f;
    for (int w = 0; w < kThreads / 64; ++w) t += sh[w];
    p.psum[(int64_t)b * p.nch2 + chunk] = t;
  }
}

// One workgroup per request: the chunk by a wave scan over the chunk sums,
// the token by a block scan over 8-element runs (one 16-byte vector per
// thread; chunks are at most 8 * kSelThreads elements).
constexpr int kSelThreads = 1024;

template <typename T>
__device__ __forceinline__ float run_weights(const AccParams& p, int64_t to, int64_t dof, int mode,
                                             float Mt, float iZt, float Md, float iZd, int v0,
                                             int v1, bool vec, float* w) {
  float xt[8], xd[8];
  if (vec && v0 + 8 <= v1) {
    Logit<T>::load8(p.tl, to + v0, xt);
    if (mode == 0) Logit<T>::load8(p.dl, dof + v0, xd);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xt[e] = v0 + e < v1 ? Logit<T>::at(p.tl, to + v0 + e) : -INFINITY;
      xd[e] = (mode == 0 && v0 + e < v1) ? Logit<T>::at(p.dl, dof + v0 + e) : -INFINITY;
    }
  }
  float run = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float pt = __builtin_amdgcn_exp2f(__builtin_fmaf(xt[e], p.c, -Mt)) * iZt;
    w[e] = v0 + e < v1
               ? (mode == 0 ? fmaxf(0.f, pt - __builtin_amdgcn_exp2f(__builtin_fmaf(xd[e], p.c, -Md)) * iZd)
                            : pt)
               : 0.f;
    run += w[e];
  }
  return run;
}

template <typename T>
__global__ __launch_bounds__(kSelThreads) void select_kernel(AccParams p) {
  __shared__ float sh[kSelThreads / 64];
  __shared__ int s_tok, s_chunk;
  __shared__ float s_rem, s_tot;
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const Decision dc = decision_of(p, b);
  const int j = dc.j;
  int mode = dc.mode;
  if (mode == 1 && p.bonus) {  // all accepted: the decision emitted the caller's bonus
    if (tid == 0) clear_slots3(dec_slots(p, b));
    return;
  }
  const float Mt = dc.Mt, iZt = dc.iZt, Md = dc.Md, iZd = dc.iZd;
  const int64_t to = trow(p, b, j);
  const int64_t dof = mode == 0 ? drow(p, b, j) : 0;
  const float u = p.u[(int64_t)b * (p.k + 1) + p.k];
  if (tid < 64) {
    // chunk sums -> inclusive wave scan (nch2 <= 64), fixed order
    const float v = tid < p.nch2 ? p.psum[(int64_t)b * p.nch2 + tid] : 0.f;
    if (tid < p.nch2) p.psum[(int64_t)b * p.nch2 + tid] = 0.f;   // the workspace ends zero
    float incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float y = __shfl_up(incl, o, 64);
      if (tid >= o) incl += y;
    }
    const float tot = __shfl(incl, 63, 64);
    const float target = u * tot;
    const uint64_t hit = __builtin_amdgcn_ballot_w64(tid < p.nch2 && incl > target);
    const uint64_t pos = __builtin_amdgcn_ballot_w64(tid < p.nch2 && v > 0.f);
    // (all 64 lanes take part in the shuffles; lane 0 publishes)
    const int cs = hit ? (int)__builtin_ctzll(hit) : 0;
    const float at_incl = __shfl(incl, cs, 64);
    const float at_v = __shfl(v, cs, 64);
    if (tid == 0) {
      s_tot = tot;
      s_tok = -1;
      if (hit) {
        s_chunk = cs;
        s_rem = target - (at_incl - at_v);
      } else {
        s_chunk = pos ? 63 - (int)__builtin_clzll(pos) : 0;
        s_rem = INFINITY;  // rounding left no crossing: last positive weight
      }
    }
  }
  __syncthreads();
  int a, e;
  const bool full = !(s_tot > 0.f);
  if (full) {
    // residual summed to zero: sample the target row itself over the whole
    // vocabulary (mirrors speculative.py:163-169), in kSelThreads * 8 slices
    mode = 1;
    a = 0;
    e = p.V;
  } else {
    a = s_chunk * p.cs2;
    e = min(p.V, a + p.cs2);
  }
  const bool vec = ((to | dof) % Logit<T>::kAlign) == 0;
  float base = 0.f;        // prefix of earlier slices (full-row fallback only)
  float target_full = 0.f;
  if (full) {
    float tot = 0.f;
    for (int v0 = a + tid * 8; v0 < e; v0 += kSelThreads * 8) {
      float w[8];
      tot += run_weights<T>(p, to, dof, mode, Mt, iZt, Md, iZd, v0, e, vec, w);
    }
    tot = wave_sum(tot);
    if ((tid & 63) == 0) sh[tid >> 6] = tot;
    __syncthreads();
    float t2 = 0.f;
    for (int w = 0; w < kSelThreads / 64; ++w) t2 += sh[w];
    __syncthreads();
    target_full = u * t2;
  }
  for (int s0 = a; s0 < e; s0 += kSelThreads * 8) {
    const int v0 = s0 + tid * 8;
    float w[8];
    const float run = v0 < e ? run_weights<T>(p, to, dof, mode, Mt, iZt, Md, iZd, v0, e, vec, w)
                             : 0.f;
    const float incl = block_incl_scan(run, sh) + base;
    const float excl = incl - run;
    const float rem = full ? target_full : s_rem;
    if (v0 < e && run > 0.f && incl > rem && !(excl > rem)) {
      float cum = 0.f;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        cum += w[q];
        if (w[q] > 0.f && excl + cum > rem) {
          atomicMax(&s_tok, v0 + q);
          break;
        }
      }
    }
    // carry the slice total into the next slice
    if (tid == kSelThreads - 1) sh[0] = incl;
    __syncthreads();
    base = sh[0];
    __syncthreads();
    if (s_tok >= 0) break;
  }
  if (s_tok < 0) {
    // rounding left no crossing: last positive weight in the range
    int last = -1;
    for (int v0 = a + tid * 8; v0 < e; v0 += kSelThreads * 8) {
      float w[8];
      run_weights<T>(p, to, dof, mode, Mt, iZt, Md, iZd, v0, e, vec, w);
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (w[q] > 0.f) last = max(last, v0 + q);
    }
    atomicMax(&s_tok, last);
    __syncthreads();
  }
  if (tid == 0) {
    p.emitted[(int64_t)b * (p.k + 1) + j] = s_tok;
    clear_slots3(dec_slots(p, b));   // zero between calls
  }
}

// ---- the decided row pair's step sums (V % 8 == 0, V <= kRsMaxV) ----
//
// The request's vocabulary is cut into kRsRanges contiguous ranges of ns
// 512-logit steps.  A wave streams one range of the decided row pair (lane l:
// logits 8 l .. 8 l + 7 of a step, 1 KB contiguous per wave load) and writes
// each step's sums of the residual max(0, pt - pd) and of pt (the
// zero-residual fallback needs no second pass), each an inclusive wave scan
// of the lanes' 8-logit runs.  One wave then picks the token: lane r sums
// range r's steps in order, a wave scan orders the ranges, the crossing lane
// finds its step, and the whole wave recomputes that one step with the same
// arithmetic (step_weights) to find the lane and the logit.  Rounding that
// leaves no crossing picks the last positive weight.
constexpr int kRsThreads = 256;
constexpr int kRsWaves = kRsThreads / 64;
constexpr int kRsSplits = 16;
constexpr int kRsRanges = kRsSplits * kRsWaves;  // 64: one per lane of select_kernel2
constexpr int kRsMaxSteps = 16;
constexpr int kRsStep = 512;
constexpr int kRsMaxV = kRsRanges * kRsMaxSteps * kRsStep;

__device__ __forceinline__ float wave_incl_scan(float x, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  return x;
}

__device__ __forceinline__ int rs_steps(int V) {
  return ((V + kRsStep - 1) / kRsStep + kRsRanges - 1) / kRsRanges;
}

// This lane's 8 logits of a step, loaded from a clamped, in-range address
// (V % 8 == 0 on this path) ...
template <typename T>
struct StepRaw {
  static constexpr int W = sizeof(T) * 8 / 16;  // 16-byte loads per 8 logits
  u32x4 t[W], d[W];
};

template <typename T>
__device__ __forceinline__ void step_load(const AccParams& p, int64_t to, int64_t dof, int mode,
                                          int v, StepRaw<T>& r) {
  const int vc = min(v, p.V - 8);
#pragma unroll
  for (int w = 0; w < StepRaw<T>::W; ++w) {
    r.t[w] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(p.tl) +
                                             (to + vc) * sizeof(T) + 16 * w);
    r.d[w] = mode == 0 ? *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(p.dl) +
                                                         (dof + vc) * sizeof(T) + 16 * w)
                       : u32x4{0u, 0u, 0u, 0u};
  }
}

// ... and its residual and target weights (zero past V) and their runs.
template <typename T>
__device__ __forceinline__ void step_weights(const AccParams& p, int mode, const Decision& d,
                                             int v, const StepRaw<T>& r, float* wres,
                                             float* wpt, float& res, float& pts) {
  res = 0.f;
  pts = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const bool in = v < p.V;
    const float pt =
        in ? __builtin_amdgcn_exp2f(__builtin_fmaf(raw_at<T>(r.t, e), p.c, -d.Mt)) * d.iZt : 0.f;
    const float rr =
        mode == 0 && in
            ? fmaxf(0.f, pt - __builtin_amdgcn_exp2f(__builtin_fmaf(raw_at<T>(r.d, e), p.c, -d.Md)) * d.iZd)
            : pt;
    wres[e] = rr;
    wpt[e] = pt;
    res += rr;
    pts += pt;
  }
}

// Streams ns steps of the decided row pair from vocabulary index v0 (this
// lane's first logit) and writes each step's sums (residual, target) -- each
// an inclusive wave scan of the lanes' 8-logit runs -- to out[0 .. ns).
template <typename T>
__device__ __forceinline__ void stream_step_sums(const AccParams& p, const Decision& d,
                                                 int64_t to, int64_t dof, int ns, int v0,
                                                 int lane, float2* out) {
  // steps whose loads are in flight together: with bf16 logits 5 covers a
  // range of vocab up to 163,840 in one round trip (batch 64, k 4, vocab
  // 151,936: 46.2 -> 45.3 us per call against 4; 6 takes 8 more registers
  // and 8 ran slower); fp32 logits keep 4 (5 would raise the kernel from 92
  // to 109 registers, one wave per SIMD fewer)
  constexpr int G = sizeof(T) == 2 ? 5 : 4;
  for (int q0 = 0; q0 < ns; q0 += G) {
    StepRaw<T> raw[G];
#pragma unroll
    for (int i = 0; i < G; ++i) step_load<T>(p, to, dof, d.mode, v0 + (q0 + i) * kRsStep, raw[i]);
    __builtin_amdgcn_sched_barrier(0);  // all G steps' loads before any arithmetic
#pragma unroll
    for (int i = 0; i < G; ++i) {
      if (q0 + i >= ns) break;
      float wr[8], wp[8], res, pts;
      step_weights<T>(p, d.mode, d, v0 + (q0 + i) * kRsStep, raw[i], wr, wp, res, pts);
      const float sr = __shfl(wave_incl_scan(res, lane), 63, 64);
      const float sp = __shfl(wave_incl_scan(pts, lane), 63, 64);
      if (lane == 0) hand_put(out + q0 + i, mark_sums(sr, sp));
    }
  }
}

// The token of request b from the step sums of R contiguous vocabulary
// ranges of ns steps each (range r: steps r*ns .. r*ns + ns - 1; its sums at
// sums[r * S .. r * S + ns)), one wave: lane r sums range r's steps in
// order, a wave scan orders the ranges, the crossing lane finds its step,
// and the whole wave recomputes that one step with the same arithmetic
// (step_weights) to find the lane and the logit.  Rounding that leaves no
// crossing picks the last positive weight.
template <typename T, int R, int S>
__device__ void select_token(const AccParams& p, int b, const Decision& d, int lane,
                             const float2* sums, int ns) {
  static_assert(R <= 64, "one range per lane");
  const int64_t to = trow(p, b, d.j);
  const int64_t dof = d.mode == 0 ? drow(p, b, d.j) : 0;
  const float u = p.u[(int64_t)b * (p.k + 1) + p.k];
  const float2* rs = sums + (int64_t)min(lane, R - 1) * S;
  float lr = 0.f, lp = 0.f;
#pragma unroll 4
  for (int q = 0; q < S; ++q) {
    const float2 v = (lane < R && q < ns) ? rs[q] : make_float2(0.f, 0.f);
    lr += v.x;
    lp += v.y;
  }
  const float tr = __shfl(wave_incl_scan(lr, lane), 63, 64);
  // residual summed to zero: sample the target row itself (speculative.py:163-169)
  const bool use_pt = d.mode == 1 || !(tr > 0.f);
  const int mode = use_pt ? 1 : 0;
  const float ls = use_pt ? lp : lr;
  const float incl = wave_incl_scan(ls, lane);
  const float excl = __shfl_up(incl, 1, 64);
  const float tot = __shfl(incl, 63, 64);
  const float target = u * tot;
  const uint64_t hitr = __builtin_amdgcn_ballot_w64(ls > 0.f && incl > target);
  const uint64_t posr = __builtin_amdgcn_ballot_w64(ls > 0.f);
  if (!posr) {  // degenerate row (no positive weight anywhere)
    if (lane == 0) p.emitted[(int64_t)b * (p.k + 1) + d.j] = -1;
    return;
  }
  bool fallback = !hitr;
  const int rsel = hitr ? (int)__builtin_ctzll(hitr) : 63 - (int)__builtin_clzll(posr);
  // the chosen range's step (sequential, in the order the range was summed)
  int qs = -1;
  float acc = lane == 0 ? 0.f : excl;
  if (lane == rsel) {  // the range's step sums again, summed in the same order
    for (int q = 0; q < ns; ++q) {
      const float2 v = rs[q];
      const float sq = use_pt ? v.y : v.x;
      if (qs < 0) {
        if (!fallback && sq > 0.f && acc + sq > target) qs = q;
        else acc += sq;
      }
    }
    if (qs < 0) {  // rounding: last positive step of the range
      fallback = true;
      for (int q = 0; q < ns; ++q) {
        const float2 v = rs[q];
        if ((use_pt ? v.y : v.x) > 0.f) qs = q;
      }
    }
  }
  qs = __shfl(qs, rsel, 64);
  acc = __shfl(acc, rsel, 64);
  fallback = __shfl((int)fallback, rsel, 64) != 0;
  // recompute that step exactly as it was summed
  const int v = (rsel * ns + qs) * kRsStep + 8 * lane;
  StepRaw<T> raw;
  step_load<T>(p, to, dof, d.mode, v, raw);
  float wr[8], wp[8], res, pts;
  step_weights<T>(p, mode, d, v, raw, wr, wp, res, pts);
  const float run = use_pt ? pts : res;
  const float* w = use_pt ? wp : wr;
  const float li = acc + wave_incl_scan(run, lane);
  const uint64_t hit = fallback ? 0 : __builtin_amdgcn_ballot_w64(run > 0.f && li > target);
  const uint64_t pos = __builtin_amdgcn_ballot_w64(run > 0.f);
  const int sel = hit ? (int)__builtin_ctzll(hit) : (pos ? 63 - (int)__builtin_clzll(pos) : 0);
  if (lane == sel) {
    float cum = li - run;  // exclusive prefix of this lane
    int tok = -1, last = -1;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      cum += w[e];
      if (w[e] > 0.f) {
        last = v + e;
        if (tok < 0 && cum > target) tok = v + e;
      }
    }
    p.emitted[(int64_t)b * (p.k + 1) + d.j] = (hit && tok >= 0) ? tok : last;
  }
}

// ---- stochastic acceptance in one launch (V % 8 == 0, V <= kRsMaxV) ----
//
// Workgroups 0 .. B*(2k+1)*nch - 1 are the chunk statistics of every row,
// request by request; request b's last one then runs b's decision in its
// wave 0 (outputs, rollback slots) and publishes it in three slots.  The
// kRsSplits workgroups per request after all of them poll those slots, and
// each of their waves streams one of the request's kRsRanges vocabulary
// ranges of the decided row pair into step sums; the request's last range
// workgroup picks the token from all of them and clears every slot it read.
// Every wait is on workgroups with smaller indices, which start first and
// never wait on later ones.  (Range blocks interleaved among later requests'
// statistics were measured slower: they compete with the statistics stream.)
template <typename T>
__global__ __launch_bounds__(kThreads) void stoch_fused_kernel(AccParams p) {
  __shared__ float2 s_sums[kRsRanges * kRsMaxSteps];   // the token pick's step sums
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int per_req = p.rpr * p.nch;
  const int t = blockIdx.x;
  if (t < p.B * per_req) {                         // statistics, request by request
    const int b = t / per_req;
    const int sub = t - b * per_req;
    const int lr = sub / p.nch;
    const bool last = sub == per_req - 1 && wave == 0;       // request b's last chunk
    const int64_t pre = last ? rollback_prefetch(p, b, lane) : -1;   // under the stream
    row_chunk_stats<T, false>(p, b, lr, sub - lr * p.nch);
    if (last) decide<T>(p, b, pre);
    return;
  }
  const int b = (t - p.B * per_req) / kRsSplits;  // then the range blocks, request by request
  const int split = t - p.B * per_req - b * kRsSplits;
  const Decision d = read_decision(p, b);           // every wave polls the three slots
  const bool draw = !(d.mode == 1 && p.bonus);     // else the decision emitted the caller's bonus
  const int ns = rs_steps(p.V);
  const int rg = split * kRsWaves + wave;
  float2* sums = p.rsum + (int64_t)b * kRsRanges * kRsMaxSteps;
  if (draw) {
    stream_step_sums<T>(p, d, trow(p, b, d.j), d.mode == 0 ? drow(p, b, d.j) : 0, ns,
                        rg * ns * kRsStep + 8 * lane, lane, sums + rg * kRsMaxSteps);
  } else if (lane < ns) {                           // mark the range done
    hand_put(sums + rg * kRsMaxSteps + lane, mark_sums(0.f, 0.f));
  }
  if (split == kRsSplits - 1 && wave == 0) {       // request b's last range workgroup
    // lane r: range r's step sums, all loads in flight, kept in LDS for the pick
    float2* mine = sums + lane * kRsMaxSteps;
    constexpr int GQ = 8;                           // loads in flight together
    for (int q0 = 0; q0 < ns; q0 += GQ) {
      uint64_t bits[GQ];
#pragma unroll
      for (int q = 0; q < GQ; ++q) bits[q] = q0 + q < ns ? hand_get_bits(mine + q0 + q) : 1;
#pragma unroll
      for (int q = 0; q < GQ; ++q) {
        if (q0 + q < ns) {
          const uint64_t v = repoll(p, mine + q0 + q, bits[q]);
          s_sums[lane * kRsMaxSteps + q0 + q] = unmark_sums(
              make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32))));
        }
      }
    }
    if (draw) select_token<T, kRsRanges, kRsMaxSteps>(p, b, d, lane, s_sums, ns);
    for (int q = 0; q < ns; ++q) clear_slot(mine + q);
    if (lane == 0) clear_slots3(dec_slots(p, b));  // every range workgroup has read it
  }
}

struct Layout {
  int rows, nch, cs, nch2, cs2;
  int64_t stats_off, dec_off, psum_off, rsum_off, xlog_off, total;
};

Layout layout(int B, int k, int V, bool greedy) {
  Layout L;
  const int rpr = greedy ? k + 1 : 2 * k + 1;
  L.rows = B * rpr;
  // a request's chunk records fit one wave's two registers per lane
  const int max_ch = std::max(1, std::min({kMaxChunks, (V + 2047) / 2048, kRecCap / rpr}));
  // at least kTargetWgs workgroups, and chunks of at most about one batch
  // of loads per thread (8 loads greedy, 12 stochastic): measured best at
  // B 64, k 4 and k 8 (V 151,936 and 128,256)
  const int cs_target = greedy ? 12288 : 20480;
  L.nch = std::max(1, std::min(max_ch, std::max((V + cs_target - 1) / cs_target,
                                               (kTargetWgs + L.rows - 1) / std::max(1, L.rows))));
  L.cs = ((V + L.nch - 1) / L.nch + 7) / 8 * 8;
  L.nch = (V + L.cs - 1) / L.cs;
  L.nch2 = std::max(1, std::min(max_ch, (kTargetWgs + B - 1) / std::max(1, B)));
  L.nch2 = std::min(kMaxChunks, std::max(L.nch2, (V + 8 * kSelThreads - 1) / (8 * kSelThreads)));
  L.cs2 = ((V + L.nch2 - 1) / L.nch2 + 7) / 8 * 8;
  L.nch2 = (V + L.cs2 - 1) / L.cs2;
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  const int rows_max = B * (2 * k + 1);  // one workspace serves both modes
  L.stats_off = kWorkspaceHeaderBytes;
  L.dec_off = L.stats_off + al((int64_t)rows_max * kMaxChunks * 8);
  L.psum_off = L.dec_off + al((int64_t)B * kDecStride * 4);
  L.rsum_off = L.psum_off + al((int64_t)B * kMaxChunks * 4);
  L.xlog_off = L.rsum_off + al((int64_t)B * kRsRanges * kRsMaxSteps * 8);
  L.total = L.xlog_off + al((int64_t)rows_max * 8);
  return L;
}

// The two-launch stochastic tail needs whole 8-logit vectors everywhere.
bool rs_path(const AccParams& p) {
  return p.V <= kRsMaxV && p.V % 8 == 0 &&
         (p.t_req | p.t_row | (p.dl ? (p.d_req | p.d_row) : 0)) % 8 == 0;
}

template <typename T>
int32_t launch_accept(const AccParams& p, int rows, hipStream_t s) {
  dim3 g1(p.nch, rows);
  if (p.greedy) {
    hipLaunchKernelGGL((greedy_fused_kernel<T>), g1, dim3(kThreads), 0, s, p);
    return launch_status("greedy_fused_kernel");
  }
  if (rs_path(p)) {
    hipLaunchKernelGGL((stoch_fused_kernel<T>), dim3(rows * p.nch + p.B * kRsSplits),
                       dim3(kThreads), 0, s, p);
    return launch_status("stoch_fused_kernel");
  }
  hipLaunchKernelGGL((stats_kernel<T, false>), g1, dim3(kThreads), 0, s, p);
  int32_t rc = launch_status("stats_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL((decide_kernel<T>), dim3(p.B), dim3(64), 0, s, p);
  rc = launch_status("decide_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL((sum_kernel<T>), dim3(p.nch2, p.B), dim3(kThreads), 0, s, p);
  rc = launch_status("sum_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL((select_kernel<T>), dim3(p.B), dim3(kSelThreads), 0, s, p);
  return launch_status("select_kernel");
}

}  // namespace
}  // namespace nsg

using namespace nsg;

extern "C" int64_t nsg_spec_accept_workspace_bytes(int32_t batch, int32_t k, int32_t vocab) {
  if (batch < 0 || k < 0 || vocab <= 0) return -1;
  return layout(batch, k, vocab, false).total;
}

namespace nsg {
namespace {

// The body of both acceptance entry points: argument checks, the workspace
// layout and the launches.  `flags` receives the device-detected error bits.
int32_t accept_impl(const void* target_logits, int64_t target_req_stride,
                    int64_t target_row_stride, const void* draft_logits,
                    int64_t draft_req_stride, int64_t draft_row_stride, int32_t logits_dtype,
                    const int64_t* draft_tokens, const float* uniforms,
                    const int64_t* bonus_tokens, int32_t batch, int32_t k, int32_t vocab,
                    float temperature, const int32_t* kv_indptr, const int32_t* kv_indices,
                    const int32_t* start_pos, int32_t page_size, int32_t* num_emitted,
                    int64_t* emitted, int64_t* rollback_slots, void* workspace,
                    int64_t workspace_bytes, int* flags, nsg_stream_t stream) {
  NSG_CHECK_ARG(batch >= 0 && batch <= kMaxBatch, "batch %d outside [0, %d]", batch, kMaxBatch);
  NSG_CHECK_ARG(k >= 0 && k <= kMaxK, "k %d outside [0, %d]", k, kMaxK);
  NSG_CHECK_ARG(vocab > 0, "vocab %d", vocab);
  NSG_CHECK_ARG(logits_dtype == 0 || logits_dtype == 1, "logits_dtype %d (0 bf16, 1 fp32)",
                logits_dtype);
  if (batch == 0) {
    clear_error();
    return NSG_OK;
  }
  const bool greedy = temperature < 1e-6f;
  NSG_CHECK_ARG(target_logits && num_emitted && emitted && workspace, "null pointer argument");
  NSG_CHECK_ARG(greedy || k == 0 || draft_logits, "draft_logits required when temperature > 0");
  NSG_CHECK_ARG(k == 0 || draft_tokens, "draft_tokens required when k > 0");
  NSG_CHECK_ARG(greedy || uniforms, "uniforms required when temperature > 0");
  NSG_CHECK_ARG(target_row_stride >= vocab && target_req_stride >= (int64_t)(k + 1) * vocab,
                "target logits strides too small");
  NSG_CHECK_ARG(greedy || k == 0 || (draft_row_stride >= vocab &&
                                     draft_req_stride >= (int64_t)k * vocab),
                "draft logits strides too small");
  int log2P = 0;
  if (rollback_slots && k > 0) {
    NSG_CHECK_ARG(kv_indptr && kv_indices && start_pos,
                  "rollback slots need kv_indptr, kv_indices and start_pos");
    NSG_CHECK_ARG(page_size > 0 && (page_size & (page_size - 1)) == 0,
                  "page_size %d must be a power of two", page_size);
    while ((1 << log2P) < page_size) ++log2P;
  }
  const Layout L = layout(batch, k, vocab, greedy);
  if (workspace_bytes < L.total) {
    set_error("workspace has %lld bytes, needs %lld", (long long)workspace_bytes,
              (long long)L.total);
    return NSG_ERR_WORKSPACE;
  }
  AccParams p{};
  p.tl = target_logits;
  p.t_req = target_req_stride;
  p.t_row = target_row_stride;
  p.dl = draft_logits;
  p.d_req = draft_req_stride;
  p.d_row = draft_row_stride;
  p.dtok = draft_tokens;
  p.u = uniforms;
  p.bonus = greedy ? nullptr : bonus_tokens;
  p.B = batch;
  p.k = k;
  p.V = vocab;
  p.c = greedy ? 0.f : kLog2e / temperature;
  p.greedy = greedy ? 1 : 0;
  p.rpr = greedy ? k + 1 : 2 * k + 1;
  p.kv_indptr = kv_indptr;
  p.kv_indices = kv_indices;
  p.start_pos = start_pos;
  p.log2P = log2P;
  p.n_out = num_emitted;
  p.emitted = emitted;
  p.rollback = k > 0 ? rollback_slots : nullptr;
  p.nch = L.nch;
  p.cs = L.cs;
  p.nch2 = L.nch2;
  p.cs2 = L.cs2;
  char* ws = static_cast<char*>(workspace);
  p.flags = flags;
  p.stats = reinterpret_cast<float2*>(ws + L.stats_off);
  p.dec = reinterpret_cast<float*>(ws + L.dec_off);
  p.psum = reinterpret_cast<float*>(ws + L.psum_off);
  p.rsum = reinterpret_cast<float2*>(ws + L.rsum_off);
  p.xlog = reinterpret_cast<float2*>(ws + L.xlog_off);
  // 16-byte vector loads need 16-byte aligned bases; rows are checked per row
  const uintptr_t mis = reinterpret_cast<uintptr_t>(target_logits) |
                        (greedy ? 0 : reinterpret_cast<uintptr_t>(draft_logits));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (logits_dtype == 0) {
    if (mis & 15) {
      set_error("logits base pointers must be 16-byte aligned");
      return NSG_ERR_ARG;
    }
    return launch_accept<bf16>(p, L.rows, s);
  }
  if (mis & 15) {
    set_error("logits base pointers must be 16-byte aligned");
    return NSG_ERR_ARG;
  }
  return launch_accept<float>(p, L.rows, s);
}

}  // namespace
}  // namespace nsg

extern "C" int32_t nsg_spec_accept(const void* target_logits, int64_t target_req_stride,
                                   int64_t target_row_stride, const void* draft_logits,
                                   int64_t draft_req_stride, int64_t draft_row_stride,
                                   int32_t logits_dtype, const int64_t* draft_tokens,
                                   const float* uniforms, const int64_t* bonus_tokens,
                                   int32_t batch, int32_t k,
                                   int32_t vocab, float temperature, const int32_t* kv_indptr,
                                   const int32_t* kv_indices, const int32_t* start_pos,
                                   int32_t page_size, int32_t* num_emitted, int64_t* emitted,
                                   int64_t* rollback_slots, void* workspace,
                                   int64_t workspace_bytes, nsg_stream_t stream) {
  return accept_impl(target_logits, target_req_stride, target_row_stride, draft_logits,
                     draft_req_stride, draft_row_stride, logits_dtype, draft_tokens, uniforms,
                     bonus_tokens, batch, k, vocab, temperature, kv_indptr, kv_indices, start_pos,
                     page_size, num_emitted, emitted, rollback_slots, workspace, workspace_bytes,
                     static_cast<int*>(workspace), stream);
}

// ---- the allocation-free variant ----
//
// Its workspace is `scratch`, a static device array of this file: every GPU
// the library runs on holds one copy of kNoAllocScratchBytes until the
// process ends.  In host code `scratch` names a host-side stand-in, so the
// array is only ever reached through the device address hipGetSymbolAddress
// returns, looked up once per device with that device current and kept in
// g_scratch_ptr.  Every call on a GPU shares that GPU's array (the kernels
// rewrite what they read and leave their counters at zero), so calls that
// overlap on one GPU race.
namespace {

constexpr int64_t kNoAllocScratchBytes = 8ll << 20;
constexpr int kMaxScratchDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

int32_t scratch_address(void** out) {
  int dev = -1;
  NSG_CHECK_HIP(hipGetDevice(&dev));
  NSG_CHECK_ARG(dev >= 0 && dev < kMaxScratchDevices, "device %d outside [0, %d)", dev,
                kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      set_error("hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                hipGetErrorString(e));
      return NSG_ERR_HIP;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return NSG_OK;
}

}  // namespace

extern "C" int64_t nsg_spec_accept_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

namespace {
// Zeroes n 16-byte words from p (a plain fill kernel rather than a memset
// node, so that a reset enqueued on a capturing stream replays correctly).
__global__ __launch_bounds__(256) void clear_words_kernel(u32x4* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    p[i] = u32x4{0u, 0u, 0u, 0u};
}
}  // namespace

extern "C" int32_t nsg_spec_accept_noalloc_reset(nsg_stream_t stream) {
  void* ws = nullptr;
  const int32_t rc = scratch_address(&ws);
  if (rc) return rc;
  const int64_t words = kNoAllocScratchBytes / 16;
  hipLaunchKernelGGL(clear_words_kernel, dim3(512), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<u32x4*>(ws), words);
  return launch_status("clear_words_kernel");
}

extern "C" int32_t nsg_spec_accept_noalloc(
    const void* target_logits, int64_t target_req_stride, int64_t target_row_stride,
    const void* draft_logits, int64_t draft_req_stride, int64_t draft_row_stride,
    int32_t logits_dtype, const int64_t* draft_tokens, const float* uniforms,
    const int64_t* bonus_tokens, int32_t batch, int32_t k, int32_t vocab, float temperature,
    const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* start_pos,
    int32_t page_size, int32_t* num_emitted, int64_t* emitted, int64_t* rollback_slots,
    int32_t* flags, nsg_stream_t stream) {
  NSG_CHECK_ARG(batch >= 0 && k >= 0 && vocab > 0, "batch %d, k %d, vocab %d", batch, k, vocab);
  const int64_t need = layout(batch, k, vocab, false).total;
  if (need > kNoAllocScratchBytes) {
    set_error("batch %d, k %d, vocab %d needs %lld bytes of workspace; the static scratch of "
              "nsg_spec_accept_noalloc holds %lld", batch, k, vocab, (long long)need,
              (long long)kNoAllocScratchBytes);
    return NSG_ERR_WORKSPACE;
  }
  void* ws = nullptr;
  const int32_t rc = scratch_address(&ws);
  if (rc) return rc;
  // without a caller word the flags land in the scratch header, unread
  return accept_impl(target_logits, target_req_stride, target_row_stride, draft_logits,
                     draft_req_stride, draft_row_stride, logits_dtype, draft_tokens, uniforms,
                     bonus_tokens, batch, k, vocab, temperature, kv_indptr, kv_indices, start_pos,
                     page_size, num_emitted, emitted, rollback_slots, ws, kNoAllocScratchBytes,
                     flags ? flags : static_cast<int*>(ws), stream);
}

// ---- greedy acceptance from the target rows' tokens ----
// The greedy rule of greedy_finalize with each target row's argmax already
// computed (nsg_linear_argmax in the verify forward's lm_head): one wave per
// request, lane i <= k holding target token i and lane i < k draft token i.
namespace nsg {
namespace {
// The rule for request b on one wave, lane i <= k holding target token t.
__device__ __forceinline__ void greedy_rule(const AccParams& p, int b, int lane, int64_t t,
                                            int64_t ds_b, int64_t ds_j, int64_t pre) {
  const int k = p.k;
  int64_t x = -1;
  if (lane < k) x = p.dtok[b * ds_b + lane * ds_j];
  if (lane < k && (x < 0 || x >= p.V) && p.flags) atomicOr(p.flags, 4);  // never matches
  const uint64_t miss = __builtin_amdgcn_ballot_w64(lane < k && x != t);
  const int j = miss ? (int)__builtin_ctzll(miss) : k;  // first mismatch, or k
  if (lane <= k) p.emitted[(int64_t)b * (k + 1) + lane] = lane < j ? x : (lane == j ? t : -1);
  if (lane == 0) p.n_out[b] = j + 1;
  rollback_lanes(p, b, j + 1, lane, pre);
}

__global__ __launch_bounds__(64) void greedy_tokens_kernel(AccParams p,
                                                           const int64_t* __restrict__ ttok,
                                                           int64_t ds_b, int64_t ds_j) {
  const int b = blockIdx.x;
  const int lane = threadIdx.x;
  const int k = p.k;
  const int64_t pre = rollback_prefetch(p, b, lane);
  const int64_t t = lane <= k ? ttok[(int64_t)b * (k + 1) + lane] : -1;
  greedy_rule(p, b, lane, t, ds_b, ds_j, pre);
}

// The same with each target row's token reduced from the lm_head's argmax
// keys in this launch (no separate reduction launch): wave w of the request's
// workgroup reduces rows w, w + waves, ... into LDS (and ttok_out, when
// given), then wave 0 applies the rule.
constexpr int kKeyWaves = 16;
__global__ __launch_bounds__(64 * kKeyWaves) void greedy_keys_kernel(
    AccParams p, const uint64_t* __restrict__ keys, int key_cols, int64_t* __restrict__ ttok_out,
    int64_t ds_b, int64_t ds_j) {
  __shared__ int64_t tok[kMaxK + 1];
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const int k = p.k;
  int64_t pre = 0;
  if (wave == 0) pre = rollback_prefetch(p, b, lane);
  for (int row = wave; row <= k; row += waves) {
    const int64_t r = (int64_t)b * (k + 1) + row;
    const int64_t t = key_token(wave_max_key(keys + r * key_cols, key_cols, lane));
    if (lane == 0) {
      tok[row] = t;
      if (ttok_out) ttok_out[r] = t;
    }
  }
  __syncthreads();
  if (wave != 0) return;
  greedy_rule(p, b, lane, lane <= k ? tok[lane] : -1, ds_b, ds_j, pre);
}
}  // namespace
}  // namespace nsg

namespace {

// The shared checks and parameters of the two greedy-from-argmax entries.
int32_t greedy_params(const int64_t* draft_tokens, int64_t draft_stride_b,
                      int64_t draft_stride_j, int32_t batch, int32_t k, int32_t vocab,
                      const int32_t* kv_indptr, const int32_t* kv_indices,
                      const int32_t* start_pos, int32_t page_size, int32_t* num_emitted,
                      int64_t* emitted, int64_t* rollback_slots, int32_t* flags, AccParams* out) {
  NSG_CHECK_ARG(num_emitted && emitted, "null pointer argument");
  NSG_CHECK_ARG(k == 0 || draft_tokens, "draft_tokens required when k > 0");
  NSG_CHECK_ARG(k == 0 || (draft_stride_b >= 0 && draft_stride_j >= 0),
                "draft token strides %lld, %lld", (long long)draft_stride_b,
                (long long)draft_stride_j);
  int log2P = 0;
  if (rollback_slots && k > 0) {
    NSG_CHECK_ARG(kv_indptr && kv_indices && start_pos,
                  "rollback slots need kv_indptr, kv_indices and start_pos");
    NSG_CHECK_ARG(page_size > 0 && (page_size & (page_size - 1)) == 0,
                  "page_size %d must be a power of two", page_size);
    while ((1 << log2P) < page_size) ++log2P;
  }
  AccParams p{};
  p.dtok = draft_tokens;
  p.B = batch;
  p.k = k;
  p.V = vocab;
  p.greedy = 1;
  p.kv_indptr = kv_indptr;
  p.kv_indices = kv_indices;
  p.start_pos = start_pos;
  p.log2P = log2P;
  p.n_out = num_emitted;
  p.emitted = emitted;
  p.rollback = k > 0 ? rollback_slots : nullptr;
  p.flags = flags;
  *out = p;
  return NSG_OK;
}

}  // namespace

extern "C" int32_t nsg_spec_accept_greedy_tokens(const int64_t* target_tokens,
                                                 const int64_t* draft_tokens,
                                                 int64_t draft_stride_b, int64_t draft_stride_j,
                                                 int32_t batch, int32_t k, int32_t vocab,
                                                 const int32_t* kv_indptr,
                                                 const int32_t* kv_indices,
                                                 const int32_t* start_pos, int32_t page_size,
                                                 int32_t* num_emitted, int64_t* emitted,
                                                 int64_t* rollback_slots, int32_t* flags,
                                                 nsg_stream_t stream) {
  NSG_CHECK_ARG(batch >= 0 && batch <= kMaxBatch, "batch %d outside [0, %d]", batch, kMaxBatch);
  NSG_CHECK_ARG(k >= 0 && k <= kMaxK, "k %d outside [0, %d]", k, kMaxK);
  NSG_CHECK_ARG(vocab > 0, "vocab %d", vocab);
  if (batch == 0) {
    clear_error();
    return NSG_OK;
  }
  NSG_CHECK_ARG(target_tokens, "null pointer argument");
  AccParams p{};
  if (int32_t rc = greedy_params(draft_tokens, draft_stride_b, draft_stride_j, batch, k, vocab,
                                 kv_indptr, kv_indices, start_pos, page_size, num_emitted,
                                 emitted, rollback_slots, flags, &p))
    return rc;
  hipLaunchKernelGGL(greedy_tokens_kernel, dim3(batch), dim3(64), 0,
                     static_cast<hipStream_t>(stream), p, target_tokens, draft_stride_b,
                     draft_stride_j);
  return launch_status("greedy_tokens_kernel");
}

extern "C" int32_t nsg_spec_accept_greedy_keys(const void* target_keys, int32_t key_cols,
                                               int64_t* target_tokens_out,
                                               const int64_t* draft_tokens,
                                               int64_t draft_stride_b, int64_t draft_stride_j,
                                               int32_t batch, int32_t k, int32_t vocab,
                                               const int32_t* kv_indptr,
                                               const int32_t* kv_indices,
                                               const int32_t* start_pos, int32_t page_size,
                                               int32_t* num_emitted, int64_t* emitted,
                                               int64_t* rollback_slots, int32_t* flags,
                                               nsg_stream_t stream) {
  NSG_CHECK_ARG(batch >= 0 && batch <= kMaxBatch, "batch %d outside [0, %d]", batch, kMaxBatch);
  NSG_CHECK_ARG(k >= 0 && k <= kMaxK, "k %d outside [0, %d]", k, kMaxK);
  NSG_CHECK_ARG(vocab > 0, "vocab %d", vocab);
  if (batch == 0) {
    clear_error();
    return NSG_OK;
  }
  NSG_CHECK_ARG(target_keys && key_cols >= 1 && (uintptr_t)target_keys % 8 == 0,
                "target_keys (8-byte aligned) and key_cols %d >= 1 required", key_cols);
  AccParams p{};
  if (int32_t rc = greedy_params(draft_tokens, draft_stride_b, draft_stride_j, batch, k, vocab,
                                 kv_indptr, kv_indices, start_pos, page_size, num_emitted,
                                 emitted, rollback_slots, flags, &p))
    return rc;
  const int waves = std::min(k + 1, kKeyWaves);
  hipLaunchKernelGGL(greedy_keys_kernel, dim3(batch), dim3(64 * waves), 0,
                     static_cast<hipStream_t>(stream), p,
                     static_cast<const uint64_t*>(target_keys), key_cols, target_tokens_out,
                     draft_stride_b, draft_stride_j);
  return launch_status("greedy_keys_kernel");
}

extern "C" int32_t nsg_spec_accept_check_flags(void* workspace, int64_t workspace_bytes,
                                               int32_t* flags_h, nsg_stream_t stream) {
  NSG_CHECK_ARG(workspace && flags_h, "null argument");
  NSG_CHECK_ARG(workspace_bytes >= (int64_t)sizeof(int32_t), "workspace_bytes %lld",
                (long long)workspace_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  NSG_CHECK_HIP(hipMemcpyAsync(flags_h, workspace, sizeof(int32_t), hipMemcpyDeviceToHost, s));
  NSG_CHECK_HIP(hipStreamSynchronize(s));
  // a hand-off gave up (bit 3): published slots may be left behind anywhere
  // in the body, so the whole workspace is cleared, not only the flag word
  const int64_t n = (*flags_h & 8) ? workspace_bytes : (int64_t)sizeof(int32_t);
  NSG_CHECK_HIP(hipMemsetAsync(workspace, 0, n, s));
  NSG_CHECK_HIP(hipStreamSynchronize(s));
  clear_error();
  return NSG_OK;
}
