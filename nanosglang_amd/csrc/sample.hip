// Temperature / top-k / top-p sampling of one token per logits row on gfx950.
//
// Reference: nano_sglang/engine/sampling.py:25-50 (sample_token: argmax when
// T < 1e-6) and :71-88 (_sample_pytorch):
//   logits / T;
//   top-k: mask logits < the k-th largest (ties with it are kept);
//   top-p: sort descending, p = softmax; mask sorted position i when
//     sum_{j<i} p_j >= top_p (the exclusive cumulative);
//   softmax, multinomial.
// Here the rule is evaluated exactly: every token's weight
// w = 2^(x*log2(e)/T - max*log2(e)/T) is held in 2^-40 fixed point (uint64),
// so every mass is an exact integer sum, independent of summation order; the
// top-p comparison is (double)prefix < top_p * (double)Z.  Among equal logits
// at the top-p boundary, the lowest vocabulary indices come first (torch's
// sort leaves that order unspecified).  The token is drawn by inverse CDF in
// vocabulary order: the first index whose inclusive kept-mass prefix exceeds
// floor(u * Z_kept).
//
// No sort: thresholds are found by radix selection over an order-preserving
// integer key of the logit (16 bits for bf16, 32 for fp32), one byte per
// level, most significant first.  Launches (the grid covers every row and
// chunk of the vocabulary; no workgroup waits on another inside a launch):
//   max_kernel   (chunks, rows): chunk max key and its first index; clears the
//                row's histograms.
//   hist_kernel  (chunks, rows), once per stage (top-k levels, then top-p
//                levels): resolves the previous stage from its histogram
//                (every workgroup, identically), then adds its chunk's
//                counts (top-k) or masses (top-p) per key byte into the row's
//                256-bin histogram (four LDS copies per wave, then
//                device-scope atomics).
//   sums_kernel  (chunks, rows): resolves the last stage -> the boundary key
//                v*, how many of its ties are kept (m*) and their weight; per
//                chunk: mass of keys > v* and count of keys == v*.
//   select_kernel (rows): kept mass per chunk (ties ranked in vocabulary
//                order), the chunk holding the draw, then a block scan of that
//                chunk.
// Greedy rows use max_kernel and select_kernel only.
#include <climits>
#include <cstring>
#include <type_traits>

#include "common.hpp"

namespace nsg {
namespace {

constexpr int kSThreads = 256;
constexpr int kSWaves = kSThreads / 64;
constexpr int kSMaxChunks = 64;
constexpr int kSTargetWgs = 1024;
constexpr int kBins = 256;
constexpr int kMaxStages = 8;   // 4 levels (fp32 keys) x 2 filters
constexpr int kMaxRows = 1 << 16;
constexpr int kPreTiles = 3;    // tiles of 8 x 256 elements loaded before a stage resolves
constexpr float kFix = 1099511627776.f;  // 2^40: fixed-point scale of the weights
constexpr float kLog2eS = 1.4426950408889634f;

typedef unsigned long long u64;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Per-row state after a stage has been resolved (written by the first
// workgroup of the launch that resolved it, read by later launches).
struct SmpState {
  uint32_t prefix;  // key bits fixed so far for the current filter
  uint32_t tk;      // top-k threshold key (every key >= tk is kept by top-k)
  uint32_t vs;      // final: boundary key v*
  uint32_t ms;      // final: how many tokens with key == v* are kept (lowest indices)
  u64 above_c;      // count of keys above the current prefix range
  u64 above_m;      // mass of keys above the current prefix range
  u64 ws;           // final: weight of one token with key == v*
  double pz;        // top_p * Z_k
};

struct SmpParams {
  const void* x;
  int64_t stride;
  int rows, V;
  float c;  // log2(e) / T
  int greedy;
  int K;    // top-k (0 = off)
  double P; // top-p (>= 1 = off)
  const float* u;
  int64_t u_stride;
  int64_t* out;
  int nch, cs;
  int levels;  // key bytes
  int nk, np;  // stages of each filter (0 or levels)
  uint2* cmax;        // [rows][nch] (max key, first index)
  uint32_t* hcnt;     // [rows][kMaxStages][256]
  u64* hmass;         // [rows][kMaxStages][256]
  SmpState* st;       // [rows][kMaxStages + 1]
  u64* csum;          // [rows][nch]
  uint32_t* ceq;      // [rows][nch]
};

template <typename T>
struct SKey;
template <>
struct SKey<bf16> {
  static constexpr int kBits = 16;
  static __device__ __forceinline__ uint32_t key(uint32_t b) {
    if (b == 0x8000u) b = 0;  // -0 == +0
    return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
  }
  static __device__ __forceinline__ float val(uint32_t b) { return __uint_as_float(b << 16); }
  static __device__ __forceinline__ uint32_t bits_of_key(uint32_t k) {
    return (k & 0x8000u) ? (k & 0x7FFFu) : (~k & 0xFFFFu);
  }
  // raw bits of 8 consecutive elements e .. e+7 (those >= end are unused)
  static __device__ __forceinline__ void load8(const void* row, int e, int end, bool vec,
                                               uint32_t* r) {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(row);
    if (vec && e + 8 <= end) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(p + e);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        r[2 * i] = v[i] & 0xFFFFu;
        r[2 * i + 1] = v[i] >> 16;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) r[i] = e + i < end ? p[e + i] : 0u;
    }
  }
};
template <>
struct SKey<float> {
  static constexpr int kBits = 32;
  static __device__ __forceinline__ uint32_t key(uint32_t b) {
    if (b == 0x80000000u) b = 0;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  }
  static __device__ __forceinline__ float val(uint32_t b) { return __uint_as_float(b); }
  static __device__ __forceinline__ uint32_t bits_of_key(uint32_t k) {
    return (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  }
  static __device__ __forceinline__ void load8(const void* row, int e, int end, bool vec,
                                               uint32_t* r) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(row);
    if (vec && e + 8 <= end) {
      const u32x4 a = *reinterpret_cast<const u32x4*>(p + e);
      const u32x4 b = *reinterpret_cast<const u32x4*>(p + e + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        r[i] = a[i];
        r[4 + i] = b[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) r[i] = e + i < end ? p[e + i] : 0u;
    }
  }
};

__device__ __forceinline__ u64 weight_of(float v, float c, float mc) {
  const float w = __builtin_amdgcn_exp2f(__builtin_fmaf(v, c, -mc));
  return (u64)(w * kFix);
}

template <typename T>
__device__ __forceinline__ const void* row_ptr(const SmpParams& p, int row) {
  return reinterpret_cast<const T*>(p.x) + (int64_t)row * p.stride;
}

__device__ __forceinline__ u64 shfl_u64(u64 v, int src) {
  const uint32_t lo = __shfl((uint32_t)v, src, 64);
  const uint32_t hi = __shfl((uint32_t)(v >> 32), src, 64);
  return ((u64)hi << 32) | lo;
}
__device__ __forceinline__ u64 shfl_up_u64(u64 v, int d) {
  const uint32_t lo = __shfl_up((uint32_t)v, d, 64);
  const uint32_t hi = __shfl_up((uint32_t)(v >> 32), d, 64);
  return ((u64)hi << 32) | lo;
}
__device__ __forceinline__ u64 wave_incl_scan_u64(u64 x, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const u64 y = shfl_up_u64(x, o);
    if (lane >= o) x += y;
  }
  return x;
}

// Row max key (and its first index) from the chunk records; one wave.
__device__ __forceinline__ uint2 row_max(const SmpParams& p, int row, int lane) {
  uint2 best = make_uint2(0u, 0x7FFFFFFFu);
  for (int c = lane; c < p.nch; c += 64) {
    const uint2 v = p.cmax[(int64_t)row * p.nch + c];
    if (v.x > best.x || (v.x == best.x && v.y < best.y)) best = v;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint32_t kx = __shfl_xor(best.x, o, 64);
    const uint32_t ky = __shfl_xor(best.y, o, 64);
    if (kx > best.x || (kx == best.x && ky < best.y)) best = make_uint2(kx, ky);
  }
  return best;
}

template <typename T>
__device__ __forceinline__ float max_c(const SmpParams& p, uint32_t maxkey) {
  return SKey<T>::val(SKey<T>::bits_of_key(maxkey)) * p.c;
}

// Resolves stage s of a row from its histogram, given the state before it,
// and returns the state after it.  Top-k stages hold counts, top-p stages
// masses.  Executed by one whole wave; lane l holds bins 4l .. 4l+3.
template <typename T>
__device__ SmpState resolve_stage(const SmpParams& p, int row, int s, SmpState in, float mc) {
  const int lane = threadIdx.x & 63;
  const bool topk = s < p.nk;
  const int level = topk ? s : s - p.nk;
  const int64_t h0 = ((int64_t)row * kMaxStages + s) * kBins + 4 * lane;
  u64 h[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) h[j] = topk ? (u64)p.hcnt[h0 + j] : p.hmass[h0 + j];
  SmpState o = in;
  const u64 incl = wave_incl_scan_u64(h[0] + h[1] + h[2] + h[3], lane);
  const u64 tot = shfl_u64(incl, 63);
  if (!topk && level == 0) {  // Z_k: every key >= tk, which this histogram holds
    o.pz = p.P * (double)tot;
    o.above_m = 0;
  }
  // cumulative from the top bin down; a = everything above this lane's bins
  u64 a = (topk ? o.above_c : o.above_m) + (tot - incl);
  int hit = -1;
  u64 ha = 0;
#pragma unroll
  for (int j = 3; j >= 0; --j) {
    const u64 n = a + h[j];
    const bool reach = topk ? n >= (u64)p.K : (double)n >= o.pz;
    if (hit < 0 && reach) {
      hit = 4 * lane + j;
      ha = a;
    }
    a = n;
  }
  // lanes below the crossing reach too: the crossing is the highest lane hit
  const uint64_t bal = __builtin_amdgcn_ballot_w64(hit >= 0);
  int src = bal ? 63 - (int)__builtin_clzll(bal) : -1;
  if (src < 0) {
    // unreachable for exact integer counts and masses (a level's bins always
    // hold the crossing); keep a defined result: the lowest bin
    src = 0;
    if (lane == 0) {
      hit = 0;
      ha = (topk ? o.above_c : o.above_m) + (tot - incl) + h[3] + h[2] + h[1];
    }
  }
  const int bin = __shfl(hit, src, 64);
  const u64 above = shfl_u64(ha, src);
  if (topk) o.above_c = above;
  else o.above_m = above;
  o.prefix = (in.prefix << 8) | (uint32_t)bin;
  if (level == p.levels - 1) {
    const uint32_t key = o.prefix;
    const u64 W = weight_of(SKey<T>::val(SKey<T>::bits_of_key(key)), p.c, mc);
    if (topk) {
      // every key >= tk is kept by top-k; without top-p that is the boundary
      o.tk = key;
      o.vs = key;
      o.ms = UINT_MAX;
      o.ws = W;
      o.prefix = 0;
      o.above_c = 0;
      o.above_m = 0;
    } else {
      // ties of v* kept: the m with (double)(S + m W) < pz, lowest indices
      // first (m = 0 always is); past their count every tie is kept
      const u64 S = o.above_m;
      u64 m0 = UINT_MAX;
      if (W > 0) {
        const double need = (o.pz - (double)S) / (double)W;
        m0 = need <= 1.0 ? 1 : (need >= (double)p.V ? (u64)p.V : (u64)ceil(need));
        while (m0 < (u64)p.V && (double)(S + m0 * W) < o.pz) ++m0;
        while (m0 > 1 && !((double)(S + (m0 - 1) * W) < o.pz)) --m0;
      }
      o.vs = key;
      o.ms = (uint32_t)m0;
      o.ws = W;
    }
  }
  return o;
}

template <typename T>
__device__ SmpState initial_state(const SmpParams& p) {
  SmpState s;
  s.prefix = 0;
  s.tk = 0;
  s.vs = 0;
  s.ms = UINT_MAX;
  s.above_c = 0;
  s.above_m = 0;
  s.ws = 0;
  s.pz = 0.0;
  return s;
}

// State before stage s (s = 0: initial; else the record stage s-1's launch
// left, resolved with histogram s-1).  One wave; the first workgroup of the
// row stores it for the next launch.
template <typename T>
__device__ SmpState state_before(const SmpParams& p, int row, int s, bool store, float mc) {
  SmpState st = initial_state<T>(p);
  if (s > 0)
    st = resolve_stage<T>(p, row, s - 1, p.st[(int64_t)row * (kMaxStages + 1) + s - 1], mc);
  if (store && (threadIdx.x & 63) == 0) p.st[(int64_t)row * (kMaxStages + 1) + s] = st;
  return st;
}

// ---- launch 1: chunk max key (first index) and histogram clearing ----
template <typename T>
__global__ __launch_bounds__(kSThreads) void max_kernel(SmpParams p, bool vec) {
  const int ch = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const int nst = p.nk + p.np;
  for (int i = ch * kSThreads + tid; i < nst * kBins; i += p.nch * kSThreads) {
    p.hcnt[(int64_t)row * kMaxStages * kBins + i] = 0;
    p.hmass[(int64_t)row * kMaxStages * kBins + i] = 0;
  }
  const void* x = row_ptr<T>(p, row);
  const int c0 = ch * p.cs, c1 = min(p.V, c0 + p.cs);
  uint32_t bk = 0, bi = 0x7FFFFFFFu;
  for (int e = c0 + 8 * tid; e < c1; e += 8 * kSThreads) {
    uint32_t r[8];
    SKey<T>::load8(x, e, c1, vec, r);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t k = SKey<T>::key(r[i]);
      if (e + i < c1 && (k > bk || bi == 0x7FFFFFFFu)) {
        bk = k;
        bi = e + i;
      }
    }
  }
  __shared__ uint2 sh[kSWaves];
  const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint32_t kx = __shfl_xor(bk, o, 64), ix = __shfl_xor(bi, o, 64);
    if (ix != 0x7FFFFFFFu && (bi == 0x7FFFFFFFu || kx > bk || (kx == bk && ix < bi))) {
      bk = kx;
      bi = ix;
    }
  }
  if (lane == 0) sh[wave] = make_uint2(bk, bi);
  __syncthreads();
  if (tid == 0) {
    uint2 b = sh[0];
    for (int w = 1; w < kSWaves; ++w) {
      const uint2 v = sh[w];
      if (v.y != 0x7FFFFFFFu && (b.y == 0x7FFFFFFFu || v.x > b.x || (v.x == b.x && v.y < b.y)))
        b = v;
    }
    p.cmax[(int64_t)row * p.nch + ch] = b;
  }
}

// ---- launch 2..: one histogram stage (counts for top-k, masses for top-p) ----
template <typename T, bool kCount>
__global__ __launch_bounds__(kSThreads) void hist_kernel(SmpParams p, int s, bool vec) {
  constexpr int kCopies = 4;  // per wave, by lane & 3: a quarter of the same-bin conflicts
  typedef typename std::conditional<kCount, uint32_t, u64>::type H;
  const int ch = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  __shared__ H lh[kSWaves * kCopies][kBins];
  __shared__ SmpState s_st;
  __shared__ float s_mc;
  const void* x = row_ptr<T>(p, row);
  const int c0 = ch * p.cs, c1 = min(p.V, c0 + p.cs);
  // the chunk's first tiles are loaded while wave 0 resolves the stage
  uint32_t pre[kPreTiles][8];
#pragma unroll
  for (int t = 0; t < kPreTiles; ++t) {
    const int e = c0 + 8 * tid + t * 8 * kSThreads;
    if (e < c1) SKey<T>::load8(x, e, c1, vec, pre[t]);
  }
  for (int i = tid; i < kSWaves * kCopies * kBins; i += kSThreads) (&lh[0][0])[i] = 0;
  if (wave == 0) {
    const uint2 mk = row_max(p, row, lane);
    const float mc = max_c<T>(p, mk.x);
    const SmpState st = state_before<T>(p, row, s, ch == 0, mc);
    if (lane == 0) {
      s_st = st;
      s_mc = mc;
    }
  }
  __syncthreads();
  const SmpState st = s_st;
  const float mc = s_mc;
  const int level = kCount ? s : s - p.nk;
  const int shift = SKey<T>::kBits - 8 * (level + 1);
  const uint32_t lo_key = kCount ? 0u : st.tk;
  H* mine = lh[wave * kCopies + (lane & 3)];
  auto tile = [&](int e, const uint32_t* r) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t k = SKey<T>::key(r[i]);
      const bool match = e + i < c1 && k >= lo_key &&
                         (level == 0 || (k >> (shift + 8)) == st.prefix);
      if (match) {
        const uint32_t bin = (k >> shift) & 0xFFu;
        if (kCount) atomicAdd(&mine[bin], (H)1);
        else atomicAdd(&mine[bin], (H)weight_of(SKey<T>::val(r[i]), p.c, mc));
      }
    }
  };
#pragma unroll
  for (int t = 0; t < kPreTiles; ++t) {
    const int e = c0 + 8 * tid + t * 8 * kSThreads;
    if (e < c1) tile(e, pre[t]);
  }
  for (int e = c0 + 8 * tid + kPreTiles * 8 * kSThreads; e < c1; e += 8 * kSThreads) {
    uint32_t r[8];
    SKey<T>::load8(x, e, c1, vec, r);
    tile(e, r);
  }
  __syncthreads();
  H t = 0;
#pragma unroll
  for (int w = 0; w < kSWaves * kCopies; ++w) t += lh[w][tid];
  if (t) {
    const int64_t o = ((int64_t)row * kMaxStages + s) * kBins + tid;
    if (kCount) atomicAdd(p.hcnt + o, (uint32_t)t);
    else atomicAdd(p.hmass + o, (u64)t);
  }
}

// ---- per-chunk kept mass above v* and ties at v* ----
template <typename T>
__global__ __launch_bounds__(kSThreads) void sums_kernel(SmpParams p, bool vec) {
  const int ch = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  __shared__ SmpState s_st;
  __shared__ float s_mc;
  __shared__ u64 sm[kSWaves];
  __shared__ uint32_t sc[kSWaves];
  const void* x = row_ptr<T>(p, row);
  const int c0 = ch * p.cs, c1 = min(p.V, c0 + p.cs);
  uint32_t pre[kPreTiles][8];
#pragma unroll
  for (int t = 0; t < kPreTiles; ++t) {
    const int e = c0 + 8 * tid + t * 8 * kSThreads;
    if (e < c1) SKey<T>::load8(x, e, c1, vec, pre[t]);
  }
  if (wave == 0) {
    const uint2 mk = row_max(p, row, lane);
    const float mc = max_c<T>(p, mk.x);
    const SmpState st = state_before<T>(p, row, p.nk + p.np, ch == 0, mc);
    if (lane == 0) {
      s_st = st;
      s_mc = mc;
    }
  }
  __syncthreads();
  const uint32_t vs = s_st.vs;
  const float mc = s_mc;
  u64 m = 0;
  uint32_t n = 0;
  auto tile = [&](int e, const uint32_t* r) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (e + i >= c1) continue;
      const uint32_t k = SKey<T>::key(r[i]);
      if (k > vs) m += weight_of(SKey<T>::val(r[i]), p.c, mc);
      n += k == vs;
    }
  };
#pragma unroll
  for (int t = 0; t < kPreTiles; ++t) {
    const int e = c0 + 8 * tid + t * 8 * kSThreads;
    if (e < c1) tile(e, pre[t]);
  }
  for (int e = c0 + 8 * tid + kPreTiles * 8 * kSThreads; e < c1; e += 8 * kSThreads) {
    uint32_t r[8];
    SKey<T>::load8(x, e, c1, vec, r);
    tile(e, r);
  }
  m = shfl_u64(wave_incl_scan_u64(m, lane), 63);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) n += __shfl_xor(n, o, 64);
  if (lane == 0) {
    sm[wave] = m;
    sc[wave] = n;
  }
  __syncthreads();
  if (tid == 0) {
    u64 tm = 0;
    uint32_t tn = 0;
    for (int w = 0; w < kSWaves; ++w) {
      tm += sm[w];
      tn += sc[w];
    }
    p.csum[(int64_t)row * p.nch + ch] = tm;
    p.ceq[(int64_t)row * p.nch + ch] = tn;
  }
}

// Block exclusive scan of one uint64 per thread (fixed order); returns the
// exclusive prefix and writes the block total to *total.
__device__ u64 block_excl_scan_u64(u64 x, u64* sh, u64* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const u64 incl = wave_incl_scan_u64(x, lane);
  if (lane == 63) sh[wave] = incl;
  __syncthreads();
  u64 pre = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kSWaves; ++w) {
    if (w < wave) pre += sh[w];
    tot += sh[w];
  }
  __syncthreads();
  *total = tot;
  return pre + incl - x;
}

// ---- the draw: one workgroup per row ----
template <typename T>
__global__ __launch_bounds__(kSThreads) void select_kernel(SmpParams p, bool vec) {
  const int row = blockIdx.x, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  __shared__ u64 sh[kSWaves];
  __shared__ int s_ch;
  __shared__ u64 s_target, s_base;
  __shared__ uint32_t s_eq0;
  __shared__ float s_mc;
  __shared__ int s_tok;
  if (p.greedy) {
    if (wave == 0) {
      const uint2 mk = row_max(p, row, lane);
      if (lane == 0) p.out[row] = mk.y;
    }
    return;
  }
  const SmpState st = p.st[(int64_t)row * (kMaxStages + 1) + p.nk + p.np];
  if (wave == 0) {
    const uint2 mk = row_max(p, row, lane);
    // kept mass per chunk: everything above v*, then the lowest-index ties
    u64 km = 0;
    uint32_t eq = 0;
    if (lane < p.nch) {
      km = p.csum[(int64_t)row * p.nch + lane];
      eq = p.ceq[(int64_t)row * p.nch + lane];
    }
    uint32_t ie = eq;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(ie, o, 64);
      if (lane >= o) ie += y;
    }
    const uint32_t before = ie - eq;
    const uint32_t kept = st.ms > before ? min(eq, st.ms - before) : 0u;
    km += (u64)kept * st.ws;
    const u64 incl = wave_incl_scan_u64(km, lane);
    const u64 Z = shfl_u64(incl, 63);
    const float u = p.u[(int64_t)row * p.u_stride];
    u64 target = (u64)((double)u * (double)Z);
    if (Z > 0 && target >= Z) target = Z - 1;
    const uint64_t hit = __builtin_amdgcn_ballot_w64(lane < p.nch && km > 0 && incl > target);
    const int ch = hit ? (int)__builtin_ctzll(hit) : -1;
    if (lane == 0) {
      s_ch = Z > 0 ? ch : -1;
      s_target = target;
      s_mc = max_c<T>(p, mk.x);
    }
    if (ch >= 0 && lane == ch) {
      s_base = incl - km;
      s_eq0 = before;
    }
  }
  __syncthreads();
  const int ch = s_ch;
  if (ch < 0) {  // no positive weight (all logits -inf)
    if (tid == 0) p.out[row] = -1;
    return;
  }
  if (tid == 0) s_tok = -1;
  const u64 target = s_target;
  const float mc = s_mc;
  u64 run = s_base;          // kept mass before the current block
  uint32_t eq_run = s_eq0;   // ties at v* before the current block
  const void* x = row_ptr<T>(p, row);
  const int c0 = ch * p.cs, c1 = min(p.V, c0 + p.cs);
  int last_kept = -1;
  for (int e0 = c0; e0 < c1; e0 += 8 * kSThreads) {
    const int e = e0 + 8 * tid;
    uint32_t r[8];
    if (e < c1) SKey<T>::load8(x, e, c1, vec, r);
    uint32_t key[8];
    uint32_t neq = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      key[i] = e + i < c1 ? SKey<T>::key(r[i]) : 0u;
      neq += (e + i < c1) && key[i] == st.vs;
    }
    u64 tot_eq;
    const uint32_t eq_before = eq_run + (uint32_t)block_excl_scan_u64(neq, sh, &tot_eq);
    u64 w[8];
    u64 tw = 0;
    uint32_t rank = eq_before;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      w[i] = 0;
      if (e + i < c1) {
        bool kept = key[i] > st.vs;
        if (key[i] == st.vs) {
          kept = rank < st.ms;
          ++rank;
        }
        if (kept) {
          w[i] = weight_of(SKey<T>::val(r[i]), p.c, mc);
          if (w[i]) last_kept = e + i;
        }
      }
      tw += w[i];
    }
    u64 tot_w;
    const u64 pre = run + block_excl_scan_u64(tw, sh, &tot_w);
    if (pre <= target && target < pre + tw) {
      u64 acc = pre;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        acc += w[i];
        if (w[i] && acc > target) {
          s_tok = e + i;
          break;
        }
      }
    }
    __syncthreads();
    if (s_tok >= 0) break;
    run += tot_w;
    eq_run += (uint32_t)tot_eq;
  }
  // rounding guard: the last kept token of the chunk (the chunk's kept mass
  // is the exact sum scanned here, so this is not reached)
  if (s_tok < 0) {
    int lk = last_kept;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) lk = max(lk, __shfl_xor(lk, o, 64));
    __shared__ int s_lk[kSWaves];
    if (lane == 0) s_lk[wave] = lk;
    __syncthreads();
    if (tid == 0) {
      int b = -1;
      for (int w2 = 0; w2 < kSWaves; ++w2) b = max(b, s_lk[w2]);
      p.out[row] = b;
    }
    return;
  }
  if (tid == 0) p.out[row] = s_tok;
}

struct SLayout {
  int nch, cs;
  int64_t cmax_off, hcnt_off, hmass_off, st_off, csum_off, ceq_off, total;
};

SLayout slayout(int rows, int V) {
  SLayout L;
  const int max_ch = std::max(1, std::min(kSMaxChunks, (V + 1023) / 1024));
  L.nch = std::max(1, std::min(max_ch, (kSTargetWgs + rows - 1) / std::max(1, rows)));
  L.cs = ((V + L.nch - 1) / L.nch + 7) / 8 * 8;
  L.nch = (V + L.cs - 1) / L.cs;
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  L.cmax_off = kWorkspaceHeaderBytes;  // the acceptance header stays untouched
  L.hcnt_off = L.cmax_off + al((int64_t)rows * kSMaxChunks * 8);
  L.hmass_off = L.hcnt_off + al((int64_t)rows * kMaxStages * kBins * 4);
  L.st_off = L.hmass_off + al((int64_t)rows * kMaxStages * kBins * 8);
  L.csum_off = L.st_off + al((int64_t)rows * (kMaxStages + 1) * sizeof(SmpState));
  L.ceq_off = L.csum_off + al((int64_t)rows * kSMaxChunks * 8);
  L.total = L.ceq_off + al((int64_t)rows * kSMaxChunks * 4);
  return L;
}

template <typename T>
int32_t launch_sample(const SmpParams& p, bool vec, hipStream_t s) {
  const dim3 g(p.nch, p.rows);
  hipLaunchKernelGGL((max_kernel<T>), g, dim3(kSThreads), 0, s, p, vec);
  int32_t rc = launch_status("sample max_kernel");
  if (rc || p.greedy) {
    if (rc) return rc;
    hipLaunchKernelGGL((select_kernel<T>), dim3(p.rows), dim3(kSThreads), 0, s, p, vec);
    return launch_status("sample select_kernel");
  }
  for (int st = 0; st < p.nk + p.np; ++st) {
    if (st < p.nk) hipLaunchKernelGGL((hist_kernel<T, true>), g, dim3(kSThreads), 0, s, p, st, vec);
    else hipLaunchKernelGGL((hist_kernel<T, false>), g, dim3(kSThreads), 0, s, p, st, vec);
    rc = launch_status("sample hist_kernel");
    if (rc) return rc;
  }
  hipLaunchKernelGGL((sums_kernel<T>), g, dim3(kSThreads), 0, s, p, vec);
  rc = launch_status("sample sums_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL((select_kernel<T>), dim3(p.rows), dim3(kSThreads), 0, s, p, vec);
  return launch_status("sample select_kernel");
}

}  // namespace
}  // namespace nsg

using namespace nsg;

extern "C" int64_t nsg_sample_workspace_bytes(int32_t rows, int32_t vocab) {
  if (rows < 0 || vocab <= 0) return -1;
  return slayout(rows, vocab).total;
}

extern "C" int32_t nsg_sample(const void* logits, int64_t row_stride, int32_t logits_dtype,
                              int32_t rows, int32_t vocab, float temperature, int32_t top_k,
                              float top_p, const float* uniforms, int64_t uniform_stride,
                              int64_t* tokens, void* workspace, int64_t workspace_bytes,
                              nsg_stream_t stream) {
  NSG_CHECK_ARG(rows >= 0 && rows <= kMaxRows, "rows %d outside [0, %d]", rows, kMaxRows);
  NSG_CHECK_ARG(vocab > 0, "vocab %d", vocab);
  NSG_CHECK_ARG(logits_dtype == 0 || logits_dtype == 1, "logits_dtype %d (0 bf16, 1 fp32)",
                logits_dtype);
  const bool greedy = temperature < 1e-6f;
  NSG_CHECK_ARG(greedy || (top_p > 0.f && top_p == top_p),
                "top_p %g must be in (0, 1] (1 = off)", (double)top_p);
  if (rows == 0) {
    clear_error();
    return NSG_OK;
  }
  NSG_CHECK_ARG(logits && tokens && workspace, "null pointer argument");
  NSG_CHECK_ARG(greedy || uniforms, "uniforms required when temperature > 0");
  NSG_CHECK_ARG(row_stride >= vocab, "row_stride %lld < vocab %d", (long long)row_stride, vocab);
  const SLayout L = slayout(rows, vocab);
  if (workspace_bytes < L.total) {
    set_error("workspace has %lld bytes, needs %lld", (long long)workspace_bytes,
              (long long)L.total);
    return NSG_ERR_WORKSPACE;
  }
  SmpParams p{};
  p.x = logits;
  p.stride = row_stride;
  p.rows = rows;
  p.V = vocab;
  p.greedy = greedy ? 1 : 0;
  p.c = greedy ? 0.f : kLog2eS / temperature;
  p.K = (!greedy && top_k > 0 && top_k < vocab) ? top_k : 0;
  p.P = (!greedy && top_p < 1.f) ? (double)top_p : 1.0;
  p.u = uniforms;
  p.u_stride = uniform_stride;
  p.out = tokens;
  p.nch = L.nch;
  p.cs = L.cs;
  const int esz = logits_dtype == 0 ? 2 : 4;
  p.levels = esz;  // one key byte per level
  p.nk = p.K > 0 ? p.levels : 0;
  p.np = p.P < 1.0 ? p.levels : 0;
  char* ws = static_cast<char*>(workspace);
  p.cmax = reinterpret_cast<uint2*>(ws + L.cmax_off);
  p.hcnt = reinterpret_cast<uint32_t*>(ws + L.hcnt_off);
  p.hmass = reinterpret_cast<u64*>(ws + L.hmass_off);
  p.st = reinterpret_cast<SmpState*>(ws + L.st_off);
  p.csum = reinterpret_cast<u64*>(ws + L.csum_off);
  p.ceq = reinterpret_cast<uint32_t*>(ws + L.ceq_off);
  const bool vec = (reinterpret_cast<uintptr_t>(logits) % 16 == 0) &&
                   ((row_stride * esz) % 16 == 0);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return logits_dtype == 0 ? launch_sample<bf16>(p, vec, s) : launch_sample<float>(p, vec, s);
}
