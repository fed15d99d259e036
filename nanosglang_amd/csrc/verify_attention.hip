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
//   tiles.  Long KV ranges are split; the last workgroup of a split group to
//   finish merges the partial (m, l, O) rows (atomic counter, agent-scope
//   fences), so one launch produces the final output.
//
// Inside a workgroup the 4 waves take 32-token KV steps round-robin; each
// wave keeps its own online-softmax state and the waves merge through LDS.
// Per 32-token step a wave:
//   - loads K rows straight into MFMA operands: lane (token = lane%16,
//     d-group = lane/16) reads 16 contiguous bytes of one token's head row;
//   - loads V rows (16-byte coalesced loads) and stages them in a per-wave
//     LDS tile [32 tokens][D + 8] bf16;
//   - computes S^T = K Q^T with v_mfma_f32_16x16x32_bf16 (M = tokens,
//     N = query rows, K = head dim), so every lane holds 4 tokens of ONE query
//     row and the row max / sum need only two cross-lane steps;
//   - converts P^T to bf16 in registers, which is already the B operand of
//     O^T += V^T P^T (M = head dim, N = query rows, K = 32 tokens); V^T comes
//     from the LDS tile with the same token order.
#include <algorithm>
#include <cstdarg>
#include <vector>

#include "common.hpp"

namespace nsg {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kTokIt = 32;           // KV tokens per wave step
constexpr float kMaskVal = -1.0e30f; // finite "minus infinity" (no inf - inf)
constexpr int64_t kHeaderBytes = 256;          // flags word + padding
constexpr int64_t kMaxCounters = 1 << 16;      // (group, kv head) merge counters
constexpr int64_t kCounterBytes = kMaxCounters * 4;
constexpr int kTargetWgPerCu = 4;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

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
  int* counters;
  float* partials;
};

__device__ __forceinline__ bf16x8 load_bf16x8(const bf16* p) {
  u32x4 v = *reinterpret_cast<const u32x4*>(p);
  return __builtin_bit_cast(bf16x8, v);
}

template <int D, int RT>
__global__ __launch_bounds__(kThreads) void verify_attn_kernel(AttnParams p) {
  constexpr int KC = D / 32;   // K-dim chunks of QK^T
  constexpr int DT = D / 16;   // d tiles of PV
  constexpr int ROWS = RT * 16;
  constexpr int VROW = D + 8;  // padded LDS row (bf16): 16-byte aligned, conflict-free reads
  constexpr int VCH = D / 8;   // 16-byte chunks per V row
  constexpr int NV = kTokIt * VCH / 64;
  constexpr int OROW = D + 4;
  constexpr int PSTRIDE = D + 4;  // partial row: O[D], m, l, 2 pad (16-byte aligned rows)
  constexpr int SMEM_V = kWaves * kTokIt * VROW * 2;
  constexpr int SMEM_M = kWaves * 16 * OROW * 4 + 2 * kWaves * 16 * 4;
  constexpr int SMEM = SMEM_V > SMEM_M ? SMEM_V : SMEM_M;
  __shared__ __attribute__((aligned(16))) char smem[SMEM];
  __shared__ int s_last;

  const int wi = blockIdx.x;
  if (wi >= p.num_work) return;
  const int h = blockIdx.y;
  const int* wk = p.work + (size_t)wi * NSG_ATTN_WORK_INTS;
  const int b = wk[0], qb = wk[1], qn = wk[2], kvb = wk[3], kve = wk[4];
  const int split = wk[5], nsplit = wk[6], group = wk[7];
  const int P = 1 << p.log2P;
  const int G = p.G;
  const int q0 = p.qo_indptr[b];
  const int ql = p.qo_indptr[b + 1] - q0;
  const int pb = p.kv_indptr[b];
  const int npg = p.kv_indptr[b + 1] - pb;
  const int L = npg > 0 ? (npg - 1) * P + p.kv_last[b] : 0;
  const int nrows = qn * G;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int g4 = lane >> 4;

  // Query fragments (B operand of S^T = K Q^T) and per-row causal limits.
  bf16x8 qf[RT][KC];
  int lim[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = rt * 16 + r16;
    const bool ok = row < nrows;
    const int tau = row / G;
    const int gam = row - tau * G;
    lim[rt] = ok ? (p.causal ? L - ql + qb + tau : L - 1) : -1;
    const bf16* qrow = p.q + ((size_t)(q0 + qb + tau) * p.Hq + h * G + gam) * D;
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      if (ok) {
        qf[rt][c] = load_bf16x8(qrow + 32 * c + 8 * g4);
      } else {
        qf[rt][c] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
      }
    }
  }

  floatx4 oacc[RT][DT];
  float m_run[RT], l_run[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m_run[rt] = kMaskVal;
    l_run[rt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[rt][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  bf16* vt = reinterpret_cast<bf16*>(smem) + wave * kTokIt * VROW;
  const size_t head_off = (size_t)h * D;
  const size_t tok_stride = (size_t)p.Hkv * D;
  const int n_it = (kve - kvb + kTokIt - 1) / kTokIt;

  for (int it = wave; it < n_it; it += kWaves) {
    const int t0 = kvb + it * kTokIt;

    // ---- K rows straight into MFMA A operands ----
    bf16x8 kf[2][KC];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int j = t0 + 16 * s + r16;
      int page = -1;
      if (j < kve) {
        page = p.kv_indices[pb + (j >> p.log2P)];
        if ((unsigned)page >= (unsigned)p.num_pages) {
          atomicOr(p.flags, 1);
          page = -1;
        }
      }
      const bf16* kp = p.kc + ((size_t)max(page, 0) * P + (j & (P - 1))) * tok_stride + head_off;
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        if (page >= 0) {
          kf[s][c] = load_bf16x8(kp + 32 * c + 8 * g4);
        } else {
          kf[s][c] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
        }
      }
    }
    // ---- V rows: coalesced 16-byte loads ----
    u32x4 vr[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = lane + 64 * i;
      const int t = e / VCH;
      const int ch = e - t * VCH;
      const int j = t0 + t;
      int page = -1;
      if (j < kve) {
        page = p.kv_indices[pb + (j >> p.log2P)];
        if ((unsigned)page >= (unsigned)p.num_pages) page = -1;
      }
      if (page >= 0) {
        vr[i] = *reinterpret_cast<const u32x4*>(
            p.vc + ((size_t)page * P + (j & (P - 1))) * tok_stride + head_off + ch * 8);
      } else {
        vr[i] = u32x4{0u, 0u, 0u, 0u};
      }
    }

    // ---- S^T = K Q^T ----
    floatx4 sacc[RT][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < KC; ++c)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[s][c], qf[rt][c], acc, 0, 0, 0);
        sacc[rt][s] = acc;
      }
    }

    // ---- stage V in this wave's LDS tile ----
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = lane + 64 * i;
      const int t = e / VCH;
      const int ch = e - t * VCH;
      *reinterpret_cast<u32x4*>(vt + t * VROW + ch * 8) = vr[i];
    }

    // ---- online softmax; P^T packed as the B operand of the PV MFMA ----
    bf16x8 pf[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float sv[8];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = t0 + 16 * s + 4 * g4 + i;
          sv[4 * s + i] = (j <= lim[rt] && j < kve) ? sacc[rt][s][i] * p.scale_log2 : kMaskVal;
        }
      }
      float mx = sv[0];
#pragma unroll
      for (int x = 1; x < 8; ++x) mx = fmaxf(mx, sv[x]);
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mnew = fmaxf(m_run[rt], mx);
      const float alpha = exp2f(m_run[rt] - mnew);
      m_run[rt] = mnew;
      float pv[8];
      float ps = 0.f;
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        pv[x] = exp2f(sv[x] - mnew);
        ps += pv[x];
      }
      l_run[rt] = l_run[rt] * alpha + ps;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) oacc[rt][dt] *= alpha;
      u32x4 pk = {pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3]),
                  pack_bf16x2(pv[4], pv[5]), pack_bf16x2(pv[6], pv[7])};
      pf[rt] = __builtin_bit_cast(bf16x8, pk);
    }

    __builtin_amdgcn_wave_barrier();
    // ---- O^T += V^T P^T; element e of lane group g4 is token
    //      4*g4 + e (e < 4) or 16 + 4*g4 + (e - 4), matching pf ----
    const uint16_t* vt16 = reinterpret_cast<const uint16_t*>(vt);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int col = dt * 16 + r16;
      uint32_t w[4];
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const int ea = 2 * e2, eb = 2 * e2 + 1;
        const int ta = ea < 4 ? 4 * g4 + ea : 16 + 4 * g4 + ea - 4;
        const int tb = eb < 4 ? 4 * g4 + eb : 16 + 4 * g4 + eb - 4;
        w[e2] = (uint32_t)vt16[ta * VROW + col] | ((uint32_t)vt16[tb * VROW + col] << 16);
      }
      const bf16x8 vf = __builtin_bit_cast(bf16x8, u32x4{w[0], w[1], w[2], w[3]});
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
        oacc[rt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[rt], oacc[rt][dt], 0, 0, 0);
    }
    __builtin_amdgcn_wave_barrier();
  }

  // ---- row sums across the 4 lane groups that share a query row ----
  float l_tot[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    float l = l_run[rt];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    l_tot[rt] = l;
  }

  // ---- merge the 4 waves through LDS, one 16-row tile at a time ----
  __syncthreads();
  float* mo = reinterpret_cast<float*>(smem);          // [kWaves][16][OROW]
  float* mm = mo + kWaves * 16 * OROW;                  // [kWaves][16]
  float* ml = mm + kWaves * 16;                         // [kWaves][16]
  constexpr int CPT = D / 16;                           // columns per thread
  const int mrow = threadIdx.x >> 4;
  const int c0 = (threadIdx.x & 15) * CPT;
  const size_t part_base = ((size_t)wi * p.Hkv + h) * ROWS * PSTRIDE;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      *reinterpret_cast<floatx4*>(&mo[(wave * 16 + r16) * OROW + dt * 16 + 4 * g4]) = oacc[rt][dt];
    if (g4 == 0) {
      mm[wave * 16 + r16] = m_run[rt];
      ml[wave * 16 + r16] = l_tot[rt];
    }
    __syncthreads();
    const int grow = rt * 16 + mrow;
    if (grow < nrows) {
      float M = mm[mrow];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) M = fmaxf(M, mm[w * 16 + mrow]);
      float wt[kWaves];
      float lsum = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        wt[w] = exp2f(mm[w * 16 + mrow] - M);
        lsum += wt[w] * ml[w * 16 + mrow];
      }
      float o[CPT];
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) acc += wt[w] * mo[(w * 16 + mrow) * OROW + c0 + c];
        o[c] = acc;
      }
      if (nsplit == 1) {
        const int tau = grow / G;
        const int gam = grow - tau * G;
        bf16* orow = p.out + ((size_t)(q0 + qb + tau) * p.Hq + h * G + gam) * D + c0;
        const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
        uint32_t pk[CPT / 2];
#pragma unroll
        for (int c = 0; c < CPT / 2; ++c) pk[c] = pack_bf16x2(o[2 * c] * inv, o[2 * c + 1] * inv);
        if constexpr (CPT == 8) {
          *reinterpret_cast<u32x4*>(orow) = u32x4{pk[0], pk[1], pk[2], pk[3]};
        } else {
          *reinterpret_cast<u32x2*>(orow) = u32x2{pk[0], pk[1]};
        }
      } else {
        float* prow = p.partials + part_base + (size_t)grow * PSTRIDE;
#pragma unroll
        for (int c = 0; c < CPT; c += 4)
          *reinterpret_cast<floatx4*>(prow + c0 + c) = floatx4{o[c], o[c + 1], o[c + 2], o[c + 3]};
        if (c0 == 0) {
          prow[D] = M;
          prow[D + 1] = lsum;
        }
      }
    }
    __syncthreads();
  }
  if (nsplit == 1) return;

  // ---- cross-split merge by the last workgroup of the group ----
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = atomicAdd(&p.counters[(size_t)group * p.Hkv + h], 1);
    s_last = (prev == nsplit - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const int wi0 = wi - split;
  for (int grow = mrow; grow < nrows; grow += kThreads / 16) {
    float M = kMaskVal;
    for (int s = 0; s < nsplit; ++s) {
      const float* prow = p.partials + ((size_t)(wi0 + s) * p.Hkv + h) * ROWS * PSTRIDE +
                          (size_t)grow * PSTRIDE;
      M = fmaxf(M, prow[D]);
    }
    float o[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c) o[c] = 0.f;
    float lsum = 0.f;
    for (int s = 0; s < nsplit; ++s) {
      const float* prow = p.partials + ((size_t)(wi0 + s) * p.Hkv + h) * ROWS * PSTRIDE +
                          (size_t)grow * PSTRIDE;
      const float wt = exp2f(prow[D] - M);
      lsum += wt * prow[D + 1];
#pragma unroll
      for (int c = 0; c < CPT; c += 4) {
        const floatx4 v = *reinterpret_cast<const floatx4*>(prow + c0 + c);
        o[c] += wt * v[0];
        o[c + 1] += wt * v[1];
        o[c + 2] += wt * v[2];
        o[c + 3] += wt * v[3];
      }
    }
    const int tau = grow / G;
    const int gam = grow - tau * G;
    bf16* orow = p.out + ((size_t)(q0 + qb + tau) * p.Hq + h * G + gam) * D + c0;
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    uint32_t pk[CPT / 2];
#pragma unroll
    for (int c = 0; c < CPT / 2; ++c) pk[c] = pack_bf16x2(o[2 * c] * inv, o[2 * c + 1] * inv);
    if constexpr (CPT == 8) {
      *reinterpret_cast<u32x4*>(orow) = u32x4{pk[0], pk[1], pk[2], pk[3]};
    } else {
      *reinterpret_cast<u32x2*>(orow) = u32x2{pk[0], pk[1]};
    }
  }
  if (threadIdx.x == 0) p.counters[(size_t)group * p.Hkv + h] = 0;
}

template <int D>
int32_t launch_d(const nsg_attn_plan_t* plan, const AttnParams& prm, hipStream_t stream) {
  dim3 grid(plan->num_work, plan->num_kv_heads);
  dim3 block(kThreads);
  switch (plan->row_tiles) {
    case 1: hipLaunchKernelGGL((verify_attn_kernel<D, 1>), grid, block, 0, stream, prm); break;
    case 2: hipLaunchKernelGGL((verify_attn_kernel<D, 2>), grid, block, 0, stream, prm); break;
    case 3: hipLaunchKernelGGL((verify_attn_kernel<D, 3>), grid, block, 0, stream, prm); break;
    case 4: hipLaunchKernelGGL((verify_attn_kernel<D, 4>), grid, block, 0, stream, prm); break;
    default: set_error("row_tiles %d out of range", plan->row_tiles); return NSG_ERR_ARG;
  }
  return launch_status("verify_attn_kernel");
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

extern "C" int32_t nsg_attn_plan(const int32_t* qo_indptr_h, const int32_t* kv_indptr_h,
                                 const int32_t* kv_last_page_len_h, int32_t batch,
                                 int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                                 int32_t page_size, int32_t causal, int32_t num_cus,
                                 int32_t* work_h, int32_t work_capacity, nsg_attn_plan_t* plan) {
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
  const int T = std::max(1, std::min(64 / G, max_ql));
  const int RT = (T * G + 15) / 16;

  struct Group { int b, qb, qn, kv_end; };
  std::vector<Group> groups;
  long long total_it = 0;
  for (int b = 0; b < batch; ++b) {
    const int ql = qo_indptr_h[b + 1] - qo_indptr_h[b];
    if (ql == 0) continue;
    const int np = kv_indptr_h[b + 1] - kv_indptr_h[b];
    const int L = np > 0 ? (np - 1) * page_size + kv_last_page_len_h[b] : 0;
    NSG_CHECK_ARG(L >= 1, "request %d has %d query tokens but an empty KV range", b, ql);
    NSG_CHECK_ARG(!causal || L >= ql, "request %d: kv length %d < query length %d", b, L, ql);
    for (int qb = 0; qb < ql; qb += T) {
      const int qn = std::min(T, ql - qb);
      const int kv_end = causal ? L - ql + qb + qn : L;
      groups.push_back({b, qb, qn, kv_end});
      total_it += (kv_end + kTokIt - 1) / kTokIt;
    }
  }
  NSG_CHECK_ARG((long long)groups.size() * num_kv_heads <= kMaxCounters,
                "%zu query tiles x %d kv heads exceed the %lld merge counters", groups.size(),
                num_kv_heads, (long long)kMaxCounters);
  const long long target_items = std::max(1, num_cus * kTargetWgPerCu / num_kv_heads);
  long long chunk_it = std::max<long long>(kWaves, (total_it + target_items - 1) / target_items);
  chunk_it = (chunk_it + kWaves - 1) / kWaves * kWaves;

  int n = 0, max_splits = 0;
  for (size_t gi = 0; gi < groups.size(); ++gi) {
    const Group& g = groups[gi];
    const long long its = (g.kv_end + kTokIt - 1) / kTokIt;
    const int ns = (int)std::max<long long>(1, (its + chunk_it - 1) / chunk_it);
    max_splits = std::max(max_splits, ns);
    for (int s = 0; s < ns; ++s) {
      if (n >= work_capacity || !work_h) {
        set_error("work list needs more than %d items", work_capacity);
        return NSG_ERR_WORKSPACE;
      }
      int32_t* w = work_h + (size_t)n * NSG_ATTN_WORK_INTS;
      w[0] = g.b;
      w[1] = g.qb;
      w[2] = g.qn;
      w[3] = (int)(s * chunk_it * kTokIt);
      w[4] = (int)std::min<long long>(g.kv_end, (s + 1) * chunk_it * kTokIt);
      w[5] = s;
      w[6] = ns;
      w[7] = (int)gi;
      ++n;
    }
  }
  plan->num_work = n;
  plan->num_groups = (int)groups.size();
  plan->row_tiles = RT;
  plan->q_tile_tokens = T;
  plan->max_splits = max_splits;
  plan->head_dim = head_dim;
  plan->num_qo_heads = num_qo_heads;
  plan->num_kv_heads = num_kv_heads;
  plan->workspace_bytes =
      kHeaderBytes + kCounterBytes + (int64_t)n * num_kv_heads * RT * 16 * (head_dim + 4) * 4;
  clear_error();
  return NSG_OK;
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
  if (workspace_bytes < plan->workspace_bytes) {
    set_error("workspace has %lld bytes, plan needs %lld", (long long)workspace_bytes,
              (long long)plan->workspace_bytes);
    return NSG_ERR_WORKSPACE;
  }
  AttnParams prm;
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
  prm.counters = reinterpret_cast<int*>(ws + kHeaderBytes);
  prm.partials = reinterpret_cast<float*>(ws + kHeaderBytes + kCounterBytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (plan->head_dim == 64) return launch_d<64>(plan, prm, s);
  if (plan->head_dim == 128) return launch_d<128>(plan, prm, s);
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
