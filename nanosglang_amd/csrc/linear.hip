// Skinny linear layers of the decode / verify forwards on gfx950.
//
// The decoder layers around the verify step (nano_sglang/model/causal_lm.py:
// q/k/v projections :229-231 and :281-283, o_proj :261 and :307, the SwiGLU
// MLP :481-482, lm_head :643-645) run on M = batch * tokens-per-request rows:
// 32 for a draft step and 160 for a verify step at batch 32, k = 4.  At such
// M a linear layer is a stream of its weight matrix W (N x K bf16) with a
// little arithmetic per byte, and the work is latency-bound rather than
// throughput-bound for the small matrices (1.6 - 17 MB).  Library GEMMs tile
// for large M; this kernel is shaped for the weight stream instead:
//
// * a workgroup owns 16 * NT rows of W (output columns) and up to 32 rows of
//   x (more rows run as 32-row groups, see launch_epi);
//   its NW waves split K in 64-element chunks (wave w takes chunks w, w + NW,
//   ...), so every lane issues its loads for the next chunk while the MFMAs
//   of the current one run, and the waves' partial sums meet in LDS;
// * W and x^T fragments go from global memory straight into the operand
//   layout of v_mfma_f32_16x16x32_bf16 (A = 16 W rows x 32 k, lane l holds
//   row l % 16, k 8 * (l / 16) .. + 8; B = 32 k x 16 x rows, same lane map),
//   so no LDS staging is needed: each W row segment is read once, x (a few
//   hundred KB at most) is served by L2;
// * the epilogue applies the bias (y = bf16(acc + bias), one rounding, as a
//   bf16 GEMM with a bias epilogue does), or the SwiGLU gate: W holds the
//   fused [gate; up] rows, and y = bf16(bf16(silu(bf16(g))) * bf16(u)), the
//   rounding order of F.silu(gate) * up on bf16 tensors (causal_lm.py:482).
#include <algorithm>
#include <cstddef>
#include <type_traits>

#include "common.hpp"
#include "lm_head.hpp"

namespace nsg {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kChunk = 64;  // K elements per wave step (two MFMA k-slices)
constexpr int kMaxMT = 10;  // up to 160 rows of x
// Partial sums of squares a folded-RMSNorm consumer reads per row: one per
// 16 columns of the producer's output, hidden sizes up to 1024.
constexpr int kMaxSumsqParts = 64;

struct LinParams {
  const bf16* x;
  const bf16* w;
  // FP8 weights (e4m3fn bytes, row stride ldw bytes) and one f32 scale per W
  // row: W[n, k] = bf16(float(w8[n, k]) * w_scale[n])
  const uint8_t* w8;
  const float* w_scale;
  const bf16* bias;
  bf16* y;
  int64_t ldx, ldw, ldy;
  int M, N, K;     // N: output columns (SwiGLU: the intermediate size I)
  int w_rows;      // rows of W (N, or 2 I for SwiGLU)
  int row_groups;  // > 1: M runs as groups of MG * MT * 16 rows, one workgroup each
  int col_tiles;   // column tiles (workgroups per row group)
  // RoPE + KV-slot epilogue (q/k/v projection): one workgroup per head
  const int64_t* pos;
  const float* cos_t;
  const float* sin_t;
  int max_pos;
  const int64_t* slots;
  int Hq, Hkv, head_dim;
  bf16* q_out;
  bf16* kc;
  bf16* vc;
  int64_t num_slots;
  int* flags;
  // RMSNorm folded into the layer's linears (the norm weight folded into the
  // consumer's W columns):
  //  consumer -- x rows are un-normalised; row m's result is scaled by
  //    rsqrt(S_m / norm_dim + norm_eps) before the epilogue, where S_m is
  //    the sum of sumsq_in[c * M + m] over c < sumsq_parts (fixed order);
  //  producer (bias epilogue) -- y = bf16(residual + bf16(x W^T + bias)),
  //    and sumsq_out[(n / 16) * M + m] = the sum of squares of y's row m
  //    over columns n .. n + 15 (one partial per 16 columns: deterministic,
  //    whatever the tile shape).
  const float* sumsq_in;
  int sumsq_parts;
  int norm_dim;
  float norm_eps;
  const bf16* residual;
  int64_t ldr;
  float* sumsq_out;
};


// The folded-RMSNorm fields of LinParams (its last 48 bytes), read from the
// kernel argument segment (the kernels here take one LinParams, at offset
// 0) by scalar loads issued where the call is and waited for at once.  The
// residual and sumsq_out pointers are accessed through the global address
// space (GlobalPtr): through a generic pointer of unknown origin the
// compiler emits flat accesses, which its wait-count pass must also take
// for LDS accesses, and every ds_bpermute of the K sweep then waits for
// every load in flight.
#define NSG_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ NSG_GLOBAL T* global_ptr(uint64_t addr) {
  return (NSG_GLOBAL T*)addr;
}
struct FoldArgs {
  const float* sumsq_in;
  int parts;
  int dim;
  float eps;
  uint64_t residual;   // bf16 rows, ldr elements apart
  int64_t ldr;
  uint64_t sumsq_out;  // float
};
typedef uint32_t u32x8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
constexpr int kFoldOff = offsetof(LinParams, sumsq_in);
static_assert(offsetof(LinParams, sumsq_parts) == kFoldOff + 8 &&
                  offsetof(LinParams, norm_dim) == kFoldOff + 12 &&
                  offsetof(LinParams, norm_eps) == kFoldOff + 16 &&
                  offsetof(LinParams, residual) == kFoldOff + 24 &&
                  offsetof(LinParams, ldr) == kFoldOff + 32 &&
                  offsetof(LinParams, sumsq_out) == kFoldOff + 40 &&
                  sizeof(LinParams) == kFoldOff + 48,
              "FoldArgs mirrors the tail of LinParams");
__device__ __forceinline__ FoldArgs fold_args_here() {
  u32x8_t a;
  u32x4_t b;
  asm volatile("s_load_dwordx8 %0, %2, %3\n\ts_load_dwordx4 %1, %2, %4\n\ts_waitcnt lgkmcnt(0)"
               : "=&s"(a), "=&s"(b)
               : "s"(__builtin_amdgcn_kernarg_segment_ptr()), "n"(kFoldOff), "n"(kFoldOff + 32));
  FoldArgs f;
  f.sumsq_in = reinterpret_cast<const float*>(((uint64_t)a[1] << 32) | a[0]);
  f.parts = (int)a[2];
  f.dim = (int)a[3];
  f.eps = __uint_as_float(a[4]);
  f.residual = ((uint64_t)a[7] << 32) | a[6];
  f.ldr = (int64_t)(((uint64_t)b[1] << 32) | b[0]);
  f.sumsq_out = ((uint64_t)b[3] << 32) | b[2];
  return f;
}

// kEpiRes: the bias epilogue of a folded-RMSNorm producer (residual add and
// partial sums of squares, see LinParams); kEpiSiluN / kEpiRopeN: the SwiGLU
// and RoPE epilogues of a folded-RMSNorm consumer (rows scaled first).
// kEpiArgmax: the bias epilogue's bf16 values, reduced to one (value,
// column) key per row and workgroup instead of being stored.
enum {
  kEpiBias = 0, kEpiSilu = 1, kEpiRope = 2, kEpiRes = 3, kEpiSiluN = 4, kEpiRopeN = 5,
  kEpiArgmax = 6
};
constexpr bool epi_silu(int e) { return e == kEpiSilu || e == kEpiSiluN; }
constexpr bool epi_rope(int e) { return e == kEpiRope || e == kEpiRopeN; }
constexpr bool epi_norm(int e) { return e == kEpiSiluN || e == kEpiRopeN; }

__device__ __forceinline__ float bf16_round(float x) {
  return bf16_bits_to_float(float_to_bf16_bits(x));
}

__device__ __forceinline__ float silu_bf16(float g) {
  return bf16_bits_to_float(float_to_bf16_bits(g / (1.f + __expf(-g))));
}

// One workgroup: output columns [16 NT * blockIdx.x, + 16 NT) (SwiGLU: NT / 2
// column tiles, each with a gate and an up row block of W), all M rows.  Its
// MG * NW waves form MG groups of NW: group g owns m tiles [g MT, g MT + MT)
// and its NW waves split K (more rows per wave would not fit the registers of
// two load stages; the groups read the same W rows, the second from L2).
// One OCP e4m3fn byte pair -> two floats (gfx950's v_cvt_pk_f32_fp8, exact),
// then the row scale and one bf16 rounding: the dequantisation
// w8.to(bf16) * scale of FP8Linear.forward (quantization.py:49-52).
__device__ __forceinline__ u32x4 dequant_fp8x8(u32x2 v, float s) {
  const floatx2_t f0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)v[0], false);
  const floatx2_t f1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)v[0], true);
  const floatx2_t f2 = __builtin_amdgcn_cvt_pk_f32_fp8((int)v[1], false);
  const floatx2_t f3 = __builtin_amdgcn_cvt_pk_f32_fp8((int)v[1], true);
  return u32x4{pack_bf16x2(f0[0] * s, f0[1] * s), pack_bf16x2(f1[0] * s, f1[1] * s),
               pack_bf16x2(f2[0] * s, f2[1] * s), pack_bf16x2(f3[0] * s, f3[1] * s)};
}

template <int MT, int MG, int NT, int NW, int EPI, bool W8 = false>
__global__ __launch_bounds__(MG * NW * 64) void linear_kernel(LinParams p) {
  static_assert(!epi_silu(EPI) || NT % 2 == 0, "SwiGLU pairs gate and up tiles");
  constexpr int NP = epi_silu(EPI) ? 2 : 1;  // physical tiles reduced together
  __shared__ floatx4 red[MG][NP][NW][MT][64];
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int wave = wid % NW;
  const int grp = wid / NW;
  const int r16 = lane & 15;

  // Workgroup -> (column tile, row group).  With row groups, the groups of
  // one column tile sit on the same XCD (workgroups go round-robin over the
  // 8 XCDs), so its W rows come from HBM once and from that XCD's L2 for the
  // other groups.
  // The empty asm takes every argument read before the first chunk's loads
  // at once, so that they arrive in one scalar memory round trip: left to
  // itself, the compiler fetches col_tiles only inside the branch below (and
  // the RoPE fields after that), one dependent round trip each.
  const int row_groups = p.row_groups, col_tiles = p.col_tiles;
  if constexpr (epi_rope(EPI))
    asm volatile("" ::"s"(row_groups), "s"(col_tiles), "s"(p.pos), "s"(p.cos_t), "s"(p.sin_t),
                 "s"(p.slots), "s"(p.head_dim), "s"(p.max_pos), "s"(p.bias));
  else
    asm volatile("" ::"s"(row_groups), "s"(col_tiles));
  int tile = blockIdx.x;
  int M = p.M;
  int m0 = 0;
  const bf16* xg = p.x;
  bf16* yg = p.y;
  if (row_groups > 1) {
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    tile = xcd + 8 * (slot / row_groups);
    if (tile >= col_tiles) return;
    m0 = (slot % row_groups) * (MG * MT * 16);
    M = min(MG * MT * 16, p.M - m0);
    xg += (int64_t)m0 * p.ldx;
    yg += (int64_t)m0 * p.ldy;
  }

  // Loads are coalesced: for a 16-row x 32-k fragment, lane l reads row
  // l / 4, 16-byte segment l % 4, so each lane quad covers one row's 64
  // contiguous bytes (the MFMA layout itself -- lane l = row l % 16 -- puts
  // four different cache lines in every quad, which the vector L1 serves at a
  // quarter of its rate).  ds_bpermute then moves segment g of row r from
  // lane 4 r + g to its MFMA lane r + 16 g.  Rows past the end are clamped
  // to a valid row; their results are not stored.
  const int lrow = lane >> 2;
  const int lseg = (lane & 3) * 8;
  const int perm_src = 4 * (4 * r16 + (lane >> 4));  // byte address of the source lane
  const bf16* wp[NT];
  const uint8_t* wp8[NT];
  float wsc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    int row;
    if constexpr (epi_silu(EPI)) {
      const int col_tile = tile * (NT / 2) + (nt >> 1);
      row = ((nt & 1) ? p.N : 0) + col_tile * 16 + lrow;
    } else if constexpr (epi_rope(EPI)) {
      // tile = (head, s): columns 16 s .. + 16 of the head and their RoPE
      // partners head_dim / 2 further on
      const int tph = p.head_dim / 32;  // tiles per half head
      row = (tile / tph) * p.head_dim + nt * (p.head_dim / 2) + (tile % tph) * 16 + lrow;
    } else {
      row = (tile * NT + nt) * 16 + lrow;
    }
    row = min(row, p.w_rows - 1);
    if constexpr (W8) {
      // FP8: lane l reads the 8 bytes (k 8 (l % 4) .. + 8 of each 32-k half)
      // that dequantise to exactly the 8 bf16 the bf16 path's 16-byte load
      // gives it, so the MFMA lane mapping below is the same
      wp8[nt] = p.w8 + (int64_t)row * p.ldw + lseg;
      wsc[nt] = p.w_scale[row];
      wp[nt] = nullptr;
    } else {
      wp[nt] = p.w + (int64_t)row * p.ldw + lseg;
      wp8[nt] = nullptr;
      wsc[nt] = 1.f;
    }
  }
  const bf16* xp[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    xp[mt] = xg + (int64_t)min((grp * MT + mt) * 16 + lrow, M - 1) * p.ldx + lseg;
  auto to_mfma = [&](u32x4 v) {
    u32x4 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = __builtin_amdgcn_ds_bpermute(perm_src, (int)v[j]);
    return __builtin_bit_cast(bf16x8, r);
  };

  floatx4 acc[NT][MT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int nchunks = p.K / kChunk;
  // workgroups start their K sweep at different chunks: otherwise all of them
  // read the same x lines at the same moment, from the same L2 channels
  const int rot = (int)((unsigned)tile % (unsigned)nchunks);
  // two register stages: loads of chunk c + NW are in flight while chunk c
  // is multiplied
  using WReg = typename std::conditional<W8, u32x2, u32x4>::type;
  WReg wa[NT][2], wb[NT][2];
  u32x4 xa[MT][2], xb[MT][2];
  auto load = [&](int c, WReg (&wv)[NT][2], u32x4 (&xv)[MT][2]) {
    int cr = c + rot;
    cr = cr >= nchunks ? cr - nchunks : cr;
    const int k0 = cr * kChunk;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if constexpr (W8) {
        wv[nt][0] = *reinterpret_cast<const u32x2*>(wp8[nt] + k0);
        wv[nt][1] = *reinterpret_cast<const u32x2*>(wp8[nt] + k0 + 32);
      } else {
        wv[nt][0] = *reinterpret_cast<const u32x4*>(wp[nt] + k0);
        wv[nt][1] = *reinterpret_cast<const u32x4*>(wp[nt] + k0 + 32);
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      xv[mt][0] = *reinterpret_cast<const u32x4*>(xp[mt] + k0);
      xv[mt][1] = *reinterpret_cast<const u32x4*>(xp[mt] + k0 + 32);
    }
  };
  auto mma = [&](const WReg (&wv)[NT][2], const u32x4 (&xv)[MT][2]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      bf16x8 wf[NT], xf[MT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        if constexpr (W8)
          wf[nt] = to_mfma(dequant_fp8x8(wv[nt][h], wsc[nt]));
        else
          wf[nt] = to_mfma(wv[nt][h]);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) xf[mt] = to_mfma(xv[mt][h]);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[nt][mt] =
              __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[nt], xf[mt], acc[nt][mt], 0, 0, 0);
    }
  };
  // RoPE epilogue operands.  A workgroup owns the 16 rotation pairs
  // (i, i + head_dim / 2), i = 16 s .. + 16, of one head: tile 0 holds the
  // first members, tile 1 the partners.  Epilogue item idx = threadIdx.x +
  // j * threads is row m = idx / 16, pair i = 16 s + idx % 16; rows past M
  // are clamped and not stored.  The loads go before the K sweep, so that
  // their latency (position, then cos / sin at that position) hides under it.
  constexpr bool kRope = epi_rope(EPI);
  constexpr int kThreads = NW * 64;
  constexpr int kItems = MT * 16 * 16;
  constexpr int kIpt = kRope ? (kItems + kThreads - 1) / kThreads : 1;  // items per thread
  constexpr int kRItems = 2 * MT * 64;  // reduction items: (tile, m tile, lane)
  constexpr int kRpt = kRope ? (kRItems + kThreads - 1) / kThreads : 1;
  static_assert(!kRope || NT == 2, "a first-half and a second-half tile");
  static_assert(!kRope || (kItems % 64 == 0 && kRItems % 64 == 0), "whole waves of items");
  const int half = p.head_dim / 2;
  const int tph = kRope ? p.head_dim / 32 : 1;
  const int head = tile / tph;
  const int pair0 = (tile % tph) * 16;
  int64_t e_pos[kIpt], e_slot[kIpt];
  float e_cos[kIpt], e_sin[kIpt];
  uint2 e_bias[kRpt];
  if constexpr (kRope) {
#pragma unroll
    for (int j = 0; j < kIpt; ++j) {
      const int idx = min((int)threadIdx.x + j * kThreads, kItems - 1);
      const int t = m0 + min(idx / 16, M - 1);
      e_pos[j] = p.pos[t];
      e_slot[j] = p.slots ? p.slots[t] : -1;
    }
#pragma unroll
    for (int j = 0; j < kRpt; ++j) {
      const int r = min((int)threadIdx.x + j * kThreads, kRItems - 1);
      const int c = head * p.head_dim + (r / (MT * 64)) * half + pair0 + 4 * ((r & 63) >> 4);
      e_bias[j] = p.bias ? *reinterpret_cast<const uint2*>(p.bias + c) : uint2{0u, 0u};
    }
  }

  // This wave's chunks are wave + NW i for i < n.  The loop body issues its
  // loads unconditionally: a load under a branch would make the wait-count
  // pass assume it might be outstanding and drain the next chunk's loads
  // before the current chunk's MFMAs.
  const int n = (nchunks - wave + NW - 1) / NW;
  if (n > 0) load(wave, wa, xa);
  // Folded RMSNorm (producer): the residual values this thread adds in the
  // epilogue (its items there, rows and columns clamped), loaded before the
  // K sweep so that their latency hides under it, but after the first
  // chunk's loads.  The fold arguments (here and in the consumer's copy
  // wave below) are read with explicit scalar loads issued after the first
  // chunk's: as ordinary argument reads the compiler hoists them to the
  // kernel's start, where every wave's first chunk waits for them.
  __builtin_amdgcn_sched_barrier(0);
  constexpr bool kRes = EPI == kEpiRes;
  constexpr bool kNorm = epi_norm(EPI);
  constexpr int kEpiIt = (MT + NW - 1) / NW;     // epilogue items per thread and tile
  FoldArgs fa{};
  u32x2 e_res[kRes ? NT : 1][kEpiIt];
  if constexpr (kRes) {
    fa = fold_args_here();
#pragma unroll
    for (int t0 = 0; t0 < NT; ++t0)
#pragma unroll
      for (int it = 0; it < kEpiIt; ++it) {
        const int idx = min((int)threadIdx.x + it * MG * NW * 64, MG * MT * 64 - 1);
        const int l = idx & 63;
        const int m = min((idx / (MT * 64) * MT + (idx >> 6) % MT) * 16 + (l & 15), M - 1);
        const int c = min((tile * NT + t0) * 16 + 4 * (l >> 4), p.N - 4);
        e_res[t0][it] = *global_ptr<const u32x2>(fa.residual + 2 * ((int64_t)(m0 + m) * fa.ldr + c));
      }
  }
  // Folded RMSNorm (consumer): the scale of each of this workgroup's rows,
  // from the producer's partial sums of squares, kept in LDS for the
  // epilogue.  The last wave copies the partials into LDS, and after its K
  // sweep sums them in one fixed order, so the scale is the same on every
  // call: row r of the R rows on R-lane groups, each lane summing every
  // (64 / R)-th partial, then an xor butterfly over the row's lanes.  The
  // copies are issued in asm, unseen by the compiler's wait-count pass:
  // through the builtin, that pass takes every later LDS operation of the K
  // sweep (the ds_bpermute shuffles) for a read of the copied words and
  // waits for every load in flight before it.  Unseen, they only make the
  // pass's wait for the first chunk wait for them as well.  (s_nop: the one
  // wait state an LDS DMA needs after an SALU write of M0.)
  constexpr int R = MG * MT * 16;
  static_assert(R <= 64 && 64 % R == 0, "rows of a workgroup on one wave");
  constexpr int LPR = 64 / R;                    // lanes per row
  constexpr int PPL = kMaxSumsqParts / LPR;      // partials per lane
  __shared__ float rscale[R];
  __shared__ float spart[kNorm ? PPL : 1][64];
  const bool copy_wave = kNorm && wid == MG * NW - 1;
  if (copy_wave) {
    fa = fold_args_here();
    const int m = m0 + min(lane % R, M - 1);
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
      if (LPR * j >= fa.parts) break;  // wave-uniform
      const int c = min(lane / R + LPR * j, fa.parts - 1);
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off"
                   :
                   : "s"(lds_addr(&spart[j][0])), "v"(fa.sumsq_in + (int64_t)c * p.M + m)
                   : "memory", "m0");
    }
  }

  if constexpr (kRope) {
#pragma unroll
    for (int j = 0; j < kIpt; ++j) {
      const int i = pair0 + ((int)threadIdx.x + j * kThreads) % 16;
      const int64_t pc = min(max(e_pos[j], (int64_t)0), (int64_t)p.max_pos - 1);
      e_cos[j] = p.cos_t[pc * half + i];
      e_sin[j] = p.sin_t[pc * half + i];
    }
  }
  int i = 0;
  // sched_barrier(0): the machine scheduler would otherwise sink the next
  // chunk's loads next to their MFMAs (to shorten live ranges), which turns
  // the two-stage pipeline back into one memory latency per chunk
  for (; i + 2 < n; i += 2) {
    load(wave + (i + 1) * NW, wb, xb);
    __builtin_amdgcn_sched_barrier(0);
    mma(wa, xa);
    __builtin_amdgcn_sched_barrier(0);
    load(wave + (i + 2) * NW, wa, xa);
    __builtin_amdgcn_sched_barrier(0);
    mma(wb, xb);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (i + 1 < n) {
    load(wave + (i + 1) * NW, wb, xb);
    __builtin_amdgcn_sched_barrier(0);
    mma(wa, xa);
    mma(wb, xb);
  } else if (i < n) {
    mma(wa, xa);
  }

  if (copy_wave) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the copies above (the sweep's loads are done)
    float ssum = 0.f;
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
      const float v = spart[j][lane];
      ssum += lane / R + LPR * j < fa.parts ? v : 0.f;
    }
#pragma unroll
    for (int o = R; o < 64; o <<= 1) ssum += __shfl_xor(ssum, o, 64);
    if (lane < R) rscale[lane] = 1.f / sqrtf(ssum / (float)fa.dim + fa.eps);
  }

  if constexpr (kRope) {
    // ---- 16 rotation pairs of one head for this row group ----
    // 1. partial sums to LDS; 2. reduce over the waves, add the bias, round
    // to bf16 (the projection's output); 3. rotate q and k heads with
    // bf16-rounded cos / sin and products (the arithmetic of bf16 tensors in
    // causal_lm.py:181-206, as rope_kv_write_kernel), write q to q_out and k
    // / v to the token's KV slot.
    static_assert(MG == 1, "one row group per workgroup");
    __shared__ floatx4 rred[2][NW][MT][64];
    __shared__ float hv[MT * 16][33];  // [m][tile * 16 + column], padded
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) rred[q][wave][mt][lane] = acc[q][mt];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kRpt; ++j) {
      const int r = threadIdx.x + j * kThreads;
      if (kRItems % kThreads == 0 || r < kRItems) {
        const int q = r / (MT * 64);
        const int mt = (r >> 6) % MT;
        const int l = r & 63;
        floatx4 sum = rred[q][0][mt][l];
#pragma unroll
        for (int w = 1; w < NW; ++w) sum += rred[q][w][mt][l];
        const uint2 bb = e_bias[j];
        const float b4[4] = {bf16_bits_to_float(bb.x & 0xffffu), bf16_bits_to_float(bb.x >> 16),
                             bf16_bits_to_float(bb.y & 0xffffu), bf16_bits_to_float(bb.y >> 16)};
        if constexpr (kNorm) sum *= rscale[mt * 16 + (l & 15)];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          hv[mt * 16 + (l & 15)][q * 16 + 4 * (l >> 4) + i] = bf16_round(sum[i] + b4[i]);
      }
    }
    __syncthreads();
    // head: q heads, then k heads, then v heads
    const bool rotate = head < p.Hq + p.Hkv;
#pragma unroll
    for (int j = 0; j < kIpt; ++j) {
      const int idx = threadIdx.x + j * kThreads;
      const int m = idx / 16;
      if ((kItems % kThreads != 0 && idx >= kItems) || m >= M) continue;
      const int il = idx % 16;
      const int i = pair0 + il;
      const int64_t t = m0 + m;
      const float x1 = hv[m][il], x2 = hv[m][16 + il];
      float y1 = x1, y2 = x2;
      if (rotate) {
        const bool pos_ok = e_pos[j] >= 0 && e_pos[j] < p.max_pos;
        const float c = pos_ok ? bf16_round(e_cos[j]) : 0.f;
        const float sn = pos_ok ? bf16_round(e_sin[j]) : 0.f;
        y1 = bf16_round(x1 * c) + bf16_round(-x2 * sn);
        y2 = bf16_round(x2 * c) + bf16_round(x1 * sn);
        if (!pos_ok && i == 0 && p.flags) atomicOr(p.flags, 1);
      }
      uint16_t* dst = nullptr;
      if (head < p.Hq) {
        dst = reinterpret_cast<uint16_t*>(p.q_out) + (t * p.Hq + head) * p.head_dim;
      } else {
        const int64_t slot = e_slot[j];
        if (slot >= 0 && slot < p.num_slots) {
          const int kh = rotate ? head - p.Hq : head - p.Hq - p.Hkv;
          dst = reinterpret_cast<uint16_t*>(rotate ? p.kc : p.vc) +
                (slot * p.Hkv + kh) * p.head_dim;
        } else if (slot >= p.num_slots && i == 0 && p.flags) {
          atomicOr(p.flags, 1);
        }
      }
      if (dst) {
        dst[i] = float_to_bf16_bits(y1);
        dst[i + half] = float_to_bf16_bits(y2);
      }
    }
    return;
  }

  // kEpiArgmax: this thread's best key over the tiles, per epilogue item
  constexpr bool kArg = EPI == kEpiArgmax;
  uint64_t best[kArg ? kEpiIt : 1] = {};
  // cross-wave reduction and epilogue, NP physical tiles at a time.  Lane l
  // of tile (nt, mt) holds y rows m = 16 mt + l % 16, columns 4 (l / 16) + i.
#pragma unroll
  for (int t0 = 0; t0 < NT; t0 += NP) {
#pragma unroll
    for (int q = 0; q < NP; ++q)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) red[grp][q][wave][mt][lane] = acc[t0 + q][mt];
    __syncthreads();
#pragma unroll
    for (int it = 0; it < kEpiIt; ++it) {
      const int idx = threadIdx.x + it * MG * NW * 64;
      if (idx >= MG * MT * 64) continue;  // wave-uniform
      const int g = idx / (MT * 64);
      const int mt = (idx >> 6) % MT;
      const int l = idx & 63;
      const int m = (g * MT + mt) * 16 + (l & 15);
      floatx4 s[NP];
#pragma unroll
      for (int q = 0; q < NP; ++q) {
        s[q] = red[g][q][0][mt][l];
#pragma unroll
        for (int w = 1; w < NW; ++w) s[q] += red[g][q][w][mt][l];
      }
      int n;
      if constexpr (epi_silu(EPI))
        n = (tile * (NT / 2) + t0 / 2) * 16 + 4 * (l >> 4);
      else
        n = (tile * NT + t0) * 16 + 4 * (l >> 4);
      const bool ok = m < M && n < p.N;
      float v[4];
      if constexpr (epi_silu(EPI)) {
        if constexpr (kNorm) {
#pragma unroll
          for (int q = 0; q < NP; ++q) s[q] *= rscale[m];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float g = bf16_bits_to_float(float_to_bf16_bits(s[0][i]));
          const float u = bf16_bits_to_float(float_to_bf16_bits(s[1][i]));
          v[i] = silu_bf16(g) * u;
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = s[0][i];
        if (p.bias && ok) {
          const u32x2 b = *reinterpret_cast<const u32x2*>(p.bias + n);
          v[0] += bf16_bits_to_float(b[0] & 0xffff);
          v[1] += bf16_bits_to_float(b[0] >> 16);
          v[2] += bf16_bits_to_float(b[1] & 0xffff);
          v[3] += bf16_bits_to_float(b[1] >> 16);
        }
        if constexpr (kRes) {
          // producer of a folded RMSNorm: the bf16 residual add, then the
          // partial sum of squares of the 16 columns n & ~15 .. + 15 of row
          // m (the four lanes l, l ^ 16, l ^ 32, l ^ 48 hold them)
          float sq = 0.f;
          if (ok) {
            const u32x2 r = e_res[t0][it];
            const float rv[4] = {bf16_bits_to_float(r[0] & 0xffff), bf16_bits_to_float(r[0] >> 16),
                                 bf16_bits_to_float(r[1] & 0xffff), bf16_bits_to_float(r[1] >> 16)};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              v[i] = bf16_round(rv[i] + bf16_round(v[i]));
              sq = __builtin_fmaf(v[i], v[i], sq);
            }
          }
          sq = sum_xor16_32(sq);
          if (ok && (l >> 4) == 0) *global_ptr<float>(fa.sumsq_out + 4 * ((int64_t)(n >> 4) * p.M + m0 + m)) = sq;
        }
      }
      if constexpr (kArg) {
        // key = (order-preserving bits of the bf16 value, ~column): the max
        // key is the largest value at its lowest column (-0 counts as +0)
        if (ok) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            uint32_t b = float_to_bf16_bits(v[i]);
            b = b == 0x8000u ? 0u : b;
            const uint32_t ord = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
            const uint64_t key = ((uint64_t)ord << 32) | (0xffffffffu - (uint32_t)(n + i));
            best[it] = key > best[it] ? key : best[it];
          }
        }
        continue;
      }
      if (!ok) continue;
      *reinterpret_cast<u32x2*>(yg + (int64_t)m * p.ldy + n) =
          u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    }
    __syncthreads();
  }
  if constexpr (kArg) {
    // the four lanes of a row's 16 columns meet, then one lane stores the
    // row's key for this workgroup's columns: keys[row * col_tiles + tile]
    uint64_t* keys = reinterpret_cast<uint64_t*>(p.y);
#pragma unroll
    for (int it = 0; it < kEpiIt; ++it) {
      const int idx = threadIdx.x + it * MG * NW * 64;
      if (idx >= MG * MT * 64) continue;  // wave-uniform
      const int l = idx & 63;
      const int m = (idx / (MT * 64) * MT + (idx >> 6) % MT) * 16 + (l & 15);
      uint64_t k = best[it];
#pragma unroll
      for (int o = 16; o < 64; o <<= 1) {
        const uint64_t other = ((uint64_t)(uint32_t)__shfl_xor((int)(k >> 32), o, 64) << 32) |
                               (uint32_t)__shfl_xor((int)(uint32_t)k, o, 64);
        k = other > k ? other : k;
      }
      if ((l >> 4) == 0 && m < M) keys[(int64_t)(m0 + m) * p.col_tiles + tile] = k;
    }
  }
}

// Per row, the largest of the lm_head workgroups' keys -> the column (token):
// one workgroup per row.
__global__ __launch_bounds__(256) void argmax_keys_kernel(const uint64_t* __restrict__ keys,
                                                          int tiles, int64_t* __restrict__ out,
                                                          int64_t out_stride) {
  const uint64_t* row = keys + (int64_t)blockIdx.x * tiles;
  uint64_t k = 0;
  for (int t = threadIdx.x; t < tiles; t += 256) k = row[t] > k ? row[t] : k;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t other = ((uint64_t)(uint32_t)__shfl_xor((int)(k >> 32), o, 64) << 32) |
                           (uint32_t)__shfl_xor((int)(uint32_t)k, o, 64);
    k = other > k ? other : k;
  }
  __shared__ uint64_t wk[4];
  if ((threadIdx.x & 63) == 0) wk[threadIdx.x >> 6] = k;
  __syncthreads();
  if (threadIdx.x == 0) {
    k = wk[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) k = wk[w] > k ? wk[w] : k;
    out[(int64_t)blockIdx.x * out_stride] = (int64_t)(0xffffffffu - (uint32_t)k);
  }
}

// Tile shape per row count: more W rows per workgroup as M grows, so that x
// (read from L2 once per workgroup) stays a small multiple of W's bytes.
template <int MT, int MG, int NT, int NW, int EPI>
int32_t launch_cfg(LinParams& p, hipStream_t s) {
  constexpr int kRows = MG * MT * 16;  // rows per workgroup
  p.row_groups = p.M > kRows ? (p.M + kRows - 1) / kRows : 1;
  if constexpr (!epi_norm(EPI) && EPI != kEpiRes && EPI != kEpiArgmax) {  // bf16 weights only
    if (p.w8) {
      const int cols_per_wg = 16 * (epi_silu(EPI) ? NT / 2 : NT);
      p.col_tiles = (p.N + cols_per_wg - 1) / cols_per_wg;
      int grid = p.col_tiles;
      if (p.row_groups > 1) grid = p.row_groups * 8 * ((p.col_tiles + 7) / 8);
      hipLaunchKernelGGL((linear_kernel<MT, MG, NT, NW, EPI, true>), dim3(grid),
                         dim3(MG * NW * 64), 0, s, p);
      return launch_status("linear_kernel");
    }
  }
  const int cols_per_wg = 16 * (epi_silu(EPI) ? NT / 2 : NT);
  p.col_tiles = (p.N + cols_per_wg - 1) / cols_per_wg;
  int grid = p.col_tiles;
  if (p.row_groups > 1) grid = p.row_groups * 8 * ((p.col_tiles + 7) / 8);
  hipLaunchKernelGGL((linear_kernel<MT, MG, NT, NW, EPI>), dim3(grid), dim3(MG * NW * 64), 0, s,
                     p);
  return launch_status("linear_kernel");
}

// Up to MG * MT * 16 rows: one workgroup per column tile.  More rows run as
// groups of that many rows, one workgroup per (column tile, group), with the
// groups of a tile on one XCD.  Tile shape per row count, measured on MI355X
// for the shapes of the verify forward (graph replay, weights cold): the
// workgroup count against 256 CUs decides most of it, since each CU streams
// its workgroups' W rows at a bounded rate.
constexpr int kWideN = 65536;
constexpr int64_t kBigWeight = 16ll << 20;  // weights of 8B-class layers and beyond
constexpr int kLongRow = 2048;   // K from which a wide output's rows count as long

template <int EPI>
int32_t launch_epi(LinParams& p, hipStream_t s) {
  if constexpr (epi_silu(EPI)) {
    // NT counts gate and up tiles: NT = 2 is one output column tile
    if (p.M <= 16) return launch_cfg<1, 1, 2, 2, EPI>(p, s);
    if (p.M <= 32) return launch_cfg<2, 1, 2, 2, EPI>(p, s);
    if (p.M <= 64) return launch_cfg<2, 1, 2, 4, EPI>(p, s);
    if (p.M <= 96) return launch_cfg<2, 1, 4, 4, EPI>(p, s);
    if (p.M <= 128) return launch_cfg<2, 1, 2, 4, EPI>(p, s);
    return launch_cfg<2, 1, 4, 2, EPI>(p, s);
  } else {
    if constexpr (EPI == kEpiBias || EPI == kEpiArgmax) {
      if (p.N >= kWideN) {  // lm_head
        if (p.M == 1) return launch_cfg<1, 1, 1, 8, EPI>(p, s);
        if (p.M <= 8) return launch_cfg<1, 1, 2, 8, EPI>(p, s);
        if (p.K >= 2048) {  // long rows (8B-class lm_head): eight column tiles
          if (p.M <= 16) return launch_cfg<2, 1, 8, 4, EPI>(p, s);
          return launch_cfg<2, 1, 8, 2, EPI>(p, s);
        }
        if (p.M <= 16) return launch_cfg<1, 1, 4, 1, EPI>(p, s);
        return launch_cfg<2, 1, 4, 2, EPI>(p, s);
      }
    }
    if (p.M <= 16) return launch_cfg<1, 1, 1, 8, EPI>(p, s);
    // up to 64 rows of weights under 16 M elements (the 0.5B o_proj and
    // down_proj, 896 output columns): 16-row groups of eight waves spread
    // the few column tiles over more CUs (down_proj at 24 - 64 rows 7.6 ->
    // 6.1 us, o_proj 3.5 -> 3.3; from 80 rows, and for 8B-class weights,
    // slower)
    if (p.M <= 64 && (int64_t)p.N * p.K < kBigWeight) return launch_cfg<1, 1, 1, 8, EPI>(p, s);
    if (p.M <= 128) return launch_cfg<2, 1, 1, 4, EPI>(p, s);
    return launch_cfg<2, 1, 2, 4, EPI>(p, s);
  }
}

// RoPE epilogue: a workgroup per (head, 16 rotation pairs) -- two column
// tiles -- and row group.  16-row groups up to 64 rows for weights under 16 M
// elements (the 0.5B q/k/v at 24 - 64 rows: 5.05 -> 4.5 us).
template <int EPI>
int32_t launch_rope(LinParams& p, hipStream_t s) {
  if (p.M <= 16 || (p.M <= 64 && (int64_t)p.N * p.K < kBigWeight))
    return launch_cfg<1, 1, 2, 8, EPI>(p, s);
  return launch_cfg<2, 1, 2, 8, EPI>(p, s);
}

}  // namespace
}  // namespace nsg

using namespace nsg;

// Where these kernels beat hipBLASLt on MI355X (measured per shape, weights
// streamed from HBM): up to 160 rows for the 0.5B-class q/k/v, o_proj,
// gate/up and down_proj shapes (weights up to 17 MB) and for the 0.5B-class
// lm_head (lm_head.hip's kernel: 69 against 101 us at 160 rows), up to 32
// for weights of 16 M elements or more (8B-class layers and lm_head, where
// the library's tiles win from about 64 rows: 212 against 219 us at 64 rows
// of the 128,256 x 4096 lm_head).
constexpr int kFastRows = 160;
constexpr int kFastRowsBig = 32;

extern "C" int32_t nsg_linear_max_rows(void) { return kMaxMT * 16; }

extern "C" int32_t nsg_linear_preferred(int32_t M, int32_t N, int32_t K) {
  if (M < 1 || K % kChunk != 0 || N % 4 != 0) return 0;
  const bool big = N >= kWideN ? K >= kLongRow : (int64_t)N * K >= kBigWeight;
  return M <= (big ? kFastRowsBig : kFastRows) ? 1 : 0;
}

namespace {

// Shared by the bf16 and FP8-weight entry points: exactly one of w / w8 is
// given; w8 rows are ldw bytes apart and w_scale holds one f32 per W row.
// Folded-RMSNorm arguments of the *_fold entry points (see LinParams).
struct NormFold {
  const float* sumsq_in;
  int32_t parts;
  int32_t dim;
  float eps;
  const void* residual;
  int64_t ldr;
  float* sumsq_out;
};

// Checks the folded-norm arguments and copies them into p.
int32_t apply_fold(LinParams& p, const NormFold* nf, int32_t N, bool consumer_ok,
                   bool producer_ok) {
  if (!nf) return NSG_OK;
  if (nf->sumsq_in) {
    NSG_CHECK_ARG(consumer_ok, "the row scale takes the SwiGLU or RoPE epilogue");
    NSG_CHECK_ARG(nf->parts >= 1 && nf->parts <= kMaxSumsqParts && nf->dim > 0 && nf->eps >= 0.f,
                  "folded norm: %d partials (1 .. %d), dim %d, eps %g", nf->parts, kMaxSumsqParts,
                  nf->dim, (double)nf->eps);
    p.sumsq_in = nf->sumsq_in;
    p.sumsq_parts = nf->parts;
    p.norm_dim = nf->dim;
    p.norm_eps = nf->eps;
  }
  if (nf->residual || nf->sumsq_out) {
    NSG_CHECK_ARG(producer_ok, "the residual add takes the bias epilogue");
    NSG_CHECK_ARG(nf->residual && nf->sumsq_out && N % 16 == 0 && nf->ldr >= N && nf->ldr % 4 == 0 &&
                      (uintptr_t)nf->residual % 8 == 0,
                  "folded norm producer: residual (8-byte aligned rows, ldr %lld >= N %d) and "
                  "sumsq_out needed, N a multiple of 16", (long long)nf->ldr, N);
    p.residual = static_cast<const bf16*>(nf->residual);
    p.ldr = nf->ldr;
    p.sumsq_out = nf->sumsq_out;
  }
  return NSG_OK;
}

// Wide outputs (lm_head) without a bias or folded norm, bf16 weights:
// lm_head.hip's kernel (x shared by 128 output columns), at any row count
// for rows shorter than 2048 (151,936 x 896: 45 against 53 - 59 us at 1 - 32
// rows), above 32 rows for longer ones (128,256 x 4096: there this kernel's
// eight-tile shapes stream faster up to 32 rows, 177 against 198 us).
// gate/up + SwiGLU (bf16 weights) from this many rows on: lm_head.hip's ring
// kernel (80-row x 48-column workgroups, W once per XCD) instead of the
// weight-streaming kernel's 32-row groups.
constexpr int kRingSwigluMinRows = 33;

bool head_route(const LinParams& p) {
  return p.w && !p.bias && p.w_rows == p.N && !p.sumsq_in && !p.residual && p.N >= kWideN &&
         (p.K < kLongRow || p.M > 32) && p.M <= kHeadMaxRows && p.K % kHeadStep == 0 &&
         p.K >= 3 * kHeadStep;
}

int32_t linear_impl(const void* x, int64_t ldx, const void* w, const void* w8, int64_t ldw,
                    const float* w_scale, const void* bias, void* y, int64_t ldy, int32_t M,
                    int32_t N, int32_t K, int32_t epilogue, nsg_stream_t stream,
                    const NormFold* nf = nullptr) {
  NSG_CHECK_ARG(M >= 0 && N > 0 && K > 0, "M %d, N %d, K %d", M, N, K);
  if (M == 0) {
    clear_error();
    return NSG_OK;
  }
  NSG_CHECK_ARG(x && (w || (w8 && w_scale)) && y, "null pointer argument");
  NSG_CHECK_ARG(epilogue == NSG_LINEAR_BIAS || epilogue == NSG_LINEAR_SILU_MUL,
                "unknown epilogue %d", epilogue);
  NSG_CHECK_ARG(!(epilogue == NSG_LINEAR_SILU_MUL && bias), "SwiGLU epilogue takes no bias");
  if (M > kMaxMT * 16) {
    set_error("M %d > %d rows (use a library GEMM)", M, kMaxMT * 16);
    return NSG_ERR_UNSUPPORTED;
  }
  if (K % kChunk != 0 || N % 4 != 0) {
    set_error("K %d must be a multiple of %d and N %d of 4", K, kChunk, N);
    return NSG_ERR_UNSUPPORTED;
  }
  NSG_CHECK_ARG(ldx >= K && ldw >= K && ldy >= N, "leading dimensions too small");
  NSG_CHECK_ARG(ldx % 8 == 0 && ldw % 8 == 0 && ldy % 4 == 0 && (uintptr_t)x % 16 == 0 &&
                    (w ? (uintptr_t)w % 16 : (uintptr_t)w8 % 8) == 0 && (uintptr_t)y % 8 == 0 &&
                    (uintptr_t)bias % 8 == 0,
                "x and bf16 w rows must be 16-byte aligned, fp8 w rows, y rows and bias 8-byte");
  LinParams p{};
  p.x = static_cast<const bf16*>(x);
  p.w = static_cast<const bf16*>(w);
  p.w8 = w ? nullptr : static_cast<const uint8_t*>(w8);
  p.w_scale = w ? nullptr : w_scale;
  p.bias = static_cast<const bf16*>(bias);
  p.y = static_cast<bf16*>(y);
  p.ldx = ldx;
  p.ldw = ldw;
  p.ldy = ldy;
  p.M = M;
  p.N = N;
  p.K = K;
  p.w_rows = epilogue == NSG_LINEAR_SILU_MUL ? 2 * N : N;
  if (int32_t rc = apply_fold(p, nf, N, epilogue == NSG_LINEAR_SILU_MUL, epilogue == NSG_LINEAR_BIAS))
    return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (epilogue == NSG_LINEAR_SILU_MUL && p.w && M >= kRingSwigluMinRows &&
      ring_swiglu_fits(M, N, K, p.sumsq_in ? p.sumsq_parts : 0)) {
    const GuParams gp{p.x, p.w, p.y, ldx, ldw, ldy, M, N, K,
                      p.sumsq_in, p.sumsq_parts, p.norm_dim, p.norm_eps};
    return launch_ring_swiglu(gp, s);
  }
  if (head_route(p)) {
    const HeadParams hp{p.x, p.w, p.y, p.ldx, p.ldw, p.ldy, M, N, K};
    int key_cols = 0;
    return launch_lm_head(hp, false, s, &key_cols);
  }
  if (epilogue == NSG_LINEAR_SILU_MUL)
    return p.sumsq_in ? launch_epi<kEpiSiluN>(p, s) : launch_epi<kEpiSilu>(p, s);
  return p.residual ? launch_epi<kEpiRes>(p, s) : launch_epi<kEpiBias>(p, s);
}

int32_t rope_impl(const void* x, int64_t ldx, const void* w, const void* w8, int64_t ldw,
                  const float* w_scale, const void* bias, int32_t M, int32_t K,
                  int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                  const int64_t* positions, const float* cos_table, const float* sin_table,
                  int32_t max_position, const int64_t* slots, void* q_out, void* k_cache,
                  void* v_cache, int64_t num_slots, int32_t* flags, nsg_stream_t stream,
                  const NormFold* nf = nullptr) {
  NSG_CHECK_ARG(M >= 0 && K > 0, "M %d, K %d", M, K);
  if (M == 0) {
    clear_error();
    return NSG_OK;
  }
  NSG_CHECK_ARG(x && (w || (w8 && w_scale)) && positions && cos_table && sin_table && q_out,
                "null pointer argument");
  NSG_CHECK_ARG(num_qo_heads > 0 && num_kv_heads > 0, "heads %d / %d", num_qo_heads, num_kv_heads);
  NSG_CHECK_ARG(!slots || (k_cache && v_cache && num_slots > 0), "slots need both caches");
  if (head_dim != 64 && head_dim != 128) {
    set_error("head_dim %d not supported (64 or 128)", head_dim);
    return NSG_ERR_UNSUPPORTED;
  }
  if (M > kMaxMT * 16 || K % kChunk != 0) {
    set_error("M %d > %d or K %d not a multiple of %d", M, kMaxMT * 16, K, kChunk);
    return NSG_ERR_UNSUPPORTED;
  }
  const int N = (num_qo_heads + 2 * num_kv_heads) * head_dim;
  NSG_CHECK_ARG(ldx >= K && ldw >= K && ldx % 8 == 0 && ldw % 8 == 0 && (uintptr_t)x % 16 == 0 &&
                    (w ? (uintptr_t)w % 16 : (uintptr_t)w8 % 8) == 0,
                "x and bf16 w rows must be 16-byte aligned, fp8 w rows 8-byte");
  NSG_CHECK_ARG(max_position > 0, "max_position %d", max_position);
  NSG_CHECK_ARG((uintptr_t)bias % 8 == 0, "bias must be 8-byte aligned");
  LinParams p{};
  p.x = static_cast<const bf16*>(x);
  p.w = static_cast<const bf16*>(w);
  p.w8 = w ? nullptr : static_cast<const uint8_t*>(w8);
  p.w_scale = w ? nullptr : w_scale;
  p.bias = static_cast<const bf16*>(bias);
  p.y = nullptr;
  p.ldx = ldx;
  p.ldw = ldw;
  p.ldy = 0;
  p.M = M;
  p.N = N;
  p.K = K;
  p.w_rows = N;
  p.pos = positions;
  p.cos_t = cos_table;
  p.sin_t = sin_table;
  p.max_pos = max_position;
  p.slots = slots;
  p.Hq = num_qo_heads;
  p.Hkv = num_kv_heads;
  p.head_dim = head_dim;
  p.q_out = static_cast<bf16*>(q_out);
  p.kc = static_cast<bf16*>(k_cache);
  p.vc = static_cast<bf16*>(v_cache);
  p.num_slots = num_slots;
  p.flags = flags;
  if (int32_t rc = apply_fold(p, nf, N, true, false)) return rc;
  return p.sumsq_in ? launch_rope<kEpiRopeN>(p, static_cast<hipStream_t>(stream))
                    : launch_rope<kEpiRope>(p, static_cast<hipStream_t>(stream));
}

}  // namespace

extern "C" int32_t nsg_linear(const void* x, int64_t ldx, const void* w, int64_t ldw,
                              const void* bias, void* y, int64_t ldy, int32_t M, int32_t N,
                              int32_t K, int32_t epilogue, nsg_stream_t stream) {
  NSG_CHECK_ARG(w, "null weight");
  return linear_impl(x, ldx, w, nullptr, ldw, nullptr, bias, y, ldy, M, N, K, epilogue, stream);
}

extern "C" int32_t nsg_linear_fp8(const void* x, int64_t ldx, const void* w8, int64_t ldw8,
                                  const float* w_scale, const void* bias, void* y, int64_t ldy,
                                  int32_t M, int32_t N, int32_t K, int32_t epilogue,
                                  nsg_stream_t stream) {
  NSG_CHECK_ARG(w8 && w_scale, "null fp8 weight or scales");
  return linear_impl(x, ldx, nullptr, w8, ldw8, w_scale, bias, y, ldy, M, N, K, epilogue, stream);
}

extern "C" int32_t nsg_linear_rope_kv(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                      const void* bias, int32_t M, int32_t K,
                                      int32_t num_qo_heads, int32_t num_kv_heads,
                                      int32_t head_dim, const int64_t* positions,
                                      const float* cos_table, const float* sin_table,
                                      int32_t max_position, const int64_t* slots, void* q_out,
                                      void* k_cache, void* v_cache, int64_t num_slots,
                                      int32_t* flags, nsg_stream_t stream) {
  NSG_CHECK_ARG(w, "null weight");
  return rope_impl(x, ldx, w, nullptr, ldw, nullptr, bias, M, K, num_qo_heads, num_kv_heads,
                   head_dim, positions, cos_table, sin_table, max_position, slots, q_out, k_cache,
                   v_cache, num_slots, flags, stream);
}

extern "C" int32_t nsg_linear_rope_kv_fp8(const void* x, int64_t ldx, const void* w8,
                                          int64_t ldw8, const float* w_scale, const void* bias,
                                          int32_t M, int32_t K, int32_t num_qo_heads,
                                          int32_t num_kv_heads, int32_t head_dim,
                                          const int64_t* positions, const float* cos_table,
                                          const float* sin_table, int32_t max_position,
                                          const int64_t* slots, void* q_out, void* k_cache,
                                          void* v_cache, int64_t num_slots, int32_t* flags,
                                          nsg_stream_t stream) {
  NSG_CHECK_ARG(w8 && w_scale, "null fp8 weight or scales");
  return rope_impl(x, ldx, nullptr, w8, ldw8, w_scale, bias, M, K, num_qo_heads, num_kv_heads,
                   head_dim, positions, cos_table, sin_table, max_position, slots, q_out, k_cache,
                   v_cache, num_slots, flags, stream);
}

// ---- RMSNorm folded into the linears around it (bf16 weights) ----
extern "C" int32_t nsg_linear_fold(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                   const void* bias, void* y, int64_t ldy, int32_t M, int32_t N,
                                   int32_t K, int32_t epilogue, const float* sumsq_in,
                                   int32_t sumsq_parts, int32_t norm_dim, float eps,
                                   const void* residual, int64_t ldr, float* sumsq_out,
                                   nsg_stream_t stream) {
  NSG_CHECK_ARG(w, "null weight");
  const NormFold nf{sumsq_in, sumsq_parts, norm_dim, eps, residual, ldr, sumsq_out};
  return linear_impl(x, ldx, w, nullptr, ldw, nullptr, bias, y, ldy, M, N, K, epilogue, stream,
                     &nf);
}

extern "C" int32_t nsg_linear_rope_kv_fold(
    const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias, int32_t M,
    int32_t K, int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
    const int64_t* positions, const float* cos_table, const float* sin_table,
    int32_t max_position, const int64_t* slots, void* q_out, void* k_cache, void* v_cache,
    int64_t num_slots, int32_t* flags, const float* sumsq_in, int32_t sumsq_parts,
    int32_t norm_dim, float eps, nsg_stream_t stream) {
  NSG_CHECK_ARG(w && sumsq_in, "null weight or sums of squares");
  const NormFold nf{sumsq_in, sumsq_parts, norm_dim, eps, nullptr, 0, nullptr};
  return rope_impl(x, ldx, w, nullptr, ldw, nullptr, bias, M, K, num_qo_heads, num_kv_heads,
                   head_dim, positions, cos_table, sin_table, max_position, slots, q_out, k_cache,
                   v_cache, num_slots, flags, stream, &nf);
}

// ---- lm_head + greedy token: argmax of the bf16 logits, never stored ----
extern "C" int64_t nsg_linear_argmax_workspace_bytes(int32_t M, int32_t N) {
  if (M <= 0 || N <= 0) return 0;
  return (int64_t)M * ((N + 15) / 16) * (int64_t)sizeof(uint64_t);
}

extern "C" int32_t nsg_linear_argmax(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                     const void* bias, int32_t M, int32_t N, int32_t K,
                                     void* workspace, int64_t workspace_bytes, int64_t* tokens,
                                     int64_t token_stride, nsg_stream_t stream) {
  NSG_CHECK_ARG(M >= 0 && N > 0 && K > 0, "M %d, N %d, K %d", M, N, K);
  if (M == 0) {
    clear_error();
    return NSG_OK;
  }
  NSG_CHECK_ARG(x && w && workspace && tokens && token_stride >= 1, "null pointer argument or token stride < 1");
  if (M > kMaxMT * 16) {
    set_error("M %d > %d rows", M, kMaxMT * 16);
    return NSG_ERR_UNSUPPORTED;
  }
  if (K % kChunk != 0 || N % 4 != 0) {
    set_error("K %d must be a multiple of %d and N %d of 4", K, kChunk, N);
    return NSG_ERR_UNSUPPORTED;
  }
  NSG_CHECK_ARG(ldx >= K && ldw >= K && ldx % 8 == 0 && ldw % 8 == 0 && (uintptr_t)x % 16 == 0 &&
                    (uintptr_t)w % 16 == 0 && (uintptr_t)bias % 8 == 0 &&
                    (uintptr_t)workspace % 8 == 0,
                "x and w rows must be 16-byte aligned, bias and workspace 8-byte");
  NSG_CHECK_ARG(workspace_bytes >= nsg_linear_argmax_workspace_bytes(M, N),
                "workspace %lld bytes < %lld", (long long)workspace_bytes,
                (long long)nsg_linear_argmax_workspace_bytes(M, N));
  LinParams p{};
  p.x = static_cast<const bf16*>(x);
  p.w = static_cast<const bf16*>(w);
  p.bias = static_cast<const bf16*>(bias);
  p.y = static_cast<bf16*>(workspace);  // the per-workgroup keys
  p.ldx = ldx;
  p.ldw = ldw;
  p.M = M;
  p.N = N;
  p.K = K;
  p.w_rows = N;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int key_cols = 0;
  if (head_route(p)) {
    const HeadParams hp{p.x, p.w, workspace, p.ldx, p.ldw, 0, M, N, K};
    if (int32_t rc = launch_lm_head(hp, true, s, &key_cols)) return rc;
  } else {
    if (int32_t rc = launch_epi<kEpiArgmax>(p, s)) return rc;
    key_cols = p.col_tiles;
  }
  hipLaunchKernelGGL(argmax_keys_kernel, dim3(M), dim3(256), 0, s,
                     static_cast<const uint64_t*>(workspace), key_cols, tokens, token_stride);
  return launch_status("argmax_keys_kernel");
}

// ---- lm_head with the final RMSNorm folded in (bf16 weights) ----
namespace {

int32_t head_fold_params(const void* x, int64_t ldx, const void* w, int64_t ldw, int32_t M,
                         int32_t N, int32_t K, const float* sumsq_in, int32_t sumsq_parts,
                         int32_t norm_dim, float eps, HeadParams* hp) {
  NSG_CHECK_ARG(x && w && sumsq_in, "null x, weight or sums of squares");
  NSG_CHECK_ARG(M >= 1 && M <= kHeadMaxRows, "M %d outside [1, %d]", M, kHeadMaxRows);
  NSG_CHECK_ARG(N >= 4 && N % 4 == 0, "N %d must be a positive multiple of 4", N);
  NSG_CHECK_ARG(K >= 3 * kHeadStep && K % kHeadStep == 0, "K %d must be a multiple of %d, >= %d",
                K, kHeadStep, 3 * kHeadStep);
  NSG_CHECK_ARG(ldx >= K && ldw >= K && ldx % 8 == 0 && ldw % 8 == 0 && (uintptr_t)x % 16 == 0 &&
                    (uintptr_t)w % 16 == 0 && (uintptr_t)sumsq_in % 16 == 0,
                "x and w rows and sumsq_in must be 16-byte aligned");
  NSG_CHECK_ARG(sumsq_parts >= 1 && norm_dim > 0 && eps >= 0.f,
                "folded norm: %d partials, dim %d, eps %g", sumsq_parts, norm_dim, (double)eps);
  if (!lm_head_fold_fits(M, sumsq_parts)) {
    set_error("the folded norm does not fit at M %d with %d partials per row", M, sumsq_parts);
    return NSG_ERR_UNSUPPORTED;
  }
  *hp = HeadParams{static_cast<const bf16*>(x), static_cast<const bf16*>(w), nullptr, ldx, ldw,
                   0, M, N, K, sumsq_in, sumsq_parts, norm_dim, eps};
  return NSG_OK;
}

}  // namespace

extern "C" int32_t nsg_lm_head_fold_supported(int32_t M, int32_t N, int32_t K,
                                              int32_t sumsq_parts) {
  return M >= 1 && M <= kHeadMaxRows && N >= 4 && N % 4 == 0 && K >= 3 * kHeadStep &&
                 K % kHeadStep == 0 && lm_head_fold_fits(M, sumsq_parts)
             ? 1
             : 0;
}

extern "C" int32_t nsg_lm_head_fold(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                    void* y, int64_t ldy, int32_t M, int32_t N, int32_t K,
                                    const float* sumsq_in, int32_t sumsq_parts, int32_t norm_dim,
                                    float eps, nsg_stream_t stream) {
  HeadParams hp{};
  if (int32_t rc = head_fold_params(x, ldx, w, ldw, M, N, K, sumsq_in, sumsq_parts, norm_dim,
                                    eps, &hp))
    return rc;
  NSG_CHECK_ARG(y && ldy >= N && ldy % 4 == 0 && (uintptr_t)y % 8 == 0,
                "y rows must be 8-byte aligned, ldy %lld >= N %d", (long long)ldy, N);
  hp.out = y;
  hp.ldy = ldy;
  int key_cols = 0;
  return launch_lm_head(hp, false, static_cast<hipStream_t>(stream), &key_cols);
}

extern "C" int32_t nsg_lm_head_fold_argmax(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                           int32_t M, int32_t N, int32_t K,
                                           const float* sumsq_in, int32_t sumsq_parts,
                                           int32_t norm_dim, float eps, void* workspace,
                                           int64_t workspace_bytes, int64_t* tokens,
                                           int64_t token_stride, nsg_stream_t stream) {
  HeadParams hp{};
  if (int32_t rc = head_fold_params(x, ldx, w, ldw, M, N, K, sumsq_in, sumsq_parts, norm_dim,
                                    eps, &hp))
    return rc;
  NSG_CHECK_ARG(workspace && tokens && token_stride >= 1 && (uintptr_t)workspace % 8 == 0,
                "null workspace or tokens, token stride < 1, or workspace not 8-byte aligned");
  NSG_CHECK_ARG(workspace_bytes >= nsg_linear_argmax_workspace_bytes(M, N),
                "workspace %lld bytes < %lld", (long long)workspace_bytes,
                (long long)nsg_linear_argmax_workspace_bytes(M, N));
  hp.out = workspace;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int key_cols = 0;
  if (int32_t rc = launch_lm_head(hp, true, s, &key_cols)) return rc;
  hipLaunchKernelGGL(argmax_keys_kernel, dim3(M), dim3(256), 0, s,
                     static_cast<const uint64_t*>(workspace), key_cols, tokens, token_stride);
  return launch_status("argmax_keys_kernel");
}

extern "C" int32_t nsg_lm_head_fold_keys(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                         int32_t M, int32_t N, int32_t K,
                                         const float* sumsq_in, int32_t sumsq_parts,
                                         int32_t norm_dim, float eps, void* keys,
                                         int64_t keys_bytes, int32_t* key_cols,
                                         nsg_stream_t stream) {
  HeadParams hp{};
  if (int32_t rc = head_fold_params(x, ldx, w, ldw, M, N, K, sumsq_in, sumsq_parts, norm_dim,
                                    eps, &hp))
    return rc;
  NSG_CHECK_ARG(keys && key_cols && (uintptr_t)keys % 8 == 0,
                "null keys or key_cols, or keys not 8-byte aligned");
  NSG_CHECK_ARG(keys_bytes >= nsg_linear_argmax_workspace_bytes(M, N), "keys %lld bytes < %lld",
                (long long)keys_bytes, (long long)nsg_linear_argmax_workspace_bytes(M, N));
  hp.out = keys;
  int kc = 0;
  if (int32_t rc = launch_lm_head(hp, true, static_cast<hipStream_t>(stream), &kc)) return rc;
  *key_cols = kc;
  return NSG_OK;
}

// ---- FP8 weights for a library GEMM (many rows, prefill) ----
// The dequantisation of FP8Linear.forward (w8.to(bf16) * scale,
// quantization.py:49-52) in one pass: 16 weight bytes per thread in, 32
// bytes of bf16 out, the same per-value arithmetic as the in-register path
// (exact e4m3 -> f32, times the row scale, one round to nearest even).
namespace nsg {
namespace {

__global__ __launch_bounds__(256) void dequant_fp8_kernel(const uint8_t* w8, int64_t ld8,
                                                          const float* scale, uint16_t* out,
                                                          int64_t ldo, int rows, int cols,
                                                          bool vec) {
  const int64_t gpr = (cols + 15) / 16;  // 16-value groups per row
  const int64_t total = (int64_t)rows * gpr;
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < total;
       g += (int64_t)gridDim.x * blockDim.x) {
    const int row = (int)(g / gpr);
    const int c0 = (int)(g % gpr) * 16;
    const float s = scale[row];
    const uint8_t* src = w8 + (int64_t)row * ld8 + c0;
    uint16_t* dst = out + (int64_t)row * ldo + c0;
    if (vec && c0 + 16 <= cols) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(src);
      *reinterpret_cast<u32x4*>(dst) = dequant_fp8x8(u32x2{v[0], v[1]}, s);
      *reinterpret_cast<u32x4*>(dst + 8) = dequant_fp8x8(u32x2{v[2], v[3]}, s);
    } else {
      for (int c = 0; c < 16 && c0 + c < cols; ++c) {
        const floatx2_t f = __builtin_amdgcn_cvt_pk_f32_fp8((int)src[c], false);
        dst[c] = float_to_bf16_bits(f[0] * s);
      }
    }
  }
}

}  // namespace
}  // namespace nsg

extern "C" int32_t nsg_dequant_fp8(const void* w8, int64_t ld8, const float* w_scale, void* out,
                                   int64_t ldo, int32_t rows, int32_t cols, nsg_stream_t stream) {
  NSG_CHECK_ARG(rows >= 0 && cols >= 0, "rows %d, cols %d", rows, cols);
  if (rows == 0 || cols == 0) {
    clear_error();
    return NSG_OK;
  }
  NSG_CHECK_ARG(w8 && w_scale && out, "null pointer argument");
  NSG_CHECK_ARG(ld8 >= cols && ldo >= cols, "ld8 %lld / ldo %lld < cols %d", (long long)ld8,
                (long long)ldo, cols);
  const bool vec = reinterpret_cast<uintptr_t>(w8) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(out) % 16 == 0 && ld8 % 16 == 0 && ldo % 8 == 0;
  const int64_t groups = (int64_t)rows * ((cols + 15) / 16);
  const int grid = (int)std::min<int64_t>((groups + 255) / 256, 8192);
  hipLaunchKernelGGL(dequant_fp8_kernel, dim3(grid), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(w8), ld8,
                     w_scale, static_cast<uint16_t*>(out), ldo, rows, cols, vec);
  return launch_status("dequant_fp8_kernel");
}
