// lm_head at verify row counts on gfx950.
//
// The vocabulary projection of the verify forward (nano_sglang/model/
// causal_lm.py:643-645, logits = lm_head(norm(h))) runs on M = batch *
// (k + 1) rows: 160 x 151,936 x 896 at batch 32, k = 4.  Its 272 MB weight
// dominates the bytes, but at 160 rows a kernel that streams W per 32-row
// group (linear.hip) re-reads it five times through the caches, and one that
// re-reads x per 16-column tile moves x's 287 KB thousands of times.  Here:
//
// * a persistent workgroup per CU walks its column tiles (128 output columns:
//   4 waves x 2 W tiles of 16) and, per tile, K in 64-element steps, one flat
//   sequence of steps across tiles, so the pipeline never drains between
//   tiles;
// * each step's x rows (all M) and W rows go from global memory into a slot
//   of an LDS ring (4 to 8 slots, as many as fit) by LDS DMA
//   (global_load_lds_dwordx4), all but one slot in flight ahead of the math:
//   W is read from HBM exactly once, x once per tile from L2;
// * up to 80 rows each wave multiplies its two W tiles by all M / 16 x tiles
//   (v_mfma_f32_16x16x32_bf16, A = W, B = x^T): a W fragment feeds MT MFMAs,
//   an x fragment two; from 96 rows the waves split the rows in two and the
//   columns in two (half the x tiles by four W tiles each: fewer fragment
//   reads);
// * an output element's whole K sum stays in one wave, in k order, so the
//   result does not depend on the grid;
// * the logits are bf16(acc), one rounding (lm_head has no bias); the argmax
//   form keeps, per row and lane, the largest bf16 value and its lowest
//   column over all the wave's tiles, and at the end stores one key per row
//   and column group of waves (linear.hip's argmax keys: ordered bf16 bits,
//   then the inverted column).
//
// The ring's 16-byte segments are XOR-swizzled per row pair (segment s of row
// r sits at s ^ ((r >> 1) & 7)): the 16 rows of an MFMA fragment read then
// fall on distinct banks of the 256-byte bank row.
//
// Folded final RMSNorm (FOLD): the rows' partial sums of squares reach the
// ring's last slot by LDS DMA before the ring's first steps are issued (that
// slot is first filled by the main loop, after its first barrier); once they
// have landed, thread t adds row t's partials in order and leaves the row
// scale in the slot's last KB, from which every lane takes the scales of its
// rows into registers.  The copies are older than the ring's, so waiting for
// them leaves the ring's first steps in flight.
#include "lm_head.hpp"

#include <algorithm>

namespace nsg {
namespace {

constexpr int kWaves = 4;
constexpr int kNT = 2;                     // 16-column W tiles per wave
constexpr int kCols = kWaves * kNT * 16;   // output columns per workgroup tile
constexpr int kRowBytes = kHeadStep * 2;   // one row's bytes per step
constexpr int kLdsMax = 160 * 1024;
constexpr int kHeadMaxParts = 64;  // folded norm: partial sums per row
constexpr int kMaxStages = 8;

template <int MT>
constexpr int stage_bytes() {
  return (MT * 16 + kWaves * kNT * 16) * kRowBytes;
}
// Ring depth: as many slots as the CU's LDS holds (4 at 160 rows, 6 at 64);
// all but one are in flight ahead of the math.
template <int MT>
constexpr int ring_stages() {
  return kLdsMax / stage_bytes<MT>() < kMaxStages ? kLdsMax / stage_bytes<MT>() : kMaxStages;
}

// One LDS DMA copy of 16 bytes per lane: lane l's 16 bytes land at LDS
// address lds + 16 l.  In asm, unseen by the compiler's wait-count pass
// (through the builtin, that pass waits for every copy in flight before each
// LDS read); the ring's own waits order them.  s_nop: the one wait state an
// LDS DMA needs after an SALU write of M0.
__device__ __forceinline__ void dma16(uint32_t lds, const void* src) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds), "v"(src)
               : "memory", "m0");
}

// The same with the non-temporal policy (W is streamed once: measured 54 ->
// 49 us at 33 rows, 78 -> 74 us at 160).
__device__ __forceinline__ void dma16_nt(uint32_t lds, const void* src) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off nt"
               :
               : "s"(lds), "v"(src)
               : "memory", "m0");
}

__device__ __forceinline__ uint64_t key_max(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Row groups of waves in the lm_head kernel: 2 from 96 rows (MT 6), else 1.
template <int MT>
constexpr int lm_row_split() {
  return MT >= 6 ? 2 : 1;
}

template <int MT, bool ARG, bool FOLD>
__global__ __launch_bounds__(kWaves * 64) void lm_head_kernel(HeadParams p) {
  static_assert(MT % 2 == 0 && MT >= 2 && MT <= kHeadMaxRows / 16, "whole x copies");
  // x: MT * 16 rows x 8 segments = 2 MT copies per step, kX per wave (the
  // last wave's surplus copies repeat the last copy: the same bytes to the
  // same place)
  constexpr int kXAll = 2 * MT;
  constexpr int kX = (kXAll + kWaves - 1) / kWaves;
  constexpr int kW = 2 * kNT;      // W copies per wave and step (its 32 rows x 8 segments)
  constexpr int NI = kX + kW;      // vector-memory instructions per wave and step
  // MFMA work of a step: RS row groups x kWaves / RS column groups of waves,
  // each wave XT x tiles by WT W tiles (from 96 rows two row groups: each
  // wave reads half of x's fragments and twice the W fragments, 9 instead of
  // 12 fragment reads per 32-k at 160 rows)
  constexpr int RS = lm_row_split<MT>();
  constexpr int XT = MT / RS;
  constexpr int WT = kNT * RS;
  constexpr int CG = kWaves / RS;
  constexpr int SB = stage_bytes<MT>();
  constexpr int kStages = ring_stages<MT>();
  static_assert(kStages >= 3 && (kStages - 2) * NI <= 63, "vmcnt counts to 63");
  __shared__ __attribute__((aligned(1024))) uint8_t ring[kStages * SB];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rh = wave % RS, cg = wave / RS;  // the wave's row group and column group
  const int nst = p.K / kHeadStep;
  const int tiles = (p.N + kCols - 1) / kCols;
  const int my_tiles = (tiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
  const int total = my_tiles * nst;

  // DMA sources.  Copy i of a wave fills ring slots (16-byte units) 64 i +
  // lane of its region: row r = slot / 8, physical segment slot % 8, which
  // holds logical segment (slot % 8) ^ ((r >> 1) & 7).  Rows past M repeat
  // row M - 1, W rows past N repeat rows of the last four columns; their
  // results are not kept.
  const uint32_t ring_lds = lds_addr(ring);
  const bf16* xsrc[kX];
  uint32_t x_lds[kX];
#pragma unroll
  for (int i = 0; i < kX; ++i) {
    const int copy = min(wave * kX + i, kXAll - 1);
    x_lds[i] = ring_lds + copy * 1024;
    const int slot = copy * 64 + lane;
    const int r = slot >> 3;
    const int seg = (slot & 7) ^ ((r >> 1) & 7);
    xsrc[i] = p.x + (int64_t)min(r, p.M - 1) * p.ldx + seg * 8;
  }
  int wrow[kW], wseg[kW];
#pragma unroll
  for (int i = 0; i < kW; ++i) {
    const int slot = i * 64 + lane;
    wrow[i] = slot >> 3;
    wseg[i] = (slot & 7) ^ ((wrow[i] >> 1) & 7);
  }
  const bf16* wsrc[kW];
  auto set_w = [&](int j) {  // W rows of this wave for the workgroup's tile j
    const int c0 = ((int)blockIdx.x + j * (int)gridDim.x) * kCols + wave * kNT * 16;
#pragma unroll
    for (int i = 0; i < kW; ++i) {
      int c = c0 + wrow[i];
      c = c < p.N ? c : p.N - 4 + (c & 3);
      wsrc[i] = p.w + (int64_t)c * p.ldw + wseg[i] * 8;
    }
  };
  const uint32_t w_lds = ring_lds + MT * 16 * kRowBytes + wave * kNT * 16 * kRowBytes;

  // issue cursor: steps issued so far, and the tile / step of the next one
  int issued = 0, i_tile = 0, i_step = 0, i_slot = 0;
  auto issue = [&]() {
    const uint32_t sb = (uint32_t)i_slot * SB;
    i_slot = i_slot + 1 == kStages ? 0 : i_slot + 1;
    const int64_t k0 = (int64_t)i_step * kHeadStep;
#pragma unroll
    for (int i = 0; i < kX; ++i) dma16(x_lds[i] + sb, xsrc[i] + k0);
#pragma unroll
    for (int i = 0; i < kW; ++i) dma16_nt(w_lds + sb + i * 1024, wsrc[i] + k0);
    ++issued;
    if (++i_step == nst) {
      i_step = 0;
      if (++i_tile < my_tiles) set_w(i_tile);
    }
  };

  // fragment reads: row T * 16 + lane % 16 of a region, logical segment
  // 4 h + lane / 16 (k 32 h + 8 (lane / 16) .. + 8 of the step)
  const int r16 = lane & 15;
  uint32_t frag_off[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) frag_off[h] = r16 * kRowBytes + 16 * ((4 * h + (lane >> 4)) ^ (r16 >> 1));

  floatx4 acc[WT][XT];
#pragma unroll
  for (int nt = 0; nt < WT; ++nt)
#pragma unroll
    for (int mt = 0; mt < XT; ++mt) acc[nt][mt] = floatx4{0.f, 0.f, 0.f, 0.f};
  // argmax: per row, this lane's largest bf16 logit and its column so far
  // (columns come in increasing order, so a strict > keeps the lowest
  // column of equal values; -0 equals +0)
  float bv[ARG ? XT : 1];
  int bc[ARG ? XT : 1];
#pragma unroll
  for (int mt = 0; mt < (ARG ? XT : 1); ++mt) {
    bv[mt] = 0.f;
    bc[mt] = -1;
  }

  if constexpr (FOLD) {  // the partial sums into the last slot, 1 KB per copy
    const int n16 = p.M * p.parts / 4;
    const int n_copies = (n16 + 63) / 64;
    const uint32_t part_lds = ring_lds + (kStages - 1) * SB;
    for (int i = wave; i < n_copies; i += kWaves)
      dma16(part_lds + i * 1024, p.sumsq + (int64_t)min(i * 64 + lane, n16 - 1) * 4);
  }
  set_w(0);
  for (int g = 0; g < kStages - 1 && g < total; ++g) issue();

  float rs[FOLD ? XT : 1];  // the row scales of this lane's rows 16 (rh XT + mt) + lane % 16
  if constexpr (FOLD) {
    wait_steps<NI, kStages - 1>(issued);  // this wave's partial copies have landed
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();  // ... and every wave's
    asm volatile("" ::: "memory");
    const float* part = reinterpret_cast<const float*>(ring + (kStages - 1) * SB);
    float* scale = reinterpret_cast<float*>(ring + kStages * SB - 1024);
    const int t = threadIdx.x;
    if (t < MT * 16) {
      // every read in flight at once, then the sum in order c = 0, 1, ..
      float v[kHeadMaxParts];
      const int tr = min(t, p.M - 1);
#pragma unroll
      for (int c = 0; c < kHeadMaxParts; ++c) v[c] = part[min(c, p.parts - 1) * p.M + tr];
      float sq = 0.f;
#pragma unroll
      for (int c = 0; c < kHeadMaxParts; ++c) sq += c < p.parts ? v[c] : 0.f;
      scale[t] = t < p.M ? 1.f / sqrtf(sq / (float)p.norm_dim + p.eps) : 0.f;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int mt = 0; mt < XT; ++mt) rs[mt] = scale[(rh * XT + mt) * 16 + r16];
    // read before the main loop's first copies refill the slot
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }

  int g = 0, c_slot = 0;
  for (int j = 0; j < my_tiles; ++j) {
    for (int s = 0; s < nst; ++s, ++g) {
      // step g landed for this wave (issued - 1 - g later steps may still be
      // in flight), then for every wave; the slot of step g - 1 is free
      wait_steps<NI, kStages - 2>(issued - 1 - g);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (issued < total) issue();
      const uint8_t* st = ring + c_slot * SB;
      c_slot = c_slot + 1 == kStages ? 0 : c_slot + 1;
      const uint8_t* xs = st;
      const uint8_t* ws = st + MT * 16 * kRowBytes + cg * WT * 16 * kRowBytes;
      bf16x8 wf[2][WT], xf[2][XT];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int nt = 0; nt < WT; ++nt)
          wf[h][nt] = *reinterpret_cast<const bf16x8*>(ws + nt * 16 * kRowBytes + frag_off[h]);
#pragma unroll
        for (int mt = 0; mt < XT; ++mt)
          xf[h][mt] = *reinterpret_cast<const bf16x8*>(xs + (rh * XT + mt) * 16 * kRowBytes +
                                                       frag_off[h]);
      }
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int nt = 0; nt < WT; ++nt)
#pragma unroll
          for (int mt = 0; mt < XT; ++mt)
            acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[h][nt], xf[h][mt],
                                                                  acc[nt][mt], 0, 0, 0);
    }

    // tile j done.  Lane l of (nt, mt) holds rows m = 16 (rh XT + mt) +
    // l % 16, columns n = c0 + 16 nt + 4 (l / 16) + i.
    const int c0 = ((int)blockIdx.x + j * (int)gridDim.x) * kCols + cg * WT * 16;
#pragma unroll
    for (int nt = 0; nt < WT; ++nt) {
      const int n = c0 + nt * 16 + 4 * (lane >> 4);
#pragma unroll
      for (int mt = 0; mt < XT; ++mt) {
        const int m = (rh * XT + mt) * 16 + r16;
        const floatx4 v = acc[nt][mt];
        if constexpr (ARG) {
          const bool ok = n < p.N;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float r = bf16_bits_to_float(float_to_bf16_bits(FOLD ? v[i] * rs[mt] : v[i]));
            const bool take = ok && (r > bv[mt] || bc[mt] < 0);
            bv[mt] = take ? r : bv[mt];
            bc[mt] = take ? n + i : bc[mt];
          }
        } else {
          if (m < p.M && n < p.N) {
            bf16* y = static_cast<bf16*>(p.out) + (int64_t)m * p.ldy + n;
            if constexpr (FOLD) {
              const float sc = rs[mt];
              *reinterpret_cast<uint2*>(y) = uint2{pack_bf16x2(v[0] * sc, v[1] * sc),
                                                   pack_bf16x2(v[2] * sc, v[3] * sc)};
            } else {
              *reinterpret_cast<uint2*>(y) =
                  uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            }
          }
        }
        acc[nt][mt] = floatx4{0.f, 0.f, 0.f, 0.f};
      }
    }
  }

  if constexpr (ARG) {
    // the four lanes of a row meet; one stores the row's key for this
    // wave's column group: keys[m * (CG * grid) + CG * workgroup + cg]
    uint64_t* keys = static_cast<uint64_t*>(p.out);
    const int cols = CG * (int)gridDim.x;
#pragma unroll
    for (int mt = 0; mt < XT; ++mt) {
      // key = (order-preserving bits of the bf16 value, ~column): the max
      // key is the largest value at its lowest column; 0 for no column
      uint32_t b = float_to_bf16_bits(bv[mt]);
      b = b == 0x8000u ? 0u : b;
      const uint32_t ord = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
      uint64_t k = bc[mt] < 0 ? 0 : ((uint64_t)ord << 32) | (0xffffffffu - (uint32_t)bc[mt]);
#pragma unroll
      for (int o = 16; o < 64; o <<= 1) {
        const uint64_t other = ((uint64_t)(uint32_t)__shfl_xor((int)(k >> 32), o, 64) << 32) |
                               (uint32_t)__shfl_xor((int)(uint32_t)k, o, 64);
        k = key_max(k, other);
      }
      const int m = (rh * XT + mt) * 16 + r16;
      if ((lane >> 4) == 0 && m < p.M) keys[(int64_t)m * cols + CG * blockIdx.x + cg] = k;
    }
  }
}

// ---- gate/up + SwiGLU on the same ring (GuParams) ----
// At 160 rows the weight-streaming linear kernel (linear.hip) takes 32-row
// groups, so a CU holds three workgroups and pulls about 510 KB through its
// L1 per call; one CU streams at most a few tens of GB/s (the bytes a ring
// or a register pipeline keeps in flight over the memory latency), so that
// traffic, not HBM, sets the time.  Here a workgroup takes 80 rows and 48
// output columns (96 W rows): x once per workgroup, W once per XCD (the two
// row groups of a column tile sit on one XCD), about 315 KB per CU.  Three
// waves, one 16-column gate tile and its up tile each, so the SwiGLU pairs
// sit in one lane; x and W reach LDS by DMA, as in the lm_head kernel.
constexpr int kGuWaves = 3;
constexpr int kGuCols = kGuWaves * 16;   // output columns per workgroup
constexpr int kGuWRows = kGuWaves * 32;  // their gate and up rows of W
constexpr int kGuMaxParts = 64;          // folded norm: partial sums per row

template <int MT>
constexpr int gu_stage_bytes() {
  return (MT * 16 + kGuWRows) * kRowBytes;
}
template <int MT>
constexpr int gu_stages() {
  return kLdsMax / gu_stage_bytes<MT>() < kMaxStages ? kLdsMax / gu_stage_bytes<MT>() : kMaxStages;
}

// 4-byte LDS DMA: lane l lands at lds + 4 l.
__device__ __forceinline__ void dma4(uint32_t lds, const void* src) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off"
               :
               : "s"(lds), "v"(src)
               : "memory", "m0");
}

// bf16(silu(g)) for a bf16 value g: F.silu on a bf16 tensor (fp32 math,
// one rounding), the same expression as linear.hip's SwiGLU epilogue.
__device__ __forceinline__ float silu_round(float g) {
  return bf16_bits_to_float(float_to_bf16_bits(g / (1.f + __expf(-g))));
}

template <int MT, bool FOLD>
__global__ __launch_bounds__(kGuWaves * 64) void ring_swiglu_kernel(GuParams p, int row_groups,
                                                                     int col_tiles) {
  constexpr int R = MT * 16;  // rows per workgroup
  constexpr int kXAll = 2 * MT;
  constexpr int kX = (kXAll + kGuWaves - 1) / kGuWaves;
  constexpr int kW = 4;  // the wave's 32 W rows: 4 copies of 8 rows
  constexpr int NI = kX + kW;
  constexpr int SB = gu_stage_bytes<MT>();
  constexpr int kStages = gu_stages<MT>();
  static_assert(kStages >= 3 && (kStages - 1) * NI <= 63, "vmcnt counts to 63");
  static_assert(kGuMaxParts * R * 4 + R * 4 <= SB, "the partials and row scales fit one slot");
  __shared__ __attribute__((aligned(1024))) uint8_t ring[kStages * SB];

  // workgroup -> (column tile, row group); the row groups of a column tile
  // on one XCD (workgroups go round-robin over the 8 XCDs)
  const int xcd = blockIdx.x & 7, slot_id = blockIdx.x >> 3;
  const int tile = xcd + 8 * (slot_id / row_groups);
  if (tile >= col_tiles) return;  // workgroup-uniform, before any barrier
  const int m0 = (slot_id % row_groups) * R;
  const int Mg = min(R, p.M - m0);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nst = p.K / kHeadStep;
  const uint32_t ring_lds = lds_addr(ring);

  // DMA sources (the lm_head kernel's layout and swizzle): x copy i of a wave
  // fills rows 8 copy .. + 8 of the x region; rows past the group repeat its
  // last row.  W: the wave's region holds its gate tile (rows 0-15) and up
  // tile (16-31); columns past N repeat column N - 1.
  const bf16* xsrc[kX];
  uint32_t x_lds[kX];
#pragma unroll
  for (int i = 0; i < kX; ++i) {
    const int copy = min(wave * kX + i, kXAll - 1);
    x_lds[i] = ring_lds + copy * 1024;
    const int sl = copy * 64 + lane;
    const int r = sl >> 3;
    const int seg = (sl & 7) ^ ((r >> 1) & 7);
    xsrc[i] = p.x + (int64_t)(m0 + min(r, Mg - 1)) * p.ldx + seg * 8;
  }
  const int c0 = tile * kGuCols + wave * 16;  // the wave's first output column
  const bf16* wsrc[kW];
#pragma unroll
  for (int i = 0; i < kW; ++i) {
    const int sl = i * 64 + lane;
    const int wr = sl >> 3;
    const int seg = (sl & 7) ^ ((wr >> 1) & 7);
    const int row = (wr < 16 ? 0 : p.N) + min(c0 + (wr & 15), p.N - 1);
    wsrc[i] = p.w + (int64_t)row * p.ldw + seg * 8;
  }
  const uint32_t w_lds = ring_lds + R * kRowBytes + wave * 32 * kRowBytes;

  int issued = 0, i_slot = 0;
  auto issue = [&]() {
    const uint32_t sb = (uint32_t)i_slot * SB;
    i_slot = i_slot + 1 == kStages ? 0 : i_slot + 1;
    const int64_t k0 = (int64_t)issued * kHeadStep;
#pragma unroll
    for (int i = 0; i < kX; ++i) dma16(x_lds[i] + sb, xsrc[i] + k0);
#pragma unroll
    for (int i = 0; i < kW; ++i) dma16_nt(w_lds + sb + i * 1024, wsrc[i] + k0);
    ++issued;
  };

  const int r16 = lane & 15;
  uint32_t frag_off[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) frag_off[h] = r16 * kRowBytes + 16 * ((4 * h + (lane >> 4)) ^ (r16 >> 1));

  floatx4 acc[2][MT];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = floatx4{0.f, 0.f, 0.f, 0.f};

  // folded norm: the group's partial sums, part[c * R + r], by LDS DMA into
  // the ring's last slot (first filled by the main loop, after its first
  // barrier), issued before the ring's first copies: waiting for them leaves
  // those in flight.  Thread t < R adds row t's partials (all reads in flight
  // at once, then the sum in order c = 0, 1, ..) and leaves the row scale
  // behind the partials, from where each lane takes its rows' scales.
  const uint32_t part_lds = ring_lds + (kStages - 1) * SB;
  if constexpr (FOLD) {
    if ((p.M & 3) == 0 && (Mg & 3) == 0) {
      // 16 bytes (4 rows of one partial) per lane: rows m0 .. m0 + Mg of
      // partial c are contiguous and 16-byte aligned
      const int n16 = p.parts * (R / 4);
      for (int i = wave; i * 64 < n16; i += kGuWaves) {
        const int u = i * 64 + lane;
        const int c = u / (R / 4);
        const int q = min(u - c * (R / 4), Mg / 4 - 1);
        dma16(part_lds + i * 1024, p.sumsq + (int64_t)min(c, p.parts - 1) * p.M + m0 + 4 * q);
      }
    } else {
      const int n_el = p.parts * R;
      for (int i = wave; i * 64 < n_el; i += kGuWaves) {
        const int e = i * 64 + lane;
        const int c = e / R;
        dma4(part_lds + i * 256,
             p.sumsq + (int64_t)min(c, p.parts - 1) * p.M + m0 + min(e - c * R, Mg - 1));
      }
    }
  }
  // with the folded norm only two steps go out before the partials are
  // added, the rest after: a wave stalls while its copies issue, so issuing
  // every first step before the sum delays the sum, and two steps in flight
  // already cover it (12.3 -> 12.0 us at 160 rows)
  for (int g = 0; g < (FOLD ? 2 : kStages - 1) && g < nst; ++g) issue();

  float rs[FOLD ? MT : 1];
  if constexpr (FOLD) {
    wait_steps<NI, kStages - 1>(issued);  // this wave's partial copies have landed
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();  // ... and every wave's
    asm volatile("" ::: "memory");
    const float* part = reinterpret_cast<const float*>(ring + (kStages - 1) * SB);
    float* scale = reinterpret_cast<float*>(ring + (kStages - 1) * SB + kGuMaxParts * R * 4);
    const int t = threadIdx.x;
    if (t < R) {
      float v[kGuMaxParts];
#pragma unroll
      for (int c = 0; c < kGuMaxParts; ++c) v[c] = part[min(c, p.parts - 1) * R + t];
      float sq = 0.f;
#pragma unroll
      for (int c = 0; c < kGuMaxParts; ++c) sq += c < p.parts ? v[c] : 0.f;
      scale[t] = t < Mg ? 1.f / sqrtf(sq / (float)p.norm_dim + p.eps) : 0.f;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) rs[mt] = scale[mt * 16 + r16];
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // before the slot is refilled
    while (issued < kStages - 1 && issued < nst) issue();  // the rest of the first steps
  }

  int c_slot = 0;
  for (int g = 0; g < nst; ++g) {
    wait_steps<NI, kStages - 2>(issued - 1 - g);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (issued < nst) issue();
    const uint8_t* st = ring + c_slot * SB;
    c_slot = c_slot + 1 == kStages ? 0 : c_slot + 1;
    const uint8_t* ws = st + R * kRowBytes + wave * 32 * kRowBytes;
    bf16x8 wf[2][2], xf[2][MT];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
        wf[h][nt] = *reinterpret_cast<const bf16x8*>(ws + nt * 16 * kRowBytes + frag_off[h]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        xf[h][mt] = *reinterpret_cast<const bf16x8*>(st + mt * 16 * kRowBytes + frag_off[h]);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[h][nt], xf[h][mt], acc[nt][mt],
                                                                0, 0, 0);
  }

  // lane l of (nt, mt) holds row 16 mt + l % 16, columns c0 + 4 (l / 16) + i
  // of the gate (nt 0) and up (nt 1) products
  const int n = c0 + 4 * (lane >> 4);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + r16;
    if (m < Mg && n < p.N) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float gs = acc[0][mt][i], us = acc[1][mt][i];
        if constexpr (FOLD) {
          gs *= rs[mt];
          us *= rs[mt];
        }
        const float g = bf16_bits_to_float(float_to_bf16_bits(gs));
        const float u = bf16_bits_to_float(float_to_bf16_bits(us));
        v[i] = silu_round(g) * u;
      }
      bf16* y = p.y + (int64_t)(m0 + m) * p.ldy + n;
      *reinterpret_cast<uint2*>(y) = uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    }
  }
}

int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

template <int MT>
int32_t launch_mt(const HeadParams& p, bool argmax, hipStream_t s, int* key_cols) {
  const int tiles = (p.N + kCols - 1) / kCols;
  const int per_cu = kLdsMax / (ring_stages<MT>() * stage_bytes<MT>());
  const int grid = std::min(tiles, device_cus() * std::max(per_cu, 1));
  *key_cols = kWaves / lm_row_split<MT>() * grid;
  const dim3 g(grid), b(kWaves * 64);
  if (p.sumsq) {
    if (argmax)
      hipLaunchKernelGGL((lm_head_kernel<MT, true, true>), g, b, 0, s, p);
    else
      hipLaunchKernelGGL((lm_head_kernel<MT, false, true>), g, b, 0, s, p);
  } else {
    if (argmax)
      hipLaunchKernelGGL((lm_head_kernel<MT, true, false>), g, b, 0, s, p);
    else
      hipLaunchKernelGGL((lm_head_kernel<MT, false, false>), g, b, 0, s, p);
  }
  return launch_status("lm_head_kernel");
}

template <int MT>
bool fold_fits_mt(int M, int parts) {
  const int64_t n16 = (int64_t)M * parts / 4;
  return ((n16 + 63) / 64) * 1024 <= stage_bytes<MT>() - 1024;
}

}  // namespace

bool lm_head_fold_fits(int M, int parts) {
  if (M < kHeadMinRows || M > kHeadMaxRows || parts < 1 || parts > kHeadMaxParts ||
      ((int64_t)M * parts) % 4 != 0)
    return false;
  const int mt = (M + 15) / 16;
  if (mt <= 2) return fold_fits_mt<2>(M, parts);
  if (mt <= 4) return fold_fits_mt<4>(M, parts);
  if (mt <= 6) return fold_fits_mt<6>(M, parts);
  if (mt <= 8) return fold_fits_mt<8>(M, parts);
  return fold_fits_mt<10>(M, parts);
}

bool ring_swiglu_fits(int M, int N, int K, int parts) {
  return M >= 1 && M <= kHeadMaxRows && N >= 4 && N % 4 == 0 && K % kHeadStep == 0 &&
         K >= 3 * kHeadStep && parts <= kGuMaxParts;
}

namespace {
template <int MT>
int32_t launch_gu_mt(const GuParams& p, hipStream_t s) {
  const int row_groups = (p.M + MT * 16 - 1) / (MT * 16);
  const int col_tiles = (p.N + kGuCols - 1) / kGuCols;
  const int grid = 8 * ((col_tiles + 7) / 8) * row_groups;
  if (p.sumsq)
    hipLaunchKernelGGL((ring_swiglu_kernel<MT, true>), dim3(grid), dim3(kGuWaves * 64), 0, s, p,
                       row_groups, col_tiles);
  else
    hipLaunchKernelGGL((ring_swiglu_kernel<MT, false>), dim3(grid), dim3(kGuWaves * 64), 0, s, p,
                       row_groups, col_tiles);
  return launch_status("ring_swiglu_kernel");
}
}  // namespace

// Rows per workgroup: two row groups above 32 rows (16-row tiles: 160 rows
// as 2 x 80, 128 as 2 x 64, 96 as 2 x 48, 64 as 2 x 32), one group up to 32.
int32_t launch_ring_swiglu(const GuParams& p, hipStream_t s) {
  const int mt = p.M <= 32 ? 2 : std::max(2, ((p.M + 1) / 2 + 15) / 16);
  if (mt <= 2) return launch_gu_mt<2>(p, s);
  if (mt <= 3) return launch_gu_mt<3>(p, s);
  if (mt <= 4) return launch_gu_mt<4>(p, s);
  return launch_gu_mt<5>(p, s);
}

int32_t launch_lm_head(const HeadParams& p, bool argmax, hipStream_t s, int* key_cols) {
  const int mt = (p.M + 15) / 16;
  if (mt <= 2) return launch_mt<2>(p, argmax, s, key_cols);
  if (mt <= 4) return launch_mt<4>(p, argmax, s, key_cols);
  if (mt <= 6) return launch_mt<6>(p, argmax, s, key_cols);
  if (mt <= 8) return launch_mt<8>(p, argmax, s, key_cols);
  return launch_mt<10>(p, argmax, s, key_cols);
}

}  // namespace nsg
