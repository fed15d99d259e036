// The wide-output linear kernel (lm_head at verify row counts), launched from
// linear.hip's entry points.
#pragma once

#include "common.hpp"

namespace nsg {

// y = x W^T (no bias) for kHeadMinRows <= M <= kHeadMaxRows rows of x and a
// wide W (vocabulary rows): logits in bf16 (out: M x N, ldy elements apart)
// or, with keys, one argmax key per row and column group of waves of the
// persistent grid
// (out: M x key_cols uint64, the keys of linear.hip's argmax epilogue).
//
// With sumsq set, the final RMSNorm is folded in (its weight already folded
// into W's columns): x holds the un-normalised rows, and row m's fp32 result
// is multiplied by rsqrt(S_m / norm_dim + eps) before its bf16 rounding,
// where S_m is the sum of sumsq[c * M + m] over c < parts, added in order
// c = 0, 1, ... (the partial sums of squares, one per 16 columns, that the
// last decoder layer's down_proj epilogue writes).
struct HeadParams {
  const bf16* x;
  const bf16* w;
  void* out;
  int64_t ldx, ldw, ldy;
  int M, N, K;
  const float* sumsq;
  int parts;
  int norm_dim;
  float eps;
};

constexpr int kHeadMinRows = 1;
constexpr int kHeadMaxRows = 160;
constexpr int kHeadStep = 64;  // K must be a multiple of this (and at least 3 steps)

// Launches the kernel (logits, or keys when argmax; *key_cols = the keys per
// row written, at most 4 * ceil(N / 128)); the shape checks are the caller's:
// 16-byte aligned rows of x and W, K % 64 == 0, K >= 192, N % 4 == 0.
int32_t launch_lm_head(const HeadParams& p, bool argmax, hipStream_t s, int* key_cols);

// Whether the folded norm fits the kernel at M rows with `parts` partial sums
// per row: the partials are staged through one ring slot (M * parts a
// multiple of 4, whole 1 KB copies, the slot's last KB left for the row
// scales).
bool lm_head_fold_fits(int M, int parts);

// gate/up projection + SwiGLU (the MLP's first half, causal_lm.py:481-482)
// at verify row counts on the same LDS ring: y[m, n] = bf16(silu(bf16(g)) *
// bf16(u)) with g = x_m . W[n], u = x_m . W[N + n] (W holds the gate rows,
// then the up rows), n < N; with sumsq set, both scaled by the folded norm's
// row scale first (as HeadParams).  A workgroup takes 48 output columns
// (three waves, one 16-column gate tile and its up tile each) and a group of
// up to 80 rows.
struct GuParams {
  const bf16* x;
  const bf16* w;
  bf16* y;
  int64_t ldx, ldw, ldy;
  int M, N, K;
  const float* sumsq;
  int parts;
  int norm_dim;
  float eps;
};

// Shape rule: 1 <= M <= kHeadMaxRows, K % kHeadStep == 0, K >= 3 * kHeadStep,
// N % 4 == 0, sumsq_parts <= 64 when folded.
bool ring_swiglu_fits(int M, int N, int K, int parts);
int32_t launch_ring_swiglu(const GuParams& p, hipStream_t s);

}  // namespace nsg
