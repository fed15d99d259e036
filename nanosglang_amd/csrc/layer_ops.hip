// Fused per-token layer ops around the verify step on gfx950:
//   RMSNorm and residual-add + RMSNorm (nano_sglang/model/causal_lm.py:
//   133-154, the FlashInfer fused_add_rmsnorm the reference credits with part
//   of its +13%, README.md:117,123) and the SwiGLU gate (causal_lm.py:482).
// Each replaces 6-10 eager elementwise launches per call with one pass that
// reads and writes each activation once.
//
// Arithmetic follows the reference's bf16 fallback: variance = mean(x^2) in
// fp32; y = bf16(w * (x * rsqrt(var + eps))) with both products in fp32
// (bf16 * fp32 promotes to fp32 in PyTorch); the residual add is a bf16 add
// (round once); silu(g) * u rounds silu(g) to bf16 before the product.
#include "common.hpp"

namespace nsg {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kNormThreads = 256;  // four rows per workgroup

// Up to R rows of H bf16 values (H % 8 == 0, H <= 512 C), one wave: lane l
// owns 16-byte chunks l + 64 c, c < C.  With ADD, s = bf16(x + residual) is
// written back to residual first (a bf16 add, one rounding); otherwise s = x.
// Then out = bf16(w * (s * rsqrt(mean(s^2) + eps))), products in fp32.  The
// sum of squares runs per lane in chunk and element order (fused
// multiply-adds), then over the wave by xor-butterfly: one fixed order.
// row[0] must be a valid row; row[r] < 0 skips row r (r > 0).  Every load
// of the batch is issued unconditionally (skipped rows and chunks past H
// read row[0] and the last chunk instead; their values are never used) and
// before the first use, so R rows cost one memory latency: a load under a
// branch would make the wait-count pass wait for each load in turn.
template <bool ADD, int R, int C>
__device__ __forceinline__ void norm_rows(const uint16_t* x, int64_t ldx, uint16_t* residual,
                                          int64_t ldr, const uint16_t* w, uint16_t* out,
                                          int64_t ldo, const int (&row)[R], int H, float eps,
                                          int lane) {
  const int nch = H >> 3;
  u32x4 a[R][C], b[R][C], wv[C];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t rl = row[r] >= 0 ? row[r] : row[0];
      const int chl = min(lane + 64 * c, nch - 1);
      a[r][c] = *reinterpret_cast<const u32x4*>(x + rl * ldx + chl * 8);
      if constexpr (ADD) b[r][c] = *reinterpret_cast<const u32x4*>(residual + rl * ldr + chl * 8);
    }
#pragma unroll
  for (int c = 0; c < C; ++c)
    wv[c] = *reinterpret_cast<const u32x4*>(w + min(lane + 64 * c, nch - 1) * 8);
  float ss[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    ss[r] = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int ch = lane + 64 * c;
      if (row[r] < 0 || ch >= nch) continue;
      if constexpr (ADD) {
        u32x4 s;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          s[i] = pack_bf16x2(
              bf16_bits_to_float(a[r][c][i] & 0xffffu) + bf16_bits_to_float(b[r][c][i] & 0xffffu),
              bf16_bits_to_float(a[r][c][i] >> 16) + bf16_bits_to_float(b[r][c][i] >> 16));
        *reinterpret_cast<u32x4*>(residual + row[r] * ldr + ch * 8) = s;
        a[r][c] = s;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lo = bf16_bits_to_float(a[r][c][i] & 0xffffu);
        const float hi = bf16_bits_to_float(a[r][c][i] >> 16);
        ss[r] = __builtin_fmaf(lo, lo, ss[r]);
        ss[r] = __builtin_fmaf(hi, hi, ss[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) ss[r] = wave_sum(ss[r]);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (row[r] < 0) continue;
    const float rs = 1.f / sqrtf(ss[r] / (float)H + eps);
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int ch = lane + 64 * c;
      if (ch >= nch) continue;
      u32x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lo = bf16_bits_to_float(wv[c][i] & 0xffffu) *
                         (bf16_bits_to_float(a[r][c][i] & 0xffffu) * rs);
        const float hi = bf16_bits_to_float(wv[c][i] >> 16) *
                         (bf16_bits_to_float(a[r][c][i] >> 16) * rs);
        o[i] = pack_bf16x2(lo, hi);
      }
      *reinterpret_cast<u32x4*>(out + row[r] * ldo + ch * 8) = o;
    }
  }
}


// One wave per token row; C 16-byte chunks per lane cover H <= 512 C.
template <bool ADD, int C>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(
    const uint16_t* __restrict__ x, uint16_t* __restrict__ residual,
    const uint16_t* __restrict__ w, uint16_t* __restrict__ out, int T, int H, float eps) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (kNormThreads / 64) + (threadIdx.x >> 6);
  if (t >= T) return;  // wave-uniform
  const int row[1] = {t};
  norm_rows<ADD, 1, C>(x, H, residual, H, w, out, H, row, H, eps, lane);
}

template <bool ADD>
void launch_rmsnorm(const uint16_t* x, uint16_t* residual, const uint16_t* w, uint16_t* out,
                    int T, int H, float eps, hipStream_t s) {
  const dim3 grid((T + kNormThreads / 64 - 1) / (kNormThreads / 64));
  if (H <= 1024)
    hipLaunchKernelGGL((rmsnorm_kernel<ADD, 2>), grid, dim3(kNormThreads), 0, s, x, residual, w,
                       out, T, H, eps);
  else if (H <= 2048)
    hipLaunchKernelGGL((rmsnorm_kernel<ADD, 4>), grid, dim3(kNormThreads), 0, s, x, residual, w,
                       out, T, H, eps);
  else if (H <= 4096)
    hipLaunchKernelGGL((rmsnorm_kernel<ADD, 8>), grid, dim3(kNormThreads), 0, s, x, residual, w,
                       out, T, H, eps);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<ADD, 16>), grid, dim3(kNormThreads), 0, s, x, residual, w,
                       out, T, H, eps);
}

// Partial sums of squares of bf16 rows for a folded-RMSNorm consumer:
// out[g * T + t] = sum over columns 16 g .. 16 g + 15 of x[t, :]^2 (one wave
// per row; lane l holds 8-column chunks l + 64 c, and the two chunks of a
// 16-column group sit on lanes 2 i, 2 i + 1).  The layout a producing linear
// writes (nsg_linear_fold), for the first layer's input.
template <int C>
__global__ __launch_bounds__(kNormThreads) void row_sumsq_kernel(const uint16_t* __restrict__ x,
                                                                  int64_t ldx, int T, int H,
                                                                  float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (kNormThreads / 64) + (threadIdx.x >> 6);
  if (t >= T) return;  // wave-uniform
  const int nch = H >> 3;
  u32x4 a[C];
#pragma unroll
  for (int c = 0; c < C; ++c)
    a[c] = *reinterpret_cast<const u32x4*>(x + (int64_t)t * ldx + min(lane + 64 * c, nch - 1) * 8);
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int ch = lane + 64 * c;
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = bf16_bits_to_float(a[c][i] & 0xffffu);
      const float hi = bf16_bits_to_float(a[c][i] >> 16);
      sq = __builtin_fmaf(lo, lo, sq);
      sq = __builtin_fmaf(hi, hi, sq);
    }
    sq += __shfl_xor(sq, 1, 64);
    if (ch < nch && (ch & 1) == 0) out[(int64_t)(ch >> 1) * T + t] = sq;
  }
}

// Embedding rows: out[r] = table[ids[b sb + j sj]] for r = b J + j (ids
// outside [0, vocab) read the nearest valid row), one wave per row, and, when
// sumsq is given, the row's per-16-column sums of squares
// sumsq[(c / 16) rows + r] (the layout row_sumsq_kernel writes).
// With keys: the ids of column key_j (rows r = b * J + key_j) are first the
// greedy tokens of keys row b (key_cols keys, the lm_head's argmax keys),
// written to ids and then looked up; the other rows read their ids.
__global__ __launch_bounds__(kNormThreads) void embed_rows_kernel(
    int64_t* __restrict__ ids, int64_t sb, int64_t sj, int J, int rows,
    const uint16_t* __restrict__ table, int64_t ldt, int vocab, int H,
    uint16_t* __restrict__ out, int64_t ldo, float* __restrict__ sumsq,
    const uint64_t* __restrict__ keys, int key_cols, int key_j) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * (kNormThreads / 64) + (threadIdx.x >> 6);
  if (r >= rows) return;  // wave-uniform
  const int b = r / J, j = r - b * J;
  int64_t raw;
  if (keys && j == key_j) {  // wave-uniform
    raw = key_token(wave_max_key(keys + (int64_t)b * key_cols, key_cols, lane));
    if (lane == 0) ids[b * sb + j * sj] = raw;
  } else {
    raw = ids[b * sb + j * sj];
  }
  const int64_t id = min(max(raw, (int64_t)0), (int64_t)vocab - 1);
  const uint16_t* src = table + id * ldt;
  uint16_t* dst = out + (int64_t)r * ldo;
  const int nseg = H >> 3;  // 16-byte segments of a row
  for (int s0 = 0; s0 < nseg; s0 += 64) {
    const int sg = s0 + lane;
    const bool ok = sg < nseg;
    const u32x4 v = *reinterpret_cast<const u32x4*>(src + min(sg, nseg - 1) * 8);
    if (ok) *reinterpret_cast<u32x4*>(dst + sg * 8) = v;
    if (sumsq) {  // kernel-uniform
      float sq = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lo = bf16_bits_to_float(v[i] & 0xffffu);
        const float hi = bf16_bits_to_float(v[i] >> 16);
        sq = __builtin_fmaf(lo, lo, sq);
        sq = __builtin_fmaf(hi, hi, sq);
      }
      sq += __shfl_xor(sq, 1, 64);
      if (ok && (sg & 1) == 0) sumsq[(int64_t)(sg >> 1) * rows + r] = sq;
    }
  }
}

// out[t, j] = bf16(bf16(silu(gu[t, j])) * gu[t, I + j]) for j < I.
__global__ void silu_mul_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ out,
                                int64_t T, int I) {
  const int64_t nv = (int64_t)T * (I / 8);
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < nv;
       g += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = g / (I / 8);
    const int j = (int)(g - t * (I / 8)) * 8;
    const u32x4 a = *reinterpret_cast<const u32x4*>(gu + t * 2 * I + j);
    const u32x4 b = *reinterpret_cast<const u32x4*>(gu + t * 2 * I + I + j);
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float x0 = bf16_bits_to_float(a[i] & 0xffff), x1 = bf16_bits_to_float(a[i] >> 16);
      x0 = bf16_bits_to_float(float_to_bf16_bits(x0 / (1.f + __expf(-x0))));
      x1 = bf16_bits_to_float(float_to_bf16_bits(x1 / (1.f + __expf(-x1))));
      o[i] = pack_bf16x2(x0 * bf16_bits_to_float(b[i] & 0xffff),
                         x1 * bf16_bits_to_float(b[i] >> 16));
    }
    *reinterpret_cast<u32x4*>(out + t * I + j) = o;
  }
}

}  // namespace
}  // namespace nsg

using namespace nsg;

extern "C" int32_t nsg_rmsnorm(const void* x, void* residual, const void* weight, void* out,
                               int32_t num_tokens, int32_t hidden, float eps,
                               nsg_stream_t stream) {
  NSG_CHECK_ARG(num_tokens >= 0, "num_tokens %d < 0", num_tokens);
  if (num_tokens == 0) {
    clear_error();
    return NSG_OK;
  }
  NSG_CHECK_ARG(x && weight && out, "null pointer argument");
  NSG_CHECK_ARG(hidden > 0 && hidden % 8 == 0 && hidden <= 8192,
                "hidden %d must be a multiple of 8 and at most 8192", hidden);
  NSG_CHECK_ARG(((uintptr_t)x | (uintptr_t)weight | (uintptr_t)out |
                 (uintptr_t)residual) % 16 == 0, "tensors must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (residual)
    launch_rmsnorm<true>(static_cast<const uint16_t*>(x), static_cast<uint16_t*>(residual),
                         static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(out),
                         num_tokens, hidden, eps, s);
  else
    launch_rmsnorm<false>(static_cast<const uint16_t*>(x), nullptr,
                          static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(out),
                          num_tokens, hidden, eps, s);
  return launch_status("rmsnorm_kernel");
}

extern "C" int32_t nsg_row_sumsq(const void* x, int64_t ldx, int32_t num_tokens, int32_t hidden,
                                 float* sumsq_out, nsg_stream_t stream) {
  NSG_CHECK_ARG(num_tokens >= 0, "num_tokens %d < 0", num_tokens);
  if (num_tokens == 0) {
    clear_error();
    return NSG_OK;
  }
  NSG_CHECK_ARG(x && sumsq_out, "null pointer argument");
  NSG_CHECK_ARG(hidden > 0 && hidden % 16 == 0 && hidden <= 1024,
                "hidden %d must be a multiple of 16 and at most 1024", hidden);
  NSG_CHECK_ARG(ldx >= hidden && ldx % 8 == 0 && (uintptr_t)x % 16 == 0,
                "x rows must be 16-byte aligned (ldx %lld)", (long long)ldx);
  const dim3 grid((num_tokens + kNormThreads / 64 - 1) / (kNormThreads / 64));
  hipLaunchKernelGGL((row_sumsq_kernel<2>), grid, dim3(kNormThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x), ldx,
                     num_tokens, hidden, sumsq_out);
  return launch_status("row_sumsq_kernel");
}

namespace {

int32_t embed_impl(int64_t* ids, int64_t id_stride_b, int64_t id_stride_j, int32_t batch,
                   int32_t per_batch, const uint64_t* keys, int32_t key_cols, int32_t key_j,
                   const void* table, int64_t ld_table, int32_t vocab, int32_t hidden, void* out,
                   int64_t ld_out, float* sumsq_out, nsg_stream_t stream) {
  NSG_CHECK_ARG(batch >= 0 && per_batch >= 0, "batch %d, per_batch %d", batch, per_batch);
  const int64_t rows = (int64_t)batch * per_batch;
  if (rows == 0) {
    clear_error();
    return NSG_OK;
  }
  NSG_CHECK_ARG(ids && table && out, "null pointer argument");
  NSG_CHECK_ARG(rows <= INT32_MAX && vocab > 0 && hidden > 0 && hidden % 16 == 0,
                "rows %lld, vocab %d, hidden %d (a multiple of 16)", (long long)rows, vocab, hidden);
  NSG_CHECK_ARG(ld_table >= hidden && ld_out >= hidden && ld_table % 8 == 0 && ld_out % 8 == 0 &&
                    (uintptr_t)table % 16 == 0 && (uintptr_t)out % 16 == 0,
                "table and out rows must be 16-byte aligned");
  const dim3 grid((unsigned)((rows + kNormThreads / 64 - 1) / (kNormThreads / 64)));
  NSG_CHECK_ARG(!keys || (key_cols >= 1 && key_j >= 0 && key_j < per_batch &&
                          (uintptr_t)keys % 8 == 0),
                "keys: key_cols %d >= 1, key_j %d in [0, per_batch %d), 8-byte aligned",
                key_cols, key_j, per_batch);
  hipLaunchKernelGGL(embed_rows_kernel, grid, dim3(kNormThreads), 0,
                     static_cast<hipStream_t>(stream), ids, id_stride_b, id_stride_j, per_batch,
                     (int)rows, static_cast<const uint16_t*>(table), ld_table, vocab, hidden,
                     static_cast<uint16_t*>(out), ld_out, sumsq_out, keys, key_cols, key_j);
  return launch_status("embed_rows_kernel");
}

}  // namespace

extern "C" int32_t nsg_embed_rows(const int64_t* ids, int64_t id_stride_b, int64_t id_stride_j,
                                  int32_t batch, int32_t per_batch, const void* table,
                                  int64_t ld_table, int32_t vocab, int32_t hidden, void* out,
                                  int64_t ld_out, float* sumsq_out, nsg_stream_t stream) {
  // without keys the kernel only reads ids
  return embed_impl(const_cast<int64_t*>(ids), id_stride_b, id_stride_j, batch, per_batch,
                    nullptr, 0, 0, table, ld_table, vocab, hidden, out, ld_out, sumsq_out,
                    stream);
}

extern "C" int32_t nsg_embed_rows_keys(int64_t* ids, int64_t id_stride_b, int64_t id_stride_j,
                                       int32_t batch, int32_t per_batch, int32_t key_j,
                                       const void* keys, int32_t key_cols, const void* table,
                                       int64_t ld_table, int32_t vocab, int32_t hidden,
                                       void* out, int64_t ld_out, float* sumsq_out,
                                       nsg_stream_t stream) {
  NSG_CHECK_ARG(keys != nullptr, "null keys");
  return embed_impl(ids, id_stride_b, id_stride_j, batch, per_batch,
                    static_cast<const uint64_t*>(keys), key_cols, key_j, table, ld_table, vocab,
                    hidden, out, ld_out, sumsq_out, stream);
}

extern "C" int32_t nsg_silu_mul(const void* gate_up, void* out, int64_t num_tokens,
                                int32_t intermediate, nsg_stream_t stream) {
  NSG_CHECK_ARG(num_tokens >= 0, "num_tokens < 0");
  if (num_tokens == 0) {
    clear_error();
    return NSG_OK;
  }
  NSG_CHECK_ARG(gate_up && out, "null pointer argument");
  NSG_CHECK_ARG(intermediate > 0 && intermediate % 8 == 0,
                "intermediate %d must be a multiple of 8", intermediate);
  NSG_CHECK_ARG(((uintptr_t)gate_up | (uintptr_t)out) % 16 == 0, "tensors must be 16-byte aligned");
  const int64_t nv = num_tokens * (intermediate / 8);
  const int threads = 256;
  const int64_t blocks = std::min<int64_t>((nv + threads - 1) / threads, 65536);
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(threads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(gate_up),
                     static_cast<uint16_t*>(out), num_tokens, intermediate);
  return launch_status("silu_mul_kernel");
}
