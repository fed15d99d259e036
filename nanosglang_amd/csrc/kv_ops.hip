// KV slot scatter / clear and Philox uniforms for the verify step, plus the
// library's error-string plumbing.
//
// nsg_kv_write replaces the index_put KV scatter of the paged path
// (nano_sglang/model/causal_lm.py:335-338) with slots built by the rule of
// nano_sglang/engine/engine.py:437-443.  nsg_kv_clear_slots zeroes rolled-back
// slots after the acceptance step.  nsg_philox_uniform supplies the verify
// step's uniforms in place of torch.rand (nano_sglang/decode/speculative.py:150).
#include <cstdarg>
#include <cstring>

#include "common.hpp"

namespace nsg {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// One thread moves 16 bytes (8 bf16); a token row is Hkv * D / 8 chunks.
__global__ void kv_write_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                int64_t src_stride, const int64_t* __restrict__ slots, int n_tok,
                                uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int row_elems,
                                int64_t num_slots, int* __restrict__ flags) {
  const int chunks = row_elems / 8;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)n_tok * chunks) return;
  const int t = (int)(gid / chunks);
  const int c = (int)(gid - (int64_t)t * chunks);
  const int64_t slot = slots[t];
  if (slot < 0) return;
  if (slot >= num_slots) {
    if (flags) atomicOr(flags, 1);
    return;
  }
  const u32x4 kv = *reinterpret_cast<const u32x4*>(k + t * src_stride + c * 8);
  const u32x4 vv = *reinterpret_cast<const u32x4*>(v + t * src_stride + c * 8);
  *reinterpret_cast<u32x4*>(kc + slot * row_elems + c * 8) = kv;
  *reinterpret_cast<u32x4*>(vc + slot * row_elems + c * 8) = vv;
}

__global__ void kv_clear_kernel(const int64_t* __restrict__ slots, int count,
                                uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                int num_layers, int64_t layer_stride, int row_elems,
                                int64_t num_slots) {
  const int chunks = row_elems / 8;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_layer = (int64_t)count * chunks;
  if (gid >= per_layer * num_layers) return;
  const int layer = (int)(gid / per_layer);
  const int64_t r = gid - layer * per_layer;
  const int t = (int)(r / chunks);
  const int c = (int)(r - (int64_t)t * chunks);
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;
  const int64_t off = layer * layer_stride + slot * row_elems + c * 8;
  *reinterpret_cast<u32x4*>(kc + off) = u32x4{0u, 0u, 0u, 0u};
  *reinterpret_cast<u32x4*>(vc + off) = u32x4{0u, 0u, 0u, 0u};
}

__device__ __forceinline__ float bf16r(float x) {  // round to bf16, back to float
  return bf16_bits_to_float(float_to_bf16_bits(x));
}

// One workgroup per token.  Work item (head hh, pair i): q / k heads are
// rotated with the half-split rule y[i] = x[i] c - x[i+D/2] s,
// y[i+D/2] = x[i+D/2] c + x[i] s, every product and the sum rounded to bf16
// and c, s rounded to bf16 first -- the arithmetic of bf16 tensors in
// nano_sglang/model/causal_lm.py:181-206.  Rotated q goes to q_out; rotated k
// and v go to the cache slot of the token (slot < 0 skips).
__global__ void rope_kv_write_kernel(const uint16_t* __restrict__ qkv, int64_t qkv_stride,
                                     const int64_t* __restrict__ positions,
                                     const float* __restrict__ cos_t,
                                     const float* __restrict__ sin_t, int max_pos,
                                     const int64_t* __restrict__ slots, int Hq, int Hkv, int D,
                                     uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc,
                                     uint16_t* __restrict__ vc, int64_t num_slots,
                                     int* __restrict__ flags) {
  const int t = blockIdx.x;
  const int half = D / 2;
  const int64_t pos = positions[t];
  const bool pos_ok = pos >= 0 && pos < max_pos;
  const int64_t slot = slots ? slots[t] : -1;
  const bool slot_ok = slot >= 0 && slot < num_slots;
  if (threadIdx.x == 0 && (!pos_ok || slot >= num_slots) && flags) atomicOr(flags, 1);
  const uint16_t* x = qkv + t * qkv_stride;
  const int items = (Hq + 2 * Hkv) * half;
  for (int it = threadIdx.x; it < items; it += blockDim.x) {
    const int hh = it / half;
    const int i = it - hh * half;
    const float x1 = bf16_bits_to_float(x[hh * D + i]);
    const float x2 = bf16_bits_to_float(x[hh * D + i + half]);
    uint16_t y1, y2;
    if (hh < Hq + Hkv) {
      const float c = pos_ok ? bf16r(cos_t[pos * half + i]) : 0.f;
      const float sn = pos_ok ? bf16r(sin_t[pos * half + i]) : 0.f;
      y1 = float_to_bf16_bits(bf16r(x1 * c) + bf16r(-x2 * sn));
      y2 = float_to_bf16_bits(bf16r(x2 * c) + bf16r(x1 * sn));
    } else {
      y1 = x[hh * D + i];
      y2 = x[hh * D + i + half];
    }
    if (hh < Hq) {
      uint16_t* qo = q_out + ((int64_t)t * Hq + hh) * D;
      qo[i] = y1;
      qo[i + half] = y2;
    } else if (slot_ok) {
      const bool is_k = hh < Hq + Hkv;
      const int kh = is_k ? hh - Hq : hh - Hq - Hkv;
      uint16_t* dst = (is_k ? kc : vc) + (slot * Hkv + kh) * D;
      dst[i] = y1;
      dst[i + half] = y2;
    }
  }
}

__device__ __forceinline__ void philox_round(uint32_t& c0, uint32_t& c1, uint32_t& c2,
                                             uint32_t& c3, uint32_t k0, uint32_t k1) {
  const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
  const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
  const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
  const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
  const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
  c0 = n0;
  c1 = lo1;
  c2 = n2;
  c3 = lo0;
}

// Each thread produces one Philox block (4 words) of the stream.
__global__ void philox_kernel(uint64_t seed, uint32_t stream_id, uint64_t offset, int64_t n,
                              float* __restrict__ out) {
  const int64_t blk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t first_block = offset / 4;
  const uint64_t b = first_block + (uint64_t)blk;
  uint32_t c0 = (uint32_t)b, c1 = (uint32_t)(b >> 32), c2 = stream_id, c3 = 0;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    philox_round(c0, c1, c2, c3, k0, k1);
  }
  const uint32_t w[4] = {c0, c1, c2, c3};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t idx = (int64_t)(b * 4 + e) - (int64_t)offset;
    if (idx >= 0 && idx < n) out[idx] = (float)(w[e] >> 8) * 5.9604644775390625e-08f;
  }
}

}  // namespace
}  // namespace nsg

using namespace nsg;

extern "C" const char* nsg_last_error(void) { return g_err; }

extern "C" int32_t nsg_abi_version(void) { return NSG_ABI_VERSION; }

extern "C" int32_t nsg_kv_write(const void* k, const void* v, int64_t src_token_stride,
                                const int64_t* slots, int32_t num_tokens, void* k_cache,
                                void* v_cache, int32_t num_kv_heads, int32_t head_dim,
                                int64_t num_slots, nsg_stream_t stream) {
  NSG_CHECK_ARG(num_tokens >= 0, "num_tokens %d < 0", num_tokens);
  if (num_tokens == 0) {
    clear_error();
    return NSG_OK;
  }
  NSG_CHECK_ARG(k && v && slots && k_cache && v_cache, "null pointer argument");
  const int row = num_kv_heads * head_dim;
  NSG_CHECK_ARG(num_kv_heads > 0 && head_dim > 0 && row % 8 == 0,
                "num_kv_heads * head_dim = %d must be a positive multiple of 8", row);
  NSG_CHECK_ARG(src_token_stride >= row && src_token_stride % 8 == 0,
                "src_token_stride %lld must be >= %d and a multiple of 8",
                (long long)src_token_stride, row);
  NSG_CHECK_ARG(((uintptr_t)k | (uintptr_t)v | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0,
                "K/V sources and caches must be 16-byte aligned");
  const int64_t total = (int64_t)num_tokens * (row / 8);
  const int threads = 256;
  hipLaunchKernelGGL(kv_write_kernel, dim3((unsigned)((total + threads - 1) / threads)),
                     dim3(threads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
                     src_token_stride, slots, num_tokens, static_cast<uint16_t*>(k_cache),
                     static_cast<uint16_t*>(v_cache), row, num_slots, (int*)nullptr);
  return launch_status("kv_write_kernel");
}

extern "C" int32_t nsg_kv_clear_slots(const int64_t* slots, int32_t count, void* k_cache,
                                      void* v_cache, int32_t num_layers, int64_t layer_stride,
                                      int32_t num_kv_heads, int32_t head_dim, int64_t num_slots,
                                      nsg_stream_t stream) {
  NSG_CHECK_ARG(count >= 0 && num_layers >= 0, "negative count");
  if (count == 0 || num_layers == 0) {
    clear_error();
    return NSG_OK;
  }
  NSG_CHECK_ARG(slots && k_cache && v_cache, "null pointer argument");
  const int row = num_kv_heads * head_dim;
  NSG_CHECK_ARG(row > 0 && row % 8 == 0, "num_kv_heads * head_dim must be a multiple of 8");
  NSG_CHECK_ARG(layer_stride >= num_slots * row && layer_stride % 8 == 0,
                "layer_stride %lld too small", (long long)layer_stride);
  NSG_CHECK_ARG(((uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0, "caches must be 16-byte aligned");
  const int64_t total = (int64_t)num_layers * count * (row / 8);
  const int threads = 256;
  hipLaunchKernelGGL(kv_clear_kernel, dim3((unsigned)((total + threads - 1) / threads)),
                     dim3(threads), 0, static_cast<hipStream_t>(stream), slots, count,
                     static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), num_layers,
                     layer_stride, row, num_slots);
  return launch_status("kv_clear_kernel");
}

extern "C" int32_t nsg_rope_kv_write(const void* qkv, int64_t qkv_token_stride,
                                     const int64_t* positions, const float* cos_table,
                                     const float* sin_table, int32_t max_position,
                                     const int64_t* slots, int32_t num_tokens,
                                     int32_t num_qo_heads, int32_t num_kv_heads,
                                     int32_t head_dim, void* q_out, void* k_cache,
                                     void* v_cache, int64_t num_slots, int32_t* flags,
                                     nsg_stream_t stream) {
  NSG_CHECK_ARG(num_tokens >= 0, "num_tokens %d < 0", num_tokens);
  if (num_tokens == 0) {
    clear_error();
    return NSG_OK;
  }
  NSG_CHECK_ARG(qkv && positions && cos_table && sin_table && q_out, "null pointer argument");
  NSG_CHECK_ARG(!slots || (k_cache && v_cache), "slots given without caches");
  NSG_CHECK_ARG(head_dim > 0 && head_dim % 2 == 0, "head_dim %d must be even", head_dim);
  NSG_CHECK_ARG(num_qo_heads > 0 && num_kv_heads > 0, "head counts must be positive");
  NSG_CHECK_ARG(qkv_token_stride >= (int64_t)(num_qo_heads + 2 * num_kv_heads) * head_dim,
                "qkv_token_stride %lld too small", (long long)qkv_token_stride);
  NSG_CHECK_ARG(max_position > 0, "max_position %d", max_position);
  hipLaunchKernelGGL(rope_kv_write_kernel, dim3(num_tokens), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(qkv),
                     qkv_token_stride, positions, cos_table, sin_table, max_position, slots,
                     num_qo_heads, num_kv_heads, head_dim, static_cast<uint16_t*>(q_out),
                     static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), num_slots,
                     flags);
  return launch_status("rope_kv_write_kernel");
}

extern "C" int32_t nsg_philox_uniform(uint64_t seed, uint32_t stream_id, uint64_t offset,
                                      int64_t n, float* out, nsg_stream_t stream) {
  NSG_CHECK_ARG(n >= 0, "n %lld < 0", (long long)n);
  if (n == 0) {
    clear_error();
    return NSG_OK;
  }
  NSG_CHECK_ARG(out != nullptr, "null output");
  const int64_t blocks = (int64_t)((offset + n + 3) / 4 - offset / 4);
  const int threads = 256;
  hipLaunchKernelGGL(philox_kernel, dim3((unsigned)((blocks + threads - 1) / threads)),
                     dim3(threads), 0, static_cast<hipStream_t>(stream), seed, stream_id, offset,
                     n, out);
  return launch_status("philox_kernel");
}
