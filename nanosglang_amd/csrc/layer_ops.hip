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
constexpr int kNormThreads = 128;

__device__ __forceinline__ float block_sum(float v, float* sh) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) sh[wave] = v;
  __syncthreads();
  float t = 0.f;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += sh[w];
  __syncthreads();
  return t;
}

// One workgroup per token row; each thread owns 8-element chunks (16 bytes).
// H must be a multiple of 8 and at most kNormThreads * 8 * kMaxChunks.
template <bool ADD>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(
    const uint16_t* __restrict__ x, uint16_t* __restrict__ residual,
    const uint16_t* __restrict__ w, uint16_t* __restrict__ out, int H, float eps) {
  constexpr int kMaxChunks = 8;  // H <= 128 * 8 * 8 = 8192
  __shared__ float sh[kNormThreads / 64];
  const int64_t row = blockIdx.x;
  const int nch = H / 8;
  float v[kMaxChunks][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int ch = threadIdx.x + c * kNormThreads;
    if (ch < nch) {
      const u32x4 a = *reinterpret_cast<const u32x4*>(x + row * H + ch * 8);
      if constexpr (ADD) {
        const u32x4 r = *reinterpret_cast<const u32x4*>(residual + row * H + ch * 8);
        u32x4 s;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float lo = bf16_bits_to_float(a[i] & 0xffff) + bf16_bits_to_float(r[i] & 0xffff);
          const float hi = bf16_bits_to_float(a[i] >> 16) + bf16_bits_to_float(r[i] >> 16);
          s[i] = pack_bf16x2(lo, hi);
        }
        *reinterpret_cast<u32x4*>(residual + row * H + ch * 8) = s;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[c][2 * i] = bf16_bits_to_float(s[i] & 0xffff);
          v[c][2 * i + 1] = bf16_bits_to_float(s[i] >> 16);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[c][2 * i] = bf16_bits_to_float(a[i] & 0xffff);
          v[c][2 * i + 1] = bf16_bits_to_float(a[i] >> 16);
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += v[c][i] * v[c][i];
    }
  }
  const float var = block_sum(ss, sh) / (float)H;
  const float r = 1.f / sqrtf(var + eps);
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int ch = threadIdx.x + c * kNormThreads;
    if (ch < nch) {
      const u32x4 wv = *reinterpret_cast<const u32x4*>(w + ch * 8);
      u32x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lo = bf16_bits_to_float(wv[i] & 0xffff) * (v[c][2 * i] * r);
        const float hi = bf16_bits_to_float(wv[i] >> 16) * (v[c][2 * i + 1] * r);
        o[i] = pack_bf16x2(lo, hi);
      }
      *reinterpret_cast<u32x4*>(out + row * H + ch * 8) = o;
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
  NSG_CHECK_ARG(hidden > 0 && hidden % 8 == 0 && hidden <= kNormThreads * 8 * 8,
                "hidden %d must be a multiple of 8 and at most 8192", hidden);
  NSG_CHECK_ARG(((uintptr_t)x | (uintptr_t)weight | (uintptr_t)out |
                 (uintptr_t)residual) % 16 == 0, "tensors must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (residual) {
    hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3(num_tokens), dim3(kNormThreads), 0, s,
                       static_cast<const uint16_t*>(x), static_cast<uint16_t*>(residual),
                       static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(out),
                       hidden, eps);
  } else {
    hipLaunchKernelGGL(rmsnorm_kernel<false>, dim3(num_tokens), dim3(kNormThreads), 0, s,
                       static_cast<const uint16_t*>(x), static_cast<uint16_t*>(nullptr),
                       static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(out),
                       hidden, eps);
  }
  return launch_status("rmsnorm_kernel");
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
