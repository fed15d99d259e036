// Shared helpers for the gfx950 verify-step kernels: error reporting across
// the C ABI, bf16 conversion, vector types and wave-level reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/nsg_spec.h"

namespace nsg {

// ---- error string (thread-local, read through nsg_last_error) ----
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define NSG_CHECK_ARG(cond, ...)             \
  do {                                       \
    if (!(cond)) {                           \
      ::nsg::set_error(__VA_ARGS__);         \
      return NSG_ERR_ARG;                    \
    }                                        \
  } while (0)

#define NSG_CHECK_HIP(expr)                                                  \
  do {                                                                       \
    hipError_t e_ = (expr);                                                  \
    if (e_ != hipSuccess) {                                                  \
      ::nsg::set_error("%s failed: %s", #expr, hipGetErrorString(e_));       \
      return NSG_ERR_HIP;                                                    \
    }                                                                        \
  } while (0)

// Checks the launch that was just enqueued.
inline int32_t launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s launch failed: %s", what, hipGetErrorString(e));
    return NSG_ERR_HIP;
  }
  clear_error();
  return NSG_OK;
}

// ---- workspaces ----
// An acceptance workspace starts with a header of kWorkspaceHeaderBytes whose
// first word holds the error flags; the sampler's layout skips the same
// header.
constexpr int64_t kWorkspaceHeaderBytes = 256;

// ---- hand-off between workgroups of one launch ----
// gfx950's L2 is per XCD and, for ordinary device memory, coherent across
// XCDs only at kernel boundaries.  The few words one workgroup hands to
// another inside a launch are therefore written and read only with
// device-scope read-modify-write atomics -- an exchange to write, an add of
// zero to read -- which the memory side performs in one order for every
// XCD.  hand_put_sync also waits for its exchange to return, so that the word
// is in place before anything this thread writes later; no L2 write-back or
// invalidate is needed, and the bulk data (logits) keeps its ordinary path.
__device__ __forceinline__ void hand_put(uint32_t* p, uint32_t v) { (void)atomicExch(p, v); }
__device__ __forceinline__ void hand_put_sync(uint32_t* p, uint32_t v) {
  const uint32_t old = atomicExch(p, v);
  asm volatile("" ::"v"(old));   // the returned word: the exchange has been performed
}
__device__ __forceinline__ uint32_t hand_get(const uint32_t* p) {
  return atomicAdd(const_cast<uint32_t*>(p), 0u);
}
__device__ __forceinline__ void hand_put(float* p, float v) {
  hand_put(reinterpret_cast<uint32_t*>(p), __float_as_uint(v));
}
__device__ __forceinline__ void hand_put_sync(float* p, float v) {
  hand_put_sync(reinterpret_cast<uint32_t*>(p), __float_as_uint(v));
}
__device__ __forceinline__ float hand_get(const float* p) {
  return __uint_as_float(hand_get(reinterpret_cast<const uint32_t*>(p)));
}
__device__ __forceinline__ uint64_t hand_get_bits(const float2* p) {
  return atomicAdd(reinterpret_cast<unsigned long long*>(const_cast<float2*>(p)), 0ull);
}
__device__ __forceinline__ void hand_put(float2* p, float2 v) {
  const unsigned long long bits =
      (unsigned long long)__float_as_uint(v.x) | ((unsigned long long)__float_as_uint(v.y) << 32);
  (void)atomicExch(reinterpret_cast<unsigned long long*>(p), bits);
}
__device__ __forceinline__ float2 hand_get(const float2* p) {
  const uint64_t bits = hand_get_bits(p);
  return make_float2(__uint_as_float((uint32_t)bits), __uint_as_float((uint32_t)(bits >> 32)));
}

// ---- device types ----
typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even float -> bf16 bits by gfx950's v_cvt_pk_bf16_f32
// (two values per instruction; the integer form u + 0x7fff + ((u >> 16) & 1)
// takes about five instructions per value).  Checked against that integer
// form on MI355X for every non-NaN float bit pattern, subnormals included:
// identical; NaN stays a quiet NaN.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float floatx2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2_t{lo, hi}), bf16x2_t));
}

__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Greedy argmax keys of the lm_head kernels: per row, one key per workgroup
// (or wave) = (order-preserving bits of its largest bf16 logit) << 32 |
// (0xffffffff - its lowest column), 0 for no column; the row's token is the
// column of the largest key.  One wave reduces a row of n keys: up to 16
// loads per lane in flight at once (addresses clamped, values past n
// dropped), then an xor butterfly; every lane returns the row's largest key.
__device__ __forceinline__ uint64_t wave_max_key(const uint64_t* row, int n, int lane) {
  constexpr int kU = 16;
  uint64_t k = 0;
  for (int c0 = 0; c0 < n; c0 += 64 * kU) {
    uint64_t v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) v[u] = row[min(c0 + u * 64 + lane, n - 1)];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const uint64_t x = c0 + u * 64 + lane < n ? v[u] : 0;
      k = x > k ? x : k;
    }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t other = ((uint64_t)(uint32_t)__shfl_xor((int)(k >> 32), o, 64) << 32) |
                           (uint32_t)__shfl_xor((int)(uint32_t)k, o, 64);
    k = other > k ? other : k;
  }
  return k;
}
__device__ __forceinline__ int64_t key_token(uint64_t k) {
  return (int64_t)(0xffffffffu - (uint32_t)k);
}

// s_waitcnt immediate that waits until at most n vector-memory ops of this
// wave are outstanding (gfx9 encoding: vmcnt bits [3:0] and [15:14]; expcnt
// and lgkmcnt left at their maxima, i.e. not waited on).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }

// s_waitcnt until at most `later` ring steps (NI DMA instructions each) of
// this wave are still in flight.  `later` is a runtime value in [0, L]; each
// case has its own immediate.  vmcnt counts to 63: a larger count waits for
// 63, which is only more conservative.
template <int NI, int L>
__device__ __forceinline__ void wait_steps(int later) {
  if constexpr (L == 0) {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  } else {
    if (later >= L) {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(L * NI < 63 ? L * NI : 63));
      return;
    }
    wait_steps<NI, L - 1>(later);
  }
}

// 32-bit LDS address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Max / sum over lanes l, l ^ 16, l ^ 32 and l ^ 48 (the four 16-lane groups
// of a 16 x 16 MFMA result that share a row or column) with gfx950's row
// swaps, which stay in the VALU:
// v_permlane32_swap with both operands x leaves lane l holding x[l % 32] in
// the first result and x[l % 32 + 32] in the second, v_permlane16_swap the
// same for the even and odd 16-lane rows.  Sums pair the same two lanes in
// both halves, so every lane ends with the same value.
__device__ __forceinline__ float max_xor16_32(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_xor16_32(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

}  // namespace nsg
