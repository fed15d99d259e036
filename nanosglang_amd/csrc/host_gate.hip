// Host gate: lets the engine queue a speculative step's graph before the
// step's inputs exist on the host.
//
// The reference's loop (nano_sglang/decode/speculative.py:50-184 per request,
// its engine's step loop around it) is synchronous: read the step's results,
// build the next step's inputs, launch.  On MI355X the launch of a captured
// step graph (about 200 kernel nodes) costs the host about 80 us, during which
// the GPU would idle.  Instead the engine queues step s + 1 (this gate, the
// input upload, the graph replay, the result copies) while step s runs; the
// gate holds the GPU until the host has written step s + 1's inputs into the
// pinned staging buffer and raised the flag, so only the input build itself
// stays between two steps.
//
// The flag lives in coherent (fine-grained) pinned host memory: the host
// writes 1, the gate's first thread reads it with system-scope loads (no GPU
// cache keeps it) and writes 0 back before it returns.  Once released, the
// gate also copies the step's pinned staging buffer to the device (a copy
// command queued after it would add its own start-up latency to the step).
// The wait is bounded: after `timeout_us` the gate gives up, sets bit 0 of
// *err, copies and returns, so a host that never raises the flag costs time,
// never a hung GPU.
#include "common.hpp"

namespace nsg {
namespace {

constexpr int kGateThreads = 1024;
constexpr int kGateUnroll = 4;  // loads in flight per thread before its stores

// Thread 0 waits for the flag; then every thread copies its share of the
// staging buffer (host -> device, 16 bytes per load), each after its own
// system-scope acquire of the flag word, so that the host's writes before it
// raised the flag are the ones read.
__global__ __launch_bounds__(kGateThreads) void host_gate_kernel(int32_t* flag, int32_t* err,
                                                                 uint64_t timeout_ticks,
                                                                 const uint4* src, uint4* dst,
                                                                 int64_t n16) {
  if (threadIdx.x == 0) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();  // 100 MHz
    for (;;) {
      if (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) != 0) break;
      if (__builtin_amdgcn_s_memrealtime() - t0 > timeout_ticks) {
        __hip_atomic_fetch_or(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(4);
    }
  }
  __syncthreads();
  (void)__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
  for (int64_t i0 = threadIdx.x; i0 < n16; i0 += kGateThreads * kGateUnroll) {
    uint4 v[kGateUnroll];
#pragma unroll
    for (int u = 0; u < kGateUnroll; ++u)
      if (i0 + u * kGateThreads < n16) v[u] = src[i0 + u * kGateThreads];
#pragma unroll
    for (int u = 0; u < kGateUnroll; ++u)
      if (i0 + u * kGateThreads < n16) dst[i0 + u * kGateThreads] = v[u];
  }
  __syncthreads();  // every thread has read the flag before it is reset
  if (threadIdx.x == 0) __hip_atomic_store(flag, 0, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// The same with the copy limited to up to kGateMaxSegs byte ranges of the
// staging buffer (the rest of the buffer is capacity a step does not use),
// spread over kGateSegGroups workgroups: one workgroup pulls pinned host
// memory at about 10 KB per microsecond.  Segment i is [off[i], off[i] +
// len[i]), 16-byte aligned; units are numbered across the segments in order
// and dealt round-robin to the threads of all workgroups.  Each workgroup
// waits on its own for *flag >= target: the host raises a gate by writing its
// target (a count that only grows), so no workgroup resets the word another
// may not have read yet.
constexpr int kGateMaxSegs = 8;
constexpr int kGateSegGroups = 8;
constexpr int kGateSegThreads = 256;
struct GateSegs {
  int64_t off[kGateMaxSegs];   // in 16-byte units
  int64_t len[kGateMaxSegs];   // in 16-byte units
  int32_t n;
};

__global__ __launch_bounds__(kGateSegThreads) void host_gate_segs_kernel(
    int32_t* flag, int32_t target, int32_t* err, uint64_t timeout_ticks, const uint4* src,
    uint4* dst, GateSegs segs) {
  if (threadIdx.x == 0) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();  // 100 MHz
    for (;;) {
      if (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) >= target) break;
      if (__builtin_amdgcn_s_memrealtime() - t0 > timeout_ticks) {
        __hip_atomic_fetch_or(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(4);
    }
  }
  __syncthreads();
  (void)__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
  int64_t total = 0;
  for (int i = 0; i < segs.n; ++i) total += segs.len[i];
  // unit u -> (segment, offset): segments in order, a short scan per unit
  auto addr = [&](int64_t u) -> int64_t {
    int i = 0;
    while (u >= segs.len[i]) u -= segs.len[i++];
    return segs.off[i] + u;
  };
  constexpr int kStride = kGateSegGroups * kGateSegThreads;
  for (int64_t u0 = (int64_t)blockIdx.x * kGateSegThreads + threadIdx.x; u0 < total;
       u0 += (int64_t)kStride * kGateUnroll) {
    uint4 v[kGateUnroll];
    int64_t a[kGateUnroll];
#pragma unroll
    for (int k = 0; k < kGateUnroll; ++k) {
      const int64_t u = u0 + (int64_t)k * kStride;
      a[k] = u < total ? addr(u) : 0;
      if (u < total) v[k] = src[a[k]];
    }
#pragma unroll
    for (int k = 0; k < kGateUnroll; ++k)
      if (u0 + (int64_t)k * kStride < total) dst[a[k]] = v[k];
  }
}

// The step's results to pinned host memory, by a kernel at the end of the
// step's graph (two copy commands after it cost about 4 us each), then the
// done word: the host polls it instead of waiting on an event.
__global__ __launch_bounds__(256) void export_kernel(const int32_t* n, const int64_t* em,
                                                     int32_t rows, int32_t cols, int32_t* n_host,
                                                     int64_t* em_host, int32_t* done) {
  for (int i = threadIdx.x; i < rows; i += 256) n_host[i] = n[i];
  for (int i = threadIdx.x; i < rows * cols; i += 256) em_host[i] = em[i];
  if (done) {
    __threadfence_system();  // this thread's result stores before the done word
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(done, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

}  // namespace
}  // namespace nsg

using namespace nsg;

extern "C" int32_t nsg_host_gate_wait_segments(int32_t* flag, int32_t target, int32_t* err,
                                               int64_t timeout_us, const void* src_host,
                                               void* dst, int64_t nbytes,
                                               const int64_t* seg_offsets,
                                               const int64_t* seg_bytes, int32_t n_segs,
                                               nsg_stream_t stream) {
  NSG_CHECK_ARG(flag != nullptr && err != nullptr, "flag and err must be set");
  NSG_CHECK_ARG(timeout_us > 0 && timeout_us <= 60000000, "timeout_us %lld outside (0, 60 s]",
                (long long)timeout_us);
  NSG_CHECK_ARG(n_segs >= 0 && n_segs <= kGateMaxSegs, "n_segs %d outside [0, %d]", n_segs,
                kGateMaxSegs);
  NSG_CHECK_ARG(n_segs == 0 || (seg_offsets && seg_bytes && src_host && dst &&
                                (reinterpret_cast<uintptr_t>(src_host) |
                                 reinterpret_cast<uintptr_t>(dst)) % 16 == 0),
                "segments need offsets, sizes and 16-byte aligned src_host and dst");
  GateSegs g{};
  g.n = n_segs;
  for (int i = 0; i < n_segs; ++i) {
    NSG_CHECK_ARG(seg_offsets[i] >= 0 && seg_bytes[i] >= 0 && seg_offsets[i] % 16 == 0 &&
                      seg_bytes[i] % 16 == 0 && seg_offsets[i] + seg_bytes[i] <= nbytes,
                  "segment %d: offset %lld and size %lld must be non-negative multiples of 16 "
                  "within the %lld-byte buffers", i, (long long)seg_offsets[i],
                  (long long)seg_bytes[i], (long long)nbytes);
    g.off[i] = seg_offsets[i] / 16;
    g.len[i] = seg_bytes[i] / 16;
  }
  NSG_CHECK_ARG(target >= 1, "target %d must be positive", target);
  hipLaunchKernelGGL(host_gate_segs_kernel, dim3(kGateSegGroups), dim3(kGateSegThreads), 0,
                     static_cast<hipStream_t>(stream), flag, target, err,
                     (uint64_t)timeout_us * 100u, static_cast<const uint4*>(src_host),
                     static_cast<uint4*>(dst), g);
  return launch_status("host_gate_segs_kernel");
}

extern "C" int32_t nsg_export_step(const int32_t* n_emitted, const int64_t* emitted,
                                   int32_t rows, int32_t cols, int32_t* n_host,
                                   int64_t* emitted_host, int32_t* done_host,
                                   nsg_stream_t stream) {
  NSG_CHECK_ARG(rows >= 0 && cols >= 0 && (int64_t)rows * cols <= (1 << 24),
                "rows %d, cols %d", rows, cols);
  NSG_CHECK_ARG(rows == 0 || (n_emitted && emitted && n_host && emitted_host),
                "null pointer");
  hipLaunchKernelGGL(export_kernel, dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream),
                     n_emitted, emitted, rows, cols, n_host, emitted_host, done_host);
  return launch_status("export_kernel");
}

extern "C" int32_t nsg_host_gate_alloc(int32_t** flag) {
  NSG_CHECK_ARG(flag != nullptr, "flag is null");
  void* p = nullptr;
  NSG_CHECK_HIP(hipHostMalloc(&p, 64, hipHostMallocCoherent | hipHostMallocMapped));
  *static_cast<volatile int32_t*>(p) = 0;
  *flag = static_cast<int32_t*>(p);
  clear_error();
  return NSG_OK;
}

extern "C" int32_t nsg_host_gate_free(int32_t* flag) {
  if (flag) NSG_CHECK_HIP(hipHostFree(flag));
  clear_error();
  return NSG_OK;
}

extern "C" int32_t nsg_host_gate_wait(int32_t* flag, int32_t* err, int64_t timeout_us,
                                      const void* src_host, void* dst, int64_t nbytes,
                                      nsg_stream_t stream) {
  NSG_CHECK_ARG(flag != nullptr && err != nullptr, "flag and err must be set");
  NSG_CHECK_ARG(timeout_us > 0 && timeout_us <= 60000000, "timeout_us %lld outside (0, 60 s]",
                (long long)timeout_us);
  NSG_CHECK_ARG(nbytes >= 0 && nbytes % 16 == 0, "nbytes %lld must be a multiple of 16",
                (long long)nbytes);
  NSG_CHECK_ARG(nbytes == 0 || (src_host && dst && (reinterpret_cast<uintptr_t>(src_host) |
                                                    reinterpret_cast<uintptr_t>(dst)) % 16 == 0),
                "src_host and dst must be set and 16-byte aligned");
  hipLaunchKernelGGL(host_gate_kernel, dim3(1), dim3(kGateThreads), 0,
                     static_cast<hipStream_t>(stream), flag, err, (uint64_t)timeout_us * 100u,
                     static_cast<const uint4*>(src_host), static_cast<uint4*>(dst), nbytes / 16);
  return launch_status("host_gate_kernel");
}
