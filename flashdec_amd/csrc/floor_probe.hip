// Measurement probes for the decode path's floor on MI355X (libflashdec_probe.so).
//
// Not part of the decode library or its C ABI: bench.py's c2-floor workload
// times these next to the shipped call, on the same rotating KV-sized buffers
// and in the same hipGraph set-up, to show what one call of that many bytes
// costs with no attention work at all:
//   * fdp_stream_read -- one kernel that reads `bytes` once with 16-byte
//     non-temporal loads (the decode kernel's load flavour), every load of a
//     thread issued before any is used: the HBM floor of a call of that size;
//   * fdp_empty -- an empty kernel: launched after fdp_stream_read on the same
//     stream it prices a dependent second launch (the reducer's launch);
//   * fdp_xcc_map -- each workgroup's XCD (hardware register XCC_ID), to check
//     the round-robin workgroup -> XCD dispatch the decode grid layout uses.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kLoadsPerThread = 4;  // 4 KB per wave in flight; 1028 workgroups for 16.8 MB

__global__ __launch_bounds__(kThreads) void stream_read_kernel(const u32x4* src, uint64_t n16, uint32_t* sink) {
  const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kThreads * kLoadsPerThread + threadIdx.x;
  u32x4 v[kLoadsPerThread];
#pragma unroll
  for (int i = 0; i < kLoadsPerThread; ++i) {
    const uint64_t idx = base + static_cast<uint64_t>(i) * kThreads;
    v[i] = idx < n16 ? __builtin_nontemporal_load(src + idx) : u32x4{0u, 0u, 0u, 0u};
  }
  uint32_t acc = 0;
#pragma unroll
  for (int i = 0; i < kLoadsPerThread; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  // a data-dependent store the compiler cannot drop (never taken on random data
  // in practice; sink holds one word per thread of a workgroup)
  if (acc == 0x9e3779b9u) sink[threadIdx.x] = acc;
}

__global__ void empty_kernel() {}

__global__ void xcc_map_kernel(uint32_t* out) {
  uint32_t x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  if (threadIdx.x == 0) out[blockIdx.x] = x & 0xfu;
}

}  // namespace

// Reads bytes (a multiple of 16, 16-byte aligned src) once; sink: >= 256 uint32 words.
// start / stop (optional HIP events) are recorded around exactly this dispatch
// (hipExtLaunchKernel), as the decode library's timing hook records its own.
extern "C" int fdp_stream_read(const void* src, uint64_t bytes, uint32_t* sink, hipStream_t stream, void* start,
                               void* stop) {
  if (src == nullptr || sink == nullptr || bytes == 0 || (bytes & 15u) || (reinterpret_cast<uintptr_t>(src) & 15u))
    return 1;
  const uint64_t n16 = bytes / 16;
  const uint64_t per_block = static_cast<uint64_t>(kThreads) * kLoadsPerThread;
  const uint64_t grid = (n16 + per_block - 1) / per_block;
  if (grid > 0x7fffffffu) return 1;
  if (start || stop)
    hipExtLaunchKernelGGL(stream_read_kernel, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, stream,
                          static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop), 0,
                          static_cast<const u32x4*>(src), n16, sink);
  else
    hipLaunchKernelGGL(stream_read_kernel, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, stream,
                       static_cast<const u32x4*>(src), n16, sink);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

extern "C" int fdp_empty(unsigned grid, unsigned block, hipStream_t stream) {
  if (grid == 0 || block == 0 || block > 1024) return 1;
  hipLaunchKernelGGL(empty_kernel, dim3(grid), dim3(block), 0, stream);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// out: >= grid uint32 words
extern "C" int fdp_xcc_map(uint32_t* out, unsigned grid, hipStream_t stream) {
  if (out == nullptr || grid == 0) return 1;
  hipLaunchKernelGGL(xcc_map_kernel, dim3(grid), dim3(64), 0, stream, out);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
