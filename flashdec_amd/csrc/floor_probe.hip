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
//     the round-robin workgroup -> XCD dispatch the decode grid layout uses;
//   * fdp_paged_read -- the split attention kernel's memory pattern with no
//     attention arithmetic: the same grid (one workgroup of four waves per
//     (request, KV head, split), XCD by XCD), each wave's block-table entry,
//     then its 32-token K and V unit (non-temporal 16-byte loads, all issued
//     before any is used), the four waves' results combined through LDS, and
//     one split partial per (query head, split) stored as the attention kernel
//     stores its partials;
//   * fdp_reduce_read -- the split reducer's memory pattern with the
//     arithmetic cut to a weighted sum: one wave per (request, query head),
//     every split's partial row and statistics loaded up front, one output
//     row stored.
// fdp_paged_read then fdp_reduce_read is the floor of a two-launch split-KV
// paged call of that shape: two dependent launches, the block-table round
// trip ahead of the K/V loads, and the round trip to the partials.
//
// Built with the decode library's kernel-argument preloading, so the probes'
// first loads issue without a kernel-argument fetch, as the decode kernels' do.

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

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kUnit16 = 512;  // one 32-token block of one KV head: 32 * 128 bf16 = 8 KB = 512 x 16 B
constexpr int kGroup = 8;     // query heads per KV head (the probe's shape: D 128, so 8 x 32 threads)

// n / d for n < 2^31 by multiply-high and shifts (Granlund and Montgomery
// 1994, Figure 4.1), as the decode kernel divides its workgroup index; the
// host computes m and the shifts (magic).
__device__ __forceinline__ uint32_t fast_div(uint32_t n, uint32_t m, int s1, int s2) {
  const uint32_t t = __umulhi(n, m);
  return (t + ((n - t) >> s1)) >> s2;
}

void magic(uint32_t d, uint32_t& m, int& s1, int& s2) {
  int l = 0;
  while ((uint64_t{1} << l) < d) ++l;
  m = static_cast<uint32_t>(((uint64_t{1} << 32) * ((uint64_t{1} << l) - d)) / d + 1);
  s1 = l < 1 ? l : 1;
  s2 = l > 1 ? l - 1 : 0;
}

// grid: batch * hkv * splits workgroups of 256 threads; per_xcd > 0: the
// i-th workgroup on XCD x is logical workgroup x * per_xcd + i.  Every
// argument the K/V loads need sits in the 14 preloaded SGPRs (56 bytes:
// the divisions by splits and hkv come as multipliers and shifts, as in the
// decode kernel); only the partials' pointers, needed at the end, are fetched.
__global__ __launch_bounds__(kThreads, 1) void paged_read_kernel(const int32_t* bt, const u32x4* k, const u32x4* v,
                                                                 int32_t kblk16, int32_t khd16, int32_t nblk,
                                                                 int32_t splits, uint32_t splits_m, uint32_t hkv_m,
                                                                 int32_t shifts, int32_t hkv_xcd, float* part,
                                                                 float* mx, float* sm) {
  const int hkv = hkv_xcd & 0xffff;
  const int per_xcd = hkv_xcd >> 16;
  const int wg = per_xcd > 0 ? (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3) : blockIdx.x;
  const int pair = static_cast<int>(fast_div(wg, splits_m, shifts & 0xff, (shifts >> 8) & 0xff));
  const int split = wg - pair * splits;
  const int b = static_cast<int>(fast_div(pair, hkv_m, (shifts >> 16) & 0xff, shifts >> 24));
  const int h = pair - b * hkv;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int per_split =
      static_cast<int>(fast_div(nblk + splits - 1, splits_m, shifts & 0xff, (shifts >> 8) & 0xff));
  int vzero = 0;  // keeps the uniform table load on the vector path, as the decode kernel does
  asm volatile("" : "+v"(vzero));
  uint32_t acc = 0;
  for (int u = wave; u < per_split; u += kThreads / 64) {
    const int bi = split * per_split + u;
    if (bi >= nblk) break;
    const int64_t blk = bt[static_cast<int64_t>(b) * nblk + bi + vzero];
    const u32x4* kb = k + blk * kblk16 + static_cast<int64_t>(h) * khd16 + lane;
    const u32x4* vb = v + blk * kblk16 + static_cast<int64_t>(h) * khd16 + lane;
    u32x4 kk[kUnit16 / 64], vv[kUnit16 / 64];
#pragma unroll
    for (int i = 0; i < kUnit16 / 64; ++i) kk[i] = __builtin_nontemporal_load(kb + 64 * i);
#pragma unroll
    for (int i = 0; i < kUnit16 / 64; ++i) vv[i] = __builtin_nontemporal_load(vb + 64 * i);
    __builtin_amdgcn_sched_barrier(0);  // all sixteen loads issue before the first use
#pragma unroll
    for (int i = 0; i < kUnit16 / 64; ++i) acc ^= kk[i].x ^ kk[i].y ^ kk[i].z ^ kk[i].w ^ vv[i].x ^ vv[i].y ^ vv[i].z ^ vv[i].w;
  }
  __shared__ uint32_t s_acc[kThreads / 64][64];
  s_acc[wave][lane] = acc;
  __syncthreads();
  const uint32_t x = s_acc[0][lane] ^ s_acc[1][lane] ^ s_acc[2][lane] ^ s_acc[3][lane];
  // thread t: query head t / 32 of this KV head, dims 4 (t % 32) .. + 3
  const int hh = threadIdx.x >> 5;
  const int64_t row = static_cast<int64_t>(b) * hkv * kGroup + h * kGroup + hh;
  const int64_t so = row * splits + split;
  const float f = static_cast<float>(x & 0xffffu);
  *reinterpret_cast<f32x4*>(part + so * 128 + 4 * (threadIdx.x & 31)) = f32x4{f, f + 1.f, f + 2.f, f + 3.f};
  if ((threadIdx.x & 31) == 0) {
    mx[so] = f;
    sm[so] = 1.f;
  }
}

constexpr int kMaxSplits = 16;

// grid: rows (= batch * hq) workgroups of one wave, XCD by XCD as above;
// splits <= 16; partials [rows, splits, 128], statistics [rows, splits]
__global__ __launch_bounds__(64) void reduce_read_kernel(const float* part, const float* mx, const float* sm,
                                                         int32_t splits, int32_t per_xcd, __bf16* out) {
  const int row = per_xcd > 0 ? (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3) : blockIdx.x;
  const int lane = threadIdx.x;
  const float* pr = part + static_cast<int64_t>(row) * splits * 128;
  const int sj = min(lane, splits - 1);
  const float lm = mx[static_cast<int64_t>(row) * splits + sj];
  const float ll = sm[static_cast<int64_t>(row) * splits + sj];
  float a[kMaxSplits][2];
#pragma unroll
  for (int j = 0; j < kMaxSplits; ++j) {
    const int s = min(j, splits - 1);
    a[j][0] = pr[s * 128 + lane];
    a[j][1] = pr[s * 128 + lane + 64];
  }
  __builtin_amdgcn_sched_barrier(0);
  float o0 = 0.f, o1 = 0.f, L = 0.f, M = -INFINITY;
#pragma unroll
  for (int j = 0; j < kMaxSplits; ++j) {
    const int src = min(j, splits - 1);
    const float lj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ll), src));
    const float m = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lm), src));
    const float w = j < splits ? lj : 0.f;
    M = j < splits ? fmaxf(M, m) : M;
    L += w;
    o0 += w * a[j][0];
    o1 += w * a[j][1];
  }
  const float inv = L > 0.f && M < INFINITY ? 1.f / L : 0.f;
  __bf16* dst = out + static_cast<int64_t>(row) * 128;
  dst[lane] = static_cast<__bf16>(o0 * inv);
  dst[lane + 64] = static_cast<__bf16>(o1 * inv);
}

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

// The attention kernel's memory pattern at a C2-like shape: a [blocks, hkv,
// 32, 128] bf16 cache (kblk_bytes / khd_bytes: block and head strides, the
// head stride 8 KB), int32 table [batch, nblk], 8 query heads per KV head;
// partials [batch * hkv * 8, splits, 128] fp32, statistics [.., splits].
extern "C" int fdp_paged_read(const int32_t* bt, int nblk, int batch, int hkv, int splits, const void* k, const void* v,
                              int64_t kblk_bytes, int64_t khd_bytes, float* part, float* mx, float* sm,
                              hipStream_t stream, void* start, void* stop) {
  if (bt == nullptr || k == nullptr || v == nullptr || part == nullptr || mx == nullptr || sm == nullptr ||
      nblk <= 0 || batch <= 0 || hkv <= 0 || splits <= 0 || splits > nblk || khd_bytes != 16 * kUnit16 ||
      kblk_bytes < hkv * khd_bytes || (kblk_bytes & 15) || kblk_bytes / 16 > 0x7fffffff ||
      ((reinterpret_cast<uintptr_t>(k) |
      reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(part)) & 15u))
    return 1;
  const int64_t grid = static_cast<int64_t>(batch) * hkv * splits;
  if (grid > 0x7fffffff || hkv > 0xffff) return 1;
  const int per_xcd = grid % 8 == 0 ? static_cast<int>(grid / 8) : 0;
  if (per_xcd > 0x7fff) return 1;
  uint32_t ms = 0, mh = 0;
  int a1 = 0, a2 = 0, b1 = 0, b2 = 0;
  magic(static_cast<uint32_t>(splits), ms, a1, a2);
  magic(static_cast<uint32_t>(hkv), mh, b1, b2);
  const int32_t shifts = a1 | (a2 << 8) | (b1 << 16) | (b2 << 24);
  const int32_t hkv_xcd = hkv | (per_xcd << 16);
  const int32_t kblk16 = static_cast<int32_t>(kblk_bytes / 16), khd16 = static_cast<int32_t>(khd_bytes / 16);
  const u32x4* k16 = static_cast<const u32x4*>(k);
  const u32x4* v16 = static_cast<const u32x4*>(v);
  if (start || stop)
    hipExtLaunchKernelGGL(paged_read_kernel, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, stream,
                          static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop), 0, bt, k16, v16, kblk16,
                          khd16, nblk, splits, ms, mh, shifts, hkv_xcd, part, mx, sm);
  else
    hipLaunchKernelGGL(paged_read_kernel, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, stream, bt, k16, v16,
                       kblk16, khd16, nblk, splits, ms, mh, shifts, hkv_xcd, part, mx, sm);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// The reducer's memory pattern over fdp_paged_read's partials: rows = batch *
// hkv * 8 output rows of 128 bf16, splits <= 16.
extern "C" int fdp_reduce_read(const float* part, const float* mx, const float* sm, int rows, int splits, void* out,
                               hipStream_t stream) {
  if (part == nullptr || mx == nullptr || sm == nullptr || out == nullptr || rows <= 0 || splits <= 0 ||
      splits > kMaxSplits)
    return 1;
  const int per_xcd = rows % 8 == 0 ? rows / 8 : 0;
  hipLaunchKernelGGL(reduce_read_kernel, dim3(static_cast<unsigned>(rows)), dim3(64), 0, stream, part, mx, sm, splits,
                     per_xcd, static_cast<__bf16*>(out));
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// out: >= grid uint32 words
extern "C" int fdp_xcc_map(uint32_t* out, unsigned grid, hipStream_t stream) {
  if (out == nullptr || grid == 0) return 1;
  hipLaunchKernelGGL(xcc_map_kernel, dim3(grid), dim3(64), 0, stream, out);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
