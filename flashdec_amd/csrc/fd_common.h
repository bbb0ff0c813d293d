// Shared helpers for the gfx950 kernels and the C-ABI glue.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/flashdec_hip.h"

namespace fd {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------- errors --
// Thread-local message for fd_last_error(); set by the host-side glue only.
std::string& last_error_slot();
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// -------------------------------------------------------- launch record --
// Off unless fd_record_launches(1): then every launch appends its kernel's
// name to a thread-local record that each public entry point clears first,
// and fd_last_launch() returns it.  Off, a launch pays one relaxed load.
bool launch_record_on();
void clear_launch_record();
void record_launch(const void* kernel, hipStream_t stream);

// ------------------------------------------------------------ conversions --
template <typename T>
__device__ __forceinline__ float to_f32(T x) {
  return static_cast<float>(x);
}

template <typename T>
__device__ __forceinline__ T from_f32(float x) {
  return static_cast<T>(x);  // RNE on gfx950 (v_cvt_pk_bf16_f32 / v_cvt_f16_f32)
}

// bf16 / f16 halves of a packed dword -> f32 (exact)
template <typename T>
__device__ __forceinline__ float lo_f32(uint32_t w);
template <typename T>
__device__ __forceinline__ float hi_f32(uint32_t w);

template <>
__device__ __forceinline__ float lo_f32<__bf16>(uint32_t w) {
  return __builtin_bit_cast(float, w << 16);
}
template <>
__device__ __forceinline__ float hi_f32<__bf16>(uint32_t w) {
  return __builtin_bit_cast(float, w & 0xffff0000u);
}
template <>
__device__ __forceinline__ float lo_f32<_Float16>(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xffffu)));
}
template <>
__device__ __forceinline__ float hi_f32<_Float16>(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
}

// two f32 -> packed 16-bit pair (lo in bits 0..15), RNE
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const uint16_t a = __builtin_bit_cast(uint16_t, from_f32<T>(lo));
  const uint16_t b = __builtin_bit_cast(uint16_t, from_f32<T>(hi));
  return static_cast<uint32_t>(a) | (static_cast<uint32_t>(b) << 16);
}

// -------------------------------------------------------------- indices --
// Branch-free read of an int32 or int64 index: the low 32-bit word of either
// (little endian).  Every index on this path (block ids, lengths, slots,
// positions) lies in int32 range -- a cache with 2^31 blocks or tokens would
// not fit in device memory -- so no information is lost, and a uniform shift
// replaces the per-load branch (and its wait) a dtype switch would compile to.
// The value stays int32 so that nothing (e.g. a sign extension) consumes the
// loaded register before its real use, which would force an early wait.
__device__ __forceinline__ int32_t load_index(const void* base, int64_t elem, int is64) {
  const char* ptr = static_cast<const char*>(base) + (elem << (is64 ? 3 : 2));
  return *reinterpret_cast<const int32_t*>(ptr);
}

// The same read for a wave-uniform index, through the scalar data cache
// (s_load, waited on with lgkmcnt): a vector load here would be followed by
// a vmcnt wait before its readfirstlane, and vmcnt retires in order, so that
// wait would also cover every K/V load issued before it.  Only for data no
// kernel of this launch writes (block tables).
__device__ __forceinline__ int32_t load_index_uniform(const void* base, int64_t elem, int is64) {
  using ConstI32 = const __attribute__((address_space(4))) int32_t;
  const char* ptr = static_cast<const char*>(base) + (elem << (is64 ? 3 : 2));
  return *(ConstI32*)(ptr);
}

// ----------------------------------------------------------- wave utils --
__device__ __forceinline__ float shfl_xor_f32(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

constexpr float kLog2e = 1.4426950408889634f;

}  // namespace fd
