// Fused split-half RoPE + paged K/V append, and the plain K/V scatter.
//
// Reference semantics (cysong2025/flashdec):
//   flashdec/rope.py:26-85              apply_rope: fp32 math, split-half
//                                       rotation, tail dims copied
//   flashdec/csrc/fused_rope_kv_append_kernel.cu:38-82
//                                       Q rotated into q_out; rotated K and raw
//                                       V written to ((blk*Hkv+h)*bs+off)*D+d
//   flashdec/csrc/kv_append_kernel.cu:10-42   K/V scatter only
//
// Bit-exactness: per request, the R/2 angles are formed exactly as
// rope.py:66-68 does in fp32 (e = fp32(-2i / R), angle = fp32(pos) * inv),
// while the two transcendental steps -- inv = base^e and cos/sin(angle) --
// are evaluated in float64 and rounded once to fp32, i.e. the correctly
// rounded values of the reference's fp32 expressions.  The rotation is
// rn(rn(a*c) -/+ rn(b*s)) with FMA contraction disabled, then RNE to the
// element dtype.  The CPU oracle defines the same numbers, so K bytes match
// bit for bit; V is a raw copy.
//
// One workgroup per request (launch-bound at decode batch sizes).
#include "fd_common.h"

#pragma clang fp contract(off)

namespace fd {

struct RopeParams {
  void* q_out;
  const void* q;
  const void* k;
  const void* v;
  void* k_cache;
  void* v_cache;
  const void* block_ids;
  const void* block_offsets;
  const void* positions;
  int idx_i64;
  int hq, hkv, head_dim, block_size, rotary_dim;
  int64_t num_blocks;
  float base;  // fp32(base): the reference's pow runs on an fp32 base
};

constexpr int kMaxHalf = 512;  // rotary_dim <= 1024

template <typename T>
__global__ __launch_bounds__(256) void rope_append_kernel(RopeParams p) {
  __shared__ float s_cos[kMaxHalf];
  __shared__ float s_sin[kMaxHalf];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int D = p.head_dim;
  const int R = p.rotary_dim;
  const int half = R / 2;
  const int64_t pos = load_index(p.positions, b, p.idx_i64);
  const float posf = static_cast<float>(pos);
  for (int i = tid; i < half; i += blockDim.x) {
    // e = -(2i) / R in fp32, as torch evaluates -arange(0, R, 2) / R
    const float e = static_cast<float>(-2 * i) / static_cast<float>(R);
    const float inv = static_cast<float>(pow(static_cast<double>(p.base), static_cast<double>(e)));
    const float ang = posf * inv;
    double sd, cd;
    sincos(static_cast<double>(ang), &sd, &cd);
    s_cos[i] = static_cast<float>(cd);
    s_sin[i] = static_cast<float>(sd);
  }
  __syncthreads();

  const int64_t blk = load_index(p.block_ids, b, p.idx_i64);
  const int64_t off = load_index(p.block_offsets, b, p.idx_i64);
  const bool write_kv = blk >= 0 && blk < p.num_blocks && off >= 0 && off < p.block_size;

  // Q: rotated into q_out
  if (p.q_out != nullptr) {
    const T* qb = static_cast<const T*>(p.q) + static_cast<int64_t>(b) * p.hq * D;
    T* ob = static_cast<T*>(p.q_out) + static_cast<int64_t>(b) * p.hq * D;
    for (int idx = tid; idx < p.hq * half; idx += blockDim.x) {
      const int h = idx / half, i = idx % half;
      const T* row = qb + h * D;
      const float x1 = to_f32(row[i]);
      const float x2 = to_f32(row[i + half]);
      const float c = s_cos[i], s = s_sin[i];
      const float a = x1 * c;
      const float bb = x2 * s;
      const float e = x2 * c;
      const float f = x1 * s;
      ob[h * D + i] = from_f32<T>(a - bb);
      ob[h * D + i + half] = from_f32<T>(e + f);
    }
    const int tail = D - R;
    for (int idx = tid; idx < p.hq * tail; idx += blockDim.x) {
      const int h = idx / tail, d = R + idx % tail;
      ob[h * D + d] = qb[h * D + d];
    }
  }
  if (!write_kv) return;
  // K: rotated into the cache slot; V: raw copy
  const T* kb = static_cast<const T*>(p.k) + static_cast<int64_t>(b) * p.hkv * D;
  const T* vb = static_cast<const T*>(p.v) + static_cast<int64_t>(b) * p.hkv * D;
  T* kc = static_cast<T*>(p.k_cache);
  T* vc = static_cast<T*>(p.v_cache);
  const int64_t hstride = static_cast<int64_t>(p.block_size) * D;
  const int64_t slot0 = (blk * p.hkv * p.block_size + off) * D;  // head 0 row of the slot
  for (int idx = tid; idx < p.hkv * half; idx += blockDim.x) {
    const int h = idx / half, i = idx % half;
    const T* row = kb + h * D;
    const float x1 = to_f32(row[i]);
    const float x2 = to_f32(row[i + half]);
    const float c = s_cos[i], s = s_sin[i];
    const float a = x1 * c;
    const float bb = x2 * s;
    const float e = x2 * c;
    const float f = x1 * s;
    T* dst = kc + slot0 + h * hstride;
    dst[i] = from_f32<T>(a - bb);
    dst[i + half] = from_f32<T>(e + f);
  }
  const int tail = D - R;
  for (int idx = tid; idx < p.hkv * tail; idx += blockDim.x) {
    const int h = idx / tail, d = R + idx % tail;
    kc[slot0 + h * hstride + d] = kb[h * D + d];
  }
  for (int idx = tid; idx < p.hkv * D; idx += blockDim.x) {
    const int h = idx / D, d = idx % D;
    vc[slot0 + h * hstride + d] = vb[h * D + d];
  }
}

// K/V scatter: one workgroup per request, 16-byte copies when rows allow.
template <typename T>
__global__ __launch_bounds__(256) void kv_append_kernel(RopeParams p) {
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int D = p.head_dim;
  const int64_t blk = load_index(p.block_ids, b, p.idx_i64);
  const int64_t off = load_index(p.block_offsets, b, p.idx_i64);
  if (!(blk >= 0 && blk < p.num_blocks && off >= 0 && off < p.block_size)) return;
  const T* kb = static_cast<const T*>(p.k) + static_cast<int64_t>(b) * p.hkv * D;
  const T* vb = static_cast<const T*>(p.v) + static_cast<int64_t>(b) * p.hkv * D;
  T* kc = static_cast<T*>(p.k_cache);
  T* vc = static_cast<T*>(p.v_cache);
  const int64_t hstride = static_cast<int64_t>(p.block_size) * D;
  const int64_t slot0 = (blk * p.hkv * p.block_size + off) * D;
  for (int idx = tid; idx < p.hkv * D; idx += blockDim.x) {
    const int h = idx / D, d = idx % D;
    kc[slot0 + h * hstride + d] = kb[h * D + d];
    vc[slot0 + h * hstride + d] = vb[h * D + d];
  }
}

namespace {

int fill_params(const fd_rope_append_args* args, RopeParams& p, bool need_rope, const char* who) {
  if (args == nullptr) return set_error(FD_E_INVALID, "%s: args is NULL", who);
  const fd_rope_append_args& a = *args;
  if (a.struct_size != sizeof(fd_rope_append_args))
    return set_error(FD_E_INVALID, "%s: struct_size %u != %zu (ABI mismatch)", who, a.struct_size,
                     sizeof(fd_rope_append_args));
  if (a.dtype != FD_DTYPE_F16 && a.dtype != FD_DTYPE_BF16 && a.dtype != FD_DTYPE_F32)
    return set_error(FD_E_UNSUPPORTED, "%s: dtype must be float16, bfloat16 or float32", who);
  if (a.batch < 0 || a.num_kv_heads <= 0 || a.head_dim <= 0 || a.block_size <= 0 || a.num_blocks <= 0)
    return set_error(FD_E_INVALID, "%s: shapes must be positive", who);
  if (a.batch > 0x7fffffffLL) return set_error(FD_E_INVALID, "%s: batch too large", who);
  if (!a.k || !a.v || !a.k_cache || !a.v_cache || !a.block_ids || !a.block_offsets)
    return set_error(FD_E_INVALID, "%s: NULL tensor pointer", who);
  if (need_rope) {
    if (a.num_q_heads <= 0 || !a.positions) return set_error(FD_E_INVALID, "%s: q heads / positions", who);
    if (a.q_out && !a.q) return set_error(FD_E_INVALID, "%s: q_out without q", who);
    if (a.rotary_dim <= 0 || a.rotary_dim > a.head_dim || a.rotary_dim % 2 != 0 || a.rotary_dim / 2 > kMaxHalf)
      return set_error(FD_E_INVALID, "%s: rotary_dim must be positive, even and <= head_dim", who);
    if (!(a.base > 0.0) || a.base > 3.4e38)
      return set_error(FD_E_INVALID, "%s: base must be a positive finite number", who);
  }
  p.q_out = a.q_out;
  p.q = a.q;
  p.k = a.k;
  p.v = a.v;
  p.k_cache = a.k_cache;
  p.v_cache = a.v_cache;
  p.block_ids = a.block_ids;
  p.block_offsets = a.block_offsets;
  p.positions = a.positions;
  p.idx_i64 = a.index_dtype == FD_INDEX_I64;
  p.hq = static_cast<int>(a.num_q_heads);
  p.hkv = static_cast<int>(a.num_kv_heads);
  p.head_dim = static_cast<int>(a.head_dim);
  p.block_size = static_cast<int>(a.block_size);
  p.rotary_dim = static_cast<int>(a.rotary_dim);
  p.num_blocks = a.num_blocks;
  p.base = static_cast<float>(a.base);
  return FD_OK;
}

template <typename T>
int launch_rope(const fd_rope_append_args& a, const RopeParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((rope_append_kernel<T>), dim3(static_cast<unsigned>(a.batch)), dim3(256), 0, stream, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(FD_E_LAUNCH, "rope append launch failed: %s", hipGetErrorString(e));
  return FD_OK;
}

template <typename T>
int launch_kv(const fd_rope_append_args& a, const RopeParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((kv_append_kernel<T>), dim3(static_cast<unsigned>(a.batch)), dim3(256), 0, stream, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(FD_E_LAUNCH, "kv append launch failed: %s", hipGetErrorString(e));
  return FD_OK;
}

}  // namespace
}  // namespace fd

using namespace fd;

extern "C" int fd_fused_rope_kv_append(const fd_rope_append_args* args, fd_stream_t stream_) {
  RopeParams p{};
  int rc = fill_params(args, p, true, "fd_fused_rope_kv_append");
  if (rc != FD_OK) return rc;
  if (args->batch == 0) return FD_OK;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  switch (args->dtype) {
    case FD_DTYPE_BF16: return launch_rope<__bf16>(*args, p, stream);
    case FD_DTYPE_F16: return launch_rope<_Float16>(*args, p, stream);
    default: return launch_rope<float>(*args, p, stream);
  }
}

extern "C" int fd_kv_append(const fd_rope_append_args* args, fd_stream_t stream_) {
  RopeParams p{};
  int rc = fill_params(args, p, false, "fd_kv_append");
  if (rc != FD_OK) return rc;
  if (args->batch == 0) return FD_OK;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  switch (args->dtype) {
    case FD_DTYPE_BF16: return launch_kv<__bf16>(*args, p, stream);
    case FD_DTYPE_F16: return launch_kv<_Float16>(*args, p, stream);
    default: return launch_kv<float>(*args, p, stream);
  }
}
