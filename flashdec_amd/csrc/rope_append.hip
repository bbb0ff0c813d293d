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
// Table mode (cos_sin_table): cos/sin come from the caller's fp32 table, row =
// position; built with the reference's torch expression on the same device,
// the output equals apply_rope there bit for bit (the rotation below is the
// same unfused arithmetic torch's elementwise ops perform).
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
// One workgroup per request (launch-bound at decode batch sizes).  Rows of
// 16-byte vectors take the vector path below, other shapes the scalar one.
#include "fd_common.h"
#include "rope_math.h"

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
  const float* tab;  // optional cos/sin table [2, tab_rows, rotary_dim / 2]
  int64_t tab_rows;
};

// cos/sin of frequency i at position pos: from the caller's table when given,
// else the correctly rounded evaluation
__device__ __forceinline__ void rope_angle(const RopeParams& p, int64_t pos, int i, float& c, float& s) {
  if (p.tab != nullptr)
    rope_table_cos_sin(p.tab, p.tab_rows, p.rotary_dim / 2, pos, i, c, s);
  else
    rope_cos_sin(p.base, p.rotary_dim, pos, i, c, s);
}

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
  for (int i = tid; i < half; i += blockDim.x) {
    // e = -(2i) / R in fp32, as torch evaluates -arange(0, R, 2) / R
    rope_angle(p, pos, i, s_cos[i], s_sin[i]);
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
      float lo, hi;
      rope_rotate(x1, x2, s_cos[i], s_sin[i], lo, hi);
      ob[h * D + i] = from_f32<T>(lo);
      ob[h * D + i + half] = from_f32<T>(hi);
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
    float lo, hi;
    rope_rotate(x1, x2, s_cos[i], s_sin[i], lo, hi);
    T* dst = kc + slot0 + h * hstride;
    dst[i] = from_f32<T>(lo);
    dst[i + half] = from_f32<T>(hi);
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

// ------------------------------------------------------------------------
// Vector path (16-byte rows): every global load of a request is issued at
// the start -- position, slot, and each thread's q/k/v vectors -- so the
// float64 cos/sin evaluation overlaps them, and the only other round trip is
// the final 16-byte stores.  Work items of one request, in order: Q rotation
// pairs (head, vector j of the low half + its partner in the high half), K
// rotation pairs, Q tail vectors, K tail vectors, V vectors.  Needs
// head_dim and rotary_dim / 2 to be multiples of the vector width and
// 16-byte aligned rows (checked on the host).
constexpr int kThreads = 256;
constexpr int kPrefetch = 2;  // work items per thread held in registers across the barrier

template <typename T>
struct VecOps {
  static constexpr int N = 16 / sizeof(T);
  __device__ static void unpack(const u32x4& w, float (&x)[N]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[2 * j] = lo_f32<T>(w[j]);
      x[2 * j + 1] = hi_f32<T>(w[j]);
    }
  }
  __device__ static u32x4 pack(const float (&x)[N]) {
    u32x4 w;
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = pack2<T>(x[2 * j], x[2 * j + 1]);
    return w;
  }
};

template <>
struct VecOps<float> {
  static constexpr int N = 4;
  // Elements go through plain scalars: __builtin_bit_cast applied directly
  // to an ext-vector element subscript (w[j]) compiled to element 0 for every
  // j with this hipcc (seen in the gfx950 assembly), broadcasting lane 0.
  __device__ static void unpack(const u32x4& w, float (&x)[N]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u = w[j];
      x[j] = __builtin_bit_cast(float, u);
    }
  }
  __device__ static u32x4 pack(const float (&x)[N]) {
    u32x4 w;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float f = x[j];
      w[j] = __builtin_bit_cast(uint32_t, f);
    }
    return w;
  }
};

struct ItemPlan {
  int nq, nk, nqt, nkt, nv, total;
  int hv, tv, dv;  // vectors per half, per tail, per row
};

// Addresses of work item `it` (element offsets from the row bases).
template <typename T>
struct Item {
  const T* src0;
  const T* src1;  // rotation partner (high half), else nullptr
  T* dst0;
  T* dst1;
  int freq0;     // first frequency index of a rotation item
  bool to_cache; // K/V item: stored only when the slot is valid
};

// SRC_ONLY: the source rows alone (destinations null), so that the first
// loads need no destination argument.
template <typename T, bool SRC_ONLY = false>
__device__ __forceinline__ Item<T> item_at(const RopeParams& p, const ItemPlan& ip, int b, int it, int64_t slot0) {
  constexpr int N = VecOps<T>::N;
  const int D = p.head_dim, half = p.rotary_dim / 2;
  const int64_t hstride = static_cast<int64_t>(p.block_size) * D;
  const T* qb = static_cast<const T*>(p.q) + static_cast<int64_t>(b) * p.hq * D;
  T* ob = SRC_ONLY ? nullptr : static_cast<T*>(p.q_out) + static_cast<int64_t>(b) * p.hq * D;
  const T* kb = static_cast<const T*>(p.k) + static_cast<int64_t>(b) * p.hkv * D;
  const T* vb = static_cast<const T*>(p.v) + static_cast<int64_t>(b) * p.hkv * D;
  T* kc = SRC_ONLY ? nullptr : static_cast<T*>(p.k_cache) + slot0;
  T* vc = SRC_ONLY ? nullptr : static_cast<T*>(p.v_cache) + slot0;
  Item<T> r{nullptr, nullptr, nullptr, nullptr, 0, false};
  if (it < ip.nq) {
    const int h = it / ip.hv, j = (it % ip.hv) * N;
    r = {qb + h * D + j, qb + h * D + half + j, ob + h * D + j, ob + h * D + half + j, j, false};
  } else if ((it -= ip.nq) < ip.nk) {
    const int h = it / ip.hv, j = (it % ip.hv) * N;
    r = {kb + h * D + j, kb + h * D + half + j, kc + h * hstride + j, kc + h * hstride + half + j, j, true};
  } else if ((it -= ip.nk) < ip.nqt) {
    const int h = it / ip.tv, d = p.rotary_dim + (it % ip.tv) * N;
    r = {qb + h * D + d, nullptr, ob + h * D + d, nullptr, 0, false};
  } else if ((it -= ip.nqt) < ip.nkt) {
    const int h = it / ip.tv, d = p.rotary_dim + (it % ip.tv) * N;
    r = {kb + h * D + d, nullptr, kc + h * hstride + d, nullptr, 0, true};
  } else {
    it -= ip.nkt;
    const int h = it / ip.dv, d = (it % ip.dv) * N;
    r = {vb + h * D + d, nullptr, vc + h * hstride + d, nullptr, 0, true};
  }
  return r;
}

template <typename T>
__device__ __forceinline__ void finish_item(const Item<T>& item, const u32x4& a, const u32x4& bvec, bool write_kv,
                                            const float* s_cos, const float* s_sin) {
  constexpr int N = VecOps<T>::N;
  if (item.to_cache && !write_kv) return;
  if (item.src1 == nullptr) {  // plain copy
    *reinterpret_cast<u32x4*>(item.dst0) = a;
    return;
  }
  float x1[N], x2[N], lo[N], hi[N];
  VecOps<T>::unpack(a, x1);
  VecOps<T>::unpack(bvec, x2);
#pragma unroll
  for (int e = 0; e < N; ++e) {
    rope_rotate(x1[e], x2[e], s_cos[item.freq0 + e], s_sin[item.freq0 + e], lo[e], hi[e]);
  }
  *reinterpret_cast<u32x4*>(item.dst0) = VecOps<T>::pack(lo);
  *reinterpret_cast<u32x4*>(item.dst1) = VecOps<T>::pack(hi);
}

// The leading scalar arguments repeat what the row loads and the work plan
// need (source and q_out rows, sizes); the library is built with
// amdgpu-kernarg-preload-count, so the command processor writes them into
// SGPRs at wave launch and the row loads issue without a kernel-argument
// round trip.
template <typename T>
__global__ __launch_bounds__(kThreads) void rope_append_vec_kernel(const void* q, const void* k, const void* v,
                                                                   void* q_out, int32_t hq, int32_t hkv,
                                                                   int32_t head_dim, int32_t rotary_dim,
                                                                   int32_t idx_i64, RopeParams pa) {
  RopeParams p = pa;
  p.q = q;
  p.k = k;
  p.v = v;
  p.q_out = q_out;
  p.hq = hq;
  p.hkv = hkv;
  p.head_dim = head_dim;
  p.rotary_dim = rotary_dim;
  p.idx_i64 = idx_i64;
  const bool has_q_out = q_out != nullptr;
  constexpr int N = VecOps<T>::N;
  __shared__ float s_cos[kMaxHalf];
  __shared__ float s_sin[kMaxHalf];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int D = p.head_dim, R = p.rotary_dim, half = R / 2;
  ItemPlan ip;
  ip.hv = half / N;
  ip.tv = (D - R) / N;
  ip.dv = D / N;
  ip.nq = has_q_out ? p.hq * ip.hv : 0;
  ip.nk = p.hkv * ip.hv;
  ip.nqt = has_q_out ? p.hq * ip.tv : 0;
  ip.nkt = p.hkv * ip.tv;
  ip.nv = p.hkv * ip.dv;
  ip.total = ip.nq + ip.nk + ip.nqt + ip.nkt + ip.nv;

  // The source rows first: their addresses need only the preloaded
  // arguments (the destination slot is not known yet, and not needed).
  u32x4 ra[kPrefetch], rb[kPrefetch];
#pragma unroll
  for (int k = 0; k < kPrefetch; ++k) {
    const int it = tid + k * kThreads;
    if (it < ip.total) {
      const Item<T> item = item_at<T, true>(p, ip, b, it, 0);
      ra[k] = *reinterpret_cast<const u32x4*>(item.src0);
      if (item.src1 != nullptr) rb[k] = *reinterpret_cast<const u32x4*>(item.src1);
    }
  }
  // then position and slot, as one batch of scalar loads with one wait
  const int64_t pos = load_index(p.positions, b, p.idx_i64);
  const int64_t blk = load_index(p.block_ids, b, p.idx_i64);
  const int64_t off = load_index(p.block_offsets, b, p.idx_i64);
  asm volatile("" ::"s"(pos), "s"(blk), "s"(off), "s"(p.num_blocks), "s"(p.block_size), "s"(p.k_cache),
               "s"(p.v_cache));
  const bool write_kv = blk >= 0 && blk < p.num_blocks && off >= 0 && off < p.block_size;
  // out-of-range slots are never stored; row 0 keeps the addresses in bounds
  const int64_t slot0 = write_kv ? (blk * p.hkv * p.block_size + off) * D : 0;
  for (int i = tid; i < half; i += kThreads) {
    rope_angle(p, pos, i, s_cos[i], s_sin[i]);
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kPrefetch; ++k) {
    const int it = tid + k * kThreads;
    if (it < ip.total) finish_item<T>(item_at<T>(p, ip, b, it, slot0), ra[k], rb[k], write_kv, s_cos, s_sin);
  }
  for (int it = tid + kPrefetch * kThreads; it < ip.total; it += kThreads) {  // very wide rows only
    const Item<T> item = item_at<T>(p, ip, b, it, slot0);
    const u32x4 a = *reinterpret_cast<const u32x4*>(item.src0);
    const u32x4 bv = item.src1 != nullptr ? *reinterpret_cast<const u32x4*>(item.src1) : a;
    finish_item<T>(item, a, bv, write_kv, s_cos, s_sin);
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
    if (a.cos_sin_table != nullptr && (a.table_rows <= 0 || (reinterpret_cast<uintptr_t>(a.cos_sin_table) & 3u)))
      return set_error(FD_E_INVALID, "%s: cos_sin_table needs table_rows > 0 and 4-byte alignment", who);
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
  p.tab = need_rope ? a.cos_sin_table : nullptr;
  p.tab_rows = a.table_rows;
  return FD_OK;
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

template <typename T>
int launch_rope(const fd_rope_append_args& a, const RopeParams& p, hipStream_t stream) {
  constexpr int N = VecOps<T>::N;
  const bool vec = a.head_dim % N == 0 && (a.rotary_dim / 2) % N == 0 && aligned16(a.q) && aligned16(a.k) &&
                   aligned16(a.v) && aligned16(a.k_cache) && aligned16(a.v_cache) &&
                   (a.q_out == nullptr || aligned16(a.q_out));
  if (vec) {
    if (launch_record_on()) record_launch(reinterpret_cast<const void*>(rope_append_vec_kernel<T>), stream);
    hipLaunchKernelGGL((rope_append_vec_kernel<T>), dim3(static_cast<unsigned>(a.batch)), dim3(kThreads), 0, stream,
                       p.q, p.k, p.v, p.q_out, p.hq, p.hkv, p.head_dim, p.rotary_dim, p.idx_i64, p);
  } else {
    if (launch_record_on()) record_launch(reinterpret_cast<const void*>(rope_append_kernel<T>), stream);
    hipLaunchKernelGGL((rope_append_kernel<T>), dim3(static_cast<unsigned>(a.batch)), dim3(256), 0, stream, p);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(FD_E_LAUNCH, "rope append launch failed: %s", hipGetErrorString(e));
  return FD_OK;
}

template <typename T>
int launch_kv(const fd_rope_append_args& a, const RopeParams& p, hipStream_t stream) {
  if (launch_record_on()) record_launch(reinterpret_cast<const void*>(kv_append_kernel<T>), stream);
  hipLaunchKernelGGL((kv_append_kernel<T>), dim3(static_cast<unsigned>(a.batch)), dim3(256), 0, stream, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(FD_E_LAUNCH, "kv append launch failed: %s", hipGetErrorString(e));
  return FD_OK;
}

}  // namespace
}  // namespace fd

using namespace fd;

extern "C" int fd_fused_rope_kv_append(const fd_rope_append_args* args, fd_stream_t stream_) {
  clear_launch_record();
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
  clear_launch_record();
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
