// Paged single-token decode attention for gfx950 (MI355X).
//
// Work decomposition: one workgroup per (request, KV head, head block of 16
// query heads, KV split).  The split covers a contiguous range of 32-token
// tiles; the waves of the workgroup take its units round-robin, each keeping
// its own online-softmax state for the block's query heads (grouped GQA), and
// the waves are merged in LDS so that one partial (or the final row) leaves
// the workgroup.
//
//  * decode_mfma_kernel  -- token-major caches with unit dim stride (vLLM
//    NHD/HND views too), head_dim 64 or 128, any group size.  QK^T and PV
//    run on v_mfma_f32_16x16x{32,16}_{bf16,f16}; V is transposed in
//    registers.  Also the body of the per-row (balanced) and cascade kernels.
//  * decode_dm_kernel    -- dim-major caches (8/16/32-token blocks): V loads
//    straight into the PV operand, K goes through LDS and comes back
//    transposed (ds_read_b64_tr_b16).
//  * decode_generic_kernel -- any strides; VALU only.
//  * split_reduce_kernel -- LSE merge of the split partials.
//
// Reference semantics followed (cysong2025/flashdec):
//   flashdec/kernels/paged_decode.py:124-327  grouped decode + fused append
//   flashdec/kernels/paged_decode.py:330-543  split stage (uniform tile split,
//                                             append owned by the last tile)
//   flashdec/kernels/paged_decode.py:546-642  LSE merge; zero rows for
//                                             seq_len == 0 / slot < 0
#include <hip/hip_ext.h>

#include <mutex>
#include <type_traits>

#include "fd_common.h"
#include "rope_math.h"

namespace fd {

// Per-wave timeline of the MFMA row kernel and the cascade kernel, in a
// measurement build only (FD_TIMELINE: libflashdec_timeline.so, read by
// bench.py's c2-timeline and c4-timeline workloads; the product library
// compiles none of it).  Lane 0 of each wave writes s_memrealtime (100 MHz)
// at the phase boundaries of decode_role / process_unit into slot
// (workgroup * 8 + wave) * 16 + phase: phases 0-9 as named at the stamps,
// 10-14 the end of the wave's units 0-4 (later units in 14), and in the
// cascade kernel slot 15 the wave's role (1 prefix, 2 tail) instead of a
// time.
#ifdef FD_TIMELINE
constexpr bool kTimeline = true;
constexpr int kTimelineWorkgroups = 8192;
__device__ uint64_t g_timeline[kTimelineWorkgroups * 8 * 16];
#else
constexpr bool kTimeline = false;
#endif

__device__ __forceinline__ void timeline_put([[maybe_unused]] int k, [[maybe_unused]] bool mark,
                                             [[maybe_unused]] uint64_t v) {
#ifdef FD_TIMELINE
  if ((threadIdx.x & 63) == 0 && blockIdx.x < kTimelineWorkgroups)
    g_timeline[(blockIdx.x * 8 + (threadIdx.x >> 6)) * 16 + k] = mark ? v : __builtin_amdgcn_s_memrealtime();
#endif
}

template <int K>
__device__ __forceinline__ void timeline_stamp() {
  timeline_put(K, false, 0);
}

struct DecodeParams {
  const void* q;
  int64_t qs0, qs1, qs2;
  void* k;
  int64_t ks0, ks1, ks2, ks3;
  void* v;
  int64_t vs0, vs1, vs2, vs3;
  const void* bt;
  int64_t bts0, bts1;
  const void* sl;
  int64_t sls;
  void* out;
  int64_t os0, os1, os2;
  float* acc;
  int64_t as0, as1, as2, as3;
  float* mx;
  float* sm;
  int64_t ss0, ss1, ss2;
  uint32_t* counters;  // in-launch merge arrival counters (nullptr: reducer kernel)
  const void* ak;
  int64_t aks0, aks1, aks2;
  const void* av;
  int64_t avs0, avs1, avs2;
  const void* slot;
  int64_t slots;
  int bt_i64, sl_i64, slot_i64, fuse;
  int num_seqs, hq, hkv, group, head_dim, block_size;
  int64_t num_blocks, max_blocks_per_seq;
  int splits;
  int hint_tiles;    // ceil(bound / 32): bound = max_seq_len or the table capacity
  int hint_tps;      // tiles per split
  // workgroup-index divisions by splits and hkv as multiply-high and shifts
  // (fast_div; set for the MFMA row kernel only)
  uint32_t div_splits_m, div_hkv_m;
  int div_shifts;  // bits 0-7 / 8-15: splits' shifts, 16-23 / 24-31: hkv's
  // cascade tail pass: row b attends tokens [tb[b], seq_len); its partials
  // take workspace splits [0, splits), the prefix pass's come after them
  const int32_t* tb;
  int hint_tb;       // guess of tb / 32 for the first unit's early loads
  // balanced splits (> 0): row b gets clamp(ceil(tiles_b / T), 1, splits)
  // splits, T = ceil(total tiles / bal_target); workgroup w takes KV head
  // w % hkv of the batch's (w / hkv)-th split
  int bal_target;
  float scale_log2;  // sm_scale * log2(e): scores live in the base-2 domain
  // fused RoPE (rope_dim 64 or 128, with the fused append): q and append_k
  // arrive unrotated and are rotated at position seq_len - 1
  int rope_dim;
  float rope_base;
  const float* rope_tab;  // optional cos/sin table [2, rope_tab_rows, rope_dim / 2]
  int64_t rope_tab_rows;
};

// Row-level bookkeeping shared by the decode kernels.
struct RowInfo {
  int64_t eff_len;     // tokens attended (0 => zero output row)
  int64_t app_tok;     // token taken from append_k/v (-1: none)
  int64_t slot;        // cache slot receiving the appended token
  int t_begin, t_end;  // 32-token tiles [t_begin, t_end) of this split
};

__device__ __forceinline__ int64_t effective_len(const DecodeParams& p, int64_t seq_len, int64_t slot) {
  bool active = seq_len > 0;
  if (p.fuse) active = active && slot >= 0;
  int64_t eff = active ? seq_len : 0;
  // never walk past the block-table row, whatever seq_lens says
  const int64_t cap = p.max_blocks_per_seq * p.block_size;
  return eff < cap ? eff : cap;
}

// Split s covers tiles [s * tps, (s + 1) * tps) of the row, tps = ceil(T / S),
// T = the row's own 32-token tile count (flashdec/kernels/paged_decode.py:
// 408-411).  The host bound (hint_tiles / hint_tps) never decides the range:
// the MFMA kernel uses it only to guess where its first tile is, so that
// tile's loads can be issued before seq_lens arrives.
// (first_tile > 0: the cascade tail pass, whose rows start after their prefix)
__device__ __forceinline__ void split_tiles(int splits, int split, int64_t eff, int first_tile, int& t0, int& t1) {
  const int total = static_cast<int>((eff + 31) / 32);
  const int span = max(total - first_tile, 0);
  const int tps = (span + splits - 1) / splits;
  t0 = first_tile + split * tps;
  t1 = min(t0 + tps, total);
}

__device__ __forceinline__ void split_range(const DecodeParams& p, int split, int64_t eff, int& t0, int& t1) {
  split_tiles(p.splits, split, eff, 0, t0, t1);
}

__device__ __forceinline__ RowInfo row_info(const DecodeParams& p, int b, int split) {
  RowInfo r;
  const int64_t seq_len = load_index(p.sl, b * p.sls, p.sl_i64);
  r.slot = p.fuse ? load_index(p.slot, b * p.slots, p.slot_i64) : -1;
  r.eff_len = effective_len(p, seq_len, r.slot);
  r.app_tok = (p.fuse && r.eff_len > 0) ? r.eff_len - 1 : -1;
  split_range(p, split, r.eff_len, r.t_begin, r.t_end);
  const int live = static_cast<int>((r.eff_len + 31) / 32);
  r.t_end = min(r.t_end, live);
  return r;
}

// ===================================================== MFMA fast path ====
template <typename T>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c);

template <>
__device__ __forceinline__ f32x4 mfma16x16x32<__bf16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma16x16x32<_Float16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                               __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// 16x16x16 MFMA (k = 16): A rows lane % 16, k = 4 * (lane / 16) + j; the
// D layout is the same as the 16x16x32 product's.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h16x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ f32x4 mfma16x16x16(u32x2 a, u32x2 b, f32x4 c);

template <>
__device__ __forceinline__ f32x4 mfma16x16x16<__bf16>(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                   0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma16x16x16<_Float16>(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h16x4, a), __builtin_bit_cast(h16x4, b), c, 0,
                                               0, 0);
}

// Work unit of one wave: UNIT = 16 or 32 consecutive tokens.  Register
// footprint for one lane (lane = 16*g + c), MT = UNIT / 16 row blocks, head
// dim D = 128 or 64:
//   kf[mt][s]: K row (token UNIT*u + 16*mt + c), dims [32*s + 8*g, +8), s < D/32  (QK A)
//   vf[i]    : V row (token UNIT*u + vrow(g, i)), dims [(D/16)*c, +D/16)  (PV, transposed)
// vrow(g, i) = 4*g + i (i < 4) or 16 + 4*g + (i - 4): the tokens whose scores
// this lane holds after QK (MFMA D layout: rows 4*g + r of each 16-row
// block), so P needs no cross-lane movement.  Four waves of 32-token units
// suit splits of about one unit per wave (their compute runs on four SIMDs
// at once); eight waves of 16-token units stream better on long splits (a
// 16.8 MB read: 4.1 vs 4.8 us) and use the 16x16x16 PV product.
//
// Load addresses depend only on the block table, never on seq_lens: tokens
// past the row's length and rows whose block id is out of range are masked
// in registers at compute time, so the K/V loads of the first unit can be in
// flight before the row length arrives.
// A lane's piece of one V row: D/16 dims (16 bytes at D = 128, 8 at 64)
template <int D>
using VPiece = std::conditional_t<D == 128, u32x4, u32x2>;

template <int UNIT, int D = 128>
struct UnitRegs {
  static_assert(D == 128 || D == 64, "head_dim 128 or 64");
  static constexpr int MT = UNIT / 16;
  static constexpr int VR = UNIT / 4;  // V rows per lane: 4 (UNIT 16) or 8 (UNIT 32)
  static constexpr int KS = D / 32;    // 32-dim pieces of a K row (QK k-steps)
  u32x4 kf[MT][KS];
  VPiece<D> vf[VR];
  uint32_t bmask;  // bit i: V row i lies in a valid physical block
};

__device__ __forceinline__ int vrow(int g, int i) { return i < 4 ? 4 * g + i : 12 + 4 * g + i; }

template <int UNIT>
constexpr int waves_for() {
  return UNIT == 32 ? 4 : 8;
}

// One K/V vector load (16 or 8 bytes).  NT: non-temporal, for K/V that a
// launch reads once (streamed past the caches: a 550 MB read runs at 6.8
// instead of 6.1 TB/s on MI355X); plain loads where rows re-read shared
// blocks.
template <bool NT, typename V = u32x4>
__device__ __forceinline__ V kv_load(const void* a) {
  if constexpr (NT)
    return __builtin_nontemporal_load(reinterpret_cast<const V*>(a));
  else
    return *reinterpret_cast<const V*>(a);
}

// Physical block ids a unit needs (wave-uniform; SCALAR: read through the
// scalar cache); pages are clamped to the table row so the read is in bounds
// whatever the row's length.  A unit spans one block, or UNIT / BS
// consecutive ones (at most four: the dim-major kernel's 32-token units on
// 8-token blocks).
struct UnitPages {
  int32_t a, b, c, d;
};

template <int BS, int UNIT, bool SCALAR = false>
__device__ __forceinline__ UnitPages fetch_pages(const DecodeParams& p, int b, int unit) {
  static_assert(BS >= UNIT / 4, "a unit spans at most four blocks");
  constexpr int kPages = BS < UNIT ? UNIT / BS : 1;
  UnitPages up{0, 0, 0, 0};
  const int64_t row = b * p.bts0;
  const int64_t width = p.max_blocks_per_seq;
  const int64_t first = (static_cast<int64_t>(unit) * UNIT) / BS;
  auto entry = [&](int i) -> int32_t {
    const int64_t pg = first + i < width ? first + i : width - 1;
    const int64_t at = row + pg * p.bts1;
    return SCALAR ? load_index_uniform(p.bt, at, p.bt_i64) : load_index(p.bt, at, p.bt_i64);
  };
  up.a = entry(0);
  if constexpr (kPages >= 2) up.b = entry(1);
  if constexpr (kPages == 4) {
    up.c = entry(2);
    up.d = entry(3);
  }
  return up;
}

template <typename T, int BS, int UNIT, bool NT, int D>
__device__ __forceinline__ void load_unit(const DecodeParams& p, int kvh, int unit, const UnitPages& up, int c,
                                          int g, UnitRegs<UNIT, D>& t) {
  const T* kbase = static_cast<const T*>(p.k);
  const T* vbase = static_cast<const T*>(p.v);
  // tt: token within the unit; its block and the row inside that block
  auto block_of = [&](int tt) -> int32_t { return (BS < UNIT && tt >= BS) ? up.b : up.a; };
  auto row_in_block = [&](int tt) -> int { return (UNIT * unit + tt) % BS; };
  // K rows 16*mt + c.  Rows in invalid blocks read row 0 of the cache (in
  // bounds, value discarded by the score mask).
#pragma unroll
  for (int mt = 0; mt < UnitRegs<UNIT, D>::MT; ++mt) {
    const int tt = 16 * mt + c;
    const int32_t blk = block_of(tt);
    const bool ok = blk >= 0 && blk < p.num_blocks;
    const int64_t off = ok ? blk * p.ks0 + kvh * p.ks1 + row_in_block(tt) * p.ks2 : 0;
    const T* row = kbase + off;
#pragma unroll
    for (int s = 0; s < UnitRegs<UNIT, D>::KS; ++s) t.kf[mt][s] = kv_load<NT>(row + 32 * s + 8 * g);
  }
  // V rows vrow(g, i)
  uint32_t bm = 0;
#pragma unroll
  for (int i = 0; i < UnitRegs<UNIT, D>::VR; ++i) {
    const int tt = vrow(g, i);
    const int32_t blk = block_of(tt);
    const bool ok = blk >= 0 && blk < p.num_blocks;
    const int64_t off = ok ? blk * p.vs0 + kvh * p.vs1 + row_in_block(tt) * p.vs2 : 0;
    bm |= ok ? (1u << i) : 0u;
    t.vf[i] = kv_load<NT, VPiece<D>>(vbase + off + (D / 16) * c);
  }
  t.bmask = bm;
}

// Byte offsets of a lane's K and V rows inside their block (head kvh, the
// row's token slot, the lane's dims).  They are the same for every unit a
// wave takes: units advance by kWaves * UNIT = 128 tokens, a multiple of the
// block size, so (UNIT * unit) % BS depends only on the wave.  The host
// checks that they fit in 32 bits.
template <int UNIT>
struct UnitOffsets {
  uint32_t k[UnitRegs<UNIT>::MT];
  uint32_t v[UnitRegs<UNIT>::VR];
};

template <typename T, int BS, int UNIT, int D>
__device__ __forceinline__ UnitOffsets<UNIT> unit_offsets(const DecodeParams& p, int kvh, int wave, int c, int g) {
  UnitOffsets<UNIT> o;
  const int u0 = UNIT * wave;
#pragma unroll
  for (int mt = 0; mt < UnitRegs<UNIT>::MT; ++mt) {
    const int row = (u0 + 16 * mt + c) % BS;
    o.k[mt] = static_cast<uint32_t>((kvh * p.ks1 + row * p.ks2 + 8 * g) * static_cast<int64_t>(sizeof(T)));
  }
#pragma unroll
  for (int i = 0; i < UnitRegs<UNIT>::VR; ++i) {
    const int row = (u0 + vrow(g, i)) % BS;
    o.v[i] = static_cast<uint32_t>((kvh * p.vs1 + row * p.vs2 + (D / 16) * c) * static_cast<int64_t>(sizeof(T)));
  }
  return o;
}

// load_unit for block sizes of 16 and 32: each 16-token row group of a unit
// lies in one block (a 32-token unit on 16-token blocks: rows < 16 in the
// first, the rest in the second), so a row's address is a uniform block base
// (scalar) plus the lane's fixed 32-bit offset -- no per-unit vector
// address arithmetic.
template <typename T, int BS, int UNIT, bool NT, int D>
__device__ __forceinline__ void load_unit_fixed(const DecodeParams& p, const UnitPages& up,
                                                const UnitOffsets<UNIT>& o, UnitRegs<UNIT, D>& t) {
  static_assert(BS >= 16, "a 16-token row group must lie in one block");
  constexpr bool kTwo = BS < UNIT;
  const bool oka = up.a >= 0 && up.a < p.num_blocks;
  const bool okb = kTwo ? (up.b >= 0 && up.b < p.num_blocks) : oka;
  constexpr int64_t E = sizeof(T);
  const char* ka = static_cast<const char*>(p.k) + (oka ? up.a : 0) * p.ks0 * E;
  const char* va = static_cast<const char*>(p.v) + (oka ? up.a : 0) * p.vs0 * E;
  const char* kb = kTwo ? static_cast<const char*>(p.k) + (okb ? up.b : 0) * p.ks0 * E : ka;
  const char* vb = kTwo ? static_cast<const char*>(p.v) + (okb ? up.b : 0) * p.vs0 * E : va;
#pragma unroll
  for (int mt = 0; mt < UnitRegs<UNIT, D>::MT; ++mt) {
    const char* base = (kTwo && mt == 1) ? kb : ka;
#pragma unroll
    for (int s = 0; s < UnitRegs<UNIT, D>::KS; ++s) t.kf[mt][s] = kv_load<NT>(base + o.k[mt] + 64 * s);
  }
  uint32_t bm = 0;
#pragma unroll
  for (int i = 0; i < UnitRegs<UNIT, D>::VR; ++i) {
    const bool second = kTwo && i >= 4;  // V rows 16 + 4g + (i - 4)
    t.vf[i] = kv_load<NT, VPiece<D>>((second ? vb : va) + o.v[i]);
    bm |= (second ? okb : oka) ? (1u << i) : 0u;
  }
  t.bmask = bm;
}

// ------------------------------------------------- dim-major caches ----
// A dim-major cache ([blocks, KV heads, head_dim, block_size], token stride
// 1) stores a head's block as head_dim rows of block_size tokens.  A 32-token
// unit is read as 16-byte pieces of those rows (eight tokens of one dim), and
// the lane tokens are reordered so that lane 16*g + c scores tokens 8*g + i,
// i < 8 (i = 4*mt + r: row 4*g + r of QK row block mt):
//   K piece i of lane l: dim 16*i + l/4, tokens 8*(l%4) + [0, 8) -- staged
//     through LDS and read back transposed into the QK A operand
//   vf[n] of lane 16*g + c: dim 16*n + c, tokens 8*g + [0, 8) -- already the
//     PV A operand (V^T row 16*n + c, k = the lane's eight tokens); one load
//     instruction reads 16 consecutive dim rows
// (D = 128: K pieces i < 8 and V operands n < 8; D = 64: four of each.)
// A piece lies in one block: quarter q of the unit is in page q (8-token
// blocks), q / 2 (16) or 0 (32).
constexpr int kDmWaves = 4;
constexpr int kDmRowBytes = 64;  // one staged dim row: 32 tokens x 2 bytes

template <int D>
struct DmRegs {
  static constexpr int KS = D / 32;  // QK k-steps
  u32x4 kf[2][KS];                   // raw K pieces, then QK A operands
  u32x4 vf[D / 16];                  // PV A operands
  uint32_t bmask;                    // bit i: token 8*g + i lies in a valid block
};

template <typename T, int BS, bool NT, int D>
__device__ __forceinline__ void load_unit_dm(const DecodeParams& p, int kvh, const UnitPages& up, int lane,
                                             DmRegs<D>& t) {
  constexpr int KS = DmRegs<D>::KS;
  static_assert(BS == 8 || BS == 16 || BS == 32, "dim-major units need 8-, 16- or 32-token blocks");
  constexpr int64_t E = sizeof(T);
  const int q = lane & 3;   // K: the lane's eight-token quarter of the unit
  const int g = lane >> 4;  // V: the lane's eight tokens
  const int c = lane & 15;
  // the block holding quarter x of the unit; invalid ids read block 0
  // (masked at compute time)
  auto page = [&](int x) -> int32_t {
    if constexpr (BS == 32) return up.a;
    else if constexpr (BS == 16) return x < 2 ? up.a : up.b;
    else return x == 0 ? up.a : x == 1 ? up.b : x == 2 ? up.c : up.d;
  };
  auto valid = [&](int32_t blk) { return blk >= 0 && blk < p.num_blocks; };
  const int32_t kpg = page(q);
  const int32_t vpg = page(g);
  const int32_t kblk = valid(kpg) ? kpg : 0;
  const int32_t vblk = valid(vpg) ? vpg : 0;
  const char* kp = static_cast<const char*>(p.k) +
                   (kblk * p.ks0 + kvh * p.ks1 + (lane >> 2) * p.ks3 + (8 * q) % BS) * E;
  const char* vp = static_cast<const char*>(p.v) + (vblk * p.vs0 + kvh * p.vs1 + c * p.vs3 + (8 * g) % BS) * E;
  const int64_t kstep = 16 * p.ks3 * E;
  const int64_t vstep = 16 * p.vs3 * E;
#pragma unroll
  for (int i = 0; i < D / 16; ++i) t.kf[i / KS][i % KS] = kv_load<NT>(kp + i * kstep);
#pragma unroll
  for (int n = 0; n < D / 16; ++n) t.vf[n] = kv_load<NT>(vp + n * vstep);
  t.bmask = valid(vpg) ? 0xffu : 0u;
}

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// The unit's raw K pieces go to the wave's LDS stage (row = dim, 64 bytes
// of tokens) and come back as QK A operands: kf[mt][s] of lane 16*g + c =
// token 8*(c/4) + 4*mt + c%4 (A row c), dims 32*s + 8*g + [0, 8).  One
// ds_read_b64_tr_b16 gives lane c of a 16-lane group element j of the
// 8-byte piece addressed by lane 4*j + c/4, element c%4; so lane c' of the
// group addresses dim row base + c'/4 at tokens 8*(c'%4) + 4*mt + [0, 4).
// A wave's LDS operations run in order, so the stage needs no barrier
// between the writes and the reads, nor before the next unit's writes.
//
// Rows 8r .. 8r+7 with r odd hold each 16-byte piece with its two 8-byte
// halves swapped.  The read of a 16-lane group covers the same 8-byte half of
// every piece in four rows; groups g and g + 1 read rows 8 apart, which without
// the swap sit on the same banks (rows 64 bytes apart, 512 bytes per 8 rows).
// Row 16i + lane/4 is odd-eighth exactly for lanes 32..63; read row
// 8g + c/4 (+4, +32s) for odd g.
template <int D>
__device__ __forceinline__ void stage_k_dm(DmRegs<D>& t, uint8_t* stage, int lane) {
  constexpr int KS = DmRegs<D>::KS;
  lds_u8* st = (lds_u8*)stage;
  const bool swap = lane >= 32;
#pragma unroll
  for (int i = 0; i < D / 16; ++i) {
    const u32x4 k = t.kf[i / KS][i % KS];
    *(lds_u32x4*)(st + (16 * i + (lane >> 2)) * kDmRowBytes + 16 * (lane & 3)) =
        swap ? u32x4{k[2], k[3], k[0], k[1]} : k;
  }
  const int c = lane & 15;
  const int g = lane >> 4;
  lds_u8* rd = st + (8 * g + (c >> 2)) * kDmRowBytes + 16 * (c & 3);
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      lds_u8* a = rd + 32 * s * kDmRowBytes + 8 * (mt ^ (g & 1));
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)a);
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(a + 4 * kDmRowBytes));
      const u32x2 l2 = __builtin_bit_cast(u32x2, lo);
      const u32x2 h2 = __builtin_bit_cast(u32x2, hi);
      t.kf[mt][s] = u32x4{l2[0], l2[1], h2[0], h2[1]};
    }
  }
}

// The appended token's pieces in this lane's operand layout: akf[s] = dims
// [32*s + 8*g, +8) of append_k, avf = dims [(D/16)*c, +D/16) of append_v.
template <int D = 128>
struct AppendRegs {
  u32x4 akf[D / 32];
  VPiece<D> avf;
};

// Fused append: store the newest token's K/V at the request's slot.  Lanes
// c == 0 write the K row (4 x D/32 x 16 B), lanes g == 0 the V row
// (16 x 2D/16 B).
template <typename T, int BS, int D>
__device__ __forceinline__ void store_append(const DecodeParams& p, int kvh, int32_t slot, int c, int g,
                                             const AppendRegs<D>& ar) {
  const int64_t blk = slot / BS, off = slot % BS;
  if (blk >= p.num_blocks) return;
  if (c == 0) {
    T* dst = static_cast<T*>(p.k) + blk * p.ks0 + kvh * p.ks1 + off * p.ks2;
#pragma unroll
    for (int s = 0; s < D / 32; ++s) *reinterpret_cast<u32x4*>(dst + 32 * s + 8 * g) = ar.akf[s];
  }
  if (g == 0) {
    T* dst = static_cast<T*>(p.v) + blk * p.vs0 + kvh * p.vs1 + off * p.vs2;
    *reinterpret_cast<VPiece<D>*>(dst + (D / 16) * c) = ar.avf;
  }
}

// Fused RoPE: rotate this lane's Q^T operand pieces and the appended K row
// in place, at position seq_len - 1 (the row's length counts the appended
// token), with the RoPE kernel's arithmetic (rope_math.h) so the cached K
// bytes and the scores are those of RoPE + append followed by decode.  Piece
// s of a lane holds dims [32*s + 8*g, +8); with half = rope_dim / 2 its
// rotation partner is piece s + half / 32 (rope_dim 64: 0 <-> 1, dims 64-127
// unrotated; 128: 0 <-> 2 and 1 <-> 3).  Lane l evaluates frequency l in
// float64 (or reads it from the caller's cos/sin table), and ds_bpermute
// hands each lane the 8 frequencies of a piece.
template <typename T>
__device__ __forceinline__ void rope_operands(const DecodeParams& p, int32_t seq_len, int lane, int g,
                                              u32x4 (&qf)[4], AppendRegs<128>& ar) {
  const int half = p.rope_dim / 2;  // 32 or 64, checked on the host
  const int64_t pos = seq_len > 0 ? seq_len - 1 : 0;
  float cl, sl;
  if (p.rope_tab != nullptr)
    rope_table_cos_sin(p.rope_tab, p.rope_tab_rows, half, pos, lane < half ? lane : 0, cl, sl);
  else
    rope_cos_sin(p.rope_base, p.rope_dim, pos, lane < half ? lane : 0, cl, sl);
  const int ci = __builtin_bit_cast(int, cl), si = __builtin_bit_cast(int, sl);
  auto rotate = [&](u32x4& lo_w, u32x4& hi_w, const float (&c)[8], const float (&sn)[8]) {
    u32x4 a = lo_w, b = hi_w;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t ua = a[w], ub = b[w];
      float l0, h0, l1, h1;
      rope_rotate(lo_f32<T>(ua), lo_f32<T>(ub), c[2 * w], sn[2 * w], l0, h0);
      rope_rotate(hi_f32<T>(ua), hi_f32<T>(ub), c[2 * w + 1], sn[2 * w + 1], l1, h1);
      a[w] = pack2<T>(l0, l1);
      b[w] = pack2<T>(h0, h1);
    }
    lo_w = a;
    hi_w = b;
  };
  auto piece = [&](int s, int partner) {
    float c[8], sn[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int src = (32 * s + 8 * g + j) * 4;
      c[j] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, ci));
      sn[j] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, si));
    }
    rotate(qf[s], qf[partner], c, sn);
    rotate(ar.akf[s], ar.akf[partner], c, sn);
  };
  if (half == 64) {
    piece(0, 2);
    piece(1, 3);
  } else {
    piece(0, 1);
  }
}

// Online-softmax state of one lane: query head c, dims (D/4)*g + (D/16)*r + n.
template <int D = 128>
struct WaveState {
  f32x4 acc[D / 16];  // acc[n][r]
  float m;            // running max (base-2 domain), uniform over g
  float l;            // partial denominator of this lane's tokens
};

// Reductions over the four lanes c, c + 16, c + 32, c + 48 (one query
// column), every lane receiving the result.  With both operands the same
// value, v_permlane16_swap leaves rows 2k and 2k + 1 of each 32-lane half in
// its two results (and v_permlane32_swap the two halves), so combining the
// pair is the xor-16 (xor-32) butterfly step, with no LDS round trip.
__device__ __forceinline__ float pair_rows16_max(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  return fmaxf(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1));
}
__device__ __forceinline__ float pair_rows32_max(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  return fmaxf(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1));
}
__device__ __forceinline__ float pair_rows16_sum(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ float pair_rows32_sum(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ float column_max(float x) { return pair_rows32_max(pair_rows16_max(x)); }
__device__ __forceinline__ float column_sum(float x) { return pair_rows32_sum(pair_rows16_sum(x)); }

// 2^x on the hardware's v_exp_f32: results below 2^-126 flush to zero, which
// only drops probabilities that small relative to the running maximum.  The
// merges (the wave merge, the split reducer and the in-launch merge) weight
// their partials with it too: the library's exp2f adds a range reduction of
// about five instructions per weight, on the merges' dependent chains (C2
// 7.58 -> 7.51 us per call), for weights that only matter above 2^-126.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// 1 / x on the hardware's v_rcp_f32 (1 ulp), for the softmax denominators of
// the stored rows: the division's correctly rounded sequence is about ten
// dependent instructions ahead of every output store.
__device__ __forceinline__ float rcp_fast(float x) { return __builtin_amdgcn_rcpf(x); }

// w * l rounded on its own (the empty asm keeps it out of any fused
// multiply-add): the terms of a merge's denominator.  Callers form it
// unconditionally and select the result: the compiler does not speculate the
// asm, so under a uniform test it became a branch per term, and the in-launch
// merge spilled its running sums around each one.
__device__ __forceinline__ float merge_term(float w, float l) {
  float t = w * l;
  asm volatile("" : "+v"(t));
  return t;
}

// The sum of 16 terms in the order a DPP row reduction gives its first lane
// (rotations by 8, 4, 2, 1): ((x0+x8)+(x4+x12)) + ((x2+x10)+(x6+x14)) and the
// same over the odd terms, then the two.  The in-launch merge sums its
// per-thread terms this way so that it matches the reducer bit for bit.
__device__ __forceinline__ float tree_sum16(const float (&x)[16]) {
  float a[8], b[4];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = x[i] + x[i + 8];
#pragma unroll
  for (int i = 0; i < 4; ++i) b[i] = a[i] + a[i + 4];
  return (b[0] + b[2]) + (b[1] + b[3]);
}

// Online-softmax step over one unit's scores of a lane (base-2 domain): the
// probabilities pr, and st updated for them.  The reference's kernels move
// the running maximum to every new block maximum and rescale acc and l each
// time (flashdec/kernels/paged_decode.py:293-312).  Here the maximum st.m
// moves only when a column's maximum exceeds it by more than kRescaleSlack:
// the probabilities, taken against st.m, stay below 2^kRescaleSlack (no
// overflow in fp32, the same relative rounding in the cache dtype), and the
// accumulator's multiply runs only on such moves instead of on most units.
// acc and l are always taken against the same st.m, so the partial they
// stand for is the same up to rounding.
constexpr float kRescaleSlack = 8.f;

template <int VR, int D>
__device__ __forceinline__ void softmax_step(const float (&sc)[VR], float (&pr)[VR], WaveState<D>& st) {
  float mx = sc[0];
#pragma unroll
  for (int i = 1; i < VR; ++i) mx = fmaxf(mx, sc[i]);
  mx = column_max(mx);
  // st.m == -inf: -inf + slack is -inf, so the first live unit moves it
  const bool move = mx > st.m + kRescaleSlack;
  const float m_ref = move ? mx : st.m;
  const float m_use = m_ref == -INFINITY ? 0.f : m_ref;
  float psum = 0.f;
#pragma unroll
  for (int i = 0; i < VR; ++i) {
    pr[i] = exp2_fast(sc[i] - m_use);
    psum += pr[i];
  }
  // while st.m is -inf, acc and l are zero: nothing to rescale
  if (__ballot(move && st.m != -INFINITY)) {
    const float alpha = exp2_fast(st.m - m_use);  // 1 where st.m stays
#pragma unroll
    for (int n = 0; n < D / 16; ++n) st.acc[n] *= alpha;
    st.l *= alpha;
  }
  st.l += psum;
  st.m = m_ref;
}

// One unit for NCB 16-column blocks of query rows: mask (row length, invalid
// blocks), splice in the appended token, QK^T, online softmax, PV.  The
// blocks share the unit's K/V registers, its mask and its V^T operands.
// `last` is the last attended token, `first` the first (0: from the row's
// start), `app` the token taken from the append registers (-1: none).  The
// probabilities enter the PV product rounded to the cache dtype, as the
// reference's grouped kernels do (flashdec/kernels/paged_decode.py:308-310);
// the denominator sums them in fp32.  Masking is skipped for units whose
// tokens are all live (wave-uniform test).
template <typename T, bool FUSE, int UNIT, int D, int NCB, bool TL = false>
__device__ __forceinline__ void process_unit(UnitRegs<UNIT, D>& t, const u32x4 (&qf)[NCB][D / 32],
                                             float scale_log2, int tok0, int first, int last, int app,
                                             const AppendRegs<D>& ar, int c, int g, WaveState<D> (&st)[NCB]) {
  constexpr int MT = UnitRegs<UNIT, D>::MT;
  constexpr int VR = UnitRegs<UNIT, D>::VR;
  constexpr int KS = UnitRegs<UNIT, D>::KS;
  constexpr int NW = D / 32;  // 32-bit words of a lane's V piece
  constexpr int NTILE = D / 16;  // PV output tiles (16 dims each)
  constexpr uint32_t kAll = (1u << VR) - 1u;
  uint32_t vmask = t.bmask;
#pragma unroll
  for (int i = 0; i < VR; ++i) {
    const int tok = tok0 + vrow(g, i);
    vmask &= (tok <= last && (first == 0 || tok >= first)) ? ~0u : ~(1u << i);
  }
  if constexpr (FUSE) {
    const int at = app - tok0;  // in [0, UNIT) only for the unit holding it
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const bool hit = at == 16 * mt + c;
#pragma unroll
      for (int s = 0; s < KS; ++s) t.kf[mt][s] = hit ? ar.akf[s] : t.kf[mt][s];
    }
#pragma unroll
    for (int i = 0; i < VR; ++i) {
      const bool hit = at == vrow(g, i);
      t.vf[i] = hit ? ar.avf : t.vf[i];
      vmask |= hit ? (1u << i) : 0u;
    }
  }
  // S^T[token][head] = K . Q^T  (MT 16-token row blocks)
  float sc[NCB][VR];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f32x4 sb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) sb = mfma16x16x32<T>(t.kf[mt][s], qf[cb][s], sb);
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[cb][4 * mt + r] = sb[r] * scale_log2;
    }
  if constexpr (TL) {
    asm volatile("" ::"v"(sc[0][0]), "v"(sc[0][VR - 1]));
    timeline_stamp<3>();  // K landed, QK done
  }
  // masked tokens: -inf scores and zero V rows (their memory may hold
  // NaN/Inf, and 0 * NaN is NaN)
  if (__ballot(vmask != kAll)) {
#pragma unroll
    for (int i = 0; i < VR; ++i) {
      const bool keep = (vmask >> i) & 1u;
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) sc[cb][i] = keep ? sc[cb][i] : -INFINITY;
#pragma unroll
      for (int k = 0; k < NW; ++k) t.vf[i][k] = keep ? t.vf[i][k] : 0u;
    }
  }
  // P^T operands (k = VR*g + i: this lane's tokens)
  uint32_t ph[NCB][VR / 2];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    float pr[VR];
    softmax_step<VR, D>(sc[cb], pr, st[cb]);
#pragma unroll
    for (int j = 0; j < VR / 2; ++j) ph[cb][j] = pack2<T>(pr[2 * j], pr[2 * j + 1]);
  }
  if constexpr (TL) {
    asm volatile("" ::"v"(ph[0][0]));
    timeline_stamp<4>();  // softmax done
  }
  // V^T operands: vt_n holds dim (D/16)*c + n of the lane's tokens
#pragma unroll
  for (int n = 0; n < NTILE; ++n) {
    const int w = n >> 1;
    const uint32_t sel = (n & 1) ? 0x07060302u : 0x05040100u;
    if constexpr (UNIT == 32) {
      u32x4 vt;
#pragma unroll
      for (int j = 0; j < 4; ++j) vt[j] = __builtin_amdgcn_perm(t.vf[2 * j + 1][w], t.vf[2 * j][w], sel);
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        u32x4 pp;
#pragma unroll
        for (int j = 0; j < 4; ++j) pp[j] = ph[cb][j];
        st[cb].acc[n] = mfma16x16x32<T>(vt, pp, st[cb].acc[n]);
      }
    } else {
      u32x2 vt;
#pragma unroll
      for (int j = 0; j < 2; ++j) vt[j] = __builtin_amdgcn_perm(t.vf[2 * j + 1][w], t.vf[2 * j][w], sel);
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        u32x2 pp;
#pragma unroll
        for (int j = 0; j < 2; ++j) pp[j] = ph[cb][j];
        st[cb].acc[n] = mfma16x16x16<T>(vt, pp, st[cb].acc[n]);
      }
    }
  }
}

// Fused append into a dim-major cache: this lane's elements of the new
// token in load_unit_dm's layout -- kd(i) = append_k dim 16*i + lane/4 (its K
// pieces), vd(n) = append_v dim 16*n + c (its V operands), two per register.
template <int D>
struct DmAppendRegs {
  uint32_t k[D / 32];  // element i in bits 16*(i%2) of word i/2
  uint32_t v[D / 32];
  __device__ __forceinline__ uint16_t kd(int i) const { return static_cast<uint16_t>(k[i >> 1] >> (16 * (i & 1))); }
  __device__ __forceinline__ uint16_t vd(int n) const { return static_cast<uint16_t>(v[n >> 1] >> (16 * (n & 1))); }
};

template <typename T, int D>
__device__ __forceinline__ void load_append_dm(const DecodeParams& p, int b, int kvh, int lane,
                                               DmAppendRegs<D>& ar) {
  const uint16_t* ak = static_cast<const uint16_t*>(p.ak) + b * p.aks0 + kvh * p.aks1;
  const uint16_t* av = static_cast<const uint16_t*>(p.av) + b * p.avs0 + kvh * p.avs1;
#pragma unroll
  for (int j = 0; j < D / 32; ++j) {
    const int kd = 32 * j + (lane >> 2), vd = 32 * j + (lane & 15);
    ar.k[j] = ak[kd * p.aks2] | (static_cast<uint32_t>(ak[(kd + 16) * p.aks2]) << 16);
    ar.v[j] = av[vd * p.avs2] | (static_cast<uint32_t>(av[(vd + 16) * p.avs2]) << 16);
  }
}

// The new token's K/V go to slot (block, offset) of the dim-major cache: one
// element per dim row.  Lanes with lane % 4 == 0 hold every K dim once, lanes
// with g == 0 every V dim.
template <typename T, int BS, int D>
__device__ __forceinline__ void store_append_dm(const DecodeParams& p, int kvh, int32_t slot, int lane,
                                                const DmAppendRegs<D>& ar) {
  const int64_t blk = slot / BS, off = slot % BS;
  if (blk >= p.num_blocks) return;
  if ((lane & 3) == 0) {
    uint16_t* dst = static_cast<uint16_t*>(p.k) + blk * p.ks0 + kvh * p.ks1 + off * p.ks2;
#pragma unroll
    for (int i = 0; i < D / 16; ++i) dst[(16 * i + (lane >> 2)) * p.ks3] = ar.kd(i);
  }
  if ((lane >> 4) == 0) {
    uint16_t* dst = static_cast<uint16_t*>(p.v) + blk * p.vs0 + kvh * p.vs1 + off * p.vs2;
#pragma unroll
    for (int n = 0; n < D / 16; ++n) dst[(16 * n + lane) * p.vs3] = ar.vd(n);
  }
}

// Element e (a token of the lane's eight) of a 16-byte piece replaced by x.
__device__ __forceinline__ void set_elem16(u32x4& piece, int e, uint16_t x) {
  const int sh = (e & 1) * 16;
  const uint32_t keep = ~(0xffffu << sh);
#pragma unroll
  for (int w = 0; w < 4; ++w)
    piece[w] = (w == (e >> 1)) ? ((piece[w] & keep) | (static_cast<uint32_t>(x) << sh)) : piece[w];
}

// process_unit for a dim-major unit (load_unit_dm's layout): the lane's
// scores and V columns are tokens 8*g + i, and V needs no transposes.
template <typename T, bool FUSE, int D>
__device__ __forceinline__ void process_unit_dm(DmRegs<D>& t, const u32x4 (&qf)[D / 32], float scale_log2,
                                                int tok0, int first, int last, int app,
                                                const DmAppendRegs<D>& ar, int lane, uint8_t* stage,
                                                WaveState<D>& st) {
  constexpr int KS = DmRegs<D>::KS;
  constexpr int NTILE = D / 16;
  const int g = lane >> 4;
  uint32_t vmask = t.bmask;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int tok = tok0 + 8 * g + i;
    vmask &= (tok <= last && (first == 0 || tok >= first)) ? ~0u : ~(1u << i);
  }
  if constexpr (FUSE) {
    // the new token comes from registers: token at = 8*qa + e of this unit
    const int at = app - tok0;
    if (at >= 0 && at < 32) {
      const int qa = at >> 3, e = at & 7;
      if ((lane & 3) == qa) {
#pragma unroll
        for (int i = 0; i < D / 16; ++i) set_elem16(t.kf[i / KS][i % KS], e, ar.kd(i));
      }
      if (g == qa) {
#pragma unroll
        for (int n = 0; n < NTILE; ++n) set_elem16(t.vf[n], e, ar.vd(n));
        vmask |= 1u << e;
      }
    }
  }
  stage_k_dm<D>(t, stage, lane);
  float sc[8];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    f32x4 sb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) sb = mfma16x16x32<T>(t.kf[mt][s], qf[s], sb);
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[4 * mt + r] = sb[r] * scale_log2;
  }
  // masked tokens: -inf scores and zeroed V elements (word w of every V
  // operand holds tokens 2w and 2w + 1)
  if (__ballot(vmask != 0xffu)) {
    uint32_t keep[4];
#pragma unroll
    for (int w = 0; w < 4; ++w)
      keep[w] = (((vmask >> (2 * w)) & 1u) ? 0x0000ffffu : 0u) | (((vmask >> (2 * w + 1)) & 1u) ? 0xffff0000u : 0u);
#pragma unroll
    for (int i = 0; i < 8; ++i) sc[i] = ((vmask >> i) & 1u) ? sc[i] : -INFINITY;
#pragma unroll
    for (int n = 0; n < NTILE; ++n)
#pragma unroll
      for (int w = 0; w < 4; ++w) t.vf[n][w] &= keep[w];
  }
  float pr[8];
  softmax_step<8, D>(sc, pr, st);
  u32x4 pp;
#pragma unroll
  for (int j = 0; j < 4; ++j) pp[j] = pack2<T>(pr[2 * j], pr[2 * j + 1]);
#pragma unroll
  for (int n = 0; n < NTILE; ++n) st.acc[n] = mfma16x16x32<T>(t.vf[n], pp, st.acc[n]);
}

constexpr int kMaxWaves = 8;          // waves per workgroup of the 16-token variant
constexpr int kWideUnitMaxTiles = 4;  // splits of at most this many tiles take 32-token units
// Floats per head row of the LDS merge slots (16-byte pieces, written and
// merged with 128-bit LDS accesses), and where a head's dims sit in its row:
// the 16-byte piece of dims [d, d + 4) starts at float acc_spread<D>() * d.
// Measured on MI355X (SQ_LDS_BANK_CONFLICT of a one-wave probe): a
// ds_write_b128 is conflict-free when each 8 consecutive lanes cover the 32
// banks once; a ds_read_b128 where each 16 lanes read 16 bytes at a 32-byte
// stride from rows 528 bytes apart is conflict-free, while 16 lanes reading
// 256 contiguous bytes from such rows is not.  So the rows are 132 floats
// apart, and head_dim-64 rows keep their pieces 32 bytes apart as head_dim
// 128's are (the merge then reads them with the same pattern).
template <int D>
constexpr int acc_pitch() {
  return 132;
}
template <int D>
constexpr int acc_spread() {
  return D == 64 ? 2 : 1;
}
// Prefix role of the cascade: up to this many 16-row MFMA column blocks per
// wave (a launch's chunk_rows / 16).  Each block is another 16 of the group's
// (member, head) rows attending the same K/V registers, so the group's
// prefix is read once per chunk instead of once per 16 rows.
constexpr int kPrefixMaxColBlocks = FD_CASCADE_MAX_CHUNK_ROWS / 16;
// Row role: groups of more than 16 query heads per KV head run this many
// 16-column blocks per wave (32 heads per workgroup on one read of the K/V,
// instead of one workgroup per 16 heads each reading it).
constexpr int kRowWideColBlocks = 2;
constexpr int kMergeChunk = 16;  // splits whose partials one merge pass loads at once
constexpr int64_t kMaxSplitTiles = 64;  // split planning: tiles of the longest row per split
// One arrival counter per 256-byte line: counters sharing a line serialise
// every workgroup's atomic on that line (measured ~3x slower arrival).
constexpr int kCounterStride = FD_SPLIT_COUNTER_STRIDE;

// An output row's eight elements.  ``out`` may be any strided view (the
// reference indexes it through its strides), so with unit dim stride the
// 16-byte store can be unaligned: gfx9+ global memory runs in the
// unaligned-access mode, which splits such a store in hardware (checked on
// views one element past an aligned base in tests/test_unaligned_views_gpu.py;
// the split partials' 16-byte stores below take caller workspaces the same way).
// N: the first 4 or all 8 elements of o.
template <typename T, int N = 8>
__device__ __forceinline__ void store_row(const DecodeParams& p, int b, int qh, int d0, const float (&o)[8],
                                          float inv) {
  static_assert(N == 4 || N == 8, "4 or 8 elements");
  T* dst = static_cast<T*>(p.out) + b * p.os0 + qh * p.os1 + d0 * p.os2;
  if (p.os2 == 1) {
    if constexpr (N == 8) {
      u32x4 w;
      w[0] = pack2<T>(o[0] * inv, o[1] * inv);
      w[1] = pack2<T>(o[2] * inv, o[3] * inv);
      w[2] = pack2<T>(o[4] * inv, o[5] * inv);
      w[3] = pack2<T>(o[6] * inv, o[7] * inv);
      *reinterpret_cast<u32x4*>(dst) = w;
    } else {
      u32x2 w;
      w[0] = pack2<T>(o[0] * inv, o[1] * inv);
      w[1] = pack2<T>(o[2] * inv, o[3] * inv);
      *reinterpret_cast<u32x2*>(dst) = w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) dst[j * p.os2] = from_f32<T>(o[j] * inv);
  }
}

// Shared-prefix (cascade) launch: groups of rows share the first
// prefix_len[g] tokens of their block tables (the same physical blocks).
// The prefix role attends a group's prefix once per 16 of its (member,
// head) rows -- MFMA column c is row 16 * chunk + c of the group: member
// (16 * chunk + c) / group, head (16 * chunk + c) % group -- reading the
// block ids from the lead member's table row, and writes its partials after
// the tail splits.  The tail role attends each row's tokens from
// row_prefix_len[b] on.
struct CascadeParams {
  const int32_t* members;     // [groups, max_members]; entry 0 is the lead
  const int32_t* prefix_len;  // [groups], tokens
  int max_members;
  int chunks;         // chunks of NCB * 16 rows per group and KV head
  int prefix_splits;  // a group's prefix tiles are spread evenly over them
  int prefix_blocks;  // workgroups of the prefix role: groups * hkv * chunks * prefix_splits
  int hint_ptps;      // guess of the prefix tiles per split (longest prefix)
};

enum class Role { kRow, kTail, kPrefix, kBalanced };

__device__ __forceinline__ int wave_sum_i32(int x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

__device__ __forceinline__ int wave_inclusive_scan_i32(int x, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    x += lane >= o ? y : 0;
  }
  return x;
}

// Balanced splits: tiles per split T for the whole batch, from every row's
// effective length (one wave; the result is the same in every lane).
__device__ __forceinline__ int balanced_tiles_per_split(const DecodeParams& p, int lane) {
  int total = 0;
  for (int r0 = 0; r0 < p.num_seqs; r0 += 64) {
    const int r = r0 + lane;
    int t = 0;
    if (r < p.num_seqs) t = static_cast<int>((effective_len(p, load_index(p.sl, r * p.sls, p.sl_i64), -1) + 31) / 32);
    total += wave_sum_i32(t);
  }
  return max(1, (total + p.bal_target - 1) / p.bal_target);
}

__device__ __forceinline__ int balanced_splits(const DecodeParams& p, int64_t eff, int tps) {
  return min(max(1, static_cast<int>((eff + 31) / 32 + tps - 1) / tps), p.splits);
}

// Wave 0 of a balanced-split workgroup: which row and split the batch's v-th
// split is (prefix sums of the rows' split counts), that row's split count and
// effective length; row -1 when v is past the batch's last split.
__device__ __forceinline__ void balanced_locate(const DecodeParams& p, int v, int lane, int* out) {
  const int tps = balanced_tiles_per_split(p, lane);
  int base = 0;
  int fb = -1, fs = 0, fn = 1, fe = 0;
  for (int r0 = 0; r0 < p.num_seqs; r0 += 64) {
    const int r = r0 + lane;
    int e = 0, n = 0;
    if (r < p.num_seqs) {
      e = static_cast<int>(effective_len(p, load_index(p.sl, r * p.sls, p.sl_i64), -1));
      n = balanced_splits(p, e, tps);
    }
    const int incl = wave_inclusive_scan_i32(n, lane);
    const bool hit = r < p.num_seqs && v >= base + incl - n && v < base + incl;
    const uint64_t m = __ballot(hit);
    if (m) {
      const int l = __builtin_ctzll(m);
      fb = r0 + l;
      fn = __builtin_amdgcn_readlane(n, l);
      fs = v - base - (__builtin_amdgcn_readlane(incl, l) - fn);
      fe = __builtin_amdgcn_readlane(e, l);
      break;
    }
    base += __builtin_amdgcn_readlane(incl, 63);
  }
  if (lane == 0) {
    out[0] = fb;
    out[1] = fs;
    out[2] = fn;
    out[3] = fe;
  }
}

// LDS of one decode workgroup: each wave's state for the merge, and the
// output row of every MFMA column.
template <int W, int P = acc_pitch<128>()>
struct alignas(16) DecodeLds {
  float acc[W][16][P];  // 16-byte rows: merged with 128-bit LDS reads
  float m[W][16];
  float l[W][16];
  int col_b[16];
  int col_h[16];
  int located[4];  // balanced splits: row, split, row's split count, effective length
  int last;
};

// The hardware dispatches consecutive workgroup ids round-robin over the
// XCDs (8 on MI355X, each with its own L2).  With per_xcd = grid / 8 (a grid
// of a multiple of 8 workgroups), the i-th workgroup on XCD x takes logical
// index x * per_xcd + i, so each run of per_xcd consecutive logical
// workgroups shares one XCD; per_xcd 0 keeps the hardware order.
__device__ __forceinline__ int xcd_logical_block(int block, int per_xcd) {
  return per_xcd > 0 ? (block & 7) * per_xcd + (block >> 3) : block;
}

// n / d for n < 2^31 from the divisor's multiplier m and shifts s1, s2
// (Granlund and Montgomery, "Division by invariant integers using
// multiplication", 1994, Figure 4.1; the host computes them in
// fast_div_magic): five scalar instructions instead of the compiler's
// reciprocal-based sequence of about twenty-five, which sat ahead of the
// block-table load.
__device__ __forceinline__ uint32_t fast_div(uint32_t n, uint32_t m, int s1, int s2) {
  const uint32_t t = __umulhi(n, m);
  return (t + ((n - t) >> s1)) >> s2;
}

// The XCD this wave runs on (hardware register XCC_ID, bits 3:0).
__device__ __forceinline__ uint32_t xcc_id() {
  uint32_t x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return x & 0xfu;
}

// DM: dim-major cache (load_unit_dm), staged through the LDS at kstage.
// PRE: the block-table arguments arrived preloaded in SGPRs (decode_mfma_kernel).
// NCB: 16-row column blocks per wave (prefix role only)
template <typename T, int BS, int FUSE, bool MERGE, int UNIT, Role ROLE, bool NT, int D = 128,
          int WAVES = waves_for<UNIT>(), bool DM = false, bool PRE = false, int NCB = 1>
__device__ __forceinline__ void decode_role(const DecodeParams& p, const CascadeParams& cp, int block,
                                            DecodeLds<WAVES, acc_pitch<D>()>& lds,
                                            [[maybe_unused]] uint8_t* kstage = nullptr) {
  static_assert(ROLE == Role::kRow || !(FUSE || MERGE),
                "cascade and balanced roles have no fused append or in-launch merge");
  static_assert(D == 128 || (ROLE == Role::kRow && FUSE != 2 && !MERGE),
                "head_dim 64 runs the row role without RoPE or in-launch merge");
  static_assert(!DM || (ROLE == Role::kRow && FUSE != 2 && !MERGE && UNIT == 32),
                "dim-major caches run the row role on 32-token units");
  static_assert(NCB == 1 || (ROLE == Role::kPrefix && NCB <= kPrefixMaxColBlocks) ||
                    (ROLE == Role::kRow && NCB == kRowWideColBlocks && FUSE != 2 && !MERGE && !DM),
                "several column blocks per wave: the prefix role, and the row role's wide groups");
  constexpr int KS = D / 32;  // 32-dim pieces of q / K rows
  constexpr int kWaves = WAVES;
  constexpr int kUnitsPerTile = 32 / UNIT;
  constexpr bool PREFIX = ROLE == Role::kPrefix;
  constexpr bool TAIL = ROLE == Role::kTail;
  constexpr bool BAL = ROLE == Role::kBalanced;
  constexpr bool ROPE = FUSE == 2;  // fused append with RoPE of q and the appended K
  // Block ids come through the scalar cache (s_load, lgkmcnt) except in the
  // kernels that stream K/V with non-temporal loads.  A vector read of the
  // id needs a vmcnt wait before its readfirstlane, and vmcnt retires in
  // order, so that wait also covers the next unit's K/V loads issued just
  // before it: each unit then waits out the next one's loads.  Kernels whose
  // K/V reads hit the caches gain from keeping them in flight (64 rows on a
  // 16384-token shared prefix: 41.9 -> 39.5 us per call; dim-major D128
  // 28.0 -> 27.0 us); the streaming kernels, already at the HBM rate,
  // measured slower with more loads in flight (36-layer B64 ctx8192 step
  // 3.14 -> 3.21 ms) and keep the vector read.
  constexpr bool kScalarPages = !(NT && ROLE != Role::kPrefix) || DM;
  if constexpr (ROLE == Role::kRow && UNIT == 32 && !PRE) {
    // Short splits (about one unit per wave) spend most of their time before
    // the first K/V loads.  Every argument those loads need goes into SGPRs
    // first: one batch of kernel-argument loads and one wait (left alone the
    // compiler fetched them in three dependent batches).
    asm volatile("" ::"s"(p.q), "s"(p.qs0), "s"(p.qs1), "s"(p.k), "s"(p.ks0), "s"(p.ks1), "s"(p.ks2), "s"(p.v),
                 "s"(p.vs0), "s"(p.vs1), "s"(p.vs2), "s"(p.bt), "s"(p.bts0), "s"(p.bts1), "s"(p.bt_i64), "s"(p.sl),
                 "s"(p.sls), "s"(p.sl_i64), "s"(p.splits), "s"(p.hkv), "s"(p.group), "s"(p.hint_tps),
                 "s"(p.max_blocks_per_seq), "s"(p.num_blocks), "s"(p.block_size));
  }

  constexpr bool TL = kTimeline && ((ROLE == Role::kRow && PRE && !DM) || PREFIX || TAIL);
  if constexpr (TL) {
    timeline_stamp<0>();  // wave start
    if constexpr (PREFIX || TAIL) timeline_put(15, true, PREFIX ? 1 : 2);
  }
  [[maybe_unused]] int tl_units = 0;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;
  int nsplit = PREFIX ? cp.prefix_splits : p.splits;
  // (request, KV head[, head block]), or (group, KV head, chunk)
  const int pair = PRE && ROLE == Role::kRow
                       ? static_cast<int>(fast_div(block, p.div_splits_m, p.div_shifts & 0xff, (p.div_shifts >> 8) & 0xff))
                       : block / nsplit;
  int split = block - pair * nsplit;
  const int G = p.group;
  // Row role: more than 16 query heads per KV head take ceil(G / (16 NCB))
  // head blocks of NCB 16-column blocks, one per workgroup (each reads the
  // K/V again).
  const int hblocks =
      ROLE == Role::kRow ? static_cast<int>(static_cast<unsigned>(G + 16 * NCB - 1) / (16u * NCB)) : 1;
  int b, kvh, chunk = 0, hb = 0;
  [[maybe_unused]] int grp = 0;  // the prefix role's group
  const int32_t* mem = nullptr;
  int64_t bal_eff = 0;
  if constexpr (BAL) {
    kvh = block % p.hkv;
    if (wave == 0) balanced_locate(p, block / p.hkv, lane, lds.located);
    __syncthreads();
    b = lds.located[0];
    if (b < 0) return;  // past the batch's last split: no work (every thread leaves here)
    split = lds.located[1];
    nsplit = lds.located[2];
    bal_eff = lds.located[3];
  } else if constexpr (PREFIX) {
    chunk = pair % cp.chunks;
    const int gk = pair / cp.chunks;
    kvh = gk % p.hkv;
    grp = gk / p.hkv;
    mem = cp.members + static_cast<int64_t>(grp) * cp.max_members;
    b = mem[0];  // the lead: its table row holds the prefix's block ids
  } else if constexpr (PRE && ROLE == Role::kRow) {
    // multiply-high divisions (the split was taken the same way above)
    const int pk = hblocks == 1 ? pair : pair / hblocks;
    hb = pair - pk * hblocks;
    b = static_cast<int>(fast_div(pk, p.div_hkv_m, (p.div_shifts >> 16) & 0xff, p.div_shifts >> 24));
    kvh = pk - b * p.hkv;
  } else {
    const int pk = pair / hblocks;
    hb = pair - pk * hblocks;
    b = pk / p.hkv;
    kvh = pk % p.hkv;
  }
  const bool lead_ok = !PREFIX || (b >= 0 && b < p.num_seqs);
  const int trow = lead_ok ? b : 0;  // table row read for K/V

  // column c of column block cb: the request's head kvh * G + 16 * (NCB * hb
  // + cb) + c (below G), or in the prefix role the group row 16 * (NCB *
  // chunk + cb) + c (member index, head)
  int col_b[NCB], col_h[NCB];
  bool col_ok[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    col_b[cb] = b;
    col_h[cb] = 16 * (NCB * hb + cb) + c;
    col_ok[cb] = col_h[cb] < G;
    if constexpr (PREFIX) {
      const int r = 16 * (NCB * chunk + cb) + c;
      const int mi = r / G;
      const int32_t m = mi < cp.max_members ? mem[mi] : -1;
      col_ok[cb] = lead_ok && m >= 0 && m < p.num_seqs;
      col_b[cb] = col_ok[cb] ? m : 0;
      col_h[cb] = r % G;
    }
  }

  // Independent loads first.  The first unit is guessed from the host bound
  // (hint tiles per split), so its block ids and K/V rows, the Q^T operand,
  // the append row and the row length / slot are all in flight together --
  // no load address depends on seq_lens.  The guess is checked below.
  int guess_begin = PREFIX ? split * cp.hint_ptps : (TAIL ? p.hint_tb : 0) + split * p.hint_tps;  // tiles
  if constexpr (BAL) {
    // the row's length is known: the first unit is not a guess
    int t1;
    split_tiles(nsplit, split, bal_eff, 0, guess_begin, t1);
  }
  int unit = kUnitsPerTile * guess_begin + wave;
  UnitPages pages = fetch_pages<BS, UNIT, kScalarPages>(p, trow, unit);  // clamped, always in bounds
  if constexpr (TL) {
    asm volatile("" ::"s"(pages.a));
    timeline_stamp<1>();  // block-table entry arrived
  }
  if constexpr (PREFIX) {
    // the prefix role's member loads needed only preloaded arguments; the
    // table, q and K/V addressing ones come in one batch of kernel-argument
    // loads, in flight together with them
    asm volatile("" ::"s"(p.bt), "s"(p.bts0), "s"(p.bts1), "s"(p.bt_i64), "s"(p.k), "s"(p.ks0), "s"(p.ks1),
                 "s"(p.ks2), "s"(p.v), "s"(p.vs0), "s"(p.vs1), "s"(p.vs2), "s"(p.num_blocks), "s"(p.q), "s"(p.qs0),
                 "s"(p.qs1), "s"(p.group), "s"(p.block_size), "s"(p.max_blocks_per_seq), "s"(cp.prefix_len));
  }
  if constexpr (ROLE == Role::kRow && UNIT == 32 && PRE) {
    // The table load above needed only preloaded arguments.  The K/V and q
    // addressing arguments come in one batch of kernel-argument loads, in
    // flight together with it.
    asm volatile("" ::"s"(p.q), "s"(p.qs0), "s"(p.qs1), "s"(p.k), "s"(p.ks0), "s"(p.ks1), "s"(p.ks2), "s"(p.v),
                 "s"(p.vs0), "s"(p.vs1), "s"(p.vs2), "s"(p.sl), "s"(p.sls), "s"(p.sl_i64), "s"(p.num_blocks),
                 "s"(p.block_size));
  }
  u32x4 qf[NCB][KS];
  // The cascade roles' waves all take the same NCB * 16 query rows.  Each of
  // the first NCB * KS waves loads one 32-dim piece of them (the piece its
  // lanes' columns need, at the same lane), the pieces meet in LDS after the
  // first unit's K/V loads have issued, and every wave reads its operand
  // there: one load of the rows per workgroup instead of one per wave (C4
  // shared prefix 11.70 -> 11.64 us, 64 x 16384 35.4 -> 34.6 us).  The row
  // kernel keeps a load per wave: there the barrier holds every wave back
  // until the slowest has issued its K/V loads (C2 7.45 -> 7.51 us).
  constexpr bool kShareQ = (PREFIX || TAIL) && NCB * KS <= kWaves;
  [[maybe_unused]] u32x4 qpiece = {0u, 0u, 0u, 0u};
  if constexpr (kShareQ) {
    const int cbw = wave / KS;
    if (wave < NCB * KS) {
      const T* qrow = static_cast<const T*>(p.q) + col_b[cbw] * p.qs0 +
                      (kvh * G + (col_ok[cbw] ? col_h[cbw] : 0)) * p.qs1;
      const u32x4 x = *reinterpret_cast<const u32x4*>(qrow + 32 * (wave % KS) + 8 * g);
      qpiece = col_ok[cbw] ? x : u32x4{0u, 0u, 0u, 0u};
    }
  } else {
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      const T* qrow =
          static_cast<const T*>(p.q) + col_b[cb] * p.qs0 + (kvh * G + (col_ok[cb] ? col_h[cb] : 0)) * p.qs1;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        u32x4 x = *reinterpret_cast<const u32x4*>(qrow + 32 * s + 8 * g);
        qf[cb][s] = col_ok[cb] ? x : u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
  AppendRegs<D> ar;
  [[maybe_unused]] DmAppendRegs<D> dar;
  if constexpr (FUSE && DM) {
    load_append_dm<T, D>(p, b, kvh, lane, dar);
  } else if constexpr (FUSE) {
    const T* ak = static_cast<const T*>(p.ak) + b * p.aks0 + kvh * p.aks1;
    const T* av = static_cast<const T*>(p.av) + b * p.avs0 + kvh * p.avs1;
#pragma unroll
    for (int s = 0; s < KS; ++s) ar.akf[s] = *reinterpret_cast<const u32x4*>(ak + 32 * s + 8 * g);
    ar.avf = *reinterpret_cast<const VPiece<D>*>(av + (D / 16) * c);
  }
  // The row length (and slot) are read here and used only after the first
  // unit's K/V loads have issued (below): a use ahead of those loads would
  // put its wait, one more round trip, in front of them.
  int64_t eff_len = 0;
  int32_t slot = -1;
  [[maybe_unused]] int32_t seq_len = 0;
  [[maybe_unused]] int64_t plen = 0;
  if constexpr (PREFIX) {
    plen = lead_ok ? cp.prefix_len[grp] : 0;
  } else if constexpr (!BAL) {
    seq_len = load_index(p.sl, b * p.sls, p.sl_i64);
    slot = FUSE ? load_index(p.slot, b * p.slots, p.slot_i64) : -1;
  }
  const int32_t first = TAIL ? max(p.tb[b], 0) : 0;
  // Long splits (16-token units, several per wave) take the fixed lane
  // offsets; short ones (32-token units, about one per wave) compute each
  // address once, which keeps the kernel-argument loads ahead of the first
  // K/V loads in fewer dependent batches (C2: 6.2 vs 7.1 us).
  constexpr bool kFixed = BS >= 16 && UNIT == 16;
  using Regs = std::conditional_t<DM, DmRegs<D>, UnitRegs<UNIT, D>>;
  Regs cur;
  [[maybe_unused]] UnitOffsets<UNIT> offs;
  if constexpr (kFixed) offs = unit_offsets<T, BS, UNIT, D>(p, kvh, wave, c, g);
  // the prefix role's blocks are read again by the group's other chunks:
  // plain loads, so the re-reads hit the caches
  constexpr bool kNT = NT && !PREFIX;
  auto load = [&](int u, const UnitPages& up, Regs& dst) {
    if constexpr (DM)
      load_unit_dm<T, BS, kNT, D>(p, kvh, up, lane, dst);
    else if constexpr (kFixed)
      load_unit_fixed<T, BS, UNIT, kNT, D>(p, up, offs, dst);
    else
      load_unit<T, BS, UNIT, kNT, D>(p, kvh, u, up, c, g, dst);
  };
  load(unit, pages, cur);
  if constexpr (TL) timeline_stamp<2>();  // first unit's K/V loads issued
  if constexpr (kShareQ) {
    __shared__ u32x4 q_stage[NCB][KS][64];
    if (wave < NCB * KS) q_stage[wave / KS][wave % KS][lane] = qpiece;
    __syncthreads();
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
      for (int s = 0; s < KS; ++s) qf[cb][s] = q_stage[cb][s][lane];
  }
  // The split partial's address for this thread's merge row, computed while
  // the K/V loads are in flight (the empty asm keeps it here, not at the
  // stores, where it sat on the kernel's last chain)
  // element offsets: the stores keep p.acc as their base, so they stay global
  // stores (a pointer through the empty asm below lost its address space and
  // stored through flat instructions: C2 7.55 -> 7.53 us with the offsets)
  [[maybe_unused]] int64_t pre_ao = 0;
  [[maybe_unused]] int64_t pre_so = 0;
  // (one-unit waves only: with several units per wave the held address
  // costs the loop registers, C5 step 3.186 -> 3.213 ms)
  constexpr bool kPreStore = ROLE == Role::kRow && NCB == 1 && !MERGE && UNIT == 32;
  if constexpr (kPreStore) {
    constexpr int kDptE = D == 128 ? 8 : 4;
    const int hE = (threadIdx.x / (D / kDptE)) & 15;
    const int dE = (threadIdx.x % (D / kDptE)) * kDptE;
    const int qhE = kvh * G + 16 * hb + hE;
    pre_ao = b * p.as0 + qhE * p.as1 + split * p.as2 + dE * p.as3;
    pre_so = b * p.ss0 + qhE * p.ss1 + split * p.ss2;
    asm volatile("" : "+v"(pre_ao), "+v"(pre_so));
  }
  // The loaded length stays in a VGPR until here (the empty asm redefines
  // it): its move to an SGPR, and the wait for the load it brings, would
  // otherwise sit at the load, ahead of the K/V loads above.
  if constexpr (PREFIX) {
    asm volatile("" : "+v"(plen));
    plen = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(plen));
  } else if constexpr (!BAL) {
    asm volatile("" : "+v"(seq_len), "+v"(slot));
    seq_len = __builtin_amdgcn_readfirstlane(seq_len);
    slot = __builtin_amdgcn_readfirstlane(slot);
  }
  if constexpr (BAL) {
    eff_len = bal_eff;
  } else if constexpr (PREFIX) {
    const int64_t cap = p.max_blocks_per_seq * p.block_size;
    eff_len = plen < 0 ? 0 : (plen < cap ? plen : cap);
  } else {
    eff_len = effective_len(p, seq_len, slot);
  }
  // the float64 cos/sin evaluation overlaps the K/V loads just issued
  if constexpr (ROPE && D == 128) rope_operands<T>(p, seq_len, lane, g, qf[0], ar);

  // token indices fit in 32 bits: eff_len <= seq_lens[b], an int32
  const int last = static_cast<int>(eff_len) - 1;
  const int app = (FUSE && eff_len > 0) ? last : -1;
  // The split's tiles come from the row's own length; its units are the
  // UNIT-token pieces of those tiles that hold at least one live token.  When
  // the host bound predicted where they start (rows as long as the bound),
  // the loads above are the right ones; otherwise the first unit is fetched
  // again.
  int t_begin, t_end;
  split_tiles(nsplit, split, eff_len, TAIL ? first / 32 : 0, t_begin, t_end);
  const int live_units = static_cast<int>((eff_len + UNIT - 1) / UNIT);
  const int u_end = min(kUnitsPerTile * t_end, live_units);
  if (t_begin != guess_begin) {
    unit = kUnitsPerTile * t_begin + wave;
    if (unit < u_end) {
      pages = fetch_pages<BS, UNIT, kScalarPages>(p, trow, unit);
      load(unit, pages, cur);
    }
  }

  WaveState<D> st[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
    for (int n = 0; n < D / 16; ++n) st[cb].acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    st[cb].m = -INFINITY;
    st[cb].l = 0.f;
  }

  if (unit < u_end) {
    UnitPages next_pages{0, 0};
    if (unit + kWaves < u_end) next_pages = fetch_pages<BS, UNIT, kScalarPages>(p, trow, unit + kWaves);
    // One unit: issue the next unit's loads into `ahead` (and the block ids
    // after it), then consume `now`; false when `now` was the last.  The two
    // buffers take turns, so no registers are copied between units.
    auto step = [&](Regs& now, Regs& ahead) -> bool {
      const int next = unit + kWaves;
      const bool more = next < u_end;
      UnitPages after{0, 0};
      if (more) {
        load(next, next_pages, ahead);
        if (next + kWaves < u_end) after = fetch_pages<BS, UNIT, kScalarPages>(p, trow, next + kWaves);
      }
      if constexpr (FUSE)
        if (app >= 0 && app / UNIT == unit && hb == 0) {
          if constexpr (DM)
            store_append_dm<T, BS, D>(p, kvh, slot, lane, dar);
          else
            store_append<T, BS, D>(p, kvh, slot, c, g, ar);
        }
      if constexpr (DM)
        process_unit_dm<T, (FUSE != 0), D>(now, qf[0], p.scale_log2, unit * UNIT, first, last, app, dar, lane,
                                           kstage + wave * D * kDmRowBytes, st[0]);
      else {
        process_unit<T, (FUSE != 0), UNIT, D, NCB, TL>(now, qf, p.scale_log2, unit * UNIT, first, last, app, ar, c,
                                                       g, st);
        if constexpr (TL) {
          timeline_stamp<5>();  // unit's PV issued
          timeline_put(10 + min(tl_units, 4), false, 0);  // the wave's unit tl_units done
          ++tl_units;
        }
      }
      unit = next;
      next_pages = after;
      return more;
    };
    Regs alt;
    if constexpr (UNIT == 16 || DM) {
      while (step(cur, alt) && step(alt, cur)) {
      }
    } else {
      // about one unit per wave: one copy of the step keeps the code small
      while (step(cur, alt)) cur = alt;
    }
  }
  if constexpr (TL) timeline_stamp<6>();  // all units done
  // merge threads: thread -> (column h, dims [d0, d0 + kDpt)), 16 threads
  // per column (8 dims each at head_dim 128, 4 at 64), so that every merge
  // read has the conflict-free pattern of acc_pitch; threads past the first
  // 256 only take part in the barriers
  constexpr int kDpt = D == 128 ? 8 : 4;
  constexpr int kDimThreads = D / kDpt;
  const int h = (threadIdx.x / kDimThreads) & 15;
  const int d0 = (threadIdx.x % kDimThreads) * kDpt;
  int ob = b, qh = kvh * G + 16 * hb + h;
  bool head_ok = threadIdx.x < 16 * kDimThreads && 16 * hb + h < G;
  // one round per column block: the waves' slots hold one block at a time
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    if (cb > 0) __syncthreads();  // every thread has read the previous block's slots
    // denominator over the four lanes (g) that share query column c
    const float lt = column_sum(st[cb].l);

    // Every wave publishes its state (one LDS slot each; eight slots take 68 KB,
    // which gfx950's LDS holds in one workgroup), then threads merge across the
    // slots.
    if (g == 0) {
      lds.m[wave][c] = st[cb].m;
      lds.l[wave][c] = lt;
      if (PREFIX && wave == 0) {
        lds.col_b[c] = col_ok[cb] ? col_b[cb] : -1;
        lds.col_h[c] = col_h[cb];
      }
    }
    constexpr int kSpread = acc_spread<D>();
    if constexpr (DM) {
      // this lane's dims 16*n + 4*g + rr (load_unit_dm's V rows)
#pragma unroll
      for (int n = 0; n < D / 16; ++n)
        *reinterpret_cast<f32x4*>(&lds.acc[wave][c][kSpread * (16 * n + 4 * g)]) = st[cb].acc[n];
    } else {
      // this lane's dims (D/4)*g + (D/16)*rr + n, n < D/16: one or two 16-byte rows
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        float* dst = &lds.acc[wave][c][kSpread * ((D / 4) * g + (D / 16) * rr)];
        const WaveState<D>& w = st[cb];
        *reinterpret_cast<f32x4*>(dst) = f32x4{w.acc[0][rr], w.acc[1][rr], w.acc[2][rr], w.acc[3][rr]};
        if constexpr (D == 128)
          *reinterpret_cast<f32x4*>(dst + 4) = f32x4{w.acc[4][rr], w.acc[5][rr], w.acc[6][rr], w.acc[7][rr]};
      }
    }
    __syncthreads();
    if constexpr (TL) timeline_stamp<7>();  // wave merge barrier passed

    // merge the slots
    if constexpr (PREFIX) {
      ob = lds.col_b[h];
      qh = kvh * G + lds.col_h[h];
      head_ok = threadIdx.x < 16 * kDimThreads && ob >= 0;
    } else if constexpr (NCB > 1) {
      const int hh = 16 * (NCB * hb + cb) + h;
      qh = kvh * G + hh;
      head_ok = threadIdx.x < 16 * kDimThreads && hh < G;
    }
    // every slot read issues before the first use: one LDS round trip after
    // the barrier instead of one per dependent step
    float mw[kWaves], lw[kWaves];
    f32x4 aw0[kWaves];
    [[maybe_unused]] f32x4 aw1[kWaves];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      mw[w] = lds.m[w][h];
      lw[w] = lds.l[w][h];
      aw0[w] = *reinterpret_cast<const f32x4*>(&lds.acc[w][h][kSpread * d0]);
      if constexpr (kDpt == 8) aw1[w] = *reinterpret_cast<const f32x4*>(&lds.acc[w][h][d0 + 4]);
    }
    __builtin_amdgcn_sched_barrier(0);
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, mw[w]);
    const float Mu = M == -INFINITY ? 0.f : M;
    float L = 0.f;
    float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float wt = exp2_fast(mw[w] - Mu);
      L += wt * lw[w];
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] += wt * aw0[w][j];
      if constexpr (kDpt == 8) {
#pragma unroll
        for (int j = 0; j < 4; ++j) o[4 + j] += wt * aw1[w][j];
      }
    }
    if (ROLE == Role::kRow && p.splits == 1) {
      if (head_ok) store_row<T, kDpt>(p, b, qh, d0, o, L > 0.f ? rcp_fast(L) : 0.f);
      continue;
    }
    // split partial: unnormalised acc, base-2 max, denominator; the prefix
    // role's partials follow the tail splits
    if (head_ok) {
      const int ws = PREFIX ? p.splits + split : split;
      float* a = p.acc + (kPreStore ? pre_ao : ob * p.as0 + qh * p.as1 + ws * p.as2 + d0 * p.as3);
      const int64_t so = kPreStore ? pre_so : ob * p.ss0 + qh * p.ss1 + ws * p.ss2;
      if constexpr (MERGE) {
        // device-coherent (sc1) stores, visible to every XCD once acknowledged;
        // the host guarantees unit dim stride and 8-byte alignment here
        uint64_t* a64 = reinterpret_cast<uint64_t*>(a);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint64_t bits = static_cast<uint64_t>(__builtin_bit_cast(uint32_t, o[2 * j])) |
                                (static_cast<uint64_t>(__builtin_bit_cast(uint32_t, o[2 * j + 1])) << 32);
          __hip_atomic_store(a64 + j, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (d0 == 0) {
          __hip_atomic_store(p.mx + so, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(p.sm + so, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      } else {
        if (p.as3 == 1) {
          *reinterpret_cast<f32x4*>(a) = f32x4{o[0], o[1], o[2], o[3]};
          if constexpr (kDpt == 8) *reinterpret_cast<f32x4*>(a + 4) = f32x4{o[4], o[5], o[6], o[7]};
        } else {
#pragma unroll
          for (int j = 0; j < kDpt; ++j) a[j * p.as3] = o[j];
        }
        if (d0 == 0) {
          p.mx[so] = M;
          p.sm[so] = L;
        }
      }
    }
  }  // column blocks
  if constexpr (TL) {
    timeline_stamp<8>();  // partials issued
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    timeline_stamp<9>();  // partials acknowledged
  }

  if constexpr (!MERGE) return;  // the reducer kernel merges
  if (p.splits == 1) return;     // rows went straight to the output

  // In-launch merge.  Partials were written with agent-scope atomic stores
  // (sc1: written through to memory, and through the writer's own XCD L2,
  // which stays coherent with them); waiting for their acknowledgement
  // (vmcnt 0) before the arrival increment is the release for them, without
  // the L2-wide write-back an agent-scope fence would do in every
  // workgroup.  The last workgroup of this (request, KV head) to arrive
  // merges and returns the arrival word to zero for the next launch.  When
  // every arrival came from its own XCD -- the hardware hands workgroup i to
  // XCD i mod 8, and the XCD-by-XCD grid layout keeps a pair's workgroups on
  // one XCD -- it reads the partials from that XCD's L2 (after invalidating
  // its own L1), otherwise with agent-scope loads from memory.  C2 on
  // MI355X: 10.65 us per call with agent-scope reads, 9.24 us with the L2
  // reads (the reducer kernel path: 8.43 us).
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  __syncthreads();
  if (threadIdx.x == 0) {
    // One 64-bit arrival word per (request, KV head): the count in bits
    // 0-15, the sum of the arrivals' XCD ids in bits 16-31 and the sum of
    // their squares in bits 32-63.  The last arrival reads all three: the
    // ids are all equal exactly when S * sum(x^2) == sum(x)^2, and then the
    // pair's partials all passed through its own XCD's L2.
    const uint32_t xcc = xcc_id();
    const uint64_t mine = 1ull | (static_cast<uint64_t>(xcc) << 16) | (static_cast<uint64_t>(xcc * xcc) << 32);
    uint64_t* word = reinterpret_cast<uint64_t*>(p.counters + pair * kCounterStride);
    const uint64_t now = __hip_atomic_fetch_add(word, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + mine;
    const uint64_t n = now & 0xffffu, sx = (now >> 16) & 0xffffu, sxx = now >> 32;
    int last = 0;
    if (n == static_cast<uint64_t>(p.splits)) {
      last = 1;
      if (n * sxx == sx * sx && sx == n * xcc) last = 2;
      __hip_atomic_store(word, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    lds.last = last;
  }
  __syncthreads();
  const int last_kind = lds.last;
  if (last_kind == 0) return;
  if (last_kind == 2 && p.splits <= kMergeChunk && p.as3 == 1 && ((p.as0 | p.as1 | p.as2) & 3) == 0 &&
      (reinterpret_cast<uintptr_t>(p.acc) & 15u) == 0) {
    // Every partial sits in this XCD's L2: all four waves read them with
    // 16-byte loads after invalidating this CU's L1.  Thread -> (head hh,
    // dims [dd, dd + DPT)): 4 dims per thread for up to 8 heads, else 8.
    const int dpt = G <= 8 ? 4 : 8;
    const int tph = D / dpt;
    const int hh = threadIdx.x / tph;
    const int dd = (threadIdx.x % tph) * dpt;
    if (hh >= G) return;
    const int qq = kvh * G + hh;
    asm volatile("buffer_inv sc0" ::: "memory");
    const float* pa = p.acc + b * p.as0 + qq * p.as1 + dd;
    const int64_t sbase = b * p.ss0 + qq * p.ss1;
    f32x4 part[kMergeChunk][2];
    float pm[kMergeChunk], pl[kMergeChunk];
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j) {
      const int ss = min(j, p.splits - 1);
      part[j][0] = *reinterpret_cast<const f32x4*>(pa + ss * p.as2);
      part[j][1] = dpt == 8 ? *reinterpret_cast<const f32x4*>(pa + ss * p.as2 + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
      pm[j] = p.mx[sbase + ss * p.ss2];
      pl[j] = p.sm[sbase + ss * p.ss2];
    }
    float cm = -INFINITY;
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j) cm = j < p.splits ? fmaxf(cm, pm[j]) : cm;
    const float nmu = cm == -INFINITY ? 0.f : cm;
    float gx[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float tl[kMergeChunk];  // the denominator's terms, summed as the reducer sums them
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j) {
      const float w = j < p.splits ? exp2_fast(pm[j] - nmu) : 0.f;
      const float t = merge_term(w, pl[j]);
      tl[j] = j < p.splits ? t : 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        gx[k] += w * part[j][0][k];
        gx[4 + k] += w * part[j][1][k];
      }
    }
    const float GLx = __builtin_fmaf(0.f, 0.f, tree_sum16(tl));
    const float inv = GLx > 0.f ? rcp_fast(GLx) : 0.f;
    T* dst = static_cast<T*>(p.out) + b * p.os0 + qq * p.os1 + dd * p.os2;
    if (p.os2 == 1 && dpt == 8) {
      u32x4 w4;
      w4[0] = pack2<T>(gx[0] * inv, gx[1] * inv);
      w4[1] = pack2<T>(gx[2] * inv, gx[3] * inv);
      w4[2] = pack2<T>(gx[4] * inv, gx[5] * inv);
      w4[3] = pack2<T>(gx[6] * inv, gx[7] * inv);
      *reinterpret_cast<u32x4*>(dst) = w4;
    } else if (p.os2 == 1) {
      u32x2 w2;
      w2[0] = pack2<T>(gx[0] * inv, gx[1] * inv);
      w2[1] = pack2<T>(gx[2] * inv, gx[3] * inv);
      *reinterpret_cast<u32x2*>(dst) = w2;
    } else {
      for (int j = 0; j < dpt; ++j) dst[j * p.os2] = from_f32<T>(gx[j] * inv);
    }
    return;
  }
  if (!head_ok) return;

  const int64_t sb = b * p.ss0 + qh * p.ss1;
  const float* ab = p.acc + b * p.as0 + qh * p.as1 + d0 * p.as3;
  float GM = -INFINITY;
  float GL = 0.f;
  float go[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // Every split ran on this XCD: its write-through stores left the L2 of
  // this XCD coherent with memory, so the partials are read from there
  // (workgroup-scope loads miss only the CU's own L1), not from memory.
  const bool local = last_kind == 2;
  for (int s0 = 0; s0 < p.splits; s0 += kMergeChunk) {
    uint64_t raw[kMergeChunk][4];
    float pm[kMergeChunk], pl[kMergeChunk];
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j) {
      const int ss = min(s0 + j, p.splits - 1);  // past the end: re-read, masked below
      const uint64_t* a64 = reinterpret_cast<const uint64_t*>(ab + ss * p.as2);
      if (local) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
          raw[j][k] = __hip_atomic_load(a64 + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        pm[j] = __hip_atomic_load(p.mx + sb + ss * p.ss2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        pl[j] = __hip_atomic_load(p.sm + sb + ss * p.ss2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k)
          raw[j][k] = __hip_atomic_load(a64 + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        pm[j] = __hip_atomic_load(p.mx + sb + ss * p.ss2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        pl[j] = __hip_atomic_load(p.sm + sb + ss * p.ss2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    float cm = -INFINITY;
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j) cm = s0 + j < p.splits ? fmaxf(cm, pm[j]) : cm;
    const float nm = fmaxf(GM, cm);
    const float nmu = nm == -INFINITY ? 0.f : nm;
    const float sc = exp2_fast(GM - nmu);
#pragma unroll
    for (int j = 0; j < 8; ++j) go[j] *= sc;
    float tl[kMergeChunk];  // the denominator's terms, summed as the reducer sums them
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j) {
      const float w = s0 + j < p.splits ? exp2_fast(pm[j] - nmu) : 0.f;
      const float t = merge_term(w, pl[j]);
      tl[j] = s0 + j < p.splits ? t : 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        go[2 * k] += w * __builtin_bit_cast(float, static_cast<uint32_t>(raw[j][k]));
        go[2 * k + 1] += w * __builtin_bit_cast(float, static_cast<uint32_t>(raw[j][k] >> 32));
      }
    }
    GL = __builtin_fmaf(GL, sc, tree_sum16(tl));
    GM = nm;
  }
  if (head_ok) store_row<T>(p, b, qh, d0, go, GL > 0.f ? rcp_fast(GL) : 0.f);
}

// FUSE: 0 none, 1 fused append, 2 fused append with RoPE of q and the new K;
// D: head_dim 128 or 64.  NCB: 16-column blocks of query heads per wave (2
// for groups of more than 16 heads per KV head).
//
// The leading scalar arguments repeat what the first block-table load needs,
// with the grid's XCD layout (xcd_blocks, for xcd_logical_block).
// The library is built with amdgpu-kernarg-preload-count, so the command
// processor writes them into SGPRs at wave launch: the table load issues
// without waiting for a kernel-argument fetch from a cold scalar cache, and
// the remaining arguments are fetched while it is in flight (C2 attention
// kernel 5.53 -> 5.33 us on MI355X).  Firmware without argument preloading
// runs the compiler's fallback prologue, which loads them from the argument
// buffer instead.
template <typename T, int BS, int FUSE, bool MERGE, int UNIT, bool NT, int D = 128, int NCB = 1>
__global__ __launch_bounds__(64 * waves_for<UNIT>(), 1) void decode_mfma_kernel(
    const void* bt, int32_t bts0, int32_t bts1, int32_t max_blocks_per_seq, int32_t splits, int32_t hkv,
    int32_t group, int32_t hint_tps, int32_t xcd_blocks, uint32_t div_splits_m, uint32_t div_hkv_m,
    int32_t div_shifts, int32_t bt_i64, DecodeParams p) {
  __shared__ DecodeLds<waves_for<UNIT>(), acc_pitch<D>()> lds;
  DecodeParams q = p;
  q.bt = bt;
  q.bts0 = bts0;
  q.bts1 = bts1;
  q.max_blocks_per_seq = max_blocks_per_seq;
  q.splits = splits;
  q.hkv = hkv;
  q.group = group;
  q.hint_tps = hint_tps;
  q.div_splits_m = div_splits_m;
  q.div_hkv_m = div_hkv_m;
  q.div_shifts = div_shifts;
  q.bt_i64 = bt_i64;
  decode_role<T, BS, FUSE, MERGE, UNIT, Role::kRow, NT, D, waves_for<UNIT>(), false, true, NCB>(
      q, CascadeParams{}, xcd_logical_block(blockIdx.x, xcd_blocks), lds);
}

// Dim-major caches: 32-token units on kDmWaves waves, K staged through LDS.
// Two workgroups per CU (67 KB of LDS each): B16 x 8192 tokens, 16 splits,
// 28.8 us against 30.0 us with one per CU and 29.9 us with one 8-wave
// workgroup per CU at its best split count.
constexpr int kDmPerCU = 2;

// FUSE: fused current-token append.  Its variant runs one workgroup per CU:
// within two per CU (256 registers a wave) the 128-dim variant spilled.
template <typename T, int BS, bool NT, int D, int FUSE>
__global__ __launch_bounds__(64 * kDmWaves, FUSE ? 1 : kDmPerCU) void decode_dm_kernel(DecodeParams p,
                                                                                       int32_t xcd_blocks) {
  __shared__ DecodeLds<kDmWaves, acc_pitch<D>()> lds;
  __shared__ __attribute__((aligned(16))) uint8_t stage[kDmWaves * D * kDmRowBytes];
  decode_role<T, BS, FUSE, false, 32, Role::kRow, NT, D, kDmWaves, true>(
      p, CascadeParams{}, xcd_logical_block(blockIdx.x, xcd_blocks), lds, stage);
}

// Balanced splits (ragged batches): the row and split of each workgroup come
// from the batch's lengths on the device.
// Four waves per workgroup and two workgroups per CU: twice the splits of
// the eight-wave layout at half the tiles each, so the heaviest CU carries
// less above the mean.
constexpr int kBalWaves = 4;
constexpr int kBalPerCU = 2;

template <typename T, int BS, bool NT>
__global__ __launch_bounds__(64 * kBalWaves, kBalPerCU) void decode_balanced_kernel(DecodeParams p) {
  __shared__ DecodeLds<kBalWaves> lds;
  decode_role<T, BS, false, false, 16, Role::kBalanced, NT, 128, kBalWaves>(p, CascadeParams{}, blockIdx.x, lds);
}

// Cascade launch: workgroups [0, prefix_blocks) take the prefix role, the
// rest the tail role (both write split partials; the reducer merges them).
// NCB: the prefix role's 16-row column blocks per wave.
//
// The leading scalar arguments repeat what the prefix role needs for its
// member and first block-id loads; the library is built with
// amdgpu-kernarg-preload-count, so they arrive in SGPRs at wave launch and
// those loads issue without a kernel-argument round trip ahead of them (C4
// shared prefix on MI355X, same box: 13.31 -> 13.06 us per call, cascade
// kernel 9.58 -> 9.18 us; 64 x 16384 36.68 -> 36.57 us).
template <typename T, int BS, int UNIT, bool NT, int NCB = 1>
__global__ __launch_bounds__(64 * waves_for<UNIT>(), 1) void cascade_decode_kernel(
    int32_t prefix_wgs, int32_t prefix_splits, int32_t chunks, int32_t hkv, int32_t hint_ptps,
    const int32_t* members, int32_t max_members, DecodeParams p, CascadeParams cp) {
  __shared__ DecodeLds<waves_for<UNIT>()> lds;
  if (static_cast<int>(blockIdx.x) < prefix_wgs) {
    CascadeParams c = cp;
    c.prefix_blocks = prefix_wgs;
    c.prefix_splits = prefix_splits;
    c.chunks = chunks;
    c.hint_ptps = hint_ptps;
    c.members = members;
    c.max_members = max_members;
    DecodeParams q = p;
    q.hkv = hkv;
    decode_role<T, BS, false, false, UNIT, Role::kPrefix, NT, 128, waves_for<UNIT>(), false, false, NCB>(
        q, c, blockIdx.x, lds);
  } else {
    decode_role<T, BS, false, false, UNIT, Role::kTail, NT>(p, cp, blockIdx.x - prefix_wgs, lds);
  }
}

// ====================================================== generic path ====
// One wave per (request, KV head, head group of <= 8 query heads, split).
// Lane = token within a 64-token tile for QK; lane = dim for PV.
constexpr int kGenHeads = 8;

template <typename T, int D>
__global__ __launch_bounds__(64) void decode_generic_kernel(DecodeParams p, int head_groups) {
  __shared__ float s_q[kGenHeads][D];
  __shared__ float s_p[kGenHeads][64];
  __shared__ int64_t s_vrow[64];  // element offset of the V row, -1 = masked, -2 = append

  const int lane = threadIdx.x;
  const int split = blockIdx.y;
  const int hg = blockIdx.x % head_groups;
  const int pair = blockIdx.x / head_groups;
  const int b = pair / p.hkv;
  const int kvh = pair % p.hkv;
  const int G = p.group;
  const int h0 = kvh * G + hg * kGenHeads;
  const int nh = min(kGenHeads, G - hg * kGenHeads);

  const T* qb = static_cast<const T*>(p.q) + b * p.qs0;
  for (int i = lane; i < kGenHeads * D; i += 64) {
    const int j = i / D, d = i % D;
    s_q[j][d] = j < nh ? to_f32(qb[(h0 + j) * p.qs1 + d * p.qs2]) : 0.f;
  }
  const RowInfo r = row_info(p, b, split);
  const T* kbase = static_cast<const T*>(p.k);
  const T* vbase = static_cast<const T*>(p.v);
  const T* akrow = p.fuse ? static_cast<const T*>(p.ak) + b * p.aks0 + kvh * p.aks1 : nullptr;
  const T* avrow = p.fuse ? static_cast<const T*>(p.av) + b * p.avs0 + kvh * p.avs1 : nullptr;

  // the split owning the appended token stores it (head group 0 only)
  if (r.app_tok >= 0 && hg == 0 && r.app_tok / 32 >= r.t_begin && r.app_tok / 32 < r.t_end) {
    const int64_t blk = r.slot / p.block_size, off = r.slot % p.block_size;
    if (blk < p.num_blocks) {
      T* kd = static_cast<T*>(p.k) + blk * p.ks0 + kvh * p.ks1 + off * p.ks2;
      T* vd = static_cast<T*>(p.v) + blk * p.vs0 + kvh * p.vs1 + off * p.vs2;
      for (int d = lane; d < D; d += 64) {
        kd[d * p.ks3] = akrow[d * p.aks2];
        vd[d * p.vs3] = avrow[d * p.avs2];
      }
    }
  }

  float m[kGenHeads], l[kGenHeads];
  float acc[kGenHeads][D / 64];
#pragma unroll
  for (int j = 0; j < kGenHeads; ++j) {
    m[j] = -INFINITY;
    l[j] = 0.f;
#pragma unroll
    for (int e = 0; e < D / 64; ++e) acc[j][e] = 0.f;
  }
  __syncthreads();

  // 64-token tiles = two 32-token split tiles
  const int64_t tok_begin = static_cast<int64_t>(r.t_begin) * 32;
  const int64_t tok_end = min(static_cast<int64_t>(r.t_end) * 32, r.eff_len);
  for (int64_t tok0 = tok_begin; tok0 < tok_end; tok0 += 64) {
    const int64_t tok = tok0 + lane;
    bool ok = tok < tok_end;
    int64_t krow = 0, vrow = -1;
    const bool is_app = ok && tok == r.app_tok;
    if (ok && !is_app) {
      const int64_t blk = load_index(p.bt, b * p.bts0 + (tok / p.block_size) * p.bts1, p.bt_i64);
      ok = blk >= 0 && blk < p.num_blocks;
      const int64_t off = tok % p.block_size;
      krow = blk * p.ks0 + kvh * p.ks1 + off * p.ks2;
      vrow = ok ? blk * p.vs0 + kvh * p.vs1 + off * p.vs2 : -1;
    }
    if (is_app) vrow = -2;
    float sc[kGenHeads];
#pragma unroll
    for (int j = 0; j < kGenHeads; ++j) sc[j] = 0.f;
    if (ok) {
      for (int d = 0; d < D; ++d) {
        const float kv = is_app ? to_f32(akrow[d * p.aks2]) : to_f32(kbase[krow + d * p.ks3]);
#pragma unroll
        for (int j = 0; j < kGenHeads; ++j) sc[j] += s_q[j][d] * kv;
      }
    }
    s_vrow[lane] = vrow;
#pragma unroll
    for (int j = 0; j < kGenHeads; ++j) {
      const float s = ok ? sc[j] * p.scale_log2 : -INFINITY;
      float mx = s;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, shfl_xor_f32(mx, o));
      const float m_new = fmaxf(m[j], mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2f(m[j] - m_use);
      const float pj = exp2f(s - m_use);
      float ps = pj;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) ps += shfl_xor_f32(ps, o);
      l[j] = l[j] * alpha + ps;
      m[j] = m_new;
#pragma unroll
      for (int e = 0; e < D / 64; ++e) acc[j][e] *= alpha;
      s_p[j][lane] = pj;
    }
    __syncthreads();
    const int n = static_cast<int>(min<int64_t>(64, tok_end - tok0));
    for (int t = 0; t < n; ++t) {
      const int64_t vr = s_vrow[t];
      if (vr == -1) continue;
#pragma unroll
      for (int e = 0; e < D / 64; ++e) {
        const int d = lane + 64 * e;
        const float vv = vr == -2 ? to_f32(avrow[d * p.avs2]) : to_f32(vbase[vr + d * p.vs3]);
#pragma unroll
        for (int j = 0; j < kGenHeads; ++j) acc[j][e] += s_p[j][t] * vv;
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < kGenHeads; ++j) {
    if (j >= nh) break;
    const int qh = h0 + j;
    if (p.splits == 1) {
      const float inv = l[j] > 0.f ? 1.f / l[j] : 0.f;
      T* dst = static_cast<T*>(p.out) + b * p.os0 + qh * p.os1;
#pragma unroll
      for (int e = 0; e < D / 64; ++e) dst[(lane + 64 * e) * p.os2] = from_f32<T>(acc[j][e] * inv);
    } else {
      float* a = p.acc + b * p.as0 + qh * p.as1 + split * p.as2;
#pragma unroll
      for (int e = 0; e < D / 64; ++e) a[(lane + 64 * e) * p.as3] = acc[j][e];
      if (lane == 0) {
        const int64_t so = b * p.ss0 + qh * p.ss1 + split * p.ss2;
        p.mx[so] = m[j];
        p.sm[so] = l[j];
      }
    }
  }
}

// ===================================================== split reducer ====
// One wave per (request, query head): out = sum_s w_s acc_s / sum_s w_s l_s,
// w_s = 2^(m_s - max_s m_s).  The kernel is pure latency, so every load is a
// vector load issued up front: lane j holds split j's (max, sum) and
// readlane broadcasts them.  Scalar loads would not do: they complete out of
// order, so each use of one waits for all (lgkmcnt(0)), which turned the
// per-split statistics into a round trip per split.  Row length and slot,
// needed only for the final zero-row select, are vector loads too.  Once the
// data has landed, one wave's instruction chain is the kernel's time: the
// splits' maximum and weights are computed across the lanes (a DPP / permlane
// reduction and one exp per lane), not as a dependent max / exp step per
// split (C2 call 8.42 -> 8.27 us, shared-prefix C4 12.43 -> 11.88 us, same
// box).
constexpr int kReduceChunk = 16;  // splits whose partial rows are in flight at once

// The reducer's own compact arguments: with the full DecodeParams the
// compiler fetched the workspace fields in a second, dependent batch of
// kernel-argument loads.
struct ReduceParams {
  const float* acc;
  const float* mx;
  const float* sm;
  void* out;
  const void* sl;
  const void* slot;  // seq_lens again when there is no fused append
  int64_t as0, as1, as2, as3;
  int64_t ss0, ss1, ss2;
  int64_t os0, os1, os2;
  int64_t sls, slots;
  int hq, splits, fuse, sl_i64, slot_i64;
  // cascade: rows with tb[b] == 0 have no prefix partials and merge only the
  // first tail_splits splits
  const int32_t* tb;
  int tail_splits;
  // balanced splits: each row's count is recomputed from the batch's lengths
  int bal_target, num_seqs;
  int64_t cap;  // table capacity in tokens (effective lengths)
};

enum ReduceMode { kReducePlain = 0, kReduceCascade = 1, kReduceBalanced = 2 };

__device__ __forceinline__ float lane_bcast(float x, int lane_idx) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane_idx));
}

// Maximum over the wave, every lane receiving it: rotations within each
// 16-lane row (DPP row_ror), then across the rows (permlane swaps).
__device__ __forceinline__ float dpp_row_ror_max(float x, int y) { return fmaxf(x, __builtin_bit_cast(float, y)); }
// Sum within each 16-lane row; the row's first lane holds it in the order of
// tree_sum16 (the other lanes hold the same terms in other orders)
__device__ __forceinline__ float dpp_row_ror_add(float x, int y) { return x + __builtin_bit_cast(float, y); }
__device__ __forceinline__ float row_sum_f32(float x) {
  x = dpp_row_ror_add(x, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false));
  x = dpp_row_ror_add(x, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x124, 0xf, 0xf, false));
  x = dpp_row_ror_add(x, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x122, 0xf, 0xf, false));
  x = dpp_row_ror_add(x, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x121, 0xf, 0xf, false));
  return x;
}

// Maximum within each 16-lane row (every lane of the row receiving it)
__device__ __forceinline__ float row_max_f32(float x) {
  x = dpp_row_ror_max(x, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false));
  x = dpp_row_ror_max(x, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x124, 0xf, 0xf, false));
  x = dpp_row_ror_max(x, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x122, 0xf, 0xf, false));
  x = dpp_row_ror_max(x, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x121, 0xf, 0xf, false));
  return x;
}
__device__ __forceinline__ float wave_max_f32(float x) {
  x = dpp_row_ror_max(x, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false));
  x = dpp_row_ror_max(x, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x124, 0xf, 0xf, false));
  x = dpp_row_ror_max(x, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x122, 0xf, 0xf, false));
  x = dpp_row_ror_max(x, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x121, 0xf, 0xf, false));
  return column_max(x);
}

// W waves per (request, query head): wave w merges the w-th quarter of the
// row's splits (W = 4, for rows with many splits: a single wave would wait
// on its chunks one after another), then wave 0 merges the waves' states.
// One (request, query head) row of the merge.  PRE (plain mode only): the
// workspace is [rows, hq, splits, D] with unit dim and statistic strides
// (as0 = hq * as1, ss0 = hq * ss1, as3 = ss2 = 1), and acc / mx / sm / as1 /
// as2 / ss1 / splits / hq arrived preloaded in SGPRs, so the partial loads
// issue at once.  Such a row needs no length or slot: every split of it was
// written by this call's attention kernel, and a row with nothing to attend
// (zero length, or a padding slot) has denominator 0 in every split, which
// selects the zero row below just as the length test does.
// FCH > 0: the row has exactly FCH splits (a power of two up to 32) in a
// contiguous [rows, FCH, D] workspace, read as one chunk.
template <typename T, int D, int MODE, int W, bool PRE, bool OUTP = false, int FCH = 0>
__device__ __forceinline__ void reduce_row(const ReduceParams& p, const int row = blockIdx.x) {
  static_assert(!PRE || MODE == kReducePlain || MODE == kReduceCascade,
                "preloaded reducer arguments are for the plain and cascade merges");
  if constexpr (!PRE) {
    // every argument in SGPRs before any use: one batch of argument loads,
    // one wait (left alone the compiler fetched the strides lazily, a second
    // dependent round trip)
    asm volatile("" ::"s"(p.acc), "s"(p.mx), "s"(p.sm), "s"(p.out), "s"(p.sl), "s"(p.slot), "s"(p.as0),
                 "s"(p.as1), "s"(p.as2), "s"(p.as3), "s"(p.ss0), "s"(p.ss1), "s"(p.ss2), "s"(p.os0), "s"(p.os1),
                 "s"(p.os2), "s"(p.sls), "s"(p.slots), "s"(p.hq), "s"(p.splits), "s"(p.fuse), "s"(p.sl_i64),
                 "s"(p.slot_i64));
  }
  const int b = row / p.hq;
  const int qh = row % p.hq;
  const int lane = threadIdx.x & 63;
  const int wave = W > 1 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0;
  constexpr int E = D / 64;  // dims per lane
  // whole chunks at head_dim 128 into a row-order output: lane l holds dims
  // 2l and 2l + 1 (one 8-byte load per split, one 4-byte store), else dims
  // l + 64e
  constexpr bool PAIR = FCH > 0 && OUTP && E == 2 && W == 1;
  // a VGPR zero keeps the uniform row-length / slot loads on the vector path
  int vzero = 0;
  asm volatile("" : "+v"(vzero));
  int32_t seq_len = 1, slot = 1;
  if constexpr (!PRE) {
    seq_len = load_index(p.sl, b * p.sls + vzero, p.sl_i64);
    slot = load_index(p.slot, b * p.slots + vzero, p.slot_i64);  // seq_lens when not fused
  }
  int splits = p.splits;
  // splits of this row that hold partials: all of them, or in the cascade
  // the tail splits only for rows without a prefix.  With preloaded
  // arguments the loads below cover every split and issue without waiting
  // for the row's prefix length; the splits past `valid` are masked.
  int valid = p.splits;
  [[maybe_unused]] int32_t row_tb = 0;
  if constexpr (MODE == kReduceCascade) {
    if constexpr (PRE) {
      row_tb = p.tb[b + vzero];  // compared after the partial loads below have issued
    } else {
      splits = __builtin_amdgcn_readfirstlane(p.tb[b + vzero]) > 0 ? p.splits : p.tail_splits;
      valid = splits;
    }
  }
  if constexpr (MODE == kReduceBalanced) {
    // the same counts as the attention kernel: T from the batch's total tiles
    auto eff_of = [&](int64_t len) -> int64_t { return len > 0 ? (len < p.cap ? len : p.cap) : 0; };
    int total = 0;
    for (int r0 = 0; r0 < p.num_seqs; r0 += 64) {
      const int r = r0 + lane;
      const int t = r < p.num_seqs ? static_cast<int>((eff_of(load_index(p.sl, r * p.sls, p.sl_i64)) + 31) / 32) : 0;
      total += wave_sum_i32(t);
    }
    const int tps = max(1, (total + p.bal_target - 1) / p.bal_target);
    const int tiles = static_cast<int>((eff_of(__builtin_amdgcn_readfirstlane(seq_len)) + 31) / 32);
    splits = min(max(1, (tiles + tps - 1) / tps), p.splits);
  }
  const int64_t sb = PRE ? row * p.ss1 : b * p.ss0 + qh * p.ss1;
  const float* ab = p.acc + (PRE ? row * p.as1 : b * p.as0 + qh * p.as1);
  const int64_t as3 = PRE ? 1 : p.as3;
  const int64_t ss2 = PRE ? 1 : p.ss2;
  float M = -INFINITY;
  float L = 0.f;
  float o[E];
#pragma unroll
  for (int e = 0; e < E; ++e) o[e] = 0.f;
  const int per = (splits + W - 1) / W;  // this wave's splits: [s_lo, s_hi)
  const int s_lo = wave * per;
  const int s_hi = min(splits, s_lo + per);
  // a whole chunk is one pass of one chunk: its loop bounds are compile-time
  // (split indices are immediates, not additions to a loop counter)
  constexpr bool kOnePass = FCH > 0;
  for (int s64 = s_lo; kOnePass ? s64 < 1 : s64 < s_hi; s64 += 64) {
    const int n = kOnePass ? FCH : min(64, s_hi - s64);  // splits of this pass, one per lane
    const int sj = s64 + min(lane, n - 1);
    const float lm = p.mx[sb + sj * ss2];
    const float ll = p.sm[sb + sj * ss2];
    constexpr bool FULL = FCH > 0;
    constexpr int CH = FULL ? FCH : kReduceChunk;
    for (int c0 = 0; kOnePass ? c0 < 1 : c0 < n; c0 += CH) {
      float a[CH][E];
      // whole chunks of D-float rows: one base, constant offsets (immediates)
      [[maybe_unused]] const float* cbase = ab + (s64 + c0) * D + (PAIR ? 2 * lane : lane);
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        if constexpr (PAIR) {
          const float2 v2 = *reinterpret_cast<const float2*>(cbase + j * D);
          a[j][0] = v2.x;
          a[j][1] = v2.y;
        } else if constexpr (FULL) {
#pragma unroll
          for (int e = 0; e < E; ++e) a[j][e] = cbase[j * D + 64 * e];
        } else {
          const int s = s64 + min(c0 + j, n - 1);  // past the end: re-read, masked below
#pragma unroll
          for (int e = 0; e < E; ++e) a[j][e] = ab[s * p.as2 + (lane + 64 * e) * as3];
        }
      }
      // keep every load above issued before the broadcasts below (they wait)
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (MODE == kReduceCascade && PRE) {
        // the row's prefix length is used here, not where it was loaded: the
        // empty asm keeps the compiler from moving the compare (and its
        // wait) ahead of this chunk's loads
        asm volatile("" : "+v"(row_tb));
        valid = row_tb > 0 ? p.splits : p.tail_splits;
      }
      // The chunk's statistics, one split per lane: their maximum by a wave
      // reduction and each split's weight 2^(m - max) by one exp per lane,
      // not a chain of dependent max and exp steps per split (the same
      // values, bit for bit: a maximum is exact in any order).
      const int cl = lane - c0;  // this lane's split within the chunk
      const bool mine = cl >= 0 && cl < CH && cl < n - c0 && s64 + lane < valid;
      // the statistics are used only from here on: on the clamped path the
      // empty asm keeps the compiler from hoisting their uses (and the wait
      // for them) above the chunk's partial loads
      float lmv = lm, llv = ll;
      if constexpr (!FULL) asm volatile("" : "+v"(lmv), "+v"(llv));
      // a whole chunk of at most 16 splits sits in lanes 0-15, the first DPP
      // row: its maximum needs no swaps across rows (the other rows' lanes
      // hold -inf and are never broadcast from)
      const float cmx = mine ? lmv : -INFINITY;
      const float nm = fmaxf(M, FULL && FCH <= 16 ? row_max_f32(cmx) : wave_max_f32(cmx));
      const float nmu = nm == -INFINITY ? 0.f : nm;
      const float sc = exp2_fast(M - nmu);
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] *= sc;
      const float wl = exp2_fast(lmv - nmu);
      {
        // the chunk's denominator: each lane's term w * l (zero for a lane
        // outside the chunk or past the row's valid splits, whatever its
        // slot holds), summed over the chunk's DPP row (two rows for a whole
        // chunk of 32) instead of one broadcast and fused multiply-add per
        // split
        const float t = merge_term(wl, llv);
        const float rs = row_sum_f32(mine ? t : 0.f);
        const float lc = CH > 16 ? lane_bcast(rs, c0) + lane_bcast(rs, c0 + 16) : lane_bcast(rs, c0);
        L = __builtin_fmaf(L, sc, lc);
      }
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        const int src = FULL ? c0 + j : min(c0 + j, n - 1);
        const bool use = FULL || (c0 + j < n && s64 + c0 + j < valid);
        if constexpr (MODE == kReduceCascade) {
          // masked splits may hold stale or NaN partials: selected away, not weighted by 0
          const float w = lane_bcast(wl, src);
#pragma unroll
          for (int e = 0; e < E; ++e) o[e] += use ? w * a[j][e] : 0.f;
        } else {
          // every split below n holds this call's partials and the loads past
          // n re-read split n - 1, so a zero weight masks them; the sums are
          // fused multiply-adds on every path (whole chunks, clamped chunks
          // and the in-launch merge round alike)
          // the broadcast runs on every path: a broadcast under the uniform
          // test becomes a branch, and the branches let the compiler sink
          // the chunk's partial loads below the statistics' wait
          const float wb = lane_bcast(wl, src);
          const float w = use ? wb : 0.f;
#pragma unroll
          for (int e = 0; e < E; ++e) o[e] += w * a[j][e];
        }
      }
      M = nm;
    }
  }
  if constexpr (W > 1) {
    // the waves' states (a wave without splits holds M = -inf, L = 0, o = 0)
    __shared__ float s_m[W], s_l[W];
    __shared__ float s_o[W][D];
    if (lane == 0) {
      s_m[wave] = M;
      s_l[wave] = L;
    }
#pragma unroll
    for (int e = 0; e < E; ++e) s_o[wave][lane + 64 * e] = o[e];
    __syncthreads();
    if (wave != 0) return;
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) mm = fmaxf(mm, s_m[w]);
    const float mu = mm == -INFINITY ? 0.f : mm;
    L = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float wt = exp2_fast(s_m[w] - mu);
      L += wt * s_l[w];
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] += wt * s_o[w][lane + 64 * e];
    }
  }
  const bool has = PRE || (seq_len > 0 && (!p.fuse || slot >= 0));
  const float inv = (has && L > 0.f) ? rcp_fast(L) : 0.f;
  // OUTP: the output is [rows, D] in row order (its pointer preloaded), so
  // the store needs no output strides from the kernel-argument buffer
  T* dst = static_cast<T*>(p.out) + (OUTP ? row * D : b * p.os0 + qh * p.os1);
  if constexpr (PAIR) {
    struct alignas(4) Two {
      T x, y;
    };
    *reinterpret_cast<Two*>(dst + 2 * lane) = Two{from_f32<T>(o[0] * inv), from_f32<T>(o[1] * inv)};
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) dst[(lane + 64 * e) * (OUTP ? 1 : p.os2)] = from_f32<T>(o[e] * inv);
  }
}

template <typename T, int D, int MODE = kReducePlain, int W = 1>
__global__ __launch_bounds__(64 * W) void split_reduce_kernel(ReduceParams p) {
  reduce_row<T, D, MODE, W, false>(p);
}

// The plain merge over a [rows, hq, splits, D] workspace, with the partials'
// addressing in leading arguments that the command processor preloads into
// SGPRs (as for decode_mfma_kernel).  Its loads then issue at wave start
// instead of after a kernel-argument round trip: with the preloaded attention
// kernel, a C2 call in a graph went from 9.37 to 8.74 us.  The preload holds
// 14 SGPRs (56 bytes of arguments): with 64-bit strides the XCD layout's
// row count fell just outside it, and its fetch held every partial load
// back by one round trip; with 32-bit strides (the host checks they fit)
// everything up to xcd_rows is preloaded (C2 8.63 -> 8.40 us per call, one
// box).  The output pointer fills the last two SGPRs: with an output in row
// order (OUTP) the kernel reads nothing from the argument buffer, whose fetch
// otherwise sat ahead of the output stores (C2 8.26 -> 8.15 us, one box).
template <typename T, int D, int W = 1, bool OUTP = false, int FCH = 0>
__global__ __launch_bounds__(64 * W) void split_reduce_pre_kernel(const float* acc, const float* mx, const float* sm,
                                                                  int32_t as1, int32_t as2, int32_t ss1,
                                                                  int32_t splits, int32_t hq, int32_t xcd_rows,
                                                                  void* out, ReduceParams p) {
  ReduceParams q = p;
  q.out = out;
  q.acc = acc;
  q.mx = mx;
  q.sm = sm;
  q.as1 = as1;
  q.as2 = as2;
  q.ss1 = ss1;
  q.splits = splits;
  q.hq = hq;
  reduce_row<T, D, kReducePlain, W, true, OUTP, FCH>(q, xcd_logical_block(blockIdx.x, xcd_rows));
}

// The cascade merge over a packed workspace (as split_reduce_pre_kernel),
// with the row prefix lengths' address preloaded too (32-bit strides make
// room for it in the 14 preloaded SGPRs): every split's partial loads issue
// without waiting for a prefix length, and rows without a prefix mask the
// prefix splits once their length arrives.
template <typename T, int D>
__global__ __launch_bounds__(64) void split_reduce_cascade_pre_kernel(const float* acc, const float* mx,
                                                                      const float* sm, int32_t as1, int32_t as2,
                                                                      int32_t ss1, int32_t splits, int32_t hq,
                                                                      const int32_t* tb, ReduceParams p) {
  ReduceParams q = p;
  q.acc = acc;
  q.mx = mx;
  q.sm = sm;
  q.as1 = as1;
  q.as2 = as2;
  q.ss1 = ss1;
  q.splits = splits;
  q.hq = hq;
  q.tb = tb;
  reduce_row<T, D, kReduceCascade, 1, true>(q);
}

// ========================================================== host glue ====
namespace {

int g_num_cus = 0;

int device_cus() {
  if (g_num_cus > 0) return g_num_cus;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) == hipSuccess &&
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0)
    g_num_cus = cus;
  else
    g_num_cus = 256;
  return g_num_cus;
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

// The MFMA row kernel: head_dim 128 or 64, unit dim strides and 16-byte
// aligned rows (groups of more than 16 query heads per KV head take several
// head blocks).  The cascade, per-row splits, fused RoPE and the in-launch
// merge need head_dim 128 and <= 16 query heads per KV head as well.
bool fast_path_ok(const fd_paged_decode_args& a, int64_t group) {
  if ((a.head_dim != 128 && a.head_dim != 64) || group > 256) return false;
  if (a.q_stride[2] != 1 || a.k_stride[3] != 1 || a.v_stride[3] != 1) return false;
  const int64_t strides[] = {a.q_stride[0], a.q_stride[1], a.k_stride[0], a.k_stride[1], a.k_stride[2],
                             a.v_stride[0], a.v_stride[1], a.v_stride[2]};
  for (int64_t s : strides)
    if (s % 8 != 0) return false;
  if (!aligned16(a.q) || !aligned16(a.k_cache) || !aligned16(a.v_cache)) return false;
  // the MFMA kernel takes the block table's strides and width as 32-bit
  // preloaded arguments
  for (int64_t t : {a.block_tables_stride[0], a.block_tables_stride[1], a.max_blocks_per_seq})
    if (t < 0 || t > INT32_MAX) return false;
  // a row's byte offset inside its block (head, token slot, dims) is a
  // 32-bit lane offset in the MFMA kernel's loads
  for (const int64_t* st : {a.k_stride, a.v_stride}) {
    if (st[0] < 0 || st[1] < 0 || st[2] < 0) return false;
    const int64_t in_block = (a.num_kv_heads - 1) * st[1] + (a.block_size - 1) * st[2] + a.head_dim;
    if (in_block * 2 > 0xffffffffLL) return false;
  }
  if (a.append_k) {
    if (a.append_k_stride[2] != 1 || a.append_v_stride[2] != 1) return false;
    const int64_t as[] = {a.append_k_stride[0], a.append_k_stride[1], a.append_v_stride[0],
                          a.append_v_stride[1]};
    for (int64_t s : as)
      if (s % 8 != 0) return false;
    if (!aligned16(a.append_k) || !aligned16(a.append_v)) return false;
  }
  return true;
}

// Dim-major caches on the MFMA path (decode_dm_kernel): 64- or 128-dim heads,
// token stride 1, 16-byte aligned dim rows (the fused append's rows may have
// any strides: they are read and stored one element at a time).
bool dm_path_ok(const fd_paged_decode_args& a, int64_t group) {
  if ((a.head_dim != 128 && a.head_dim != 64) || group > 256) return false;
  if (a.q_stride[2] != 1 || a.k_stride[2] != 1 || a.v_stride[2] != 1) return false;
  const int64_t strides[] = {a.q_stride[0], a.q_stride[1], a.k_stride[0], a.k_stride[1], a.k_stride[3],
                             a.v_stride[0], a.v_stride[1], a.v_stride[3]};
  for (int64_t s : strides)
    if (s % 8 != 0) return false;
  return aligned16(a.q) && aligned16(a.k_cache) && aligned16(a.v_cache);
}

// One dispatch; events given are recorded at its start / end (profiling hook).
template <typename F, typename... Args>
void dispatch(F kernel, dim3 grid, dim3 block, hipStream_t stream, void* start, void* stop, Args... args) {
  if (launch_record_on()) record_launch(reinterpret_cast<const void*>(kernel), stream);
  if (start || stop)
    hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, static_cast<hipEvent_t>(start),
                          static_cast<hipEvent_t>(stop), 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, 0, stream, args...);
}

// Workgroups per (request, KV head, split) of the MFMA row kernel: one for
// up to 16 query heads per KV head, else one per 32 (two column blocks).
int64_t row_head_blocks(int64_t group) {
  return group > 16 ? (group + 16 * kRowWideColBlocks - 1) / (16 * kRowWideColBlocks) : 1;
}

// A streaming row kernel's grid is laid out XCD by XCD (xcd_logical_block)
// when it is a multiple of 8 workgroups and each (request, KV head) has at
// least kXcdMinPairBlocks of them (splits x head blocks): they then share the
// q rows, the block-table row and, across head blocks, the K/V through one
// XCD's L2 instead of fetching them into several.  Same-box MI355X A/B,
// us/call: C2 (B8 ctx2048, 16 splits) 8.74 -> 8.41, attention kernel 5.39 ->
// 5.18; B16 x 8192 G71 D64 (3 head blocks, 5 splits) 27.4 -> 22.8; G32 32.2
// -> 31.6; dim-major D128 27.0 -> 26.5.  With 2 splits (B64 ctx8192) the
// kernel measured 1 % slower (91.7 -> 92.7 us), hence the threshold.  Cached
// loads (kv_reuse) keep the hardware order: rows sharing a prefix then read
// its tiles on the same XCDs (consecutive workgroups are splits of one row,
// and a split's tile range recurs on the same XCD every 4 rows at 10
// splits), which the XCD-by-XCD layout breaks: 64 rows on a 16384-token
// prefix, 94.8 -> 114.0 us.
constexpr int64_t kXcdMinPairBlocks = 4;

// Workgroups per XCD for xcd_logical_block (0: hardware order)
int32_t row_xcd_blocks(unsigned grid, int64_t pair_blocks, bool nt) {
  return nt && grid % 8 == 0 && pair_blocks >= kXcdMinPairBlocks ? static_cast<int32_t>(grid / 8) : 0;
}

// Multiplier and shifts (bits 0-7 s1, 8-15 s2) for fast_div by d >= 1:
// l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1, s1 = min(l, 1),
// s2 = max(l - 1, 0).
void fast_div_magic(uint32_t d, uint32_t& m, int& shifts) {
  int l = 0;
  while ((uint64_t{1} << l) < d) ++l;
  m = static_cast<uint32_t>(((uint64_t{1} << 32) * ((uint64_t{1} << l) - d)) / d + 1);
  shifts = (l < 1 ? l : 1) | ((l > 1 ? l - 1 : 0) << 8);
}

// decode_mfma_kernel's arguments: the block-table fields and the workgroup
// index's divisors (all within the 14 preloaded SGPRs: 32-bit table strides,
// which fast_path_ok checks), then the parameter block
template <typename K>
void dispatch_mfma(K kernel, dim3 grid, dim3 block, hipStream_t stream, void* const* ev, const DecodeParams& p,
                   bool nt) {
  uint32_t ms = 0, mh = 0;
  int ss = 0, sh = 0;
  fast_div_magic(static_cast<uint32_t>(p.splits), ms, ss);
  fast_div_magic(static_cast<uint32_t>(p.hkv), mh, sh);
  dispatch(kernel, grid, block, stream, ev[0], ev[1], p.bt, static_cast<int32_t>(p.bts0), static_cast<int32_t>(p.bts1),
           static_cast<int32_t>(p.max_blocks_per_seq), p.splits, p.hkv, p.group, p.hint_tps,
           row_xcd_blocks(grid.x, p.splits * row_head_blocks(p.group), nt), ms, mh, ss | (sh << 16), p.bt_i64, p);
}

template <typename T, int BS, int UNIT, bool NT>
void launch_mfma_unit(const DecodeParams& p, dim3 grid, hipStream_t stream, void* const* ev) {
  const bool merge = p.counters != nullptr;
  const dim3 block(64 * waves_for<UNIT>());
  if (p.head_dim == 64) {
    // head_dim 64: the host gives it no RoPE and no in-launch merge
    if (p.fuse)
      dispatch_mfma(decode_mfma_kernel<T, BS, 1, false, UNIT, NT, 64>, grid, block, stream, ev, p, NT);
    else
      dispatch_mfma(decode_mfma_kernel<T, BS, 0, false, UNIT, NT, 64>, grid, block, stream, ev, p, NT);
    return;
  }
  if (p.fuse && p.rope_dim > 0) {
    // the host refuses RoPE with the in-launch merge
    dispatch_mfma(decode_mfma_kernel<T, BS, 2, false, UNIT, NT>, grid, block, stream, ev, p, NT);
  } else if (p.fuse) {
    if (merge)
      dispatch_mfma(decode_mfma_kernel<T, BS, 1, true, UNIT, NT>, grid, block, stream, ev, p, NT);
    else
      dispatch_mfma(decode_mfma_kernel<T, BS, 1, false, UNIT, NT>, grid, block, stream, ev, p, NT);
  } else {
    if (merge)
      dispatch_mfma(decode_mfma_kernel<T, BS, 0, true, UNIT, NT>, grid, block, stream, ev, p, NT);
    else
      dispatch_mfma(decode_mfma_kernel<T, BS, 0, false, UNIT, NT>, grid, block, stream, ev, p, NT);
  }
}

// 32-token units on four waves when a split holds about one unit per wave
// (C2: 4 tiles per split, 6.4 vs 6.7 us), 16-token units on eight waves for
// longer splits (ragged B32: 70 -> 60 us; C5 layer: 97 -> 93 us).  8-token
// blocks always take 16-token units (a unit spans at most two blocks).
// Groups of more than 16 query heads per KV head: two 16-column blocks per
// wave on 16-token units (the head dims and fused append as above; the host
// gives them no RoPE and no in-launch merge).
template <typename T, int BS, bool NT>
void launch_mfma_wide(const DecodeParams& p, dim3 grid, hipStream_t stream, void* const* ev) {
  constexpr int W = kRowWideColBlocks;
  const dim3 block(64 * waves_for<16>());
  if (p.head_dim == 64) {
    if (p.fuse)
      dispatch_mfma(decode_mfma_kernel<T, BS, 1, false, 16, NT, 64, W>, grid, block, stream, ev, p, NT);
    else
      dispatch_mfma(decode_mfma_kernel<T, BS, 0, false, 16, NT, 64, W>, grid, block, stream, ev, p, NT);
  } else {
    if (p.fuse)
      dispatch_mfma(decode_mfma_kernel<T, BS, 1, false, 16, NT, 128, W>, grid, block, stream, ev, p, NT);
    else
      dispatch_mfma(decode_mfma_kernel<T, BS, 0, false, 16, NT, 128, W>, grid, block, stream, ev, p, NT);
  }
}

template <typename T, int BS, bool NT>
void launch_mfma(const DecodeParams& p, dim3 grid, hipStream_t stream, void* const* ev) {
  if (p.group > 16) {
    launch_mfma_wide<T, BS, NT>(p, grid, stream, ev);
    return;
  }
  if constexpr (BS >= 16) {
    if (p.hint_tps <= kWideUnitMaxTiles) {
      launch_mfma_unit<T, BS, 32, NT>(p, grid, stream, ev);
      return;
    }
  }
  launch_mfma_unit<T, BS, 16, NT>(p, grid, stream, ev);
}

template <typename T, int BS>
void launch_mfma(const DecodeParams& p, bool nt, dim3 grid, hipStream_t stream, void* const* ev) {
  if (nt)
    launch_mfma<T, BS, true>(p, grid, stream, ev);
  else
    launch_mfma<T, BS, false>(p, grid, stream, ev);
}

template <typename T, int D, int FUSE>
void launch_dm(const DecodeParams& p, int64_t block_size, bool nt, dim3 grid, dim3 block, hipStream_t stream,
               void* const* ev, int32_t xcd) {
  if (block_size == 8)
    nt ? dispatch(decode_dm_kernel<T, 8, true, D, FUSE>, grid, block, stream, ev[0], ev[1], p, xcd)
       : dispatch(decode_dm_kernel<T, 8, false, D, FUSE>, grid, block, stream, ev[0], ev[1], p, xcd);
  else if (block_size == 16)
    nt ? dispatch(decode_dm_kernel<T, 16, true, D, FUSE>, grid, block, stream, ev[0], ev[1], p, xcd)
       : dispatch(decode_dm_kernel<T, 16, false, D, FUSE>, grid, block, stream, ev[0], ev[1], p, xcd);
  else
    nt ? dispatch(decode_dm_kernel<T, 32, true, D, FUSE>, grid, block, stream, ev[0], ev[1], p, xcd)
       : dispatch(decode_dm_kernel<T, 32, false, D, FUSE>, grid, block, stream, ev[0], ev[1], p, xcd);
}

ReduceParams reduce_params(const DecodeParams& p) {
  ReduceParams r{};
  r.acc = p.acc;
  r.mx = p.mx;
  r.sm = p.sm;
  r.out = p.out;
  r.sl = p.sl;
  r.slot = p.fuse ? p.slot : p.sl;
  r.as0 = p.as0;
  r.as1 = p.as1;
  r.as2 = p.as2;
  r.as3 = p.as3;
  r.ss0 = p.ss0;
  r.ss1 = p.ss1;
  r.ss2 = p.ss2;
  r.os0 = p.os0;
  r.os1 = p.os1;
  r.os2 = p.os2;
  r.sls = p.sls;
  r.slots = p.fuse ? p.slots : p.sls;
  r.hq = p.hq;
  r.splits = p.splits;
  r.fuse = p.fuse;
  r.sl_i64 = p.sl_i64;
  r.slot_i64 = p.fuse ? p.slot_i64 : p.sl_i64;
  r.tb = nullptr;
  r.tail_splits = p.splits;
  r.bal_target = p.bal_target;
  r.num_seqs = p.num_seqs;
  r.cap = p.max_blocks_per_seq * p.block_size;
  return r;
}

// The plain merge's workspace has the layout split_reduce_pre_kernel assumes
bool reduce_layout_packed(const ReduceParams& r) {
  return r.as3 == 1 && r.ss2 == 1 && r.as0 == r.hq * r.as1 && r.ss0 == r.hq * r.ss1;
}

// xcd_rows: the plain merge of a row kernel laid out XCD by XCD takes the same
// layout (grid / 8 rows per XCD), so that each row's merge runs on the XCD
// whose workgroups wrote its partials; false keeps the hardware order.
template <typename T, int MODE>
int launch_reduce(const fd_paged_decode_args& a, const ReduceParams& r, hipStream_t stream, bool xcd_rows = false) {
  const dim3 grid(static_cast<unsigned>(a.num_seqs * a.num_q_heads));
  void* e0 = a.timing_events[2];
  void* e1 = a.timing_events[3];
  // 32-bit strides keep every argument the partials' addresses need inside
  // the 14 preloaded SGPRs
  auto fits = [](int64_t x) { return x >= 0 && x <= INT32_MAX; };
  const bool pre_ok = reduce_layout_packed(r) && fits(r.as1) && fits(r.as2) && fits(r.ss1);
  if (MODE == kReducePlain && pre_ok) {
    // the partials' addressing leads the argument list (preloaded into SGPRs)
    auto pre = [&](auto kernel, dim3 block) {
      dispatch(kernel, grid, block, stream, e0, e1, r.acc, r.mx, r.sm, static_cast<int32_t>(r.as1),
               static_cast<int32_t>(r.as2), static_cast<int32_t>(r.ss1), r.splits, r.hq,
               xcd_rows && grid.x % 8 == 0 ? static_cast<int32_t>(grid.x / 8) : 0, r.out, r);
    };
    // output rows in order: [requests, q heads, head_dim] with unit dim stride
    const bool outp = r.os2 == 1 && r.os1 == a.head_dim && r.os0 == r.hq * r.os1;
    if (r.splits > 32) {
      if (a.head_dim == 64)
        outp ? pre(split_reduce_pre_kernel<T, 64, 4, true>, dim3(256)) : pre(split_reduce_pre_kernel<T, 64, 4>, dim3(256));
      else
        outp ? pre(split_reduce_pre_kernel<T, 128, 4, true>, dim3(256))
             : pre(split_reduce_pre_kernel<T, 128, 4>, dim3(256));
    } else if (outp && r.as2 == a.head_dim && r.as1 == r.splits * a.head_dim && r.ss1 == r.splits &&
               (r.splits == 2 || r.splits == 4 || r.splits == 8 || r.splits == 16 || r.splits == 32) &&
               (reinterpret_cast<uintptr_t>(r.acc) & 7) == 0 && (reinterpret_cast<uintptr_t>(r.out) & 3) == 0) {
      // contiguous [rows, splits, D] partials with a power-of-two split count
      // (the library's own workspaces: C2 has 16, its ctx1024 companion 8):
      // every partial load is an immediate offset from one base, with no
      // clamp, no per-split address and no select
      auto full = [&](auto k2, auto k4, auto k8, auto k16, auto k32) {
        switch (r.splits) {
          case 2: pre(k2, dim3(64)); break;
          case 4: pre(k4, dim3(64)); break;
          case 8: pre(k8, dim3(64)); break;
          case 16: pre(k16, dim3(64)); break;
          default: pre(k32, dim3(64)); break;
        }
      };
      if (a.head_dim == 64)
        full(split_reduce_pre_kernel<T, 64, 1, true, 2>, split_reduce_pre_kernel<T, 64, 1, true, 4>,
             split_reduce_pre_kernel<T, 64, 1, true, 8>, split_reduce_pre_kernel<T, 64, 1, true, 16>,
             split_reduce_pre_kernel<T, 64, 1, true, 32>);
      else
        full(split_reduce_pre_kernel<T, 128, 1, true, 2>, split_reduce_pre_kernel<T, 128, 1, true, 4>,
             split_reduce_pre_kernel<T, 128, 1, true, 8>, split_reduce_pre_kernel<T, 128, 1, true, 16>,
             split_reduce_pre_kernel<T, 128, 1, true, 32>);
    } else if (a.head_dim == 64) {
      outp ? pre(split_reduce_pre_kernel<T, 64, 1, true>, dim3(64)) : pre(split_reduce_pre_kernel<T, 64>, dim3(64));
    } else {
      outp ? pre(split_reduce_pre_kernel<T, 128, 1, true>, dim3(64)) : pre(split_reduce_pre_kernel<T, 128>, dim3(64));
    }
  } else if (MODE == kReduceCascade && pre_ok && r.splits <= 32 && a.head_dim == 128) {
    dispatch(split_reduce_cascade_pre_kernel<T, 128>, grid, dim3(64), stream, e0, e1, r.acc, r.mx, r.sm,
             static_cast<int32_t>(r.as1), static_cast<int32_t>(r.as2), static_cast<int32_t>(r.ss1), r.splits, r.hq,
             r.tb, r);
  } else if (r.splits > 32) {
    // more than 32 splits: four waves per row share them
    if (a.head_dim == 64)
      dispatch(split_reduce_kernel<T, 64, MODE, 4>, grid, dim3(256), stream, e0, e1, r);
    else
      dispatch(split_reduce_kernel<T, 128, MODE, 4>, grid, dim3(256), stream, e0, e1, r);
  } else if (a.head_dim == 64) {
    dispatch(split_reduce_kernel<T, 64, MODE>, grid, dim3(64), stream, e0, e1, r);
  } else {
    dispatch(split_reduce_kernel<T, 128, MODE>, grid, dim3(64), stream, e0, e1, r);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(FD_E_LAUNCH, "split reduce launch failed: %s", hipGetErrorString(e));
  return FD_OK;
}


template <typename T>
int launch_decode(const fd_paged_decode_args& a, DecodeParams& p, hipStream_t stream) {
  const int64_t pairs = a.num_seqs * a.num_kv_heads;
  const bool fast = fast_path_ok(a, p.group);
  const bool nt = a.kv_reuse == 0;  // stream K/V past the caches
  // the in-launch merge exists only in the MFMA kernel and writes the
  // workspace with 8-byte stores (unit dim stride, 8-byte aligned rows)
  const bool narrow = a.head_dim == 128 && p.group <= 16;  // one head block of 128-dim heads
  if (!fast || !narrow || p.splits == 1 || p.as3 != 1 || (p.as2 & 1) || (p.as1 & 1) || (p.as0 & 1) ||
      (reinterpret_cast<uintptr_t>(p.acc) & 7u))
    p.counters = nullptr;
  // balanced splits need the MFMA kernel with one head block of 128-dim
  // heads, no fused append and a workspace
  const bool balanced = p.bal_target > 0 && fast && narrow && !p.fuse && p.splits > 1;
  if (!balanced) p.bal_target = 0;
  bool xcd = false;  // the row kernel's grid laid out XCD by XCD
  if (balanced) {
    p.counters = nullptr;
    // sum over rows of ceil(tiles_b / T) <= bal_target + num_seqs
    const dim3 grid(static_cast<unsigned>(a.num_kv_heads * (p.bal_target + a.num_seqs)));
    const dim3 block(64 * kBalWaves);
    void* const* ev = a.timing_events;
    switch (a.block_size) {
      case 8:
        nt ? dispatch(decode_balanced_kernel<T, 8, true>, grid, block, stream, ev[0], ev[1], p)
           : dispatch(decode_balanced_kernel<T, 8, false>, grid, block, stream, ev[0], ev[1], p);
        break;
      case 16:
        nt ? dispatch(decode_balanced_kernel<T, 16, true>, grid, block, stream, ev[0], ev[1], p)
           : dispatch(decode_balanced_kernel<T, 16, false>, grid, block, stream, ev[0], ev[1], p);
        break;
      default:
        nt ? dispatch(decode_balanced_kernel<T, 32, true>, grid, block, stream, ev[0], ev[1], p)
           : dispatch(decode_balanced_kernel<T, 32, false>, grid, block, stream, ev[0], ev[1], p);
        break;
    }
  } else if (fast) {
    const int64_t hblocks = row_head_blocks(p.group);
    const dim3 grid(static_cast<unsigned>(pairs * hblocks * p.splits));
    xcd = row_xcd_blocks(grid.x, p.splits * hblocks, nt) > 0;
    switch (a.block_size) {
      case 8: launch_mfma<T, 8>(p, nt, grid, stream, a.timing_events); break;
      case 16: launch_mfma<T, 16>(p, nt, grid, stream, a.timing_events); break;
      default: launch_mfma<T, 32>(p, nt, grid, stream, a.timing_events); break;
    }
  } else if (dm_path_ok(a, p.group)) {
    const int64_t hblocks = (p.group + 15) / 16;
    const dim3 grid(static_cast<unsigned>(pairs * hblocks * p.splits));
    const dim3 block(64 * kDmWaves);
    void* const* ev = a.timing_events;
    const int32_t per_xcd = row_xcd_blocks(grid.x, p.splits * hblocks, nt);
    xcd = per_xcd > 0;
    if (a.head_dim == 64)
      p.fuse ? launch_dm<T, 64, 1>(p, a.block_size, nt, grid, block, stream, ev, per_xcd)
             : launch_dm<T, 64, 0>(p, a.block_size, nt, grid, block, stream, ev, per_xcd);
    else
      p.fuse ? launch_dm<T, 128, 1>(p, a.block_size, nt, grid, block, stream, ev, per_xcd)
             : launch_dm<T, 128, 0>(p, a.block_size, nt, grid, block, stream, ev, per_xcd);
  } else {
    const int hg = static_cast<int>((p.group + kGenHeads - 1) / kGenHeads);
    const dim3 grid(static_cast<unsigned>(pairs * hg), static_cast<unsigned>(p.splits));
    void* const* ev = a.timing_events;
    if (a.head_dim == 64)
      dispatch(decode_generic_kernel<T, 64>, grid, dim3(64), stream, ev[0], ev[1], p, hg);
    else
      dispatch(decode_generic_kernel<T, 128>, grid, dim3(64), stream, ev[0], ev[1], p, hg);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(FD_E_LAUNCH, "decode launch failed: %s", hipGetErrorString(e));
  if (p.splits > 1 && p.counters == nullptr) {
    const ReduceParams r = reduce_params(p);
    const int rc =
        balanced ? launch_reduce<T, kReduceBalanced>(a, r, stream) : launch_reduce<T, kReducePlain>(a, r, stream, xcd);
    if (rc != FD_OK) return rc;
  }
  return FD_OK;
}


// Cascade: one launch of prefix- and tail-role workgroups, then the reducer
// over tail + prefix partials.  The attention timing events bracket it.
// cascade_decode_kernel's arguments: the preloaded prefix-role fields, then the parameter blocks
template <typename K>
void dispatch_cascade(K kernel, dim3 grid, dim3 block, hipStream_t stream, void* const* ev, const DecodeParams& p,
                      const CascadeParams& cp) {
  dispatch(kernel, grid, block, stream, ev[0], ev[1], static_cast<int32_t>(cp.prefix_blocks),
           static_cast<int32_t>(cp.prefix_splits), static_cast<int32_t>(cp.chunks), p.hkv,
           static_cast<int32_t>(cp.hint_ptps), cp.members, static_cast<int32_t>(cp.max_members), p, cp);
}

template <typename T, int BS, bool NT>
void launch_cascade_kernel(const DecodeParams& p, const CascadeParams& cp, int col_blocks, int64_t pairs,
                           hipStream_t stream, void* const* ev) {
  const dim3 grid(static_cast<unsigned>(cp.prefix_blocks + pairs * p.splits));
  if (col_blocks == 2) {
    // long prefixes shared by many rows: 16-token units, two column blocks
    dispatch_cascade(cascade_decode_kernel<T, BS, 16, NT, 2>, grid, dim3(64 * waves_for<16>()), stream, ev, p, cp);
    return;
  }
  if constexpr (BS >= 16) {
    if (p.hint_tps <= kWideUnitMaxTiles && cp.hint_ptps <= kWideUnitMaxTiles) {
      dispatch_cascade(cascade_decode_kernel<T, BS, 32, NT>, grid, dim3(64 * waves_for<32>()), stream, ev, p, cp);
      return;
    }
  }
  dispatch_cascade(cascade_decode_kernel<T, BS, 16, NT>, grid, dim3(64 * waves_for<16>()), stream, ev, p, cp);
}

// NT applies to the tail role; the prefix role always uses plain loads
template <typename T, int BS>
void launch_cascade_kernel(const DecodeParams& p, const CascadeParams& cp, int col_blocks, bool nt, int64_t pairs,
                           hipStream_t stream, void* const* ev) {
  if (nt)
    launch_cascade_kernel<T, BS, true>(p, cp, col_blocks, pairs, stream, ev);
  else
    launch_cascade_kernel<T, BS, false>(p, cp, col_blocks, pairs, stream, ev);
}

template <typename T>
int launch_cascade(const fd_paged_decode_args& a, const DecodeParams& p, const CascadeParams& cp, int col_blocks,
                   hipStream_t stream) {
  const int64_t pairs = a.num_seqs * a.num_kv_heads;
  const bool nt = a.kv_reuse == 0;
  void* const* ev = a.timing_events;
  switch (a.block_size) {
    case 8: launch_cascade_kernel<T, 8>(p, cp, col_blocks, nt, pairs, stream, ev); break;
    case 16: launch_cascade_kernel<T, 16>(p, cp, col_blocks, nt, pairs, stream, ev); break;
    default: launch_cascade_kernel<T, 32>(p, cp, col_blocks, nt, pairs, stream, ev); break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(FD_E_LAUNCH, "cascade decode launch failed: %s", hipGetErrorString(e));
  ReduceParams r = reduce_params(p);
  r.splits = p.splits + cp.prefix_splits;
  r.tb = p.tb;
  r.tail_splits = p.splits;
  return launch_reduce<T, kReduceCascade>(a, r, stream);
}

}  // namespace

}  // namespace fd

#ifdef FD_TIMELINE
// Measurement build only: the device address and size of the timeline slots.
extern "C" int fd_timeline_buffer(void** ptr, uint64_t* bytes) {
  if (ptr == nullptr || bytes == nullptr) return FD_E_INVALID;
  if (hipGetSymbolAddress(ptr, HIP_SYMBOL(fd::g_timeline)) != hipSuccess) return FD_E_LAUNCH;
  *bytes = sizeof(fd::g_timeline);
  return FD_OK;
}
#endif

using namespace fd;

extern "C" int fd_paged_decode_balance_target(int64_t num_seqs, int64_t num_kv_heads) {
  if (num_seqs <= 0 || num_kv_heads <= 0)
    return set_error(FD_E_INVALID, "fd_paged_decode_balance_target: non-positive shape");
  // One round of workgroups (kBalPerCU per CU): sum over rows of S_b <=
  // V + B, so V = kBalPerCU * CUs / Hkv - B keeps the grid within it.
  // Ragged B32 on MI355X (Σ L = 206 k, max 30.7 k): attention 58.4 us with
  // 16 uniform splits; one 8-wave workgroup per CU, V = 64 / 96 / 128 / 224:
  // 46.9 / 41.9 / 56.2 / 44.2 us; two 4-wave workgroups per CU, V = 224:
  // 38.7 us.  A batch that already fills a round gets 0: uniform splits.
  const int64_t v = kBalPerCU * device_cus() / num_kv_heads - num_seqs;
  return v >= num_seqs && v <= (1 << 20) ? static_cast<int>(v) : 0;
}

extern "C" int fd_paged_decode_plan(int64_t num_seqs, int64_t num_q_heads, int64_t num_kv_heads,
                                    int64_t head_dim, int64_t max_seq_len, int64_t total_seq_len) {
  if (num_seqs <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || max_seq_len < 0 ||
      total_seq_len < 0)
    return set_error(FD_E_INVALID, "fd_paged_decode_plan: non-positive shape");
  const int64_t tiles = (max_seq_len + 31) / 32;
  // groups of more than 16 query heads per KV head: one workgroup per head
  // block of 32, each reading the row's K/V
  const int64_t group = num_q_heads / num_kv_heads;
  const int64_t hblocks = (head_dim == 128 || head_dim == 64) ? row_head_blocks(group) : 1;
  const int64_t pairs = num_seqs * num_kv_heads * hblocks;
  const int64_t cus = device_cus();
  // one workgroup per CU for a batch of equal rows: fewer, longer splits
  // measured best for long uniform rows (36-layer B64 ctx8192 step: 2 splits
  // 4.28 ms, 4 splits 4.45 ms)
  int64_t s = (cus + pairs - 1) / pairs;
  // The longest row's splits must not outlast the average CU's share:
  // max_tiles / S <= total_tiles / CUs.  Unknown totals assume the worst
  // spread and keep the longest row's splits at <= kMaxSplitTiles tiles.
  int64_t balance;
  if (total_seq_len > 0) {
    // in tokens, with 1/8 slack so rounding never lifts a uniform batch
    const int64_t work = 8 * total_seq_len * num_kv_heads * hblocks;
    balance = (7 * max_seq_len * cus + work - 1) / work;
  } else {
    balance = (tiles + kMaxSplitTiles - 1) / kMaxSplitTiles;
  }
  if (s < balance) s = balance;
  // Whole waves of workgroups: a grid of 2.5 workgroups per CU ends with a
  // half-empty wave (one C5 layer, 128 pairs: 4 or 6 splits 109 us, 5 splits
  // 116 us), so round up to the next count that fills every CU (at most 2x).
  bool whole = false;
  for (int64_t t = s; t <= 2 * s && !whole; ++t)
    if ((pairs * t) % cus == 0) {
      s = t;
      whole = true;
    }
  if (!whole) {
    // No count up to 2x fills whole waves (the pair count shares too few
    // factors with the CU count: 48 pairs took 6 splits, 288 workgroups, a
    // second wave of 32).  Take the count from the balance bound up whose
    // last wave is fullest; on a tie, fewer workgroups (48 pairs: 5 splits,
    // one wave of 240).
    int64_t best = s;
    int64_t best_num = 0, best_den = 1;  // fullness best_num / best_den
    for (int64_t t = balance > 1 ? balance : 1; t <= 2 * s; ++t) {
      const int64_t wgs = pairs * t;
      const int64_t den = (wgs + cus - 1) / cus * cus;
      if (wgs * best_den > best_num * den) {
        best = t;
        best_num = wgs;
        best_den = den;
      }
    }
    s = best;
  }
  int64_t cap = (2 * tiles + kMaxWaves - 1) / kMaxWaves;  // >= one unit per wave
  // Rows of at most 8 tiles: two splits of one unit per wave lose to one
  // split of two (16-token) units per wave, which needs no reducer launch
  // (same-box graphs, us/call, S = 1 vs 2: B2/B32/B64 ctx256 D128 5.95/7.69/
  // 8.17 vs 6.85/8.06/9.07; B4 ctx256 D64 5.06 vs 6.19).  Longer rows keep
  // their splits (B8 ctx512 D64: 4 splits 6.54, 1 split 7.22 us).
  if (cap == 2) cap = 1;
  if (s > cap) s = cap;
  if (s > 256) s = 256;
  if (s < 1) s = 1;
  return static_cast<int>(s);
}

// Validates the launch arguments shared by the decode entry points and fills
// the kernel parameters; fn names the entry point in error messages.
static int fill_decode_params(const fd_paged_decode_args* args, const char* fn, DecodeParams& p) {
  if (args == nullptr) return set_error(FD_E_INVALID, "%s: args is NULL", fn);
  const fd_paged_decode_args& a = *args;
  if (a.struct_size != sizeof(fd_paged_decode_args))
    return set_error(FD_E_INVALID, "%s: struct_size %u != %zu (ABI mismatch)", fn, a.struct_size,
                     sizeof(fd_paged_decode_args));
  if (a.dtype != FD_DTYPE_F16 && a.dtype != FD_DTYPE_BF16)
    return set_error(FD_E_UNSUPPORTED, "%s: dtype must be float16 or bfloat16", fn);
  if (a.num_seqs <= 0 || a.num_q_heads <= 0 || a.num_kv_heads <= 0 || a.num_blocks <= 0 ||
      a.max_blocks_per_seq <= 0)
    return set_error(FD_E_INVALID, "%s: shapes must be positive", fn);
  if (a.num_q_heads % a.num_kv_heads != 0)
    return set_error(FD_E_INVALID, "%s: num_q_heads must be divisible by num_kv_heads", fn);
  if (a.head_dim != 64 && a.head_dim != 128)
    return set_error(FD_E_UNSUPPORTED, "%s: head_dim must be 64 or 128", fn);
  if (a.block_size != 8 && a.block_size != 16 && a.block_size != 32)
    return set_error(FD_E_UNSUPPORTED, "%s: block_size must be 8, 16 or 32", fn);
  if (!a.q || !a.k_cache || !a.v_cache || !a.block_tables || !a.seq_lens || !a.out)
    return set_error(FD_E_INVALID, "%s: NULL tensor pointer", fn);
  if (a.num_splits < 1 || a.num_splits > 4096)
    return set_error(FD_E_INVALID, "%s: num_splits must be in [1, 4096]", fn);
  if (a.num_splits > 1 && (!a.split_acc || !a.split_max || !a.split_sum))
    return set_error(FD_E_INVALID, "%s: split workspace required for num_splits > 1", fn);
  const bool fuse = a.append_k != nullptr;
  if (fuse != (a.append_v != nullptr) || fuse != (a.slot_mapping != nullptr))
    return set_error(FD_E_INVALID, "%s: append_k, append_v and slot_mapping go together", fn);
  const int64_t pairs = a.num_seqs * a.num_kv_heads;
  const int64_t hblocks = (a.num_q_heads / a.num_kv_heads + 15) / 16;
  if (pairs * hblocks * a.num_splits > 0x7fffffffLL || a.num_seqs * a.num_q_heads > 0x7fffffffLL)
    return set_error(FD_E_INVALID, "%s: launch grid too large", fn);

  p = DecodeParams{};
  p.q = a.q;
  p.qs0 = a.q_stride[0];
  p.qs1 = a.q_stride[1];
  p.qs2 = a.q_stride[2];
  p.k = a.k_cache;
  p.ks0 = a.k_stride[0];
  p.ks1 = a.k_stride[1];
  p.ks2 = a.k_stride[2];
  p.ks3 = a.k_stride[3];
  p.v = a.v_cache;
  p.vs0 = a.v_stride[0];
  p.vs1 = a.v_stride[1];
  p.vs2 = a.v_stride[2];
  p.vs3 = a.v_stride[3];
  p.bt = a.block_tables;
  p.bts0 = a.block_tables_stride[0];
  p.bts1 = a.block_tables_stride[1];
  p.bt_i64 = a.block_tables_dtype == FD_INDEX_I64;
  p.sl = a.seq_lens;
  p.sls = a.seq_lens_stride;
  p.sl_i64 = a.seq_lens_dtype == FD_INDEX_I64;
  p.out = a.out;
  p.os0 = a.out_stride[0];
  p.os1 = a.out_stride[1];
  p.os2 = a.out_stride[2];
  p.acc = a.split_acc;
  p.as0 = a.split_acc_stride[0];
  p.as1 = a.split_acc_stride[1];
  p.as2 = a.split_acc_stride[2];
  p.as3 = a.split_acc_stride[3];
  p.mx = a.split_max;
  p.sm = a.split_sum;
  p.ss0 = a.split_stats_stride[0];
  p.ss1 = a.split_stats_stride[1];
  p.ss2 = a.split_stats_stride[2];
  p.counters = a.num_splits > 1 ? a.split_counters : nullptr;
  if (p.counters != nullptr && (reinterpret_cast<uintptr_t>(p.counters) & 7u) != 0)
    return set_error(FD_E_INVALID, "%s: split_counters must be 8-byte aligned", fn);
  p.fuse = fuse ? 1 : 0;
  if (fuse) {
    p.ak = a.append_k;
    p.aks0 = a.append_k_stride[0];
    p.aks1 = a.append_k_stride[1];
    p.aks2 = a.append_k_stride[2];
    p.av = a.append_v;
    p.avs0 = a.append_v_stride[0];
    p.avs1 = a.append_v_stride[1];
    p.avs2 = a.append_v_stride[2];
    p.slot = a.slot_mapping;
    p.slots = a.slot_mapping_stride;
    p.slot_i64 = a.slot_mapping_dtype == FD_INDEX_I64;
  }
  p.num_seqs = static_cast<int>(a.num_seqs);
  p.hq = static_cast<int>(a.num_q_heads);
  p.hkv = static_cast<int>(a.num_kv_heads);
  p.group = static_cast<int>(a.num_q_heads / a.num_kv_heads);
  p.head_dim = static_cast<int>(a.head_dim);
  p.block_size = static_cast<int>(a.block_size);
  p.num_blocks = a.num_blocks;
  p.max_blocks_per_seq = a.max_blocks_per_seq;
  p.splits = a.num_splits;
  if (a.max_seq_len < 0) return set_error(FD_E_INVALID, "%s: max_seq_len must be >= 0", fn);
  if (a.balance_target < 0 || a.balance_target > (1 << 20))
    return set_error(FD_E_INVALID, "%s: balance_target must be in [0, 2^20]", fn);
  if (a.num_kv_heads * (a.balance_target + a.num_seqs) > 0x7fffffffLL)
    return set_error(FD_E_INVALID, "%s: launch grid too large", fn);
  p.bal_target = a.balance_target;
  if (a.kv_reuse != 0 && a.kv_reuse != 1) return set_error(FD_E_INVALID, "%s: kv_reuse must be 0 or 1", fn);
  if (a.rotary_dim != 0) {
    if (a.rotary_dim != 64 && a.rotary_dim != 128)
      return set_error(FD_E_UNSUPPORTED, "%s: rotary_dim must be 0, 64 or 128", fn);
    if (!fuse)
      return set_error(FD_E_INVALID, "%s: rotary_dim needs the fused append (append_k, append_v, slot_mapping)", fn);
    if (!(a.rope_base > 0.0) || a.rope_base > 3.4e38)
      return set_error(FD_E_INVALID, "%s: rope_base must be a positive finite number", fn);
    if (a.head_dim != 128 || p.group > 16 || !fast_path_ok(a, p.group))
      return set_error(FD_E_UNSUPPORTED,
                       "%s: fused RoPE needs head_dim 128, <= 16 query heads per KV head, unit dim stride and "
                       "16-byte rows",
                       fn);
    if (p.counters != nullptr)
      return set_error(FD_E_UNSUPPORTED, "%s: fused RoPE does not combine with the in-launch merge", fn);
    p.rope_dim = static_cast<int>(a.rotary_dim);
    p.rope_base = static_cast<float>(a.rope_base);  // the reference's pow runs on an fp32 base
    if (a.rope_cos_sin_table != nullptr) {
      if (a.rope_table_rows <= 0 || (reinterpret_cast<uintptr_t>(a.rope_cos_sin_table) & 3u))
        return set_error(FD_E_INVALID, "%s: rope_cos_sin_table needs rope_table_rows > 0 and 4-byte alignment", fn);
      p.rope_tab = a.rope_cos_sin_table;
      p.rope_tab_rows = a.rope_table_rows;
    }
  } else if (a.rope_cos_sin_table != nullptr) {
    return set_error(FD_E_INVALID, "%s: rope_cos_sin_table needs rotary_dim (fused RoPE)", fn);
  }
  {
    // first-tile guess of the MFMA kernel: from max_seq_len when given, else
    // from the table width; each row's split range uses its own length
    const int64_t cap = a.max_blocks_per_seq * a.block_size;
    const int64_t bound = (a.max_seq_len > 0 && a.max_seq_len < cap) ? a.max_seq_len : cap;
    p.hint_tiles = static_cast<int>((bound + 31) / 32);
    p.hint_tps = (p.hint_tiles + p.splits - 1) / p.splits;
  }
  p.scale_log2 = a.sm_scale * kLog2e;
  return FD_OK;
}

extern "C" int fd_paged_decode(const fd_paged_decode_args* args, fd_stream_t stream_) {
  clear_launch_record();
  DecodeParams p;
  const int rc = fill_decode_params(args, "fd_paged_decode", p);
  if (rc != FD_OK) return rc;
  const fd_paged_decode_args& a = *args;

  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (a.dtype == FD_DTYPE_BF16) return launch_decode<__bf16>(a, p, stream);
  return launch_decode<_Float16>(a, p, stream);
}

// ------------------------------------------------ no-allocation entry ----
// Split partials of fd_paged_decode_noalloc live in this file-scope array:
// one copy per GPU, held until the process ends, cut into
// FD_NOALLOC_STREAM_SLOTS slots of FD_NOALLOC_SCRATCH_BYTES.  Each of the
// first FD_NOALLOC_STREAM_SLOTS distinct streams that use it on a device owns
// one slot for the rest of the process, so calls on different streams never
// share partials, and the calls of one stream run in its order.  Host code
// never passes the array's name to a kernel (on the host it is only a
// stand-in for the symbol): the device address comes from
// hipGetSymbolAddress, once per device.
static __device__ __align__(256) float scratch[FD_NOALLOC_STREAM_SLOTS * (FD_NOALLOC_SCRATCH_BYTES / sizeof(float))];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};
// slot owners per device (a stream handle; the null stream is a stream too)
hipStream_t g_slot_owner[kMaxDevices][FD_NOALLOC_STREAM_SLOTS] = {};
bool g_slot_used[kMaxDevices][FD_NOALLOC_STREAM_SLOTS] = {};

// Base of the stream's scratch slot on its device (the current device for
// the null stream).  The array's address is looked up on the first call on
// that device, with it current; the stream takes a free slot on its first
// call.  Host bookkeeping only: nothing here launches or allocates.
int scratch_address(hipStream_t stream, const char* fn, float** out) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return set_error(FD_E_LAUNCH, "%s: hipGetDevice failed: %s", fn, hipGetErrorString(e));
  int dev = cur;
  if (stream != nullptr) {
    e = hipStreamGetDevice(stream, &dev);
    if (e != hipSuccess) return set_error(FD_E_LAUNCH, "%s: hipStreamGetDevice failed: %s", fn, hipGetErrorString(e));
  }
  if (dev < 0 || dev >= kMaxDevices) return set_error(FD_E_UNSUPPORTED, "%s: device %d >= %d", fn, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess)
      return set_error(FD_E_LAUNCH, "%s: hipSetDevice(%d) failed: %s", fn, dev, hipGetErrorString(e));
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    const hipError_t restored = dev != cur ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess || ptr == nullptr)
      return set_error(FD_E_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", fn, dev,
                       hipGetErrorString(e));
    if (restored != hipSuccess)
      return set_error(FD_E_LAUNCH, "%s: restoring device %d failed: %s", fn, cur, hipGetErrorString(restored));
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  int slot = -1;
  for (int i = 0; i < FD_NOALLOC_STREAM_SLOTS && slot < 0; ++i)
    if (g_slot_used[dev][i] && g_slot_owner[dev][i] == stream) slot = i;
  for (int i = 0; i < FD_NOALLOC_STREAM_SLOTS && slot < 0; ++i)
    if (!g_slot_used[dev][i]) {
      g_slot_used[dev][i] = true;
      g_slot_owner[dev][i] = stream;
      slot = i;
    }
  if (slot < 0)
    return set_error(FD_E_UNSUPPORTED,
                     "%s: device %d's %d no-allocation scratch slots are taken by other streams (one per stream, "
                     "for the life of the process); use fewer streams or fd_paged_decode with a workspace",
                     fn, dev, FD_NOALLOC_STREAM_SLOTS);
  *out = g_scratch_ptr[dev] + static_cast<size_t>(slot) * (FD_NOALLOC_SCRATCH_BYTES / sizeof(float));
  return FD_OK;
}
}  // namespace

extern "C" int fd_paged_decode_noalloc_prepare(fd_stream_t stream_) {
  clear_launch_record();
  float* base = nullptr;
  return scratch_address(reinterpret_cast<hipStream_t>(stream_), "fd_paged_decode_noalloc_prepare", &base);
}

extern "C" int fd_paged_decode_noalloc(const fd_paged_decode_args* args, fd_stream_t stream_) {
  clear_launch_record();
  static const char* fn = "fd_paged_decode_noalloc";
  if (args == nullptr) return set_error(FD_E_INVALID, "%s: args is NULL", fn);
  if (args->struct_size != sizeof(fd_paged_decode_args))
    return set_error(FD_E_INVALID, "%s: struct_size %u != %zu (ABI mismatch)", fn, args->struct_size,
                     sizeof(fd_paged_decode_args));
  if (args->split_acc || args->split_max || args->split_sum || args->split_counters)
    return set_error(FD_E_INVALID,
                     "%s: split_acc, split_max, split_sum and split_counters must be NULL (the library's scratch "
                     "holds the split partials)",
                     fn);
  fd_paged_decode_args a = *args;
  const bool split = a.num_splits > 1;
  int64_t rows = 0;
  if (split) {
    // stand-in pointers so the shared validation below passes; the scratch
    // address replaces them after it
    a.split_acc = a.split_max = a.split_sum = reinterpret_cast<float*>(alignof(float));
    // fp32 partials: acc [B, Hq, S, D], then max and sum planes [B, Hq, S]
    // (shapes that fail here are reported by the shared validation)
    if (a.num_seqs > 0 && a.num_q_heads > 0 && a.num_seqs < (int64_t{1} << 31) && a.num_q_heads < (int64_t{1} << 31) &&
        a.num_seqs * a.num_q_heads <= 0x7fffffffLL && (a.head_dim == 64 || a.head_dim == 128) &&
        a.num_splits <= 4096) {
      rows = a.num_seqs * a.num_q_heads * a.num_splits;
      const int64_t bytes = rows * (a.head_dim + 2) * static_cast<int64_t>(sizeof(float));
      if (bytes > static_cast<int64_t>(FD_NOALLOC_SCRATCH_BYTES))
        return set_error(FD_E_INVALID,
                         "%s: %lld sequences x %lld query heads x %d splits x (head_dim %lld + 2) fp32 partials "
                         "(%lld bytes) exceed the %lld-byte scratch; use fewer splits or fd_paged_decode",
                         fn, static_cast<long long>(a.num_seqs), static_cast<long long>(a.num_q_heads), a.num_splits,
                         static_cast<long long>(a.head_dim), static_cast<long long>(bytes),
                         static_cast<long long>(FD_NOALLOC_SCRATCH_BYTES));
    }
  }
  DecodeParams p;
  const int rc = fill_decode_params(&a, fn, p);
  if (rc != FD_OK) return rc;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (split) {
    float* base = nullptr;
    const int rs = scratch_address(stream, fn, &base);
    if (rs != FD_OK) return rs;
    const int64_t S = a.num_splits, D = a.head_dim;
    p.acc = base;
    p.as0 = a.num_q_heads * S * D;
    p.as1 = S * D;
    p.as2 = D;
    p.as3 = 1;
    p.mx = base + rows * D;
    p.sm = p.mx + rows;
    p.ss0 = a.num_q_heads * S;
    p.ss1 = S;
    p.ss2 = 1;
  }
  p.counters = nullptr;  // the reducer kernel merges the splits
  if (a.dtype == FD_DTYPE_BF16) return launch_decode<__bf16>(a, p, stream);
  return launch_decode<_Float16>(a, p, stream);
}

extern "C" int fd_paged_decode_cascade(const fd_paged_decode_args* args, const fd_cascade_args* cascade,
                                       fd_stream_t stream_) {
  clear_launch_record();
  static const char* fn = "fd_paged_decode_cascade";
  DecodeParams p;
  const int rc = fill_decode_params(args, fn, p);
  if (rc != FD_OK) return rc;
  const fd_paged_decode_args& a = *args;
  if (cascade == nullptr) return set_error(FD_E_INVALID, "%s: cascade is NULL", fn);
  const fd_cascade_args& c = *cascade;
  if (c.struct_size != sizeof(fd_cascade_args))
    return set_error(FD_E_INVALID, "%s: cascade struct_size %u != %zu (ABI mismatch)", fn, c.struct_size,
                     sizeof(fd_cascade_args));
  if (p.fuse) return set_error(FD_E_UNSUPPORTED, "%s: fused append is not supported (append first)", fn);
  if (a.head_dim != 128 || p.group > 16 || !fast_path_ok(a, p.group))
    return set_error(FD_E_UNSUPPORTED,
                     "%s: needs head_dim 128, <= 16 query heads per KV head, unit dim stride and 16-byte rows", fn);
  if (c.num_groups < 0 || c.max_members < 1 || c.prefix_splits < 1)
    return set_error(FD_E_INVALID, "%s: num_groups must be >= 0, max_members and prefix_splits >= 1", fn);
  if (a.num_splits + static_cast<int64_t>(c.prefix_splits) > 4096)
    return set_error(FD_E_INVALID, "%s: num_splits + prefix_splits must be <= 4096", fn);
  if (!a.split_acc || !a.split_max || !a.split_sum)
    return set_error(FD_E_INVALID, "%s: split workspace required", fn);
  if (!c.row_prefix_len || (c.num_groups > 0 && (!c.group_members || !c.group_prefix_len)))
    return set_error(FD_E_INVALID, "%s: NULL group pointer", fn);
  if (c.max_prefix_len < 0) return set_error(FD_E_INVALID, "%s: max_prefix_len must be >= 0", fn);
  if (c.chunk_rows != 0 && c.chunk_rows != 16 && c.chunk_rows != FD_CASCADE_MAX_CHUNK_ROWS)
    return set_error(FD_E_INVALID, "%s: chunk_rows must be 0, 16 or %d", fn, FD_CASCADE_MAX_CHUNK_ROWS);
  const int chunk_rows = c.chunk_rows == 0 ? 16 : c.chunk_rows;
  const int64_t chunks = (static_cast<int64_t>(c.max_members) * p.group + chunk_rows - 1) / chunk_rows;
  const int64_t prefix_blocks = static_cast<int64_t>(c.num_groups) * a.num_kv_heads * chunks * c.prefix_splits;
  if (prefix_blocks + a.num_seqs * a.num_kv_heads * a.num_splits > 0x7fffffffLL)
    return set_error(FD_E_INVALID, "%s: launch grid too large", fn);

  p.counters = nullptr;
  p.tb = c.row_prefix_len;
  const int64_t cap = a.max_blocks_per_seq * a.block_size;
  const int64_t pre = c.max_prefix_len < cap ? c.max_prefix_len : cap;
  {
    // tail-role guess of each split's first tile, for a row of the longest
    // prefix and the bound length
    p.hint_tb = static_cast<int>(pre / 32);
    const int span = max(p.hint_tiles - p.hint_tb, 0);
    p.hint_tps = (span + p.splits - 1) / p.splits;
  }
  CascadeParams cp{};
  cp.members = c.group_members;
  cp.prefix_len = c.group_prefix_len;
  cp.max_members = c.max_members;
  cp.chunks = static_cast<int>(chunks);
  cp.prefix_splits = c.prefix_splits;
  cp.prefix_blocks = static_cast<int>(prefix_blocks);
  cp.hint_ptps = static_cast<int>(((pre + 31) / 32 + c.prefix_splits - 1) / c.prefix_splits);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (a.dtype == FD_DTYPE_BF16) return launch_cascade<__bf16>(a, p, cp, chunk_rows / 16, stream);
  return launch_cascade<_Float16>(a, p, cp, chunk_rows / 16, stream);
}
