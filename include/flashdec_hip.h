/*
 * flashdec_hip.h -- C ABI of the MI355X (gfx950) paged-decode data path.
 *
 * Every entry point allocates no device memory, never synchronises, launches
 * on the caller's hipStream_t and returns an int status (FD_OK or a negative
 * FD_E* code).  All are stateless and re-entrant except
 * fd_paged_decode_noalloc, whose calls share one scratch array per GPU.  On error, fd_last_error() returns
 * a thread-local, human-readable message.  Nothing here throws across the ABI.
 *
 * Tensors are passed as raw device pointers plus element strides, so strided
 * views (vLLM's [block, plane, token, head, dim] cache, NHD/HND permutations,
 * dim-major caches) are consumed in place without copies.  fd_paged_decode
 * runs an MFMA kernel (head_dim 64 or 128, up to 256 query heads per KV head,
 * strides multiples of 8 and 16-byte aligned bases) for token-major caches with unit
 * dim stride and for dim-major caches with unit token stride; other views run
 * a VALU kernel with the same results within rounding.
 *
 * Reference interfaces replaced (paths relative to cysong2025/flashdec):
 *   fd_paged_decode          flashdec/kernels/paged_decode.py:972-1264
 *                            (paged_decode_attention_into) and :728-919
 *                            (_vllm_paged_decode_attention_into); the four
 *                            Triton kernels at :28-642
 *   fd_fused_rope_kv_append  flashdec/csrc/fused_rope_kv_append.cpp:90-124
 *                            (bound from _fused_rope_kv_append.py:148-176)
 *   fd_kv_append             flashdec/csrc/kv_append.cpp:60-73
 *                            (bound from _cuda_kv_append.py:116-137)
 *   fd_paged_decode_plan     flashdec/vllm_backend.py:168-188 chooses split
 *                            counts for its launcher; this is the MI355X policy
 *   fd_paged_decode_cascade  no counterpart (shared-prefix decode over the
 *                            prefixes of flashdec/cache.py:192-276)
 *   fd_paged_decode_balance_target  no counterpart: the per-row split
 *                            policy for ragged batches (balance_target)
 */
#ifndef FLASHDEC_HIP_H_
#define FLASHDEC_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FD_ABI_VERSION 9

/* status codes */
#define FD_OK 0
#define FD_E_INVALID (-1)     /* argument / shape / stride contract violated */
#define FD_E_UNSUPPORTED (-2) /* valid but not implemented (dtype, head_dim) */
#define FD_E_LAUNCH (-3)      /* hipLaunchKernel / hipGetLastError failure   */

/* uint32 words between the split arrival counters of two (request, KV head)
 * pairs: one 256-byte line each */
#define FD_SPLIT_COUNTER_STRIDE 64

/* element dtypes */
#define FD_DTYPE_F16 0
#define FD_DTYPE_BF16 1
#define FD_DTYPE_F32 2
/* index dtypes */
#define FD_INDEX_I32 0
#define FD_INDEX_I64 1

typedef struct ihipStream_t* fd_stream_t; /* == hipStream_t */

/*
 * Paged single-token decode attention.
 *
 * out[b, h, :] = softmax(q[b, h] . K_b^T * sm_scale) . V_b over the first
 * seq_lens[b] tokens of request b, whose token t lives at physical block
 * block_tables[b, t / block_size], offset t % block_size, KV head
 * h / (num_q_heads / num_kv_heads).  seq_lens[b] == 0 gives a zero row.
 *
 * Cache strides are [block, head, token, dim] in elements; a 5-D vLLM cache
 * is described by these strides plus the plane offset baked into the K and
 * V base pointers.
 *
 * num_splits: 1 = single pass, S > 1 = split-KV with the caller's fp32
 * workspace (split_acc [>=B, >=Hq, >=S, >=D], split_max/split_sum
 * [>=B, >=Hq, >=S], identical strides for max and sum), followed by the LSE
 * merge.  split_max holds base-2 log-domain maxima (internal format).
 *
 * split_counters (optional, S > 1): >= num_seqs * num_kv_heads *
 * FD_SPLIT_COUNTER_STRIDE uint32 words (one 256-byte line per (request,
 * KV head), whose first two words form one 64-bit arrival word), 8-byte
 * aligned, all zero before the first launch.  With it the merge happens inside the
 * same launch (the last workgroup of each (request, KV head) to finish
 * merges, then returns its counter to zero, so the buffer is zero again
 * after every launch and replays of a captured graph stay valid).  Launches
 * that share one counter buffer must not run concurrently (e.g. on two
 * streams).  Without it a second, reducer kernel performs the merge.
 *
 * max_seq_len: optional hint (0 = none), e.g. the batch's longest row.
 * Each row's split range comes from its own seq_lens[b] (tiles split evenly
 * over num_splits), so any value is correct; for rows whose length matches
 * the hint the first tile's block-table and K/V reads are issued before
 * seq_lens[b] is read, other rows fetch their first tile after it.
 *
 * Fused append (append_k, append_v, slot_mapping all non-NULL): the
 * request's newest token (position seq_lens[b]-1) is taken from
 * append_k/append_v instead of the cache, and written into the cache at
 * slot_mapping[b] = block * block_size + offset by the split that owns it.
 * Rows with slot_mapping[b] < 0 or seq_lens[b] == 0 are inert: no cache
 * write and a zero output row (vLLM's graph-padding rows).
 */
typedef struct fd_paged_decode_args {
  uint32_t struct_size; /* sizeof(fd_paged_decode_args): ABI guard */
  int32_t dtype;        /* FD_DTYPE_F16 or FD_DTYPE_BF16 */
  int64_t num_seqs;
  int64_t num_q_heads;
  int64_t num_kv_heads;
  int64_t head_dim;  /* 64 or 128 */
  int64_t block_size; /* 8, 16 or 32 */
  int64_t num_blocks; /* physical blocks; ids outside [0, num_blocks) are masked */
  int64_t max_blocks_per_seq;

  const void* q;
  int64_t q_stride[3]; /* seq, head, dim */
  void* k_cache;
  int64_t k_stride[4]; /* block, head, token, dim */
  void* v_cache;
  int64_t v_stride[4];
  const void* block_tables;
  int32_t block_tables_dtype; /* FD_INDEX_I32 / FD_INDEX_I64 */
  int64_t block_tables_stride[2];
  const void* seq_lens;
  int32_t seq_lens_dtype;
  int64_t seq_lens_stride;
  void* out;
  int64_t out_stride[3];

  float sm_scale;
  int32_t num_splits;
  float* split_acc;
  int64_t split_acc_stride[4]; /* seq, head, split, dim */
  float* split_max;
  float* split_sum;
  int64_t split_stats_stride[3]; /* seq, head, split */
  uint32_t* split_counters;     /* optional in-launch merge, see above */
  int64_t max_seq_len;          /* optional hint, 0 = none: the batch's longest
                                   row.  Rows of any length are correct; rows
                                   this long start their K/V loads before
                                   seq_lens is read. */

  const void* append_k; /* optional fused append, all-or-none */
  int64_t append_k_stride[3];
  const void* append_v;
  int64_t append_v_stride[3];
  const void* slot_mapping;
  int32_t slot_mapping_dtype;
  int64_t slot_mapping_stride;

  /* Optional profiling hook, all NULL = off.  Caller-created hipEvent_t
   * handles recorded around exactly one dispatch each (hipExtLaunchKernel):
   * [0]/[1] around the attention kernel, [2]/[3] around the split reducer
   * when the call launches one.  No counterpart in the reference; it lets a
   * caller time the attention kernel alone on its own stream. */
  void* timing_events[4];

  /* Balanced splits for ragged batches (0 = off: every row gets num_splits
   * splits).  With balance_target = V > 0, row b gets
   *   S_b = clamp(ceil(tiles_b / T), 1, num_splits),  T = ceil(Σ tiles / V)
   * splits (tiles = 32-token tiles of the row's length), computed on the
   * device from seq_lens, so long rows get more splits and every split holds
   * at most T tiles.  The launch has num_kv_heads * (V + num_seqs)
   * workgroups, the ones past the batch's Σ S_b exit at once.  S_b <= V, so
   * a workspace of num_splits = min(V, ceil(max_len / 32)) splits suffices.
   * Needs the token-major MFMA path with head_dim 128 and <= 16 query heads
   * per KV head, num_splits > 1 and no fused append (otherwise ignored);
   * costs one extra round trip (the lengths) per workgroup.  No
   * counterpart in the reference, whose split count is per launch
   * (flashdec/kernels/paged_decode.py:408-411). */
  int32_t balance_target;

  /* K/V read policy.  0 (default): every K/V row is read once per launch,
   * so the loads are non-temporal (streamed past the caches; 6-11 % faster
   * on unique K/V).  1: rows share blocks (a common prefix in several rows'
   * tables) and re-reads should hit the caches: plain loads.  The cascade's
   * prefix pass always uses plain loads.  Results are identical either way.
   * No counterpart in the reference. */
  int32_t kv_reuse;

  /* Fused RoPE: 0 = off; 64 or 128 = rotary width (head_dim 128, at most 16
   * query heads per KV head, split-half rotation as flashdec/rope.py:26-85,
   * frequencies rope_base^(-2i/R)).  Needs
   * the fused append: q and append_k are then unrotated, both are rotated at
   * position seq_len - 1 (the appended token's index) and the cache receives
   * the rotated K.  Bit-identical to fd_fused_rope_kv_append at those
   * positions followed by fd_paged_decode on the rotated q.  Refused with the
   * in-launch merge.  No counterpart in the reference, which runs RoPE +
   * append as its own kernel. */
  int32_t rotary_dim;
  double rope_base;
  /* Optional with fused RoPE: fp32 cos/sin table [2, rope_table_rows,
   * rotary_dim / 2], contiguous (plane 0 cos, plane 1 sin, row = position),
   * used instead of the kernel's own evaluation -- see cos_sin_table of
   * fd_rope_append_args.  NULL = off.  Needs rotary_dim != 0. */
  const float* rope_cos_sin_table;
  int64_t rope_table_rows;
} fd_paged_decode_args;

int fd_paged_decode(const fd_paged_decode_args* args, fd_stream_t stream);

/* bytes of one stream's slot of the per-GPU scratch behind
 * fd_paged_decode_noalloc (8 MiB), and the slots per GPU (32 MiB in all) */
#define FD_NOALLOC_SCRATCH_BYTES 8388608
#define FD_NOALLOC_STREAM_SLOTS 4

/*
 * fd_paged_decode without a caller workspace and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under hipGraph capture, tight serving loops, harnesses
 * that forbid hipMalloc).
 *
 * Same arguments, kernels and results as fd_paged_decode, except that
 * split_acc, split_max, split_sum and split_counters must be NULL: the split
 * partials go to a file-scope device array of FD_NOALLOC_STREAM_SLOTS slots
 * of FD_NOALLOC_SCRATCH_BYTES per GPU, which each GPU the library runs on
 * holds until the process ends.  A launch with num_splits > 1 needs
 *   num_seqs * num_q_heads * num_splits * (head_dim + 2) * 4 bytes
 * of a slot (B8 Hq16 D128: up to 126 splits; B64 Hq16: up to 15); larger
 * launches are rejected with FD_E_INVALID before anything runs.  The splits
 * are merged by the reducer kernel (no in-launch merge).  Nothing in the
 * array needs to start at zero.
 *
 * Slots: each of the first FD_NOALLOC_STREAM_SLOTS distinct streams (the NULL
 * stream counts as one) that calls this function (or
 * fd_paged_decode_noalloc_prepare) on a GPU owns one slot there for the rest
 * of the process.  Calls on different streams therefore never share
 * partials, from any number of host threads, and the calls of one stream
 * run in its order.  A call from a further stream fails with
 * FD_E_UNSUPPORTED before anything runs.  A call captured into a hipGraph
 * keeps the slot of the stream it was captured on: replaying that graph on
 * another stream while the capturing stream runs no-allocation calls, or
 * replaying it twice at once, races.  The array's address on a device is
 * looked up once (hipGetSymbolAddress) by fd_paged_decode_noalloc_prepare
 * or, failing that, by the first call on the device; no call allocates or
 * frees memory.
 */
int fd_paged_decode_noalloc(const fd_paged_decode_args* args, fd_stream_t stream);

/*
 * Set-up of fd_paged_decode_noalloc on the stream's device (the current
 * device for a NULL stream): looks the scratch array's device address up,
 * once per device, with that device current, takes the stream's scratch slot
 * (FD_E_UNSUPPORTED when every slot belongs to another stream), and launches
 * nothing.  Call it (or make one eager fd_paged_decode_noalloc call) on every
 * device before capturing fd_paged_decode_noalloc into a hipGraph, so that
 * no lookup runs inside the capture.  Allocates nothing; idempotent.  No
 * counterpart in the reference.
 */
int fd_paged_decode_noalloc_prepare(fd_stream_t stream);

/*
 * Shared-prefix (cascade) decode: the result of fd_paged_decode, with the
 * K/V of a prefix shared by a group of rows read once per 16 (member, query
 * head) rows of the group.  No counterpart in the reference, which reads
 * every row's prefix separately (flashdec/kernels/paged_decode.py:330-543);
 * groups are the rows attached to one registered prefix of PagedKVCache
 * (flashdec/cache.py:192-276).
 *
 * Group g lists up to max_members row indices in group_members[g, :] (row
 * stride max_members; entries outside [0, num_seqs), e.g. -1, are padding)
 * that share their first group_prefix_len[g] tokens: whole blocks, the same
 * physical block ids leading each member's block-table row, and no more
 * tokens than any member's seq_lens.  Entry 0 is the lead: the prefix's
 * block ids are read from its table row.  row_prefix_len[b] is that length
 * for each member row and 0 for rows in no group; a row belongs to at most
 * one group.  One launch holds prefix-role workgroups -- one per (group, KV
 * head, chunk of chunk_rows of the group's member x query-head rows, prefix
 * split), writing
 * prefix_splits partials per (row, head) at workspace splits
 * [num_splits, num_splits + prefix_splits) -- and tail-role workgroups
 * attending tokens [row_prefix_len[b], seq_lens[b]) of each row at splits
 * [0, num_splits); the reducer merges them (tail splits only for rows with
 * no prefix).
 *
 * Needs the token-major MFMA path (head_dim 128, <= 16 query heads per KV
 * head, unit dim stride, 16-byte aligned rows), a split workspace of num_splits +
 * prefix_splits splits and no fused append (append first).  max_prefix_len
 * is a hint (the longest group prefix) for where each split starts.  The
 * timing events [0]/[1] bracket the attention launch, [2]/[3] the reducer.
 */
/* chunk_rows: member x query-head rows of a group that one prefix-role
 * workgroup attends (16 per MFMA column block of its waves), 16 or
 * FD_CASCADE_MAX_CHUNK_ROWS; 0 means 16.  The prefix is read once per
 * chunk; a chunk of 32 rows doubles each wave's work per K/V unit, which pays
 * for long prefixes shared by many rows.  There are ceil(max_members * G /
 * chunk_rows) chunks per (group, KV head). */
#define FD_CASCADE_MAX_CHUNK_ROWS 32

typedef struct fd_cascade_args {
  uint32_t struct_size; /* sizeof(fd_cascade_args): ABI guard */
  int32_t num_groups;
  int32_t max_members;
  int32_t prefix_splits;
  const int32_t* group_members;    /* [num_groups, max_members] */
  const int32_t* group_prefix_len; /* [num_groups], tokens */
  const int32_t* row_prefix_len;   /* [num_seqs], tokens */
  int64_t max_prefix_len;
  int32_t chunk_rows;              /* 0, 16 or FD_CASCADE_MAX_CHUNK_ROWS (see above) */
} fd_cascade_args;

int fd_paged_decode_cascade(const fd_paged_decode_args* args, const fd_cascade_args* cascade,
                            fd_stream_t stream);

/*
 * Split count the library would pick for a launch of this shape on the
 * current device (num_splits argument of fd_paged_decode).  max_seq_len is
 * the longest row (or a bound such as max_blocks_per_seq * block_size);
 * total_seq_len is the sum of seq_lens when the caller knows it (0 =
 * unknown), which lets the plan tell a ragged batch (long rows need more
 * splits) from a uniform one (fewer, longer splits).
 * Returns >= 1, or a negative FD_E* code.
 */
int fd_paged_decode_plan(int64_t num_seqs, int64_t num_q_heads,
                         int64_t num_kv_heads, int64_t head_dim,
                         int64_t max_seq_len, int64_t total_seq_len);

/*
 * balance_target (fd_paged_decode_args) the library would use for a ragged
 * batch of this shape on the current device: about one round of workgroups
 * (two per CU) after the per-row rounding.  0 = not worth it (the batch
 * fills a round already): use uniform splits.  The matching workspace is
 * num_splits = min(V, ceil(max_seq_len / 32)).
 */
int fd_paged_decode_balance_target(int64_t num_seqs, int64_t num_kv_heads);

/*
 * Fused split-half (NeoX) RoPE of Q and K plus paged append of rotated K and
 * raw V for one layer.  q/k/v/q_out are contiguous [B, H, D]; caches are
 * contiguous token-major [num_blocks, Hkv, block_size, D].  Row b is written
 * at (block_ids[b], block_offsets[b]) and rotated with positions[b].
 *
 * The rotation is bit-exact by construction: inv_freq and cos/sin are
 * evaluated in float64 and rounded once to float32 (the correctly rounded
 * values of flashdec/rope.py:66-71), then
 *   out_lo = rn(rn(x_lo * cos) - rn(x_hi * sin)),
 *   out_hi = rn(rn(x_hi * cos) + rn(x_lo * sin))
 * without FMA contraction, rounded to the element dtype (RNE).  Dimensions
 * past rotary_dim are copied.  Block ids and offsets are range-checked in
 * the kernel: a row whose block id is outside [0, num_blocks) or whose
 * offset is outside [0, block_size) writes no K/V (its q_out row is still
 * produced).  Positions are not checked here; callers validate them
 * (non-negative) before the launch.
 */
typedef struct fd_rope_append_args {
  uint32_t struct_size;
  int32_t dtype; /* FD_DTYPE_F16 / BF16 / F32 */
  int64_t batch;
  int64_t num_q_heads;
  int64_t num_kv_heads;
  int64_t head_dim;
  int64_t block_size;
  int64_t num_blocks;
  int64_t rotary_dim;
  double base;
  void* q_out; /* may be NULL: K/V only */
  const void* q;
  const void* k;
  const void* v;
  void* k_cache;
  void* v_cache;
  const void* block_ids;
  const void* block_offsets;
  const void* positions;
  int32_t index_dtype; /* FD_INDEX_I32 / FD_INDEX_I64, shared by the three */
  /* Optional fp32 cos/sin table [2, table_rows, rotary_dim / 2], contiguous:
   * plane 0 cos, plane 1 sin, row p = the angles of position p.  When given,
   * cos/sin are read from it instead of being evaluated, and only the
   * rotation above runs: a table built with flashdec/rope.py:66-70's torch
   * expression on the same device makes q_out and the K bytes equal that
   * apply_rope bit for bit.  Positions must be < table_rows (a position
   * outside reads the nearest row; nothing is read out of bounds).  NULL =
   * off (the correctly rounded evaluation).  fd_kv_append ignores it.
   * No counterpart in the reference. */
  const float* cos_sin_table;
  int64_t table_rows;
} fd_rope_append_args;

int fd_fused_rope_kv_append(const fd_rope_append_args* args, fd_stream_t stream);

/*
 * K/V scatter without RoPE: k_cache[block_ids[b], h, block_offsets[b], :]
 * = k[b, h, :] (same for v).  Uses fd_rope_append_args with q, q_out,
 * positions, rotary_dim and base ignored.  Bit-exact copy.
 */
int fd_kv_append(const fd_rope_append_args* args, fd_stream_t stream);

/* thread-local message for the last failing call on this thread */
const char* fd_last_error(void);

/* FD_ABI_VERSION of the loaded library */
int fd_abi_version(void);

/*
 * Launch record (no counterpart in the reference; for tests and debugging).
 * fd_record_launches(1) turns it on for the process: each fd_paged_decode*,
 * fd_fused_rope_kv_append and fd_kv_append call then clears this thread's
 * record and appends the demangled name of every kernel it launches
 * ("fd::decode_mfma_kernel<__bf16, 32, 0, false, 32, true, 128, 1>;
 * fd::split_reduce_pre_kernel<__bf16, 128, 1>"), which fd_last_launch()
 * returns.  Off by default; off, a launch pays one relaxed load.
 */
void fd_record_launches(int on);
const char* fd_last_launch(void);

#ifdef __cplusplus
}
#endif

#endif /* FLASHDEC_HIP_H_ */
