/*
 * int8kv.h -- C ABI of the MI355X (gfx950) INT8 KV-cache library, libint8kv.so.
 *
 * Two hot operations of a static per-head symmetric INT8 KV cache:
 *   1. the paged cache write (slot_mapping scatter, RNE quantisation, clamp to [-127, 127]);
 *   2. PagedAttention decode over an INT8 cache (or a 16-bit cache, same kernel family),
 *      split over equal ranges of the batch's token stream with online-softmax partials and a
 *      merge pass.
 *
 * Conventions shared by every entry point:
 *   - All pointers are device pointers except the `*_strides` arrays, which are host arrays.
 *   - Strides are in ELEMENTS of the tensor they describe (torch's Tensor.stride()).
 *   - `stream` is a hipStream_t passed as void* (NULL = the legacy default stream).
 *   - Nothing here allocates, frees or synchronises; every launch is enqueued on `stream`.
 *   - The return value is 0 on success, a negative INT8KV_E* code for a rejected argument
 *     (nothing was launched), or a positive hipError_t from the launch.
 *   - No C++ exception crosses this boundary.
 *
 * Reference interfaces replaced (paths relative to the cjsmt/Int8-kvcache checkout):
 *   int8kv_cache_write   <- src/triton_ops/int8_cache_write.py:85-149  (int8_kv_cache_write)
 *   int8kv_dynamic_cache_write <- vllm_int8/vllm_int8_cache_ops.py:134-210 (reshape_and_cache_int8)
 *   int8kv_paged_decode  <- src/triton_ops/int8_paged_attention.py:683-769 (int8_paged_attention,
 *                           the V4 kernel :61-327 plus the split merge :330-388) and
 *                           src/triton_ops/bf16_paged_attention.py:118-165 (bf16_paged_attention)
 *   int8kv_decode_workspace_bytes <- the partial-buffer allocation of
 *                           src/triton_ops/int8_paged_attention.py:594-603
 *   int8kv_decode_auto_ranges <- the split-count heuristic _choose_num_splits,
 *                           src/triton_ops/int8_paged_attention.py:39-49
 *   int8kv_decode_plan   <- the dispatcher's host-side choices, _choose_num_splits and _auto_impl
 *                           (src/triton_ops/int8_paged_attention.py:39-58, used at :726-763)
 */
#ifndef INT8KV_H
#define INT8KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type codes. */
enum int8kv_dtype {
  INT8KV_F32 = 0,
  INT8KV_F16 = 1,
  INT8KV_BF16 = 2,
  INT8KV_I8 = 3,
  INT8KV_I32 = 4,
  INT8KV_I64 = 5
};

/* Argument errors (negative return values). */
#define INT8KV_OK 0
#define INT8KV_E_NULL (-1)      /* a required pointer is NULL */
#define INT8KV_E_DTYPE (-2)     /* unsupported element type for this argument */
#define INT8KV_E_SHAPE (-3)     /* unsupported or inconsistent size */
#define INT8KV_E_STRIDE (-4)    /* innermost stride != 1 or rows not 16-byte aligned */
#define INT8KV_E_WORKSPACE (-5) /* workspace missing or smaller than required */
#define INT8KV_E_SCRATCH (-6)   /* needed scratch exceeds INT8KV_DECODE_SCRATCH_BYTES */

/* Flags of int8kv_paged_decode. */
#define INT8KV_DECODE_MAIN 1u   /* run the range decode kernel */
#define INT8KV_DECODE_MERGE 2u  /* run the split merge kernel */
#define INT8KV_DECODE_ALL 3u
#define INT8KV_DECODE_QUANTIZE_Q 4u  /* quantise q to int8 per (sequence, head) first */
#define INT8KV_DECODE_PER_SEQUENCE 8u  /* one workgroup per (sequence, kv head), no merge */
#define INT8KV_DECODE_SPLIT_SEQUENCES 16u  /* several workgroups per (sequence, kv head) */

/*
 * Static per-head INT8 quantisation of K and V plus the slot_mapping scatter into the paged
 * caches (replaces src/triton_ops/int8_cache_write.py:85-149 and its kernel :6-82).
 *
 *   for every token t with s = slot_mapping[t] in [0, num_blocks * block_size):
 *     key_cache[s / block_size, s % block_size, h, :] =
 *         clamp(rint(float(key[t, h, :]) / max(k_scale[h], 1e-6)), -127, 127)   (IEEE fp32 divide)
 *   (value likewise with v_scale).  Tokens with s < 0 are skipped; slots at or beyond
 *   num_blocks * block_size are skipped as well so that no access leaves the caches.
 *
 *   key/value:      [num_tokens, num_kv_heads, head_dim] of src_dtype (F32, F16, BF16),
 *                   innermost stride 1, each (token, head) row 16-byte aligned.
 *   key_cache/value_cache: int8 [num_blocks, block_size, num_kv_heads, head_dim],
 *                   innermost stride 1, rows 8-byte aligned.
 *   slot_mapping:   [num_tokens] of slot_dtype (I32 or I64), contiguous.
 *   k_scale/v_scale: fp32 [num_kv_heads], contiguous.
 *   head_dim must be a multiple of 8.
 */
int int8kv_cache_write(const void* key, const void* value, int src_dtype, int64_t num_tokens,
                       int32_t num_kv_heads, int32_t head_dim, const int64_t key_strides[3],
                       const int64_t value_strides[3], void* key_cache, void* value_cache,
                       int64_t num_blocks, int32_t block_size, const int64_t key_cache_strides[4],
                       const int64_t value_cache_strides[4], const void* slot_mapping,
                       int slot_dtype, const float* k_scale, const float* v_scale, void* stream);

/*
 * Dynamic per-(token, head) INT8 quantisation of K and V plus the slot_mapping scatter, with the
 * scales stored beside the codes (replaces reshape_and_cache_int8 and its Triton kernel,
 * vllm_int8/vllm_int8_cache_ops.py:13-210):
 *
 *   for every token t with s = slot_mapping[t] in [0, num_blocks * block_size), every head h:
 *     scale = max(absmax(key[t, h, :]) / 127, 1e-6)                       (IEEE fp32)
 *     key_cache[s / block_size, s % block_size, h, :] =
 *         round_half_away_from_zero(clamp(key[t, h, :] / scale, -127, 127))
 *     k_scale_cache[s / block_size, s % block_size, h] = scale
 *   (value likewise into value_cache / v_scale_cache).  Tokens with s < 0 (or past the cache)
 *   are skipped; nothing else is written.
 *
 *   Layouts as int8kv_cache_write; k_scale_cache/v_scale_cache: fp32 [num_blocks, block_size,
 *   num_kv_heads], any element strides.  head_dim / 8 must be a power of two <= 64
 *   (head_dim in {8, 16, ..., 512}).
 */
int int8kv_dynamic_cache_write(const void* key, const void* value, int src_dtype,
                               int64_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                               const int64_t key_strides[3], const int64_t value_strides[3],
                               void* key_cache, void* value_cache, int64_t num_blocks,
                               int32_t block_size, const int64_t key_cache_strides[4],
                               const int64_t value_cache_strides[4], float* k_scale_cache,
                               float* v_scale_cache, const int64_t k_scale_cache_strides[3],
                               const int64_t v_scale_cache_strides[3], const void* slot_mapping,
                               int slot_dtype, void* stream);

/*
 * Automatic range count of int8kv_paged_decode (num_ranges = 0) on the current device: the
 * token stream of a decode call is cut into at most this many equal ranges, one wave per SIMD
 * (4 x compute units / num_kv_heads: 256 for 4 kv heads on MI355X).
 * At head_dim 64 with an even num_kv_heads and at most 8 query heads per kv head, the decode
 * takes kv heads in pairs (one wave per pair) and its automatic count is that of
 * num_kv_heads / 2; with more than 16 query heads per kv head each kv head takes
 * ceil(group / 16) waves (column tiles of 16 query heads) and the count is that of
 * num_kv_heads x ceil(group / 16).  int8kv_decode_workspace_bytes(..., 0) accounts for both.
 */
int32_t int8kv_decode_auto_ranges(int32_t num_kv_heads);

/*
 * Bytes of device workspace int8kv_paged_decode needs (the split partials: one running max,
 * one running sum and one accumulator of head_dim rounded up to 64, 128 or 256 elements per
 * range, slot and query head, and per range a
 * 32-byte descriptor of the cut sequence it starts); independent of the batch, the context
 * lengths and the block-table width.  num_ranges is the value that will
 * be passed to int8kv_paged_decode (0 = automatic, for the current device).  Returns 0 for
 * sizes int8kv_paged_decode would reject.
 */
size_t int8kv_decode_workspace_bytes(int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                     int32_t block_size, int32_t num_ranges);

/* Layouts and merge kernels reported by int8kv_decode_plan. */
#define INT8KV_LAYOUT_RANGES 0       /* equal ranges of the batch's token stream */
#define INT8KV_LAYOUT_PER_SEQUENCE 1 /* one workgroup per (sequence, kv head), no merge */
#define INT8KV_LAYOUT_SPLIT 2        /* `split` workgroups per (sequence, kv head) + merge */
#define INT8KV_MERGE_NONE 0
#define INT8KV_MERGE_BY_SEQUENCE 1   /* one workgroup per (sequence, query head) */
#define INT8KV_MERGE_BY_RANGE 2      /* one wave per (range, query head) */
#define INT8KV_MERGE_SPLIT 3         /* the split layout's records, one wave per (sequence, q head) */

/* What int8kv_paged_decode does for given sizes (int8kv_decode_plan). */
typedef struct int8kv_decode_plan_t {
  int32_t layout;               /* INT8KV_LAYOUT_* */
  int32_t kernels;              /* kernel launches of a call with INT8KV_DECODE_ALL (0 for batch 0) */
  int32_t num_ranges;           /* ranges layout: most ranges the token stream is cut into; every
                                   layout: the range count the workspace is sized by */
  int32_t min_tiles;            /* ranges layout: smallest range, in 32-token tiles */
  int32_t seq_cost;             /* ranges layout: stream units charged per sequence start */
  int32_t ranges_per_workgroup; /* ranges layout: 1, or 2 (paired ranges); 0 otherwise */
  int32_t depth;                /* 32-token tiles of K/V loads in flight per wave */
  int32_t kv_pair;              /* 1: head_dim 64, two kv heads per wave as one 128-wide head */
  int32_t split;                /* split layout: workgroups per (sequence, kv head); else 0 */
  int32_t non_temporal;         /* 1: K/V loads carry the non-temporal hint */
  int32_t merge;                /* INT8KV_MERGE_* (the second kernel) */
  int32_t merge_waves;          /* waves per merge workgroup (0 without a merge) */
  int32_t merge_fold;           /* merge by sequence: records per lane slot and round */
  int32_t compute_units;        /* compute units the plan was made for */
  uint64_t workspace_bytes;     /* workspace the call needs */
} int8kv_decode_plan_t;

/*
 * The plan int8kv_paged_decode (no_alloc = 0) or int8kv_paged_decode_noalloc (no_alloc = 1)
 * follows for these sizes, without launching, allocating or reading device memory.  The
 * arguments mean what they mean there; key_head_stride / value_head_stride are the caches'
 * strides between kv heads in elements (key_cache_strides[2] / value_cache_strides[2]: head_dim
 * 64 takes kv heads in pairs only when both equal head_dim).  compute_units: the device's CU
 * count (256 on MI355X), or 0 for the current device (the only case that makes a HIP call).
 * Returns 0 and fills *plan, or the negative code int8kv_paged_decode returns for these sizes.
 * (The reference decides its split count and kernel on the host as well,
 * src/triton_ops/int8_paged_attention.py:39-58.)
 */
int int8kv_decode_plan(int query_dtype, int cache_dtype, int64_t batch, int32_t num_q_heads,
                       int32_t num_kv_heads, int32_t head_dim, int64_t num_blocks,
                       int32_t block_size, int64_t table_width, int64_t key_head_stride,
                       int64_t value_head_stride, int32_t num_ranges, int32_t min_tiles,
                       uint32_t flags, int32_t compute_units, int32_t no_alloc,
                       int8kv_decode_plan_t* plan);

/*
 * Paged decode attention, one query token per sequence, GQA group = num_q_heads / num_kv_heads
 * (replaces int8_paged_attention, src/triton_ops/int8_paged_attention.py:683-769, and
 * bf16_paged_attention, src/triton_ops/bf16_paged_attention.py:118-165):
 *
 *   out[b, h, :] = sum_{t < L_b} softmax_t(<q[b, h], k_t> * ks * sm_scale) * v_t * vs
 *   with g = h / group, k_t = key_cache[block_tables[b, t / bs], t % bs, g, :],
 *   ks = max(k_scale[g], 1e-6), vs = max(v_scale[g], 1e-6) for an I8 cache and ks = vs = 1 for
 *   a 16-bit cache, L_b = clamp(seq_lens[b], 0, table_width * block_size).  L_b = 0 gives 0.
 *
 *   query:        [batch, num_q_heads, head_dim] of query_dtype (F32, F16, BF16), innermost
 *                 stride 1, rows 16-byte aligned.
 *   key_cache/value_cache: [num_blocks, block_size, num_kv_heads, head_dim] of cache_dtype
 *                 (I8, BF16 or F16), innermost stride 1, rows 16-byte aligned.
 *   block_tables: [batch, table_width] of table_dtype (I32 or I64), any strides; entries for
 *                 the blocks a sequence covers must lie in [0, num_blocks) (others are clamped
 *                 into range so that every access stays inside the caches).
 *   seq_lens:     [batch] of seq_lens_dtype (I32 or I64), contiguous.
 *   k_scale/v_scale: fp32 [num_kv_heads] for an I8 cache; ignored (may be NULL) otherwise.
 *   out:          [batch, num_q_heads, head_dim] of query_dtype, innermost stride 1, rows
 *                 16-byte aligned.
 *   workspace:    at least int8kv_decode_workspace_bytes(...) bytes, 16-byte aligned; it needs
 *                 no initialisation.  Calls that share a workspace must not overlap.
 *   num_ranges:   the 32-token tiles of all sequences (each non-empty sequence also charged
 *                 a fixed start cost) form one stream per kv head, cut into
 *                 P = min(num_ranges, ceil(units / min_tiles)) equal ranges, one workgroup
 *                 each; a sequence cut by range bounds is combined by the merge kernel.
 *                 0 = automatic (int8kv_decode_auto_ranges).  num_ranges = batch gives one
 *                 range per sequence when all lengths are equal (a single pass).  With an
 *                 INT8 cache, twice the automatic count (two waves per SIMD) puts two ranges
 *                 in each workgroup once every range holds 16 units or more.
 *   min_tiles:    smallest range in tiles (0 = automatic: 2, or 4 when 2-tile ranges could cut
 *                 one sequence into more than 128 ranges; decided from batch, table width and
 *                 block size only).
 *                 With num_ranges = 0 and min_tiles = 0, short calls take the per-sequence layout
 *                 below instead (decided from head_dim, batch, num_kv_heads, group, table width
 *                 and block size only, with tokens = table width x block size and W = batch x
 *                 num_kv_heads x ceil(group / 16) workgroups; "head_dim" in these rules is
 *                 head_dim rounded up to 64, 128 or 256; head_dim 128, INT8 cache: W <= CUs,
 *                 and tokens <= 768,
 *                 or tokens <= 2048 with W >= (tiles per wave - 3) x CUs / 8, at most CUs / 2,
 *                 except with W <= CUs / 8, 3 or more tiles per wave and W x tiles >= CUs (then
 *                 the split layout below);
 *                 head_dim 128, 16-bit cache: W <= 3 CUs, and tokens <= 512, or tokens <= 1024
 *                 with W >= CUs / 2; head_dim 64: W <= 4 CUs, and for an INT8 cache tokens <=
 *                 1536, or tokens <= 2048 with W >= CUs / 8; for a 16-bit cache tokens <= 1024;
 *                 head_dim 256: W <= 3 CUs, and for an INT8 cache tokens <= 512 (not with W <=
 *                 CUs / 8 above 256 tokens: the split layout below), or tokens <= 1024 with
 *                 CUs / 2 <= W <= CUs; for a 16-bit cache tokens <= 256, or tokens <=
 *                 512 with W >= CUs / 2).
 *   flags:        INT8KV_DECODE_ALL normally; MAIN and MERGE separately let a caller time the
 *                 two kernels on their own (MERGE must follow MAIN with identical arguments).
 *                 OR INT8KV_DECODE_QUANTIZE_Q to quantise each (sequence, query head) row of q
 *                 to int8 first, as the reference's quantize_q=True
 *                 (src/triton_ops/int8_paged_attention.py:137-146): q_scale = max(absmax/127,
 *                 1e-6), q8 = clamp(round_half_away_from_zero(q / q_scale), -127, 127).
 *                 OR INT8KV_DECODE_PER_SEQUENCE for the per-sequence layout: one workgroup per
 *                 (sequence, kv head), whose waves split the sequence and combine their partial
 *                 softmax states on chip; one kernel, the workspace is not touched and MERGE
 *                 does nothing.  Suited to short sequences (each workgroup streams its whole
 *                 sequence on one compute unit).
 *                 OR INT8KV_DECODE_SPLIT_SEQUENCES for the split per-sequence layout: Z such
 *                 workgroups per (sequence, kv head), each over 1/Z of the sequence's tiles,
 *                 leave one partial record per query head in the workspace, and MERGE combines
 *                 the Z records (below Z = 2 it is the plain per-sequence layout); Z =
 *                 min(num_ranges / batch, 64) for a given num_ranges (S splits per sequence:
 *                 num_ranges = S x batch), else min(CUs / (batch x num_kv_heads), 64,
 *                 2 x automatic ranges / batch).  Suited to a few long sequences.  The automatic choice (num_ranges = 0, min_tiles = 0, when the
 *                 per-sequence layout is not taken) uses it when batch x num_kv_heads <= CUs / 8
 *                 and each wave then holds at most 4 tiles of 32 tokens (2 at head_dim 64) of
 *                 the longest possible sequence (table width x block size).
 *
 * Supported sizes: head_dim a multiple of 16 in [16, 256] (64, 128 and 256 run their own
 * kernels; the others run the next of them with the elements past head_dim neither loaded into
 * an output nor stored: 80, 96 and 112 on the 128-wide kernels, for example), block_size a
 * power of two in [16, 65536] (16 and 32 are vLLM's usual values), any integer group =
 * num_q_heads / num_kv_heads with num_kv_heads x ceil(group / 16) <= 65535 (a kv head's query
 * heads are taken 16 at a time, one wave or workgroup per 16: multi-query attention with 64
 * query heads runs 4 waves per kv head).  Other sizes return INT8KV_E_SHAPE.
 */
int int8kv_paged_decode(const void* query, int query_dtype, int64_t batch, int32_t num_q_heads,
                        int32_t head_dim, const int64_t query_strides[3], const void* key_cache,
                        const void* value_cache, int cache_dtype, int64_t num_blocks,
                        int32_t block_size, int32_t num_kv_heads,
                        const int64_t key_cache_strides[4], const int64_t value_cache_strides[4],
                        const void* block_tables, int table_dtype, int64_t table_width,
                        const int64_t table_strides[2], const void* seq_lens, int seq_lens_dtype,
                        const float* k_scale, const float* v_scale, float sm_scale, void* out,
                        const int64_t out_strides[3], void* workspace, size_t workspace_bytes,
                        int32_t num_ranges, int32_t min_tiles, uint32_t flags, void* stream);

/*
 * int8kv_paged_decode without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP-graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference: it is the same operation as int8kv_paged_decode (same
 * arguments, kernels and results) with the split partials kept in a fixed array of
 * INT8KV_DECODE_SCRATCH_BYTES per GPU inside the library (held from the GPU's first call until
 * the process ends) instead of a caller's workspace.  It calls no allocator.
 *
 *   - The array belongs to the current device (hipGetDevice); `stream` must be on it.
 *   - With num_ranges = 0 the automatic range count is lowered, if need be, to the most ranges
 *     whose partials fit INT8KV_DECODE_SCRATCH_BYTES (16 MiB: the full automatic count of 256
 *     ranges at 4 kv heads for a GQA group of up to 15 query heads per kv head at head_dim
 *     128, 7 at 256; larger groups get fewer, longer ranges; int8kv_decode_plan(..., no_alloc
 *     = 1, ...) reports the count).  A given num_ranges whose partials exceed the array
 *     (int8kv_decode_workspace_bytes(...) > INT8KV_DECODE_SCRATCH_BYTES) returns
 *     INT8KV_E_SCRATCH and launches nothing.
 *   - Every call on one GPU shares that GPU's array: calls that overlap on one GPU (two streams,
 *     two threads) race and must be serialised by the caller.  The array keeps the last call's
 *     contents; the kernels need no clearing between calls.
 */
#define INT8KV_DECODE_SCRATCH_BYTES ((size_t)16 << 20)
int int8kv_paged_decode_noalloc(const void* query, int query_dtype, int64_t batch,
                                int32_t num_q_heads, int32_t head_dim,
                                const int64_t query_strides[3], const void* key_cache,
                                const void* value_cache, int cache_dtype, int64_t num_blocks,
                                int32_t block_size, int32_t num_kv_heads,
                                const int64_t key_cache_strides[4],
                                const int64_t value_cache_strides[4], const void* block_tables,
                                int table_dtype, int64_t table_width,
                                const int64_t table_strides[2], const void* seq_lens,
                                int seq_lens_dtype, const float* k_scale, const float* v_scale,
                                float sm_scale, void* out, const int64_t out_strides[3],
                                int32_t num_ranges, int32_t min_tiles, uint32_t flags,
                                void* stream);

/* Library version string, e.g. "int8kv 0.1.0 gfx950". */
const char* int8kv_version(void);

#ifdef __cplusplus
}
#endif

#endif /* INT8KV_H */
