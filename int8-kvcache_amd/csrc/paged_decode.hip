// PagedAttention decode for gfx950: one kernel family over INT8 and 16-bit paged caches.
//
// Replaces src/triton_ops/int8_paged_attention.py (V4 GQA kernel :61-327, split merge :330-388,
// dispatcher :683-769) and src/triton_ops/bf16_paged_attention.py:9-165.  The mathematics is
// the reference's (src/attention_ref.py:19-28 on the dequantised cache,
// src/triton_ops/int8_paged_attention.py:776-814): softmax over <q, k_t> * k_scale * sm_scale,
// weights times v_t * v_scale, with v_scale applied once at the end (:291-292).
//
// Work decomposition (MI355X-first, not the reference's grid):
//   * Every sequence is cut into 32-token tiles.  The batch, in order, becomes one stream of
//     units per kv head: a non-empty sequence is a few "start" units (the cost of reaching its
//     first tile) followed by its tiles.  The stream is divided into P equal contiguous ranges
//     (P = one wave per SIMD by default, fewer for short batches: at least min_tiles units per
//     range), so a ragged batch costs every workgroup the same whatever the length
//     distribution.  The unit counts and the range bounds are computed on the device from
//     seq_lens; the host never reads them.
//   * A workgroup owns a range for W kv heads, one wave per (range, kv head).  The W waves of a
//     range read the same cache rows (their head slices of the same 16-token row groups) at the
//     same time.  A wave handles all query heads of its GQA group on the matrix cores, so every
//     K/V byte is read from HBM exactly once, and needs no barrier.  With a range count of two
//     waves per SIMD (a caller's choice) INT8 workgroups own a pair of ranges instead, waves
//     0..W-1 the first and W..2W-1 the second; the first range of a pair is the longer one: of
//     two waves sharing a SIMD the first streams faster (see kFirstShare).
//   * A sequence wholly inside one range is finished by that wave (output written directly).
//     A sequence cut by range bounds leaves (max, sum, accumulator) partials in the workspace,
//     at most two per range and head; a merge kernel combines them: merge_kernel (one workgroup
//     per sequence and query head, which finds its ranges from seq_lens) for batches below half
//     the range count, merge_by_range_kernel (one per range and query head, from the descriptor
//     of the cut sequence each range starts, which the decode kernel writes) otherwise.
//   * Per 32-token tile and wave:  S^T = K * Q^T  (2 x 4 MFMA 16x16x32; rows = tokens, cols =
//     heads), online softmax in the exp2 domain, then out^T += V^T * P^T (2 x 8 MFMA 16x16x32,
//     P split into 16-bit hi + lo parts; rows = head_dim, cols = heads).  The MFMA accumulator
//     layout puts one head per lane column, so the probabilities never leave registers.
//   * INT8 K/V are read with non-temporal loads when a call can stream more than the 256 MB
//     Infinity Cache holds: every byte is used once, and keeping the stream out of L2 and the
//     Infinity Cache raises the delivered bandwidth by ~10 % on MI355X (large ragged batch,
//     5.4 -> 6.1 TB/s).  Smaller pools, which the cache keeps between calls, and 16-bit caches use
//     plain loads (see stream_load).
//   * DEPTH tiles are in flight per wave: K(t+DEPTH) is requested as soon as the scores of tile
//     t are formed and V(t+DEPTH) as soon as its P*V is done.  DEPTH is 2 (a 16 KB BF16 tile
//     keeps 32 KB in flight per wave), or 4 for INT8 waves with long ranges, so that one wave
//     per SIMD has the bytes in flight of two.  The block ids of up to 256 tiles are staged
//     in LDS per wave ahead of use, every load in the tile loop is unconditional (requests past
//     the end of a range repeat its last tile), and the loop body is straight-line code per
//     DEPTH tiles, so no wait for a table read or a branch drains the pipeline.
//   * INT8 K/V are dequantised in registers to fp16 with the exact magic-number conversion
//     (0x6400 | (x ^ 0x80)) - 1152 = x, two elements per v_pk_add_f16.  Q is scaled by a power
//     of two into the upper fp16 range (exact for bf16 input); k_scale * sm_scale * log2(e) and
//     that power of two are applied to the fp32 scores, v_scale to the final output.  With
//     INT8KV_DECODE_QUANTIZE_Q, q is first quantised per (sequence, head) to int8 with
//     half-away rounding (src/triton_ops/int8_paged_attention.py:137-149) and its scale folded
//     into the score scale.
//   * A running max is only moved when a tile's max exceeds it by more than 8 (log2 units), so
//     most tiles skip the accumulator rescale; probabilities are then <= 2^8 (fits fp16/bf16).

#include <algorithm>
#include <atomic>
#include <cmath>
#include <mutex>

#include "paged_decode_kernels.h"

using namespace int8kv;


namespace {

constexpr int kMaxRangesLimit = 1 << 20;
// Stream units charged per sequence start (make_plan).  A wave that moves on to another
// sequence inside its range lets its pipeline run dry and refills it after two dependent loads
// (block ids, then the first tiles), which costs about 2 x DEPTH tile times for 8 KB INT8 tiles
// and half as many tile times for 16 KB 16-bit tiles.  Measured on MI355X (per-wave exit stamps
// and sweeps of the charge): with 2 units the INT8 ranges that start a second sequence
// finished ~2.3 us after the others and set the end of the call; 6 (four tiles in flight) and
// 4 (two) gave B=128 x U[1,4096] 58.0 -> 54.1 us, B=256 x U[1,2048] 64.1 -> 58.4 us,
// B=64 x U[1,8192] 51.9 -> 49.9 us, B=32 x U[1,4096] 17.8 -> 16.9 us and the large ragged
// batch 190.5 -> 188.8 us, and were neutral on uniform lengths; larger charges lose again.
// 16-bit caches measured best at 2-3.
constexpr int kSeqStartCost = 2;        // host-side bounds, and 16-bit caches
constexpr int kSeqStartCostI8 = 4;      // INT8, two tiles in flight
constexpr int kSeqStartCostI8Deep = 6;  // INT8, four tiles in flight
// Smallest automatic range (see auto_min_tiles).
constexpr int kMinTilesSmall = 2;
constexpr int kMinTilesLarge = 4;
constexpr int64_t kMaxMergeRanges = 128;  // ranges per sequence the merge takes in 4 rounds
// Resident decode waves per CU the automatic range count targets: one per SIMD.  Against two
// per SIMD (the second of which streams ~30 % slower) it measured 3-11 % faster on every
// shape tried on MI355X from B=1 x 32k to B=128 x 2048 tokens and on cfg3's BF16 call, and
// equal on cfg3's INT8 call with four tiles in flight.
constexpr int kWavesPerCU = 4;
// INT8 ranges of at least this many units (host-side bound) keep four tiles in flight per wave;
// shorter ones two (the deeper prologue and its unused refills cost 2-3 us on short ranges).
constexpr int64_t kDeepMinUnits = 32;
// INT8 K/V loads carry the non-temporal hint when a call may read more than this (half of
// MI355X's 256 MB Infinity Cache): such a stream does not stay resident across calls, and
// keeping it out of the caches stops it from evicting other lines.  Measured with half the cache
// against the whole: B=16 x 16k 48.5 vs 50.0 us on one pool and 49.4 vs 55.7 us rotating over 4
// layers' pools, B=8 x 32k 47.7 vs 52.2 / 49.6 vs 55.8 us (both ~268 MB, just at the old
// bound), no change at 135 and 250 MB; cache-resident pools (config 2, <= 34 MB) read ~10 %
// slower with the hint, so they keep plain loads.
constexpr int64_t kNonTemporalMinBytes = 128LL << 20;
// Share (1/256) of a range pair's units given to the first half of the workgroup.  Two waves
// share each SIMD, and the first (waves 0..W-1) streams ~30 % faster than the second on
// MI355X; with equal halves the second then runs alone for the last quarter of the call.
// 160 (62.5 %) measured best between cfg3 (~152) and B=32 x 8320 (~168): -2 us at both.
constexpr int32_t kFirstShare = 160;

// Compute units of the current device, queried on every call (no state is kept between calls;
// the runtime answers from its cached device properties).  256 on MI355X.
int cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  return n;
}

// Smallest automatic range, from host-side bounds only.  A call whose units stay below the range
// cap is latency-bound: 2-tile ranges need one K/V round trip instead of two (MI355X: 1.5-2 us
// less per call for B <= 16 at 512-8192 tokens), unless that cuts a sequence into more than
// kMaxMergeRanges ranges, whose merge then costs more (one 32k-token sequence cut 512 ways: +6 us).
// 4 tiles also keep the partial records (3.6 KB per kv head and range) under a quarter of a
// range's K/V bytes.
int32_t auto_min_tiles(int64_t batch, int64_t table_width, int32_t block_size, int32_t ranges) {
  const double tiles = std::ceil((double)table_width * block_size / 32.0);  // longest sequence
  const double units = (double)batch * (tiles + kSeqStartCost);
  const double p = std::fmin(std::ceil(units / kMinTilesSmall), (double)ranges);
  return p <= (double)kMaxMergeRanges * (double)batch ? kMinTilesSmall : kMinTilesLarge;
}

// The automatic choice of the per-sequence layout (group_kernel), from host-side bounds only:
// the longest possible sequence (table width x block size) and the workgroup count.  It saves the
// merge launch and the range plan, but each workgroup streams a whole sequence on one CU, so it
// pays when the waves hold few tiles or the workgroups cover enough of the chip.  Measured on
// MI355X (INT8, graph replays, uniform lengths, op time per call against the range layout): with
// at most 3 tiles per wave it wins at every batch (ctx 640-768: 10.0-10.6 vs 10.6-12.2 us, B = 1
// to 16); with 4 from 32 workgroups on (ctx 1024: B = 8 11.77 vs 11.89, B = 16 11.84 vs 13.22,
// B = 24 12.27 vs 14.44 us; B = 1-4 lose 0.3-0.45 us); with 6 from ~96 (ctx 1536: B = 24 15.58 vs
// 16.54 us, B = 16 loses 0.9 us); with 8 from 128 (ctx 2048 B = 32 even, B = 16 loses 2.1 us).
// So an INT8 call needs (tiles per wave - 3) x CUs / 8 workgroups, at most CUs / 2, and past one
// workgroup per CU the two layouts trade places by +-3 us (B = 32-192, 28/4 and 32/8 heads), so
// it stops there.  BF16 tiles hold twice the bytes: up to 2 tiles per wave at any count, up to 4
// from CUs / 2 workgroups, and it keeps winning up to 3 workgroups per CU (28/4 heads: B = 128 x
// 512 25.8 vs 29.9 us, B = 192 x 1024 78.3 vs 82.4; at 4 per CU it loses, 50.9 vs 46.7).
// At head_dim 64 the workgroup's LDS state is half as large and the range layout's 64-wide loads
// are shorter (32/8 heads): INT8 wins up to 6 tiles per wave at any count (B = 1 x 1536 10.6 vs
// 12.5 us), up to 8 from CUs / 8 workgroups (B = 4 x 2048 12.9 vs 13.3, B = 128 x 2048 45.5 vs
// 56.8), and up to 4 workgroups per CU (B = 128 x 1024 26.4 vs 32.6; at 6 per CU with 4 tiles
// per wave 54.3 vs 45.0, at 8 per CU it loses at every length); BF16 wins up to 4 tiles per wave
// at any count (B = 8 x 1024 9.5 vs 12.8 us) and loses from 6 on.  At head_dim 256 (16/8 heads,
// four waves per workgroup): INT8 wins up to 4 tiles per wave at any count up to 3 workgroups
// per CU (B = 1 x 256 10.2 vs 14.2 us, B = 32 x 512 17.8 vs 22.8, B = 96 x 512 42.7 vs 47.1; at
// 4 per CU 44.0 vs 29.5), with 8 from CUs / 2 to CUs workgroups (B = 32 x 1024 27.4 vs 32.4;
// B = 1 and 8 x 1024 lose 4.1 and 0.6); 16-bit caches up to 2 tiles per wave (B = 1 x 256 10.9
// vs 14.6), 4 from CUs / 2 workgroups (B = 16 x 512 18.3 vs 22.4; B = 1-8 lose 0.7-0.8).
// Workgroups per (sequence, kv head) of the split per-sequence layout: one on every CU, at most
// 64 (one merge lane each) and at most 2 x num_ranges / batch (the records use the range-record
// rows of the workspace, 2 x num_ranges per query head); at head_dim 128 also at most
// max(16, tiles / 4) for the longest possible sequence's tiles, so that short sequences do not
// leave workgroups without tiles: B = 1 x 1024 / 2048 / 4096 tokens (32 / 64 / 128 tiles) measured
// best at Z = 16-32 / 16-32 / 32 (INT8 9.3-9.4 / 9.7 / 10.5 us, BF16 8.7 / 9.5-9.8 / 10.6 us,
// HIP-graph replays) against 10.5 / 10.8 / 11.6 (INT8) at Z = 64.  Below 2 it is the plain
// layout.
int32_t split_count(int64_t batch, int32_t num_kv_heads, int32_t num_ranges, int64_t cu,
                    int32_t head_dim, int64_t table_width, int32_t block_size) {
  int64_t z = cu / (batch * num_kv_heads);
  z = std::min<int64_t>(z, 64);
  z = std::min<int64_t>(z, 2 * (int64_t)num_ranges / batch);
  if (head_dim == 128) {
    const int64_t tiles = ((int64_t)table_width * block_size + 31) / 32;  // longest sequence
    z = std::min<int64_t>(z, std::max<int64_t>(16, tiles / 4));
  }
  return z >= 2 ? (int32_t)z : 0;
}

bool use_per_sequence(bool int8_cache, int32_t head_dim, int64_t batch, int32_t num_kv_heads,
                      int64_t table_width, int32_t block_size, int64_t cu) {
  const int64_t wgs = batch * num_kv_heads;
  const double tiles = std::ceil((double)table_width * block_size / 32.0);  // longest sequence
  const int nw = head_dim > 128 ? group_waves<256>() : group_waves<128>();
  const int64_t per_wave = (int64_t)std::ceil(tiles / nw);
  if (head_dim > 128) {  // four waves per workgroup, so twice the tiles per wave
    if (wgs > 3 * cu) return false;
    if (!int8_cache) return per_wave <= 2 || (per_wave <= 4 && 2 * wgs >= cu);
    // Few workgroups with 3 or more tiles per wave: the split layout (use_split) spreads them
    // over every CU (B = 1 / 2 / 4 x 512: 13.1 / 13.1 / 13.3 -> 11.2 / 10.5 / 11.2 us).
    if (8 * wgs <= cu && per_wave >= 3) return false;
    return per_wave <= 4 || (per_wave <= 8 && 2 * wgs >= cu && wgs <= cu);
  }
  if (head_dim == 64) {
    if (wgs > 4 * cu) return false;
    if (!int8_cache) return per_wave <= 4;
    return per_wave <= 6 || (per_wave <= 8 && wgs >= cu / 8);
  }
  if (!int8_cache) {
    // Few workgroups: the split layout, once each of its workgroups gets a tile, beats the
    // per-sequence one for 16-bit caches even at 2 tiles per wave (B = 1 / 2 / 4 / 8 x 512:
    // 8.04 / 8.02 / 8.20 / 8.59 vs 8.99 / 9.02 / 9.10 / 9.19 us).
    if (8 * wgs <= cu &&
        tiles >= (double)split_count(batch, num_kv_heads, 1 << 20, cu, head_dim, table_width,
                                     block_size))
      return false;
    return wgs <= 3 * cu && (per_wave <= 2 || (per_wave <= 4 && 2 * wgs >= cu));
  }
  if (wgs > cu) return false;
  // Few workgroups with 3 or more tiles per wave: the split layout (use_split) spreads them over
  // every CU once each of its workgroups gets a tile (B = 8 x 1024 11.7 -> 9.8 us, 8 x 768 10.5
  // -> 8.9, 4 x 768 10.3 -> 9.6; B = 1 x 768, under a tile per split workgroup, 10.3 vs 10.9).
  if (8 * wgs <= cu && per_wave >= 3 && tiles * (double)wgs >= (double)cu) return false;
  if (per_wave <= 3) return true;
  if (per_wave > 8) return false;
  const int64_t need = (per_wave - 3) * cu / 8;
  return wgs >= (need < cu / 2 ? need : cu / 2);
}

// The automatic choice of the split per-sequence layout, for few long sequences (when the
// per-sequence layout itself is not taken): the range layout cuts such a sequence into up to 256
// ranges per kv head, whose records the merge then reads on one CU per query head (one 32k-token
// sequence: 133 KB per query head, ~5.8 us of its 7 us), while the split layout leaves Z <= 64
// records, already combined over the workgroup's waves in LDS.  Taken with at least 8 workgroups per
// (sequence, kv head) and at most 4 tiles per wave (2 at head_dim 64, whose 64-wide loads lose to
// the range layout's paired kv heads beyond that).  Measured on MI355X (HIP-graph replays, op
// time, automatic range layout vs split, us): 28/4 heads at head_dim 128, INT8: B = 1 x 32768
// 18.7 vs 15.3, 1 x 16384 15.2 vs 13.2, 1 x 8192 13.5 vs 12.2, 1 x 65536 23.4 vs 22.4, 2 x 8192
// 14.5 vs 11.8, 4 x 4096 13.2 vs 11.1, 8 x 8192 21.4 vs 20.6 (1 x 4096 loses 0.3); 8 tiles per
// wave or more lose (8 x 32768 53.2 vs 53.9, 4 workgroups: 16 x 8192 29.9 vs 31.6); BF16 cache
// 1 x 8192 15.0 vs 11.9; 16/8 heads at 256: 1 x 16384 26.5 vs 22.4; 32/8 heads at 64: 1 x 8192
// 15.1 vs 9.6, 4 tiles per wave ties (1 x 32768 18.7 vs 19.0) and 8 lose (4 x 16384 21.3 vs 28.7).
bool use_split(int32_t head_dim, int64_t batch, int32_t num_kv_heads, int64_t table_width,
               int32_t block_size, int64_t cu) {
  const int64_t wgs = batch * num_kv_heads;
  if (8 * wgs > cu) return false;
  const int64_t z = split_count(batch, num_kv_heads, 1 << 20, cu, head_dim, table_width, block_size);
  if (z < 2) return false;
  const double tiles = std::ceil((double)table_width * block_size / 32.0);  // longest sequence
  const int nw = head_dim > 128 ? group_waves<256>() : group_waves<128>();
  return tiles / (double)(z * nw) <= (head_dim == 64 ? 2.0 : 4.0);
}

// head_dim 64 with an even kv-head count and GQA groups of at most 8: a wave can take two kv
// heads as one 128-wide head (their rows sit side by side in the cache when the head stride is
// head_dim), 2 G <= 16 query heads in the MFMA columns.  Loads then have HD = 128's shape
// (32-byte K runs, 8-byte V pieces per lane and token row) instead of 16- and 4-byte ones.
bool kv_pair_shape(int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim) {
  return head_dim == 64 && num_kv_heads % 2 == 0 && num_q_heads / num_kv_heads <= 8;
}

int32_t auto_ranges(int32_t num_kv_heads, int64_t cu) {
  const int64_t p = cu * kWavesPerCU / num_kv_heads;
  return (int32_t)(p < 1 ? 1 : (p > kMaxRangesLimit ? kMaxRangesLimit : p));
}

// Per range: 2 x num_q_heads partial records (head_dim + 2 floats each) and the 32-byte
// cut-sequence descriptor.  The records' bytes are a multiple of 16, so the descriptors that
// follow them stay 16-byte aligned.
size_t workspace_bytes(int32_t num_q_heads, int32_t ranges, int32_t head_dim) {
  return (size_t)ranges * (2 * num_q_heads * (head_dim + 2) * sizeof(float) + 4 * sizeof(int64_t));
}

bool aligned16(const void* p, int64_t stride_bytes) {
  return ((uintptr_t)p % 16) == 0 && (stride_bytes % 16) == 0;
}

// Cache block sizes: powers of two from one 16-token row group up to kMaxBlock.
constexpr int32_t kMaxBlock = 1 << 16;

bool block_size_ok(int32_t block_size) {
  return block_size >= kRows && block_size <= kMaxBlock && (block_size & (block_size - 1)) == 0;
}

// head_dim: a multiple of 16 from 16 to 256 (the kernels run at 64, 128 or 256, padded_head_dim;
// 16-byte K pieces and V columns of whole 16-element groups stay inside the cache row).  Any GQA
// group: above 16 query heads per kv head the grid takes ceil(group / 16) column tiles of 16 per
// kv head (col_tiles), up to 65535 grid heads.
bool shape_ok(int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size) {
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0) return false;
  const int64_t tiles = (num_q_heads / num_kv_heads + kMaxGroup - 1) / kMaxGroup;
  return (int64_t)num_kv_heads * tiles <= 65535 && head_dim >= 16 && head_dim <= 256 &&
         head_dim % 16 == 0 && block_size_ok(block_size);
}

// MFMA column tiles of 16 query heads per kv head, and the grid's heads (kv heads x tiles).
int32_t col_tiles(int32_t num_q_heads, int32_t num_kv_heads) {
  return (num_q_heads / num_kv_heads + kMaxGroup - 1) / kMaxGroup;
}

int32_t grid_heads(int32_t num_q_heads, int32_t num_kv_heads) {
  return num_kv_heads * col_tiles(num_q_heads, num_kv_heads);
}

}  // namespace

extern "C" int32_t int8kv_decode_auto_ranges(int32_t num_kv_heads) {
  if (num_kv_heads <= 0) return 1;
  return auto_ranges(num_kv_heads, cu_count());
}

extern "C" size_t int8kv_decode_workspace_bytes(int32_t num_q_heads, int32_t num_kv_heads,
                                                int32_t head_dim, int32_t block_size,
                                                int32_t num_ranges) {
  if (!shape_ok(num_q_heads, num_kv_heads, head_dim, block_size) || num_ranges < 0 ||
      num_ranges > kMaxRangesLimit)
    return 0;
  if (num_ranges == 0)
    num_ranges = auto_ranges(kv_pair_shape(num_q_heads, num_kv_heads, head_dim)
                                 ? num_kv_heads / 2
                                 : grid_heads(num_q_heads, num_kv_heads),
                             cu_count());
  return workspace_bytes(num_q_heads, num_ranges, padded_head_dim(head_dim));
}

// ------------------------------------------------------------------ no-allocation scratch
// Split partials of int8kv_paged_decode_noalloc: a fixed array in the code object, so a call
// allocates nothing.  Each GPU the library runs on holds its own copy (kScratchBytes) until the
// process ends.  In host code `scratch` names a host-side stand-in, not device memory: its
// device address is looked up once per device with hipGetSymbolAddress and only that address is
// ever passed to a kernel.  Every call on a GPU shares that GPU's array (calls that overlap on one
// GPU race); the decode kernel writes every partial record and range descriptor the merge kernel
// reads, so nothing needs clearing between calls.
constexpr size_t kScratchBytes = INT8KV_DECODE_SCRATCH_BYTES;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {

constexpr int kMaxScratchDevices = 64;
std::atomic<void*> g_scratch_addr[kMaxScratchDevices];
std::mutex g_scratch_lookup;

// Device address of the current device's scratch array (looked up on its first use there).
int current_scratch(void** addr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxScratchDevices) return INT8KV_E_SCRATCH;
  void* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_lookup);
    p = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return (int)e;
      if (p == nullptr) return INT8KV_E_SCRATCH;
      g_scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *addr = p;
  return INT8KV_OK;
}

// Merge kernel of the range layout's merge indexed by sequence: waves per workgroup and records
// per lane slot and round, from an estimate of the ranges per sequence (ranges / batch, bounded
// by the longest sequence the table allows: a range holds at least min_tiles units, so no
// sequence spans more than units_max / min_tiles + 1 ranges).  One round of a wave takes
// 2 x FOLD ranges (at head_dim 128).  More waves and eight records per round only for long cut
// sequences (MI355X, op = decode + merge): one 32k-token sequence cut 256 ways 21.3 -> 18.4 us
// with 8 waves x 8, B = 1 x 4096 (67 ranges) 12.1 -> 11.6 us and B = 2 x 16384 (128 ranges each)
// 18.4 -> 17.4 us with 4 x 8, while at 32-36 ranges per sequence (B = 8 x 4096, 1 x 2048,
// 4 x 2048) eight per round costs 0.2-0.3 us and eight waves 1 us.
void merge_shape(int64_t batch, int64_t table_width, int32_t block_size, int32_t tile_tokens,
                 int32_t seq_cost, int32_t min_tiles, int32_t num_ranges, int32_t* waves,
                 int32_t* fold) {
  const int64_t units_max =
      ((int64_t)table_width * block_size + tile_tokens - 1) / tile_tokens + seq_cost;
  const int64_t span_max = (units_max + min_tiles - 1) / min_tiles + 1;
  int64_t per_seq = ((int64_t)num_ranges + batch - 1) / batch;
  if (per_seq > span_max) per_seq = span_max;
  *fold = per_seq <= 48 ? 4 : 8;
  *waves = per_seq <= 8 ? 1 : per_seq <= 16 ? 2 : per_seq <= 128 ? 4 : 8;
}

// The host's whole decision for one call (argument checks on sizes and dtypes included; no
// pointer is looked at).  cus: compute units of the device the call runs on.  scratch_cap: the
// no-allocation entry point's workspace limit (0 = none); an automatic range count is lowered
// to fit it.
int plan_call(int query_dtype, int cache_dtype, int64_t batch, int32_t num_q_heads,
              int32_t num_kv_heads, int32_t head_dim, int64_t num_blocks, int32_t block_size,
              int64_t table_width, int64_t key_head_stride, int64_t value_head_stride,
              int32_t num_ranges, int32_t min_tiles, uint32_t flags, int64_t cus,
              size_t scratch_cap, HostPlan* hp) {
  if (query_dtype != INT8KV_F32 && query_dtype != INT8KV_F16 && query_dtype != INT8KV_BF16)
    return INT8KV_E_DTYPE;
  if (cache_dtype != INT8KV_I8 && cache_dtype != INT8KV_BF16 && cache_dtype != INT8KV_F16)
    return INT8KV_E_DTYPE;
  if (batch < 0 || !shape_ok(num_q_heads, num_kv_heads, head_dim, block_size) ||
      num_blocks <= 0 || table_width <= 0 || table_width > 0x7fffffffLL || num_ranges < 0 ||
      num_ranges > kMaxRangesLimit || min_tiles < 0 || batch > 0x7fffffffLL || cus <= 0)
    return INT8KV_E_SHAPE;
  const bool i8 = cache_dtype == INT8KV_I8;
  const int64_t ce = i8 ? 1 : 2;
  const bool automatic = num_ranges == 0 && min_tiles == 0;
  const bool auto_ranges_req = num_ranges == 0;
  // The kernels run at hd (head_dim padded to 64, 128 or 256) over the grid heads hv (kv heads,
  // times the column tiles of groups above 16 query heads).  Every layout rule below is stated
  // for the kernels' shape; the padded instances keep one range per workgroup with two tiles in
  // flight.
  const int32_t hd = padded_head_dim(head_dim);
  const bool pad = hd != head_dim;
  const int32_t hv = grid_heads(num_q_heads, num_kv_heads);
  const bool kv_pair_ok = kv_pair_shape(num_q_heads, num_kv_heads, head_dim) &&
                          key_head_stride == head_dim && value_head_stride == head_dim;
  const int32_t wave_heads = kv_pair_ok ? num_kv_heads / 2 : hv;  // per range
  if (num_ranges == 0) num_ranges = auto_ranges(wave_heads, cus);
  if (scratch_cap > 0 && auto_ranges_req) {
    // The partials of the automatic count may exceed the fixed scratch array (large GQA groups
    // or head_dim 256): take the most ranges it holds instead.
    const size_t fit = scratch_cap / workspace_bytes(num_q_heads, 1, hd);
    if (fit < 1) return INT8KV_E_SCRATCH;
    if ((size_t)num_ranges > fit) num_ranges = (int32_t)fit;
  }
  if (min_tiles == 0) min_tiles = auto_min_tiles(batch, table_width, block_size, num_ranges);
  HostPlan p{};
  p.cus = cus;
  p.hd = hd;
  p.pad = pad;
  p.grid_heads = hv;
  p.col_tiles = col_tiles(num_q_heads, num_kv_heads);
  p.num_ranges = num_ranges;
  p.min_tiles = min_tiles;
  p.need = workspace_bytes(num_q_heads, num_ranges, hd);
  if (scratch_cap > 0 && p.need > scratch_cap) return INT8KV_E_SCRATCH;
  // (An empty batch launches nothing; the rules below divide by it.)
  p.group_mode = (flags & INT8KV_DECODE_PER_SEQUENCE) != 0 ||
                 (automatic && batch > 0 &&
                  use_per_sequence(i8, hd, batch, hv, table_width, block_size, cus));
  p.split = 0;
  if (batch > 0 && ((flags & INT8KV_DECODE_SPLIT_SEQUENCES) != 0 ||
                    (automatic && !p.group_mode &&
                     use_split(hd, batch, hv, table_width, block_size, cus)))) {
    p.group_mode = true;
    // A caller's range count fixes the split count (num_ranges / batch workgroups per sequence
    // and kv head, e.g. the reference's num_splits); the automatic one fills the chip.
    p.split = auto_ranges_req
                  ? split_count(batch, hv, num_ranges, cus, hd, table_width, block_size)
                  : (int32_t)std::min<int64_t>(64, num_ranges / batch);
    if (p.split < 2) p.split = 0;
  }
  p.kv_pair = kv_pair_ok && !p.group_mode;
  const int32_t tile_tokens = kRows * (i8 ? tile_blocks<kI8>() : tile_blocks<kBF16>());
  p.seq_cost = kSeqStartCost;
  {
    // Paired layout (two ranges per workgroup, the first one longer) for INT8 calls whose
    // range count reaches a pair per CU (two waves per SIMD: only an explicit num_ranges does)
    // and that can fill it: P >= pair_min needs at least pair_min * min_tiles units, bounded
    // here by batch x (longest possible sequence).  16-bit caches (1 % slower paired) keep one
    // range per workgroup.
    const int64_t wgs_y = wave_heads / waves_per_wg(wave_heads);  // workgroups per range
    const int64_t pair_min = (2LL * cus + wgs_y - 1) / wgs_y;
    const double units_max =
        (double)batch * (std::ceil((double)table_width * block_size / tile_tokens) + p.seq_cost);
    const bool paired = i8 && hd <= 128 && !pad && num_ranges >= pair_min &&
                        units_max >= (double)pair_min * min_tiles &&
                        units_max >= (double)pair_min * kPairMinUnits;
    p.halves = paired ? 2 : 1;
    p.pair_min = paired ? (int32_t)pair_min : 0x7fffffff;
    // One wave per SIMD at most (every range's waves resident at once) and long ranges: INT8
    // waves keep four tiles in flight instead of two, the bytes in flight of two waves.
    p.depth = i8 && !paired && hd <= 128 && !pad &&
                      (int64_t)num_ranges * wave_heads <= 4LL * cus &&
                      units_max >= (double)kDeepMinUnits * num_ranges
                  ? 4
                  : 2;
  }
  // The layout above was chosen with the base charge; the plan itself charges what a sequence
  // start costs at the chosen depth (kSeqStartCost*).  decode_kernel and merge_kernel read the
  // same value, so their range bounds agree.
  if (i8) p.seq_cost = p.depth == 4 ? kSeqStartCostI8Deep : kSeqStartCostI8;
  // Four tiles in flight leave no registers for an fp32 query's lo operands: two for those.
  p.launch_depth = p.group_mode ? 2 : (p.depth == 4 && query_dtype != INT8KV_F32 ? 4 : 2);
  // Units of one sequence are at most ceil(table_width x block_size / 32) + seq_cost (lengths are
  // clamped to the table); 64 of them fit the 32-bit wave scans unless one sequence could hold
  // more than 2^25 tiles.
  p.scan32 = (double)kWave * (std::ceil((double)table_width * block_size / tile_tokens) +
                              p.seq_cost) < 2147483647.0;
  // The merge indexed by range (from descriptors the decode kernel then writes) for batches of
  // at least half the range count, where its grid is the smaller one; below that, the merge
  // indexed by sequence, and no descriptors.
  p.cut_desc = 2 * batch >= (int64_t)num_ranges;
  if (p.group_mode) {
    p.merge = p.split > 0 ? kMergeSplit : kMergeNone;
    p.merge_waves = p.split > 0 ? 1 : 0;
    p.merge_fold = 0;
  } else if (p.cut_desc) {
    p.merge = kMergeByRange;
    p.merge_waves = 1;
    p.merge_fold = 0;
  } else {
    p.merge = kMergeBySequence;
    merge_shape(batch > 0 ? batch : 1, table_width, block_size, tile_tokens, p.seq_cost,
                min_tiles, num_ranges, &p.merge_waves, &p.merge_fold);
  }
  // Non-temporal K/V loads when the call may stream more than kNonTemporalMinBytes: the most it
  // can read is min(pool, batch x table width) blocks of K and V (host-side sizes only).  INT8
  // lanes read K in 32-byte runs at every head_dim (k_run).  With one 64-byte run per lane at
  // head_dim 256 the hint had made those calls 13-15 % slower; with two 32-byte runs it makes
  // them 10 % faster (Gemma-2-9B shape, B = 64 x U[1, 16384]: 347 -> 313 us, 6.44 TB/s).
  // 16-bit caches take it at head_dim 128 only, where their K loads follow k_spread (a 64-byte
  // half line per token and instruction): cfg3 BF16 404 -> 360 us, B = 32 x 8256 99.0 -> 89.5,
  // B = 16 x 16384 99.7 -> 90.2 (in runs of k_run the hint made the same calls 10-11 % slower);
  // at head_dim 256 it measured 1 % slower (659 -> 666 us), and padded head_dims and kv-head
  // pairs (k_run order) are not measured with it.  The per-sequence kernels read without it.
  const int64_t touch_blocks = batch * table_width < num_blocks ? batch * table_width : num_blocks;
  p.nt = (i8 || (hd == 128 && !p.pad && !p.kv_pair)) && !p.group_mode &&
         (double)touch_blocks * block_size * num_kv_heads * head_dim * ce * 2 >
             (double)kNonTemporalMinBytes;
  *hp = p;
  return INT8KV_OK;
}

// Shared body of int8kv_paged_decode and int8kv_paged_decode_noalloc.  from_scratch: take the
// current device's scratch array as the workspace (after every argument check, so a rejected
// call touches no device).
int decode_entry(
    const void* query, int query_dtype, int64_t batch, int32_t num_q_heads, int32_t head_dim,
    const int64_t query_strides[3], const void* key_cache, const void* value_cache,
    int cache_dtype, int64_t num_blocks, int32_t block_size, int32_t num_kv_heads,
    const int64_t key_cache_strides[4], const int64_t value_cache_strides[4],
    const void* block_tables, int table_dtype, int64_t table_width, const int64_t table_strides[2],
    const void* seq_lens, int seq_lens_dtype, const float* k_scale, const float* v_scale,
    float sm_scale, void* out, const int64_t out_strides[3], void* workspace,
    size_t workspace_bytes_given, int32_t num_ranges, int32_t min_tiles, uint32_t flags,
    void* stream, bool from_scratch) {
  if (!query_strides || !key_cache_strides || !value_cache_strides || !table_strides ||
      !out_strides)
    return INT8KV_E_NULL;
  if (table_dtype != INT8KV_I32 && table_dtype != INT8KV_I64) return INT8KV_E_DTYPE;
  if (seq_lens_dtype != INT8KV_I32 && seq_lens_dtype != INT8KV_I64) return INT8KV_E_DTYPE;
  HostPlan hp;
  {
    // Sizes and dtypes first (the plan checks them); the CU count only once they pass.
    const int st = plan_call(query_dtype, cache_dtype, batch, num_q_heads, num_kv_heads, head_dim,
                             num_blocks, block_size, table_width, key_cache_strides[2],
                             value_cache_strides[2], num_ranges, min_tiles, flags, 256,
                             from_scratch ? kScratchBytes : 0, &hp);
    if (st != INT8KV_OK) return st;
  }
  if (batch == 0) return INT8KV_OK;
  if (!query || !key_cache || !value_cache || !block_tables || !seq_lens || !out)
    return INT8KV_E_NULL;
  if (cache_dtype == INT8KV_I8 && (!k_scale || !v_scale)) return INT8KV_E_NULL;

  const int64_t qe = query_dtype == INT8KV_F32 ? 4 : 2;
  const int64_t ce = cache_dtype == INT8KV_I8 ? 1 : 2;
  if (query_strides[2] != 1 || out_strides[2] != 1 || key_cache_strides[3] != 1 ||
      value_cache_strides[3] != 1)
    return INT8KV_E_STRIDE;
  if (!aligned16(query, query_strides[0] * qe) || !aligned16(query, query_strides[1] * qe) ||
      !aligned16(out, out_strides[0] * qe) || !aligned16(out, out_strides[1] * qe))
    return INT8KV_E_STRIDE;
  for (int i = 0; i < 3; ++i) {
    if (!aligned16(key_cache, key_cache_strides[i] * ce) ||
        !aligned16(value_cache, value_cache_strides[i] * ce))
      return INT8KV_E_STRIDE;
  }
  {
    const int st = plan_call(query_dtype, cache_dtype, batch, num_q_heads, num_kv_heads, head_dim,
                             num_blocks, block_size, table_width, key_cache_strides[2],
                             value_cache_strides[2], num_ranges, min_tiles, flags, cu_count(),
                             from_scratch ? kScratchBytes : 0, &hp);
    if (st != INT8KV_OK) return st;
  }
  if (from_scratch) {
    const int st = current_scratch(&workspace);
    if (st != INT8KV_OK) return st;
    workspace_bytes_given = kScratchBytes;
  }
  if (workspace == nullptr || workspace_bytes_given < hp.need || ((uintptr_t)workspace % 16) != 0)
    return INT8KV_E_WORKSPACE;

  DecodeArgs a;
  a.q = static_cast<const char*>(query);
  a.q_sb = query_strides[0];
  a.q_sh = query_strides[1];
  a.kc = static_cast<const char*>(key_cache);
  a.vc = static_cast<const char*>(value_cache);
  a.kc_sb = key_cache_strides[0] * ce;
  a.kc_ss = key_cache_strides[1] * ce;
  a.kc_sh = key_cache_strides[2] * ce;
  a.vc_sb = value_cache_strides[0] * ce;
  a.vc_ss = value_cache_strides[1] * ce;
  a.vc_sh = value_cache_strides[2] * ce;
  a.bt = block_tables;
  a.bt_sb = table_strides[0];
  a.bt_sl = table_strides[1];
  a.sl = seq_lens;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.out = static_cast<char*>(out);
  a.o_sb = out_strides[0];
  a.o_sh = out_strides[1];
  const int64_t recs = (int64_t)hp.num_ranges * 2 * num_q_heads;
  float* ws = static_cast<float*>(workspace);
  a.ws_acc = ws;
  a.ws_m = ws + recs * hp.hd;
  a.ws_l = ws + recs * (hp.hd + 1);
  a.ws_cut = reinterpret_cast<int64_t*>(ws + recs * (hp.hd + 2));
  a.head_dim = head_dim;
  a.num_blocks = num_blocks;
  a.batch = batch;
  a.num_kv_heads = hp.grid_heads;
  a.num_q_heads = num_q_heads;
  a.group = num_q_heads / num_kv_heads;
  a.col_tiles = hp.col_tiles;
  a.width = (int32_t)table_width;
  a.max_ranges = hp.num_ranges;
  a.min_tiles = hp.min_tiles;
  a.seq_cost = hp.seq_cost;
  a.quantize_q = (flags & INT8KV_DECODE_QUANTIZE_Q) != 0;
  a.group_mode = hp.group_mode;
  a.split = hp.split;
  a.kv_pair = hp.kv_pair;
  a.block_shift = __builtin_ctz((unsigned)block_size);
  a.tile_tokens = kRows * (cache_dtype == INT8KV_I8 ? tile_blocks<kI8>() : tile_blocks<kBF16>());
  a.bt_is64 = table_dtype == INT8KV_I64;
  a.sl_is64 = seq_lens_dtype == INT8KV_I64;
  a.sm_scale_log2e = sm_scale * kLog2e;
  a.first_share = kFirstShare;
  a.halves = hp.halves;
  a.pair_min = hp.pair_min;
  a.depth = hp.depth;
  a.scan32 = hp.scan32;
  a.cut_desc = hp.merge == kMergeByRange;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (cache_dtype) {
    case INT8KV_I8:
      return hp.pad ? launch_cache_int8_pad(a, hp, query_dtype, flags, s)
                    : launch_cache_int8(a, hp, query_dtype, flags, s);
    case INT8KV_BF16:
      return hp.pad ? launch_cache_bf16_pad(a, hp, query_dtype, flags, s)
                    : launch_cache_bf16(a, hp, query_dtype, flags, s);
    default:
      return hp.pad ? launch_cache_fp16_pad(a, hp, query_dtype, flags, s)
                    : launch_cache_fp16(a, hp, query_dtype, flags, s);
  }
}

}  // namespace

extern "C" int int8kv_decode_plan(int query_dtype, int cache_dtype, int64_t batch,
                                  int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                  int64_t num_blocks, int32_t block_size, int64_t table_width,
                                  int64_t key_head_stride, int64_t value_head_stride,
                                  int32_t num_ranges, int32_t min_tiles, uint32_t flags,
                                  int32_t compute_units, int32_t no_alloc,
                                  int8kv_decode_plan_t* plan) {
  if (plan == nullptr) return INT8KV_E_NULL;
  if (compute_units < 0) return INT8KV_E_SHAPE;
  const int64_t cus = compute_units > 0 ? compute_units : cu_count();
  HostPlan hp;
  const int st = plan_call(query_dtype, cache_dtype, batch, num_q_heads, num_kv_heads, head_dim,
                           num_blocks, block_size, table_width, key_head_stride,
                           value_head_stride, num_ranges, min_tiles, flags, cus,
                           no_alloc ? kScratchBytes : 0, &hp);
  if (st != INT8KV_OK) return st;
  int8kv_decode_plan_t p{};
  p.layout = !hp.group_mode ? INT8KV_LAYOUT_RANGES
             : hp.split > 0 ? INT8KV_LAYOUT_SPLIT
                            : INT8KV_LAYOUT_PER_SEQUENCE;
  p.kernels = batch == 0 ? 0 : (hp.merge == kMergeNone ? 1 : 2);
  p.num_ranges = hp.num_ranges;
  p.min_tiles = hp.min_tiles;
  p.seq_cost = hp.seq_cost;
  p.ranges_per_workgroup = hp.group_mode ? 0 : hp.halves;
  p.depth = hp.launch_depth;
  p.kv_pair = hp.kv_pair ? 1 : 0;
  p.split = hp.split;
  p.non_temporal = hp.nt ? 1 : 0;
  p.merge = hp.merge;
  p.merge_waves = hp.merge_waves;
  p.merge_fold = hp.merge_fold;
  p.compute_units = (int32_t)cus;
  p.workspace_bytes = hp.need;
  *plan = p;
  return INT8KV_OK;
}

extern "C" int int8kv_paged_decode(
    const void* query, int query_dtype, int64_t batch, int32_t num_q_heads, int32_t head_dim,
    const int64_t query_strides[3], const void* key_cache, const void* value_cache,
    int cache_dtype, int64_t num_blocks, int32_t block_size, int32_t num_kv_heads,
    const int64_t key_cache_strides[4], const int64_t value_cache_strides[4],
    const void* block_tables, int table_dtype, int64_t table_width, const int64_t table_strides[2],
    const void* seq_lens, int seq_lens_dtype, const float* k_scale, const float* v_scale,
    float sm_scale, void* out, const int64_t out_strides[3], void* workspace,
    size_t workspace_bytes_given, int32_t num_ranges, int32_t min_tiles, uint32_t flags,
    void* stream) {
  return decode_entry(query, query_dtype, batch, num_q_heads, head_dim, query_strides, key_cache,
                      value_cache, cache_dtype, num_blocks, block_size, num_kv_heads,
                      key_cache_strides, value_cache_strides, block_tables, table_dtype,
                      table_width, table_strides, seq_lens, seq_lens_dtype, k_scale, v_scale,
                      sm_scale, out, out_strides, workspace, workspace_bytes_given, num_ranges,
                      min_tiles, flags, stream, false);
}

extern "C" int int8kv_paged_decode_noalloc(
    const void* query, int query_dtype, int64_t batch, int32_t num_q_heads, int32_t head_dim,
    const int64_t query_strides[3], const void* key_cache, const void* value_cache,
    int cache_dtype, int64_t num_blocks, int32_t block_size, int32_t num_kv_heads,
    const int64_t key_cache_strides[4], const int64_t value_cache_strides[4],
    const void* block_tables, int table_dtype, int64_t table_width, const int64_t table_strides[2],
    const void* seq_lens, int seq_lens_dtype, const float* k_scale, const float* v_scale,
    float sm_scale, void* out, const int64_t out_strides[3], int32_t num_ranges,
    int32_t min_tiles, uint32_t flags, void* stream) {
  return decode_entry(query, query_dtype, batch, num_q_heads, head_dim, query_strides, key_cache,
                      value_cache, cache_dtype, num_blocks, block_size, num_kv_heads,
                      key_cache_strides, value_cache_strides, block_tables, table_dtype,
                      table_width, table_strides, seq_lens, seq_lens_dtype, k_scale, v_scale,
                      sm_scale, out, out_strides, nullptr, 0, num_ranges, min_tiles, flags, stream,
                      true);
}
