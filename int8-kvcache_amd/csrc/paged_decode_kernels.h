// Kernels of the paged decode (INT8 and 16-bit caches) and their launchers, shared by the
// translation units that instantiate them: paged_decode_int8.hip, paged_decode_bf16.hip and
// paged_decode_fp16.hip each compile one cache type's kernels (in parallel), paged_decode.hip
// holds the host side (planner, entry points of include/int8kv.h).  The design notes are at the
// top of paged_decode.hip.

#ifndef INT8KV_PAGED_DECODE_KERNELS_H
#define INT8KV_PAGED_DECODE_KERNELS_H

#include <cmath>
#include <type_traits>

#include "int8kv_common.h"

namespace int8kv {

// head_dim: 64, 128 or 256 (template parameter HD of the kernels).
constexpr int kRows = 16;           // tokens per MFMA row group (half a tile)
constexpr int kMaxGroup = 16;       // query heads per kv head (MFMA column count)
constexpr int kChunkTiles = 256;    // tiles whose block ids a wave stages in LDS at a time
constexpr int kMaxWavesPerWG = 4;

// 16-token row groups per wave iteration ("tile"): 32 tokens, one MFMA k-step of P*V.
template <int CACHE>
constexpr int tile_blocks() {
  return 2;
}
constexpr float kLazyRescale = 8.0f;
constexpr float kLog2e = 1.4426950408889634f;

// ---- Measurement build only: libint8kv_stamps.so, every source compiled with -DINT8KV_STAMPS
// (bench.py --stamps).  Each wave of decode_kernel, group_kernel and probe_decode_kernel keeps
// s_memrealtime stamps (the GPU's constant 100 MHz counter) in registers at fixed points and
// stores them once, at its end, into its translation unit's g_stamps (slot = workgroup x waves
// per workgroup + wave); int8kv_stamps_read_<unit> copies them out.  Stamps:
//   0 entry; 1 sequence lengths read (group) / plan made (ranges); 2 first segment: its block
//   ids staged and its first tiles requested; 3 its query operand built; 4 its first tile's
//   scores done (K arrived and dequantised); 5 that tile's P*V done (V arrived); 6 the
//   segment's tiles done; 7 end (ranges, probe) / after the workgroup barrier (group); 8 the
//   wave's XCD (HW_REG_XCC_ID); 9 first segment entered.
// In the product build (no INT8KV_STAMPS) every macro below is empty.
#ifdef INT8KV_STAMPS
constexpr int kStampSlots = 10;
constexpr int kStampWaves = 16384;
struct Stamps {
  unsigned long long t[kStampSlots];
};
__device__ unsigned long long g_stamps[kStampWaves * kStampSlots];
__device__ __forceinline__ unsigned long long stamp_now() {
  __builtin_amdgcn_sched_barrier(0);
  const unsigned long long t = __builtin_amdgcn_s_memrealtime();
  __builtin_amdgcn_sched_barrier(0);
  return t;
}
__device__ __forceinline__ void store_stamps(Stamps& st, int waves_per_wg, int wave, int lane) {
  // HW_REG_XCC_ID (hardware register 20), bits [3:0]: the XCD the wave runs on.
  st.t[8] = (unsigned)__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u;
  const long long slot =
      (((long long)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * waves_per_wg +
      wave;
  if (lane == 0 && slot < kStampWaves) {
#pragma unroll
    for (int i = 0; i < kStampSlots; ++i) g_stamps[slot * kStampSlots + i] = st.t[i];
  }
}
#define INT8KV_STAMPS_DECL Stamps stamps_{};
#define INT8KV_STAMP(i) (stamps_.t[i] = stamp_now())
#define INT8KV_STAMP_ONCE(i) \
  do {                       \
    if (stamps_.t[i] == 0) stamps_.t[i] = stamp_now(); \
  } while (0)
#define INT8KV_STAMP_SEG(i)                                        \
  do {                                                             \
    if (stamps_p && stamps_p->t[i] == 0) stamps_p->t[i] = stamp_now(); \
  } while (0)
#define INT8KV_STAMPS_PARAM , Stamps* stamps_p = nullptr
#define INT8KV_STAMPS_ARG , &stamps_
#define INT8KV_STAMPS_ARG_NO_GROUP , nullptr, nullptr, nullptr, nullptr, &stamps_
#define INT8KV_STAMPS_STORE(waves_per_wg, wave, lane) store_stamps(stamps_, waves_per_wg, wave, lane)
#define INT8KV_STAMPS_ACCESSORS(unit)                                                          \
  extern "C" int int8kv_stamps_read_##unit(void* dst, size_t bytes) {                         \
    if (bytes > sizeof(int8kv::g_stamps)) return 1;                                            \
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(int8kv::g_stamps), bytes, 0,               \
                                    hipMemcpyDeviceToHost);                                    \
  }                                                                                            \
  extern "C" int int8kv_stamps_clear_##unit() {                                                \
    static unsigned long long zero[int8kv::kStampWaves * int8kv::kStampSlots];                 \
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(int8kv::g_stamps), zero, sizeof(zero), 0,        \
                                  hipMemcpyHostToDevice);                                      \
  }
#else
#define INT8KV_STAMPS_DECL
#define INT8KV_STAMP(i) ((void)0)
#define INT8KV_STAMP_ONCE(i) ((void)0)
#define INT8KV_STAMP_SEG(i) ((void)0)
#define INT8KV_STAMPS_PARAM
#define INT8KV_STAMPS_ARG
#define INT8KV_STAMPS_ARG_NO_GROUP
#define INT8KV_STAMPS_STORE(waves_per_wg, wave, lane) ((void)0)
#define INT8KV_STAMPS_ACCESSORS(unit)
#endif

struct DecodeArgs {
  const char* q;
  int64_t q_sb, q_sh;  // element strides
  const char* kc;
  const char* vc;
  int64_t kc_sb, kc_ss, kc_sh;  // byte strides
  int64_t vc_sb, vc_ss, vc_sh;
  const void* bt;
  int64_t bt_sb, bt_sl;  // element strides
  const void* sl;
  const float* k_scale;
  const float* v_scale;
  char* out;
  int64_t o_sb, o_sh;  // element strides
  float* ws_acc;       // [max_ranges * 2][num_q_heads][head_dim]
  float* ws_m;         // [max_ranges * 2][num_q_heads]
  float* ws_l;         // [max_ranges * 2][num_q_heads]
  int64_t* ws_cut;     // [max_ranges][4]: (sequence, unit of its last tile) of the cut sequence a
                       // range starts (its tile 0 lies in the range and its tiles run past it;
                       // sequence -1 when the range starts none), then the plan (U; P, share,
                       // paired packed), from which the merge finds the sequence's last range
  int64_t num_blocks;
  int64_t batch;
  int32_t num_kv_heads;  // heads of the grid: kv heads x col_tiles (see head_map)
  int32_t num_q_heads;
  int32_t group;        // query heads per kv head
  int32_t col_tiles;    // MFMA column tiles of 16 query heads per kv head: ceil(group / 16)
  int32_t width;       // block-table width in blocks
  int32_t max_ranges;  // P upper bound (= grid.x of decode_kernel)
  int32_t min_tiles;   // P <= ceil(U / min_tiles)
  int32_t seq_cost;    // stream units charged for starting a sequence (see make_plan)
  int32_t quantize_q;  // quantise q per (sequence, head) to int8 first (the reference's option)
  int32_t tile_tokens;  // 16 * tile_blocks<CACHE>()
  int32_t block_shift;  // log2(cache block size); the block size is a power of two >= 16
  int32_t bt_is64;
  int32_t sl_is64;
  float sm_scale_log2e;
  int32_t first_share;  // of a range pair's units, the first range's share in 1/256
  int32_t pair_min;     // ranges are paired when P >= pair_min (every CU gets a whole pair)
  int32_t halves;       // ranges per workgroup (1, or 2 with the paired layout)
  int32_t depth;        // tiles of K/V loads in flight per wave (2, or 4: INT8, one range per WG)
  int32_t group_mode;   // one workgroup per (sequence, kv head), states merged in LDS
  int32_t head_dim;     // the cache's head_dim: a multiple of 16, at most the kernels' HD
  int32_t scan32;       // a 64-sequence chunk's units fit 32 bits (see units_scan)
  int32_t cut_desc;     // write ws_cut (merge_by_range_kernel follows)
  int32_t kv_pair;      // head_dim 64: each wave takes kv heads 2k and 2k + 1 as one 128-wide head
  int32_t split;        // per-sequence layout over `split` workgroups per (sequence, kv head), whose
                        // records merge_split_kernel combines (0: one workgroup, no records)
};

// A grid head (a wave's or workgroup's "kv head") is one column tile of up to 16 query heads of
// one kv head: grid head vh is kv head vh / col_tiles and its query heads q0 .. q0 + g - 1,
// q0 = kv head x group + 16 (vh % col_tiles).  With at most 16 query heads per kv head (every
// shape but the largest multi-query ones) it is the kv head itself.
struct HeadMap {
  int kv;  // kv head (cache head, its scales)
  int q0;  // first query head
  int g;   // query heads in this tile (the MFMA columns used)
};

__device__ __forceinline__ HeadMap head_map(const DecodeArgs& a, int vh) {
  if (a.col_tiles == 1) return {vh, vh * a.group, a.group};
  const int kv = vh / a.col_tiles;
  const int t = vh - kv * a.col_tiles;
  const int rest = a.group - 16 * t;
  return {kv, kv * a.group + 16 * t, rest < 16 ? rest : 16};
}

// ------------------------------------------------------------------------ wave utilities
// Combines x over the four 16-lane rows of the wave (lanes l, l ^ 16, l ^ 32, l ^ 48: one MFMA
// column's four lane groups) with gfx950's row swaps, v_permlane32_swap then v_permlane16_swap:
// two VALU exchanges instead of two LDS permutes (ds_bpermute, whose round trips sat on the
// critical path of every tile's softmax and of each segment's start).  Every lane gets the same
// bits: op(op(x0, x2), op(x1, x3)) for rows 0-3 (op commutative).
template <typename Op>
__device__ __forceinline__ float across_rows(float x, Op op) {
  const uint32_t b = __float_as_uint(x);
  const auto h = __builtin_amdgcn_permlane32_swap(b, b, false, false);  // rows {0,1} <-> {2,3}
  const float y = op(__uint_as_float(h[0]), __uint_as_float(h[1]));
  const uint32_t c = __float_as_uint(y);
  const auto r = __builtin_amdgcn_permlane16_swap(c, c, false, false);  // rows 0 <-> 1, 2 <-> 3
  return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float rows_max(float x) {
  return across_rows(x, [](float u, float v) { return fmaxf(u, v); });
}

__device__ __forceinline__ float rows_sum(float x) {
  return across_rows(x, [](float u, float v) { return u + v; });
}

__device__ __forceinline__ int64_t wave_sum(int64_t x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

__device__ __forceinline__ int64_t wave_inclusive_scan(int64_t x, int lane) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int64_t y = __shfl_up(x, (unsigned)o);
    if (lane >= o) x += y;
  }
  return x;
}

// Inclusive prefix sum of a 32-bit value over the wave (all 64 lanes active): DPP row shifts
// by 1, 2, 4, 8 inside each 16-lane row, then the totals of the rows below (lanes 15, 31, 47,
// read before they change) added to each row.  A few dozen VALU cycles, against six
// dependent LDS permutes per 32-bit word for a __shfl_up / __shfl_xor ladder.
__device__ __forceinline__ int32_t wave_scan32(int32_t x, int lane) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  const int32_t r0 = __builtin_amdgcn_readlane(x, 15);
  const int32_t r1 = __builtin_amdgcn_readlane(x, 31);
  const int32_t r2 = __builtin_amdgcn_readlane(x, 47);
  const int row = lane >> 4;
  return x + (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
}

__device__ __forceinline__ int64_t readlane64(int64_t x, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)x >> 32), lane);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// ------------------------------------------------------------------------ work plan
// Sequence b's token count L_b = clamp(seq_lens[b], 0, width * 16) and tile count
// n_b = ceil(L_b / tile_tokens).  The batch becomes a stream of units: a non-empty sequence
// contributes seq_cost "start" units (the latency of its first block ids and tiles, which a
// range pays again for every sequence it starts) followed by its n_b tiles.  With U units in
// all, P = clamp(ceil(U / min_tiles), 1, max_ranges) and the uniform bounds are b_r = r U / P,
// so every range costs the same whatever the lengths.  When P >= pair_min (enough ranges for a
// pair on every CU), ranges come in pairs (2k, 2k + 1), the two halves of one workgroup, and
// the bound between them moves from b_{2k+1} to first_share / 256 of the pair's units (an
// unpaired last range keeps its bounds): the first half, which streams faster on a shared
// SIMD, gets the larger share.
__device__ __forceinline__ int64_t seq_len_of(const DecodeArgs& a, int64_t b) {
  if (b >= a.batch) return 0;
  int64_t L = load_index(a.sl, b, a.sl_is64);
  const int64_t cap = (int64_t)a.width << a.block_shift;
  return L < 0 ? 0 : (L > cap ? cap : L);
}

// seq_len_of for a sequence b < batch that the whole workgroup shares (the per-sequence kernels'
// blockIdx.x), without branches: the low word at b x (4 or 8) bytes and, for 64-bit lengths, the
// high word after it (else the same word again), both requested at once.  seq_len_of's bounds
// test and its branch on the index type put two dependent scalar round trips (the type flag,
// then the length) in front of everything these kernels do.
__device__ __forceinline__ int64_t seq_len_uniform(const DecodeArgs& a, int64_t b) {
  const char* p = static_cast<const char*>(a.sl) + (b << (a.sl_is64 ? 3 : 2));
  const uint32_t lo = *reinterpret_cast<const uint32_t*>(p);
  const uint32_t hi = *reinterpret_cast<const uint32_t*>(p + (a.sl_is64 ? 4 : 0));
  const int64_t L = a.sl_is64 ? (int64_t)(((uint64_t)hi << 32) | lo) : (int64_t)(int32_t)lo;
  const int64_t cap = (int64_t)a.width << a.block_shift;
  return L < 0 ? 0 : (L > cap ? cap : L);
}

// Lengths (as seq_len_of) of sequences (c0 + k) 64 + lane, k < K, with all K loads issued before
// any is used (the index clamped into the batch, 0 past it): seq_len_of's bounds test around
// each load made every chunk wait for the previous one.
template <int K>
__device__ __forceinline__ void seq_len_chunks(const DecodeArgs& a, int64_t c0, int lane,
                                               int64_t (&L)[K]) {
  const int64_t last = a.batch - 1;
  if (a.sl_is64) {
    const int64_t* t = reinterpret_cast<const int64_t*>(a.sl);
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int64_t i = (c0 + k) * kWave + lane;
      L[k] = t[i < last ? i : last];
    }
  } else {
    const int32_t* t = reinterpret_cast<const int32_t*>(a.sl);
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int64_t i = (c0 + k) * kWave + lane;
      L[k] = t[i < last ? i : last];
    }
  }
  const int64_t cap = (int64_t)a.width << a.block_shift;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int64_t x = L[k] < 0 ? 0 : (L[k] > cap ? cap : L[k]);
    L[k] = (c0 + k) * kWave + lane <= last ? x : 0;
  }
}

__device__ __forceinline__ int64_t tiles_of(const DecodeArgs& a, int64_t L) {
  static_assert(tile_blocks<kI8>() == 2 && tile_blocks<kBF16>() == 2, "32-token tiles");
  return (L + 2 * kRows - 1) / (2 * kRows);
}

__device__ __forceinline__ int64_t units_of(const DecodeArgs& a, int64_t n) {
  return n > 0 ? n + a.seq_cost : 0;
}

// Inclusive scan / total of the lanes' unit counts over one 64-sequence chunk.  32-bit DPP
// scan when the host has bounded a chunk's units below 2^31 (scan32: no sequence can exceed
// 2^25 tiles), else the 64-bit permute ladder.
__device__ __forceinline__ int64_t units_scan(const DecodeArgs& a, int64_t u, int lane) {
  if (a.scan32) return (int64_t)wave_scan32((int32_t)u, lane);
  return wave_inclusive_scan(u, lane);
}

__device__ __forceinline__ int64_t units_sum(const DecodeArgs& a, int64_t u, int lane) {
  if (a.scan32) return (int64_t)__builtin_amdgcn_readlane(wave_scan32((int32_t)u, lane), kWave - 1);
  return wave_sum(u);
}

// a / b for a >= 0, b > 0, with a 32-bit divide when both fit (the plan's bounds always do in
// practice; the 64-bit divide is a long instruction sequence on the GPU).
__device__ __forceinline__ int64_t udiv(int64_t a, int64_t b) {
  if ((((uint64_t)a | (uint64_t)b) >> 32) == 0) return (int64_t)((uint32_t)a / (uint32_t)b);
  return a / b;
}

// Ranges are paired only when they average at least this many units: short ranges are
// latency-bound, and shifting a unit or two between them costs more than the balance gains.
constexpr int kPairMinUnits = 16;

struct Plan {
  int64_t U;
  int64_t P;
  int32_t share;  // first_share
  bool paired;
};

// A plan's P, share and paired in one word (P < 2^31, share < 2^8), and back, with U.
__device__ __forceinline__ int64_t pack_plan(const Plan& p) {
  return p.P | ((int64_t)p.share << 32) | ((int64_t)p.paired << 40);
}

__device__ __forceinline__ Plan unpack_plan(int64_t U, int64_t w) {
  return {U, w & 0x7fffffff, (int32_t)((w >> 32) & 0xff), ((w >> 40) & 1) != 0};
}

// The plan of a batch of U units.
__device__ __forceinline__ Plan plan_of_units(const DecodeArgs& a, int64_t U) {
  int64_t P = udiv(U + a.min_tiles - 1, a.min_tiles);
  P = P < 1 ? 1 : (P > a.max_ranges ? a.max_ranges : P);
  return {U, P, a.first_share, P >= a.pair_min && U >= (int64_t)kPairMinUnits * P};
}

// L0: this lane's seq_len_of(a, lane), the first 64 sequences' lengths, which the caller keeps
// in a register for its own walk over the batch (most batches have at most 64 sequences).
__device__ __forceinline__ Plan make_plan(const DecodeArgs& a, int lane, int64_t L0) {
  int64_t U = units_sum(a, units_of(a, tiles_of(a, L0)), lane);
  for (int64_t base = kWave; base < a.batch; base += kWave)
    U += units_sum(a, units_of(a, tiles_of(a, seq_len_of(a, base + lane))), lane);
  return plan_of_units(a, U);
}

// Bound between the ranges of pair k (2k + 1 < P): first_share of the pair's units, at least
// one unit on each side (P <= U keeps every uniform range non-empty).
__device__ __forceinline__ int64_t pair_split(const Plan& p, int64_t k) {
  const int64_t ps = udiv(2 * k * p.U, p.P);
  const int64_t pe = udiv((2 * k + 2) * p.U, p.P);
  int64_t h = ((pe - ps) * p.share) >> 8;
  h = h < 1 ? 1 : (h > pe - ps - 1 ? pe - ps - 1 : h);
  return ps + h;
}

__device__ __forceinline__ int64_t range_start(const Plan& p, int64_t r) {
  if (p.paired && (r & 1) && r < p.P) return pair_split(p, r >> 1);
  return udiv(r * p.U, p.P);
}

// The range holding stream unit x (0 <= x < U): the largest r with range_start(r) <= x.
__device__ __forceinline__ int64_t range_of(const Plan& p, int64_t x) {
  const int64_t r0 = udiv((x + 1) * p.P - 1, p.U);  // uniform range
  const int64_t k = r0 >> 1;
  if (!p.paired || 2 * k + 1 >= p.P) return r0;  // uniform, or the unpaired last range
  return 2 * k + (x >= pair_split(p, k) ? 1 : 0);
}

// Partial-record slot of a sequence cut by a range: 0 if it started in an earlier range, 1 if
// it starts in this range and continues after it.  A range cuts at most one sequence of each
// kind (its first and its last), so the two slots never collide.
__device__ __forceinline__ int64_t cut_slot(int64_t first_tile) { return first_tile > 0 ? 0 : 1; }

// ------------------------------------------------------------------------ tile registers
// Registers holding the K or the V half of one tile (NB 16-token row groups) for one lane, for
// head_dim HD (64, 128 or 256).
//   K: lane (i = lane % 16, g = lane / 16) holds token i of row group s, head_dim elements
//      [HD/4 g, HD/4 (g + 1)): HD/4 elements, HD E / 64 16-byte pieces.
//   V: lane (i, g) holds tokens 4g + r (r = 0..3) of row group s, head_dim elements
//      [HD/16 i, HD/16 (i + 1)): HD E / 64 dwords per token row.
template <int CACHE, int HD>
constexpr int k_pieces() {
  return HD * (CACHE == kI8 ? 1 : 2) / 64;
}
template <int CACHE, int HD>
constexpr int v_dwords() {
  return HD * (CACHE == kI8 ? 1 : 2) / 64;
}
template <int CACHE, int NB, int HD>
struct KTile {
  u32x4 k[NB][k_pieces<CACHE, HD>()];
};
template <int CACHE, int NB, int HD>
struct VTile {
  uint32_t v[NB][4][v_dwords<CACHE, HD>()];
};

template <int CACHE>
struct MfmaOp;
template <>
struct MfmaOp<kI8> {
  typedef f16x8 T;
  typedef _Float16 E;
};
template <>
struct MfmaOp<kF16> {
  typedef f16x8 T;
  typedef _Float16 E;
};
template <>
struct MfmaOp<kBF16> {
  typedef bf16x8 T;
  typedef __bf16 E;
};

__device__ __forceinline__ f32x4 mfma(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Exact int8 x int8 -> int32 product of a 16x64 and a 64x16 tile (lane (i, g): row/column i,
// 16 k-slots of group g).
__device__ __forceinline__ i32x4 mfma_i8(u32x4 a, i32x4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a), b, c, 0, 0, 0);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Byte permute: result byte k = byte sel_k of the 8-byte value {hi, lo} (0-3 from lo).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

constexpr uint32_t kMagic = 0x64646464u;     // fp16 exponent byte of 1024.0
constexpr uint32_t kSignFlip = 0x80808080u;  // int8 -> offset binary (x + 128)
constexpr uint32_t kSelLo = 0x04010400u;     // [b0, 0x64, b1, 0x64]
constexpr uint32_t kSelHi = 0x04030402u;     // [b2, 0x64, b3, 0x64]

// Four offset-binary bytes of d0 and four of d1 -> 8 exact fp16 values of the signed bytes.
__device__ __forceinline__ f16x8 i8x8_to_f16(uint32_t d0, uint32_t d1) {
  u32x4 w;
  w[0] = perm(kMagic, d0, kSelLo);
  w[1] = perm(kMagic, d0, kSelHi);
  w[2] = perm(kMagic, d1, kSelLo);
  w[3] = perm(kMagic, d1, kSelHi);
  return __builtin_bit_cast(f16x8, w) - (f16x8)(_Float16)1152.0f;
}

template <int DT>
constexpr int esize() {
  return DT == kF32 ? 4 : (DT == kI8 ? 1 : 2);
}

// Stores 8 consecutive fp32 values as DT (16-byte aligned destination).
template <int DT>
__device__ __forceinline__ void store8(char* p, const float (&x)[8]) {
  if constexpr (DT == kF32) {
    f32x4* q = reinterpret_cast<f32x4*>(p);
    q[0] = f32x4{x[0], x[1], x[2], x[3]};
    q[1] = f32x4{x[4], x[5], x[6], x[7]};
  } else if constexpr (DT == kF16) {
    f16x8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = (_Float16)x[i];
    *reinterpret_cast<f16x8*>(p) = h;
  } else {
    bf16x8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = (__bf16)x[i];
    *reinterpret_cast<bf16x8*>(p) = h;
  }
}

// Stores N (4, 8 or 16) consecutive fp32 values as DT (aligned to min(N, 8) elements).
template <int DT, int N>
__device__ __forceinline__ void store_n(char* p, const float (&x)[N]) {
  static_assert(N == 4 || N == 8 || N == 16, "4, 8 or 16 elements");
  if constexpr (N == 16) {
    const float lo[8] = {x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]};
    const float hi[8] = {x[8], x[9], x[10], x[11], x[12], x[13], x[14], x[15]};
    store8<DT>(p, lo);
    store8<DT>(p + 8 * esize<DT>(), hi);
  } else if constexpr (N == 8) {
    store8<DT>(p, x);
  } else if constexpr (DT == kF32) {
    *reinterpret_cast<f32x4*>(p) = f32x4{x[0], x[1], x[2], x[3]};
  } else if constexpr (DT == kF16) {
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
    *reinterpret_cast<f16x4*>(p) = f16x4{(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]};
  } else {
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    *reinterpret_cast<bf16x4*>(p) = bf16x4{(__bf16)x[0], (__bf16)x[1], (__bf16)x[2], (__bf16)x[3]};
  }
}

// Cache-stream load.  NT (chosen per call by the host, INT8 caches only): the non-temporal hint,
// +10 % delivered bandwidth on MI355X when the call streams more K/V than the Infinity Cache
// holds; a small pool that the cache keeps between calls is read faster without it.  16-bit
// caches always use plain loads: their wider per-lane rows (64 B of K per lane) measured ~12 %
// slower with the hint.
template <int CACHE, bool NT, typename T>
__device__ __forceinline__ T stream_load(const T* p) {
  if constexpr (NT)
    return __builtin_nontemporal_load(p);
  else
    return *p;
}

// Where each 16-token row group of a tile starts: its cache block and its first row in the block.
template <int NB>
struct TileRows {
  int32_t id[NB];
  int32_t row[NB];
};

// The lane's HD/4 K elements of its token: one contiguous run [HD/4 lg, HD/4 (lg + 1)) up to
// head_dim 128; at 256 two runs of HD/8, [HD/8 lg, ...) and [HD/2 + HD/8 lg, ...), so that an
// INT8 lane reads 32 contiguous bytes per run as at 128 (the order the lane's elements are held
// in, run 0 then run 1, is the order issue_query loads the query in, so the products pair the
// same elements).
template <int HD>
__device__ __forceinline__ constexpr int k_run(int run, int lg) {
  return HD > 128 ? run * (HD / 2) + lg * (HD / 8) : lg * (HD / 4);
}

// SPREAD (16-bit caches outside kv-head pairs): k-step j of lane group lg holds head_dim
// elements 32 j + 8 lg .. + 7 instead of the runs of k_run, so the four lane groups of a token
// read one contiguous 64-byte half line per load instruction (its 16-byte piece j at byte
// 64 j + 16 lg); in runs of HD/4 (64 bytes per lane) each 16-byte load of the four touched both
// 128-byte lines of a 256-byte row, and with the non-temporal hint the kernel ran 10-11 % slower
// instead of 11 % faster.  An INT8 row is one 128-byte line, which each of its loads already
// meets as one line: the same order measured within noise there (cfg3 191.7 vs 191.5 us).  Any
// assignment of head_dim elements to k-steps gives the same dot products as long as K and the
// query use the same one.
__device__ __forceinline__ constexpr int k_spread(int j, int lg) { return 32 * j + 8 * lg; }

// PAD (head_dim D < HD): a lane's 16-byte pieces at or past element D read the row's first piece
// instead, which keeps every access inside the row; their products meet query elements that are
// zero, and the V columns at or past D feed output columns that are never stored.
template <int CACHE, int NB, bool NT, int HD, bool PAD = false, bool SPREAD = false>
__device__ __forceinline__ void issue_k(KTile<CACHE, NB, HD>& r, const char* kb,
                                        const TileRows<NB>& ph, const DecodeArgs& a, int li,
                                        int lg) {
  constexpr int E = esize<CACHE>();
  constexpr int kRuns = HD > 128 ? 2 : 1;
  constexpr int PR = k_pieces<CACHE, HD>() / kRuns;  // 16-byte pieces per run
#pragma unroll
  for (int s = 0; s < NB; ++s) {
    const char* row = kb + ph.id[s] * a.kc_sb + (ph.row[s] + li) * a.kc_ss;
    if constexpr (SPREAD) {
      static_assert(E == 2, "16-bit caches: one 16-byte piece per k-step");
#pragma unroll
      for (int j = 0; j < k_pieces<CACHE, HD>(); ++j) {
        const int e = k_spread(j, lg);
        r.k[s][j] = stream_load<CACHE, NT>(reinterpret_cast<const u32x4*>(
            row + (!PAD || e < a.head_dim ? e * E : 0)));
      }
      continue;
    }
#pragma unroll
    for (int run = 0; run < kRuns; ++run) {
      if constexpr (PAD) {
#pragma unroll
        for (int i = 0; i < PR; ++i) {
          const int e = k_run<HD>(run, lg) + i * (16 / E);
          r.k[s][run * PR + i] = stream_load<CACHE, NT>(
              reinterpret_cast<const u32x4*>(row + (e < a.head_dim ? e * E : 0)));
        }
      } else {
        const u32x4* k4 = reinterpret_cast<const u32x4*>(row + k_run<HD>(run, lg) * E);
#pragma unroll
        for (int i = 0; i < PR; ++i) r.k[s][run * PR + i] = stream_load<CACHE, NT>(&k4[i]);
      }
    }
  }
}

template <int CACHE, int NB, bool NT, int HD, bool PAD = false>
__device__ __forceinline__ void issue_v(VTile<CACHE, NB, HD>& r, const char* vb,
                                        const TileRows<NB>& ph, const DecodeArgs& a, int li,
                                        int lg) {
  constexpr int E = esize<CACHE>();
  constexpr int DW = v_dwords<CACHE, HD>();
  const int vcol = PAD && HD / 16 * li >= a.head_dim ? 0 : li * (HD / 16 * E);
#pragma unroll
  for (int s = 0; s < NB; ++s) {
    const char* vp = vb + ph.id[s] * a.vc_sb + (ph.row[s] + 4 * lg) * a.vc_ss + vcol;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const char* rp = vp + rr * a.vc_ss;
      if constexpr (DW == 1) {
        r.v[s][rr][0] = stream_load<CACHE, NT>(reinterpret_cast<const uint32_t*>(rp));
      } else if constexpr (DW == 2) {
        const u32x2 x = stream_load<CACHE, NT>(reinterpret_cast<const u32x2*>(rp));
        r.v[s][rr][0] = x[0];
        r.v[s][rr][1] = x[1];
      } else {
        static_assert(DW % 4 == 0, "whole 16-byte pieces");
#pragma unroll
        for (int h = 0; h < DW / 4; ++h) {
          const u32x4 x = stream_load<CACHE, NT>(reinterpret_cast<const u32x4*>(rp) + h);
#pragma unroll
          for (int k = 0; k < 4; ++k) r.v[s][rr][4 * h + k] = x[k];
        }
      }
    }
  }
}

// Scores of one tile (NB row groups) and the online-softmax update: rescales acc/l_part when
// the running max moves and returns the P^T operands (one per MFMA k-step of 32 tokens) as a
// hi + lo pair of 16-bit values (p = hi + lo to about 2^-22 relative), so that P*V on the
// 16-bit matrix cores keeps fp32 accuracy: the rounding of p would otherwise dominate the error
// (2^-12 relative for fp16, 2^-9 for bf16).
//   valid: number of tokens of this tile inside the sequence (1..16 NB).
//   QSPLIT (an fp32 query): q is held as 16-bit hi + lo operands and each k-step takes two MFMAs,
//   so the scores keep ~2^-22 (fp16) / 2^-16 (bf16) relative accuracy instead of one rounding of q.
//   QQ (INT8 cache with a quantised query): the scores are the exact integer products of the
//   int8 K rows and q8 on the int8 matrix cores (2 k-steps of 64, no K conversion); otherwise
//   K is converted to 16-bit operands (4 k-steps of 32).
template <int CACHE, int NB, bool QQ, int HD, bool QSPLIT>
__device__ __forceinline__ void tile_scores(const KTile<CACHE, NB, HD>& r,
                                            const typename MfmaOp<CACHE>::T (&qop)[HD / 32],
                                            const typename MfmaOp<CACHE>::T (&qlo)[HD / 32],
                                            const i32x4 (&q8op)[HD / 64], f32x4 (&acc)[HD / 16],
                                            float& m_run, float& l_part, int valid, int lg,
                                            float s_scale,
                                            typename MfmaOp<CACHE>::T (&pop)[NB / 2][2]) {
  typedef typename MfmaOp<CACHE>::T OpT;
  constexpr int kTileTokens = NB * kRows;
  // ---- scores S^T[token][head] for each row group of the tile ----
  f32x4 S[NB];
#pragma unroll
  for (int s = 0; s < NB; ++s) {
    if constexpr (QQ) {
      i32x4 si = (i32x4)(0);
#pragma unroll
      for (int ks = 0; ks < HD / 64; ++ks) si = mfma_i8(r.k[s][ks], q8op[ks], si);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) S[s][rr] = (float)si[rr];
      continue;
    }
    S[s] = (f32x4)(0.0f);
#pragma unroll
    for (int ks = 0; ks < HD / 32; ++ks) {
      OpT kop;
      if constexpr (CACHE == kI8) {
        const uint32_t d0 = r.k[s][ks >> 1][(ks & 1) * 2] ^ kSignFlip;
        const uint32_t d1 = r.k[s][ks >> 1][(ks & 1) * 2 + 1] ^ kSignFlip;
        kop = i8x8_to_f16(d0, d1);
      } else {
        kop = __builtin_bit_cast(OpT, r.k[s][ks]);
      }
      S[s] = mfma(kop, qop[ks], S[s]);
      if constexpr (QSPLIT) S[s] = mfma(kop, qlo[ks], S[s]);
    }
  }

  // ---- online softmax (exp2 domain); lane column = head, rows = tokens 16s + 4lg + r ----
  float sv[4 * NB];
#pragma unroll
  for (int s = 0; s < NB; ++s)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) sv[4 * s + rr] = S[s][rr] * s_scale;
  if (valid < kTileTokens) {
#pragma unroll
    for (int s = 0; s < NB; ++s)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        if (16 * s + 4 * lg + rr >= valid) sv[4 * s + rr] = -INFINITY;
  }
  float mx = sv[0];
#pragma unroll
  for (int e = 1; e < 4 * NB; ++e) mx = fmaxf(mx, sv[e]);
  mx = rows_max(mx);
  const bool need = mx > m_run + kLazyRescale;
  if (__any(need)) {
    const float m_new = need ? mx : m_run;
    const float alpha = exp2_fast(m_run - m_new);
    m_run = m_new;
    l_part *= alpha;
#pragma unroll
    for (int dt = 0; dt < HD / 16; ++dt) acc[dt] *= alpha;
  }
  typedef typename MfmaOp<CACHE>::E E;
#pragma unroll
  for (int e = 0; e < 4 * NB; ++e) {
    const float pe = exp2_fast(sv[e] - m_run);
    l_part += pe;
    const E hi = (E)pe;
    pop[e / 8][0][e % 8] = hi;
    pop[e / 8][1][e % 8] = (E)(pe - (float)hi);
  }
}

// out^T[dim][head] += V^T[dim][token] * P^T[token][head] for one tile.
// MFMA row i of dim tile dt is head_dim element (HD/16) i + dt; k-slot e of lane group g in
// k-step kst is token (row group 2 kst + e / 4, row 4g + e % 4), matching the P^T operands.
template <int CACHE, int NB, int HD>
__device__ __forceinline__ void tile_pv(VTile<CACHE, NB, HD>& r,
                                        const typename MfmaOp<CACHE>::T (&pop)[NB / 2][2],
                                        f32x4 (&acc)[HD / 16], int valid, int lg) {
  typedef typename MfmaOp<CACHE>::T OpT;
  constexpr int DW = v_dwords<CACHE, HD>();
  if constexpr (CACHE != kI8) {
    // 16-bit rows past the sequence end may hold non-finite garbage; 0 * NaN would leak.
    if (valid < NB * kRows) {
#pragma unroll
      for (int s = 0; s < NB; ++s)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          if (16 * s + 4 * lg + rr >= valid) {
#pragma unroll
            for (int k = 0; k < DW; ++k) r.v[s][rr][k] = 0u;
          }
    }
  }
#pragma unroll
  for (int kst = 0; kst < NB / 2; ++kst) {
    const int s0 = 2 * kst;
    if constexpr (CACHE == kI8) {
      uint32_t pk[2][2][DW][2];  // [row group][token pair][row dword][byte pair 01/23]
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int rp = 0; rp < 2; ++rp)
#pragma unroll
          for (int hsel = 0; hsel < DW; ++hsel) {
            const uint32_t a0 = r.v[s0 + s][2 * rp][hsel] ^ kSignFlip;
            const uint32_t b0 = r.v[s0 + s][2 * rp + 1][hsel] ^ kSignFlip;
            pk[s][rp][hsel][0] = perm(a0, b0, 0x01050004u);  // [a.b0, b.b0, a.b1, b.b1]
            pk[s][rp][hsel][1] = perm(a0, b0, 0x03070206u);  // [a.b2, b.b2, a.b3, b.b3]
          }
#pragma unroll
      for (int dt = 0; dt < HD / 16; ++dt) {
        const int hsel = dt >> 2, bp = (dt >> 1) & 1;
        const uint32_t sel = (dt & 1) ? kSelHi : kSelLo;
        u32x4 w;
        w[0] = perm(kMagic, pk[0][0][hsel][bp], sel);
        w[1] = perm(kMagic, pk[0][1][hsel][bp], sel);
        w[2] = perm(kMagic, pk[1][0][hsel][bp], sel);
        w[3] = perm(kMagic, pk[1][1][hsel][bp], sel);
        const f16x8 vop = __builtin_bit_cast(f16x8, w) - (f16x8)(_Float16)1152.0f;
        acc[dt] = mfma(vop, pop[kst][0], acc[dt]);
        acc[dt] = mfma(vop, pop[kst][1], acc[dt]);
      }
    } else {
#pragma unroll
      for (int dt = 0; dt < HD / 16; ++dt) {
        const int wd = dt >> 1;
        const uint32_t sel = (dt & 1) ? 0x07060302u : 0x05040100u;
        u32x4 w;
        w[0] = perm(r.v[s0][1][wd], r.v[s0][0][wd], sel);
        w[1] = perm(r.v[s0][3][wd], r.v[s0][2][wd], sel);
        w[2] = perm(r.v[s0 + 1][1][wd], r.v[s0 + 1][0][wd], sel);
        w[3] = perm(r.v[s0 + 1][3][wd], r.v[s0 + 1][2][wd], sel);
        const OpT vop = __builtin_bit_cast(OpT, w);
        acc[dt] = mfma(vop, pop[kst][0], acc[dt]);
        acc[dt] = mfma(vop, pop[kst][1], acc[dt]);
      }
    }
  }
}

// Raw query row piece of one lane: head li, its HD/4 elements (the runs of k_run) as loaded.
template <int QT, int HD>
struct QueryRaw {
  u32x4 w[HD / 32];  // HD/4 16-bit elements
};
template <int HD>
struct QueryRaw<kF32, HD> {
  f32x4 w[HD / 16];  // HD/4 fp32 elements
};

// Issues the query loads (no wait): lane (head li, group lg) fetches the HD/4 elements of
// q[b, kvh * G + li] whose K elements it holds (the runs of k_run, in the same order); lanes of
// padding heads (li >= G) hold zeros.
//   PAIR (head_dim 64 as kv heads kvh, kvh + 1 side by side, HD = 128): column li < 2G is query
//   head kvh G + li; its 64 elements go to the lanes of its own kv head's half (lg / 2 = 0 for
//   li < G, 1 above) and the other half's lanes hold zeros, so each column's scores use only its
//   own kv head's K elements.
//   hm: the grid head's query heads (head_map).  PAD: elements at or past head_dim are zero.
template <int QT, int HD, bool PAIR = false, bool PAD = false, bool SPREAD = false>
__device__ __forceinline__ void issue_query(const DecodeArgs& a, int64_t b, const HeadMap& hm,
                                            int li, int lg, QueryRaw<QT, HD>& raw) {
  constexpr int QE = esize<QT>();
  typedef typename std::remove_reference<decltype(raw.w[0])>::type Vec;
  constexpr int N = sizeof(raw.w) / sizeof(raw.w[0]);
  constexpr int kRuns = HD > 128 ? 2 : 1;
  const int kvh = hm.kv;
  if constexpr (SPREAD) {  // k-step j: elements k_spread(j, lg) .. + 7 (issue_k)
    static_assert(!PAIR, "kv-head pairs keep the runs of k_run");
    constexpr int VE = sizeof(Vec) / QE;  // elements per vector: 8 (16-bit) or 4 (fp32)
    constexpr int PV = 8 / VE;            // vectors per k-step
    if (li < hm.g) {
      const char* qrow = a.q + ((int64_t)b * a.q_sb + (int64_t)(hm.q0 + li) * a.q_sh) * QE;
#pragma unroll
      for (int j = 0; j < HD / 32; ++j)
#pragma unroll
        for (int h = 0; h < PV; ++h) {
          const int e = k_spread(j, lg) + h * VE;
          raw.w[j * PV + h] = !PAD || e < a.head_dim
                                  ? *reinterpret_cast<const Vec*>(qrow + e * QE)
                                  : (Vec)(0);
        }
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) raw.w[i] = (Vec)(0);
    }
    return;
  }
  if constexpr (PAIR) {
    static_assert(HD == 128, "pairs of 64-wide kv heads");
    if (li < 2 * a.group && (lg >> 1) == (li >= a.group ? 1 : 0)) {
      const Vec* qp = reinterpret_cast<const Vec*>(
          a.q + ((int64_t)b * a.q_sb + (int64_t)(kvh * a.group + li) * a.q_sh + 32 * (lg & 1)) * QE);
#pragma unroll
      for (int i = 0; i < N; ++i) raw.w[i] = qp[i];
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) raw.w[i] = (Vec)(0);
    }
    return;
  }
  // Up to head_dim 128 the lane's elements are one run and its address is one expression: built
  // from a row pointer plus k_run's offset instead, hipcc's allocation of the depth-2 INT8
  // kernel put a wait for the older loads before each V load of the tile loop (137 instead of
  // 100 s_waitcnt), which cost 0.3-0.45 us per call at B = 1 x 32768 and B = 8 x 4096.
  if constexpr (PAD) {
    constexpr int VE = sizeof(Vec) / QE;  // elements per vector
    if (li < hm.g) {
      const char* qrow = a.q + ((int64_t)b * a.q_sb + (int64_t)(hm.q0 + li) * a.q_sh) * QE;
#pragma unroll
      for (int run = 0; run < kRuns; ++run)
#pragma unroll
        for (int i = 0; i < N / kRuns; ++i) {
          const int e = k_run<HD>(run, lg) + i * VE;
          raw.w[run * (N / kRuns) + i] =
              e < a.head_dim ? *reinterpret_cast<const Vec*>(qrow + e * QE) : (Vec)(0);
        }
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) raw.w[i] = (Vec)(0);
    }
    return;
  }
  if (kRuns == 1 && li < hm.g) {
    const Vec* qp = reinterpret_cast<const Vec*>(
        a.q + ((int64_t)b * a.q_sb + (int64_t)(hm.q0 + li) * a.q_sh + HD / 4 * lg) * QE);
#pragma unroll
    for (int i = 0; i < N; ++i) raw.w[i] = qp[i];
  } else if (li < hm.g) {
    const char* qrow = a.q + ((int64_t)b * a.q_sb + (int64_t)(hm.q0 + li) * a.q_sh) * QE;
#pragma unroll
    for (int run = 0; run < kRuns; ++run) {
      const Vec* qp = reinterpret_cast<const Vec*>(qrow + k_run<HD>(run, lg) * QE);
#pragma unroll
      for (int i = 0; i < N / kRuns; ++i) raw.w[run * (N / kRuns) + i] = qp[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) raw.w[i] = (Vec)(0);
  }
}

__device__ __forceinline__ float round_half_away(float x) {
  return x >= 0.0f ? floorf(x + 0.5f) : -floorf(-x + 0.5f);
}

// Builds the Q^T operand (lane (li, lg) holds element 8 ks + e of its HD/4 query elements, in
// k_run order: q[li][HD/4 lg + 8 ks + e] up to head_dim 128) from the raw loads and
// returns the lane's fp32 factor turning MFMA scores into log2-domain logits.
//   * default: q is scaled by 2^e so the largest |q| of the wave lands in [2^14, 2^15) for fp16
//     operands (exact for bf16 input, never overflows); bf16 operands take q as is;
//   * quantize_q: per (sequence, head) q_scale = max(absmax / 127, 1e-6) and
//     q8 = clamp(round_half_away(q / q_scale), -127, 127) (src/triton_ops/int8_paged_attention.py:
//     137-146, :798-802); the operand is q8 and q_scale joins the score factor.  With QQ the
//     q8 values are packed as int8 operands instead (q8op[ks] byte e of lane (li, lg) =
//     lane element 16 ks + e of q8, matching the int8 K bytes the lane holds).
//   HEADWISE: the 2^e scale per query head (the 4 lanes holding a head's elements, whose score
//   column is the same lane's), two lane exchanges instead of six; the per-sequence kernels use
//   it (their short calls wait on every exchange: ~0.15 us of a 6.5 us kernel on MI355X).
template <int CACHE, int QT, bool QQ, int HD, bool PAIR = false, bool HEADWISE = false>
__device__ __forceinline__ float finish_query(const DecodeArgs& a, const QueryRaw<QT, HD>& raw,
                                              const float (&ksc)[2],
                                              typename MfmaOp<CACHE>::T (&qop)[HD / 32],
                                              typename MfmaOp<CACHE>::T (&qlo)[HD / 32],
                                              i32x4 (&q8op)[HD / 64]) {
  constexpr int KS = HD / 32;  // 16-bit k-steps
  float x[KS][8];
  if constexpr (QT == kF32) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) x[ks][e] = raw.w[2 * ks + e / 4][e % 4];
  } else {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int e = 0; e < 4; ++e) unpack2<QT>(raw.w[ks][e], x[ks][2 * e], x[ks][2 * e + 1]);
  }
  float amax = 0.0f;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(x[ks][e]));
  float s_scale = a.sm_scale_log2e;
  if constexpr (CACHE == kI8) {
    // ksc: the K scales of the wave's kv head and (PAIR) the next one, whose columns start at G.
    const float ks = PAIR && (int)(__lane_id() & 15) >= a.group ? ksc[1] : ksc[0];
    s_scale *= fmaxf(ks, 1e-6f);
  }
  if (a.quantize_q) {
    // absmax over the head's HD elements: the 4 lanes (li, lg = 0..3) of this head column
    amax = rows_max(amax);
    const float qs = fmaxf(amax / 127.0f, 1e-6f);
    if constexpr (QQ) {
#pragma unroll
      for (int ks = 0; ks < HD / 64; ++ks)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          uint32_t word = 0;
#pragma unroll
          for (int bb = 0; bb < 4; ++bb) {
            const int d = 16 * ks + 4 * w + bb;  // element of the lane's HD / 4
            const float v = fminf(fmaxf(round_half_away(x[d / 8][d % 8] / qs), -127.0f), 127.0f);
            word |= ((uint32_t)(int32_t)v & 0xffu) << (8 * bb);
          }
          q8op[ks][w] = (int32_t)word;
        }
      return s_scale * qs;
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        qop[ks][e] = (typename MfmaOp<CACHE>::E)fminf(fmaxf(round_half_away(x[ks][e] / qs), -127.0f),
                                                      127.0f);
    return s_scale * qs;
  }
  float qmul = 1.0f;
  if constexpr (CACHE != kBF16) {
    if constexpr (!HEADWISE) {
      amax = fmaxf(amax, __shfl_xor(amax, 1));
      amax = fmaxf(amax, __shfl_xor(amax, 2));
      amax = fmaxf(amax, __shfl_xor(amax, 4));
      amax = fmaxf(amax, __shfl_xor(amax, 8));
    }
    amax = rows_max(amax);
    if (amax > 0.0f && amax < INFINITY) {
      const int e = 14 - ilogbf(amax);
      qmul = ldexpf(1.0f, e);
      s_scale = ldexpf(s_scale, -e);
    }
  }
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = x[ks][e] * qmul;  // exact: a power of two
      qop[ks][e] = (typename MfmaOp<CACHE>::E)v;
      if constexpr (QT == kF32) qlo[ks][e] = (typename MfmaOp<CACHE>::E)(v - (float)qop[ks][e]);
    }
  return s_scale;
}

// Stages the physical block ids of tiles [c0, c1) of sequence b (nblk blocks) in this wave's
// LDS slots, one per 16-token row group: ids[NB * (t - c0) + s] = the block holding row group s
// of tile t (tokens 16 (NB t + s) .. + 15; consecutive row groups share a block when the block
// size exceeds 16), 0 past the sequence's last block and clamped into [0, num_blocks) so every
// access stays inside the caches.
template <int NB>
__device__ __forceinline__ void stage_block_ids(const DecodeArgs& a, int32_t* ids, int64_t b,
                                                int64_t c0, int64_t c1, int64_t nblk, int lane) {
  const int n = (int)(NB * (c1 - c0));
  const int64_t hi = a.num_blocks - 1;
  const int gshift = a.block_shift - 4;  // row groups per block = 2^gshift
  for (int j = lane; j < n; j += kWave) {
    const int64_t blk = (NB * c0 + j) >> gshift;
    int64_t p = 0;
    if (blk < nblk) p = load_index(a.bt, b * a.bt_sb + blk * a.bt_sl, a.bt_is64);
    ids[j] = (int32_t)(p < 0 ? 0 : (p > hi ? hi : p));
  }
}

// Output rows of an empty sequence: zeros for the grid head's query heads (one wave).  PAD: only
// the columns below head_dim.  (The mask is compiled in only where it is needed: in the
// depth-2 INT8 range kernels this runtime test alone made hipcc place a wait before each V load
// of the tile loop, 139 s_waitcnt instead of 100.)
template <int QT, int HD, bool PAD = false>
__device__ __forceinline__ void write_zero_rows(const DecodeArgs& a, int64_t b, const HeadMap& hm,
                                                int lane) {
  const int li = lane & 15;
  const int lg = lane >> 4;
  if (li >= hm.g) return;
  char* op = a.out + (b * a.o_sb + (int64_t)(hm.q0 + li) * a.o_sh) * esize<QT>();
  float z[HD / 16];
#pragma unroll
  for (int i = 0; i < HD / 16; ++i) z[i] = 0.0f;
#pragma unroll
  for (int rr = 0; rr < 4; ++rr)
    if (!PAD || HD / 4 * lg + HD / 16 * rr < a.head_dim)
      store_n<QT, HD / 16>(op + (HD / 4 * lg + HD / 16 * rr) * esize<QT>(), z);
}

// Processes tiles [ta, tb) of sequence b (length L) for kv head kvh with one wave, then writes
// either the final output (full == true) or a partial record.  ids: this wave's LDS slots.
// DEPTH: tiles of K/V loads kept in flight (register buffers).  GROUP: leave the state
// (running max, sum, accumulators) in this wave's LDS slot (g_acc [HD/4][64], g_m, g_l [16])
// for the workgroup to merge, instead of an output row or a partial record.
// vh: the grid head (head_map); with PAIR the first kv head of the pair.  PAD: head_dim below HD
// (issue_k); the output columns at or past head_dim are not stored.
// QPRE: the caller requested the query (issue_query into *qpre) before the sequence length was
// known; its operand is then built while the first block ids are in flight (below).
template <int CACHE, int QT, bool NT, bool QQ, int HD, int DEPTH, bool GROUP = false,
          bool PAIR = false, bool PAD = false, bool QPRE = false>
__device__ __forceinline__ void run_segment(const DecodeArgs& a, int32_t* ids, int64_t b,
                                            int64_t L, int vh, int64_t ta, int64_t tb,
                                            bool full, int64_t rec, int lane,
                                            float* g_acc = nullptr, float* g_m = nullptr,
                                            float* g_l = nullptr,
                                            const QueryRaw<QT, HD>* qpre = nullptr
                                                INT8KV_STAMPS_PARAM) {
  typedef typename MfmaOp<CACHE>::T OpT;
  constexpr bool kSpread = CACHE != kI8 && !PAIR;  // k_spread (issue_k, issue_query)
  const int li = lane & 15;
  const int lg = lane >> 4;
  const HeadMap hm = head_map(a, vh);
  const int kvh = hm.kv;
  const int G = hm.g;

  f32x4 acc[HD / 16];
#pragma unroll
  for (int dt = 0; dt < HD / 16; ++dt) acc[dt] = (f32x4)(0.0f);
  float m_run = -INFINITY;
  float l_part = 0.0f;

  const char* kb = a.kc + (int64_t)kvh * a.kc_sh;
  const char* vb = a.vc + (int64_t)kvh * a.vc_sh;
  const int64_t nblk = (L + (1 << a.block_shift) - 1) >> a.block_shift;
  constexpr int NB = tile_blocks<CACHE>();
  constexpr int kTileTokens = NB * kRows;

  auto valid_of = [&](int64_t t) -> int {
    const int64_t v = L - t * kTileTokens;
    return v >= kTileTokens ? kTileTokens : (int)v;
  };

  // The tiles are processed in chunks of at most kChunkTiles whose block ids are staged in LDS
  // (read through the LDS counter, so the waits on tile loads below only ever count tile loads).
  int64_t c0 = ta;
  int64_t c1 = (tb - c0 > kChunkTiles) ? c0 + kChunkTiles : tb;
  const int gmask = (1 << (a.block_shift - 4)) - 1;  // row group within its block
  auto blocks_of = [&](int64_t t, TileRows<NB>& ph) {
    const int j = NB * (int)(t - c0);
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      ph.id[s] = __builtin_amdgcn_readfirstlane(ids[j + s]);
      ph.row[s] = (((int)t * NB + s) & gmask) * kRows;
    }
  };

  // DEPTH K and DEPTH V register buffers, refilled as soon as they are consumed: K(t + DEPTH)
  // is requested right after the scores of tile t, V(t + DEPTH) right after its P*V, so up to
  // DEPTH tiles of loads are in flight while a tile is computed.  The main loop body handles
  // DEPTH tiles as one straight-line block and every load in it is unconditional, so the
  // compiler's wait counts are exact and no wait drains the pipeline; only the chunk's last
  // full block refills conditionally (its waits may be coarser: the pipeline is ending there).
  KTile<CACHE, NB, HD> kt[DEPTH];
  VTile<CACHE, NB, HD> vt[DEPTH];
  TileRows<NB> ph[DEPTH];
  OpT pop[NB / 2][2];
  auto issue_first_tiles = [&]() {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      blocks_of(c0 + d < c1 ? c0 + d : c1 - 1, ph[d]);
      issue_k<CACHE, NB, NT, HD, PAD, kSpread>(kt[d], kb, ph[d], a, li, lg);
      issue_v<CACHE, NB, NT, HD, PAD>(vt[d], vb, ph[d], a, li, lg);
    }
  };
  auto chunk_prologue = [&]() {
    stage_block_ids<NB>(a, ids, b, c0, c1, nblk, lane);
    issue_first_tiles();
  };

  // The query, the first chunk's block ids and its first DEPTH tiles are requested back to
  // back; the query operand is built once they are all in flight (otherwise three memory
  // latencies would line up at every segment start).
  // An fp32 query keeps a lo part (QSPLIT); a quantised query is exact in one operand.
  constexpr bool QSPLIT = QT == kF32 && !QQ;
  OpT qop[HD / 32];
  OpT qlo[HD / 32];  // unused (and removed by the compiler) unless QSPLIT
  i32x4 q8op[HD / 64];
  float s_scale;
  {
    // The K scale is requested first: loaded where it is used, its scalar load was issued after
    // the tile loads and its wait sat between the query conversion and the first tile.
    float ksc[2] = {1.0f, 1.0f};
    if constexpr (CACHE == kI8) {
      ksc[0] = a.k_scale[kvh];
      if constexpr (PAIR) ksc[1] = a.k_scale[kvh + 1];
    }
    if constexpr (QPRE) {
      // The query arrived (or is arriving) while the sequence length was read, so its operand is
      // built between the first round of block-id loads and their wait: one unconditional pair
      // of 32-bit loads per lane (the index clamped into the sequence's blocks, the low word and,
      // for 64-bit tables, the high word) keeps the compiler's wait before the build down to the
      // query loads.  Built after the first tile requests instead, it sat between the first
      // tiles' arrival and their scores (0.12 us for a 16-bit query of a 16-bit cache, 0.24 us
      // with the fp16 query scaling of an INT8 cache, at one tile per wave).  The first tiles are
      // requested at the top of the chunk loop below, the one place every chunk's are.
      const int n = (int)(NB * (c1 - c0));  // >= NB: this segment has a tile
      const int64_t hi = a.num_blocks - 1;
      const int gshift = a.block_shift - 4;
      const int64_t blk = (NB * c0 + (lane < n ? lane : n - 1)) >> gshift;
      const int64_t blkc = blk < nblk ? blk : nblk - 1;
      const char* ip = static_cast<const char*>(a.bt) +
                       ((b * a.bt_sb + blkc * a.bt_sl) << (a.bt_is64 ? 3 : 2));
      const uint32_t wlo = *reinterpret_cast<const uint32_t*>(ip);
      const uint32_t whi = *reinterpret_cast<const uint32_t*>(ip + (a.bt_is64 ? 4 : 0));
      s_scale = finish_query<CACHE, QT, QQ, HD, PAIR, GROUP>(a, *qpre, ksc, qop, qlo, q8op);
      INT8KV_STAMP_SEG(3);
      const int64_t p = blk >= nblk ? 0
                        : a.bt_is64 ? (int64_t)(((uint64_t)whi << 32) | wlo)
                                    : (int64_t)(int32_t)wlo;
      if (lane < n) ids[lane] = (int32_t)(p < 0 ? 0 : (p > hi ? hi : p));
      for (int j = lane + kWave; j < n; j += kWave) {  // chunks of more than 64 row groups
        const int64_t bj = (NB * c0 + j) >> gshift;
        int64_t pj = 0;
        if (bj < nblk) pj = load_index(a.bt, b * a.bt_sb + bj * a.bt_sl, a.bt_is64);
        ids[j] = (int32_t)(pj < 0 ? 0 : (pj > hi ? hi : pj));
      }
    } else {
      QueryRaw<QT, HD> qraw;
      issue_query<QT, HD, PAIR, PAD, kSpread>(a, b, hm, li, lg, qraw);
      chunk_prologue();
      INT8KV_STAMP_SEG(2);
      s_scale = finish_query<CACHE, QT, QQ, HD, PAIR, GROUP>(a, qraw, ksc, qop, qlo, q8op);
      INT8KV_STAMP_SEG(3);
    }
  }

  // Tile t + d (buffer d): scores, refill K with tile t + d + DEPTH, P*V, refill V.  refill is a
  // compile-time true inside the main loop; in the chunk's last full block it stops the refills
  // at the chunk's end, so no request repeats a tile there (with non-temporal loads a repeated
  // tile is read from HBM again: 1-4 tiles per segment, ~2 % of a large call's bytes).
  // sched_barrier(0) keeps the compiler's scheduler from sinking the refills past the compute
  // that follows them (which would shorten the prefetch distance).
  auto tile_step = [&](int64_t t, int d, bool refill) {
    const int valid = valid_of(t + d);
    tile_scores<CACHE, NB, QQ, HD, QSPLIT>(kt[d], qop, qlo, q8op,
                                           acc, m_run, l_part, valid, lg, s_scale, pop);
    INT8KV_STAMP_SEG(4);
    if (refill) {
      blocks_of(t + d + DEPTH, ph[d]);
      issue_k<CACHE, NB, NT, HD, PAD, kSpread>(kt[d], kb, ph[d], a, li, lg);
    }
    __builtin_amdgcn_sched_barrier(0);
    tile_pv<CACHE, NB, HD>(vt[d], pop, acc, valid, lg);
    INT8KV_STAMP_SEG(5);
    if (refill) issue_v<CACHE, NB, NT, HD, PAD>(vt[d], vb, ph[d], a, li, lg);
    __builtin_amdgcn_sched_barrier(0);
  };

  bool staged = QPRE;  // QPRE: the first chunk's ids are staged, its tiles not yet requested
  while (true) {
    if constexpr (QPRE) {
      // One request site for every chunk's first tiles: with a second one before the loop, hipcc
      // merged the two into the loop header behind a wait for every load in flight.
      if (!staged) stage_block_ids<NB>(a, ids, b, c0, c1, nblk, lane);
      staged = false;
      issue_first_tiles();
      INT8KV_STAMP_SEG(2);
    }
    int64_t t = c0;
    // Every refill of these blocks lies inside the chunk.
    for (; t + 2 * DEPTH - 1 < c1; t += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) tile_step(t, d, true);
    }
    // The chunk's last full block refills only the tiles the chunk still has.
    if (t + DEPTH - 1 < c1) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) tile_step(t, d, t + d + DEPTH < c1);
      t += DEPTH;
    }
    // The last c1 - t < DEPTH tiles of the chunk are in buffers 0, 1, ...
#pragma unroll
    for (int d = 0; d + 1 < DEPTH; ++d) {
      if (t + d < c1) {
        const int valid = valid_of(t + d);
        tile_scores<CACHE, NB, QQ, HD, QSPLIT>(kt[d], qop, qlo,
                                               q8op, acc, m_run, l_part, valid, lg, s_scale,
                                       pop);
        INT8KV_STAMP_SEG(4);
        tile_pv<CACHE, NB, HD>(vt[d], pop, acc, valid, lg);
        INT8KV_STAMP_SEG(5);
      }
    }
    if (c1 >= tb) break;
    c0 = c1;
    c1 = (tb - c0 > kChunkTiles) ? c0 + kChunkTiles : tb;
    if constexpr (!QPRE) chunk_prologue();
  }

  INT8KV_STAMP_SEG(6);
  l_part = rows_sum(l_part);
  if constexpr (PAIR) {
    // Columns li < 2G; a column's rows are its own kv head's half of the 128 (lg / 2 = 0 for
    // li < G, 1 above: real head_dim elements 32 (lg % 2) + 8 rr + dt); the other half's rows
    // mixed this column's probabilities with the other kv head's V and are dropped.
    static_assert(!GROUP && HD == 128, "pairs of 64-wide kv heads, range layout only");
    const int upper = li >= G ? 1 : 0;
    if (li >= 2 * G) return;
    const int h = kvh * G + li;
    const int64_t row = rec * a.num_q_heads + h;
    if (!full && lg == 2 * upper) {
      a.ws_m[row] = m_run;
      a.ws_l[row] = l_part;
    }
    if ((lg >> 1) != upper) return;
    const int d0 = 32 * (lg & 1);
    if (full) {
      const float vscale = (CACHE == kI8) ? fmaxf(a.v_scale[kvh + upper], 1e-6f) : 1.0f;
      const float inv = l_part > 0.0f ? vscale / l_part : 0.0f;
      char* op = a.out + (b * a.o_sb + (int64_t)h * a.o_sh) * esize<QT>();
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        float o[8];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[dt] = acc[dt][rr] * inv;
        store_n<QT, 8>(op + (d0 + 8 * rr) * esize<QT>(), o);
      }
    } else {
      char* pp = reinterpret_cast<char*>(a.ws_acc + row * 64);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        float o[8];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[dt] = acc[dt][rr];
        store_n<kF32, 8>(pp + (d0 + 8 * rr) * 4, o);
      }
    }
    return;
  }
  if (li >= G) return;
  if constexpr (GROUP) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
#pragma unroll
      for (int dt = 0; dt < HD / 16; ++dt) g_acc[(rr * (HD / 16) + dt) * kWave + lane] = acc[dt][rr];
    if (lg == 0) {
      g_m[li] = m_run;
      g_l[li] = l_part;
    }
    return;
  }
  const int h = hm.q0 + li;
  if (full) {
    const float vscale = (CACHE == kI8) ? fmaxf(a.v_scale[kvh], 1e-6f) : 1.0f;
    const float inv = l_part > 0.0f ? vscale / l_part : 0.0f;
    char* op = a.out + (b * a.o_sb + (int64_t)h * a.o_sh) * esize<QT>();
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      float o[HD / 16];
#pragma unroll
      for (int dt = 0; dt < HD / 16; ++dt) o[dt] = acc[dt][rr] * inv;
      if (!PAD || HD / 4 * lg + HD / 16 * rr < a.head_dim)
        store_n<QT, HD / 16>(op + (HD / 4 * lg + HD / 16 * rr) * esize<QT>(), o);
    }
  } else {
    const int64_t row = rec * a.num_q_heads + h;
    char* pp = reinterpret_cast<char*>(a.ws_acc + row * HD);
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      float o[HD / 16];
#pragma unroll
      for (int dt = 0; dt < HD / 16; ++dt) o[dt] = acc[dt][rr];
      store_n<kF32, HD / 16>(pp + (HD / 4 * lg + HD / 16 * rr) * 4, o);
    }
    if (lg == 0) {
      a.ws_m[row] = m_run;
      a.ws_l[row] = l_part;
    }
  }
}

// grid (ceil(max_ranges / HALVES), num_kv_heads / W), block HALVES * W waves; wave w of
// workgroup (x, y) handles kv head y * W + w % W over stream range x (HALVES = 1), or, with two
// ranges per workgroup, 2x + w / W (paired ranges) or x + (w / W) grid.x.  DEPTH: tiles in flight
// per wave (4 only in the one-wave-per-SIMD layout, whose register budget allows it).
// Register budget: one wave per SIMD (512 registers) for INT8 waves with four tiles in flight,
// for head_dim 256 (twice the tile and accumulator registers) and for 16-bit caches, whose 16 KB
// tiles spilled to scratch under the two-wave budget (their automatic range count is one wave
// per SIMD anyway); two waves per SIMD otherwise.
template <int CACHE, int DEPTH, int HD>
constexpr int decode_waves_per_eu() {
  return (DEPTH > 2 || CACHE != kI8 || HD > 128) ? 1 : 2;
}

template <int CACHE, int QT, bool NT, bool QQ, int HALVES, int HD, int DEPTH, bool PAIR = false,
          bool PAD = false>
__global__ __launch_bounds__(256 * HALVES) __attribute__((amdgpu_waves_per_eu(decode_waves_per_eu<CACHE, DEPTH, HD>()))) void decode_kernel(DecodeArgs a) {
  __shared__ int32_t s_ids[HALVES * kMaxWavesPerWG][kChunkTiles * tile_blocks<CACHE>()];
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int W = blockDim.x / (HALVES * kWave);  // kv heads per workgroup
  const int kvh = blockIdx.y * W + (HALVES == 1 ? wave : wave % W);  // the wave's (pair of) kv heads
  const int kv0 = PAIR ? 2 * kvh : kvh;  // first kv head of the wave
  const int half = HALVES == 1 ? 0 : wave / W;
  INT8KV_STAMPS_DECL
  INT8KV_STAMP(0);

  const int64_t L0 = seq_len_of(a, lane);
  const Plan plan = make_plan(a, lane, L0);
  INT8KV_STAMP(1);
  // One range per workgroup, or two: ranges 2x and 2x + 1 when paired, else x and x + grid.x
  // (the second only when the batch needs more ranges than there are workgroups).
  int64_t r = blockIdx.x;
  if constexpr (HALVES == 2)
    r = plan.paired ? 2 * (int64_t)blockIdx.x + half
                    : (int64_t)blockIdx.x + half * (int64_t)gridDim.x;
  // The range's cut-sequence descriptor for merge_by_range_kernel: "none" first, overwritten by
  // the same lane below if the range starts a cut sequence.  Every range below max_ranges gets
  // one per call, so the workspace needs no initialisation.  It holds only values the walk
  // already has (the merge derives the last range from them), so the walk keeps no more of the
  // plan live than before.
  const bool cut_writer = a.cut_desc && kvh == 0 && lane == 0 && r < a.max_ranges;
  if (cut_writer) {
    a.ws_cut[4 * r] = -1;
    a.ws_cut[4 * r + 2] = plan.U;
    a.ws_cut[4 * r + 3] = pack_plan(plan);
  }
  if (r >= plan.P) return;
  const int64_t u0 = range_start(plan, r);
  const int64_t u1 = range_start(plan, r + 1);
  const bool last_range = r == plan.P - 1;

  int64_t cum = 0;  // units of the sequences before this 64-sequence chunk
  int64_t L = L0;
  for (int64_t base = 0; base < a.batch; base += kWave) {
    if (base > 0) L = seq_len_of(a, base + lane);
    const int64_t n = tiles_of(a, L);
    const int64_t u = units_of(a, n);
    const int64_t incl = units_scan(a, u, lane) + cum;
    const int64_t excl = incl - u;
    const int64_t chunk_end = readlane64(incl, kWave - 1);
    if (chunk_end >= u0) {
      // Empty sequences occupy no units: the range holding their position writes their zeros.
      uint64_t zmask = __ballot(base + lane < a.batch && n == 0 && excl >= u0 &&
                                (excl < u1 || (last_range && excl == plan.U)));
      while (zmask) {
        const int j = __builtin_ctzll(zmask);
        zmask &= zmask - 1;
        if constexpr (PAIR) {
          write_zero_rows<QT, 64>(a, base + j, head_map(a, kv0), lane);
          write_zero_rows<QT, 64>(a, base + j, head_map(a, kv0 + 1), lane);
        } else {
          write_zero_rows<QT, HD, PAD>(a, base + j, head_map(a, kvh), lane);
        }
      }
      // Sequences whose tiles (units past the start cost) meet [u0, u1).
      uint64_t mask = __ballot(n > 0 && incl > u0 && excl + a.seq_cost < u1);
      while (mask) {
        const int j = __builtin_ctzll(mask);
        mask &= mask - 1;
        const int64_t first = readlane64(excl, j) + a.seq_cost;  // unit of tile 0
        const int64_t nb = readlane64(n, j);
        const int64_t Lb = readlane64(L, j);
        const int64_t ta = (u0 > first ? u0 : first) - first;
        const int64_t te = (u1 < first + nb ? u1 : first + nb) - first;
        if (ta >= te) continue;
        const bool full = ta == 0 && te == nb;
        if (cut_writer && ta == 0 && te < nb) {  // b starts here and runs past this range
          a.ws_cut[4 * r] = base + j;
          a.ws_cut[4 * r + 1] = first + nb - 1;
        }
        INT8KV_STAMP_ONCE(9);
        run_segment<CACHE, QT, NT, QQ, HD, DEPTH, false, PAIR, PAD>(
            a, s_ids[wave], base + j, Lb, kv0, ta, te, full, 2 * r + cut_slot(ta),
            lane INT8KV_STAMPS_ARG_NO_GROUP);
      }
    }
    if (chunk_end >= u1 && !last_range) break;
    cum = chunk_end;
  }
  INT8KV_STAMP(7);
  INT8KV_STAMPS_STORE(HALVES * W, wave, lane);
}

// Short sequences, one workgroup per (sequence b = blockIdx.x, kv head blockIdx.y): its
// group_waves<HD>() waves take equal shares of the sequence's tiles, leave their softmax states in
// LDS, and waves 0-3 merge them into the output rows.  No partial records and no merge kernel: a
// call costs one launch and the dependent loads of one segment.  Eight waves (two per SIMD) up
// to head_dim 128; four at 256, one per SIMD as its registers need, whose states then take
// 64 KB of LDS (eight would need 128 KB and spill).
// SPLIT (few long sequences): gridDim.z workgroups per (sequence, kv head), workgroup z taking
// tiles [z n / Z, (z + 1) n / Z) of the sequence's n; each leaves one record per query head
// (row (b Z + z) Hq + h, the layout of the range records) for merge_split_kernel, and an empty
// sequence leaves none (that kernel writes its zero rows).
template <int HD>
constexpr int group_waves() {
  return HD > 128 ? 4 : 8;
}

// Whether share v of nw equal shares of a span (share v of s tiles: [v s / nw, (v + 1) s / nw))
// is non-empty for some span of at most smax tiles.
__device__ __forceinline__ bool share_may_hold(int v, int smax, int nw) {
  if (smax >= nw) return true;
  for (int s = 1; s <= smax; ++s)
    if ((v + 1) * s / nw > v * s / nw) return true;
  return false;
}

template <int CACHE, int QT, bool QQ, int HD, bool SPLIT, bool PAD = false>
__global__ __launch_bounds__(group_waves<HD>() * 64) __attribute__((amdgpu_waves_per_eu(HD > 128 ? 1 : 2))) void group_kernel(DecodeArgs a) {
  constexpr int NW = group_waves<HD>();
  __shared__ int32_t s_ids[NW][kChunkTiles * tile_blocks<CACHE>()];
  __shared__ float s_acc[NW][HD / 4 * kWave];
  __shared__ float s_m[NW][16];
  __shared__ float s_l[NW][16];
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int64_t b = blockIdx.x;
  const int vh = blockIdx.y;  // grid head (head_map)
  INT8KV_STAMPS_DECL
  INT8KV_STAMP(0);
  // The span's NW equal shares go to the waves SIMD by SIMD (wave w runs on SIMD w % 4): wave w
  // takes share (w % 4) (NW / 4) + w / 4, so with fewer tiles than waves the waves that get one
  // sit on different SIMDs.  (In wave order two tiles went to waves 3 and 7, which share SIMD 3.)
  const int v = NW > 4 ? (wave % 4) * (NW / 4) + wave / 4 : wave;
  QueryRaw<QT, HD> qraw;
  bool early_q = false;
  int64_t L;
  if constexpr (SPLIT) {
    L = seq_len_uniform(a, b);  // first: every later step waits for it
  } else {
    // The query rows do not depend on the length, so the waves whose share can hold a tile (for
    // the longest sequence the table holds) request them right behind it: their operand is then
    // built while the block ids are in flight (run_segment, QPRE).  The length's load goes
    // first (a query load ahead of it delayed it by ~0.7 us); in the split layout, whose waves
    // hold one tile each at these sizes, the waiting length outweighed the gain (0.2-0.6 us
    // slower per call), so its kernel keeps the query in run_segment.
    const char* slp = static_cast<const char*>(a.sl) + (b << (a.sl_is64 ? 3 : 2));
    const uint32_t sl_lo = *reinterpret_cast<const uint32_t*>(slp);
    const uint32_t sl_hi = *reinterpret_cast<const uint32_t*>(slp + (a.sl_is64 ? 4 : 0));
    __builtin_amdgcn_sched_barrier(0);
    const int64_t nmax = tiles_of(a, (int64_t)a.width << a.block_shift);
    early_q = share_may_hold(v, nmax < (int64_t)NW ? (int)nmax : NW, NW);
    if (early_q)
      issue_query<QT, HD, false, PAD, CACHE != kI8>(a, b, head_map(a, vh), li, lg, qraw);
    const int64_t Lr =
        a.sl_is64 ? (int64_t)(((uint64_t)sl_hi << 32) | sl_lo) : (int64_t)(int32_t)sl_lo;
    const int64_t cap = (int64_t)a.width << a.block_shift;
    L = Lr < 0 ? 0 : (Lr > cap ? cap : Lr);
  }
  INT8KV_STAMP(1);
  const HeadMap hm = head_map(a, vh);
  const int G = hm.g;
  const int64_t n = tiles_of(a, L);
  if (n == 0) {  // uniform over the workgroup: every wave leaves before the barrier
    if (!SPLIT && wave == 0) write_zero_rows<QT, HD, PAD>(a, b, hm, lane);
    return;
  }
  // Loaded before the tile loop: after the barrier it would add a memory latency to every call.
  const float vscale = (CACHE == kI8 && !SPLIT) ? fmaxf(a.v_scale[hm.kv], 1e-6f) : 1.0f;
  int64_t t0 = 0, span = n;  // this workgroup's tiles of the sequence
  if constexpr (SPLIT) {
    t0 = (int64_t)blockIdx.z * n / gridDim.z;
    span = ((int64_t)blockIdx.z + 1) * n / gridDim.z - t0;
  }
  const int64_t ta = t0 + v * span / NW;
  const int64_t tb = t0 + (v + 1) * span / NW;
  if (ta < tb) {
    INT8KV_STAMP(9);
    // (Without SPLIT early_q holds whenever the share is non-empty; requested here, the query
    // still precedes the block-id loads, which is all run_segment's waits assume.)
    if (!SPLIT && !early_q)
      issue_query<QT, HD, false, PAD, CACHE != kI8>(a, b, hm, li, lg, qraw);
    run_segment<CACHE, QT, false, QQ, HD, 2, true, false, PAD, !SPLIT>(
        a, s_ids[wave], b, L, vh, ta, tb, false, 0, lane, s_acc[wave], s_m[wave], s_l[wave],
        &qraw INT8KV_STAMPS_ARG);
  } else if (li < G) {  // no tiles for this wave: the neutral state
#pragma unroll
    for (int j = 0; j < HD / 4; ++j) s_acc[wave][j * kWave + lane] = 0.0f;
    if (lg == 0) {
      s_m[wave][li] = -INFINITY;
      s_l[wave][li] = 0.0f;
    }
  }
  __syncthreads();
  INT8KV_STAMP(7);
  INT8KV_STAMPS_STORE(NW, wave, lane);
  // Online-softmax merge of the NW states (exp2 domain), as merge_kernel does for records.  The
  // four row groups rr of the accumulator layout are independent, so waves 0..3 take one each
  // (head_dim elements HD/4 lg + HD/16 rr + [0, HD/16) of lane (li, lg)): wave 0 merging all
  // of them took 2.3 us of a 9.4 us call at B = 1 x 512 tokens.
  if (wave >= 4 || li >= G) return;
  const int rr = wave;
  float M = -INFINITY, Ls = 0.0f;
  float O[HD / 16];
#pragma unroll
  for (int dt = 0; dt < HD / 16; ++dt) O[dt] = 0.0f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const float m = s_m[w][li];
    const float l = s_l[w][li];
    float A[HD / 16];
#pragma unroll
    for (int dt = 0; dt < HD / 16; ++dt) A[dt] = s_acc[w][(rr * (HD / 16) + dt) * kWave + lane];
    const float Mn = fmaxf(M, m);
    if (Mn == -INFINITY) {  // nothing finite yet: add unscaled (a NaN still reaches the output)
      Ls += l;
#pragma unroll
      for (int dt = 0; dt < HD / 16; ++dt) O[dt] += A[dt];
    } else {
      const float ca = exp2_fast(M - Mn);
      const float cb = exp2_fast(m - Mn);
      Ls = Ls * ca + l * cb;
#pragma unroll
      for (int dt = 0; dt < HD / 16; ++dt) O[dt] = O[dt] * ca + A[dt] * cb;
      M = Mn;
    }
  }
  if constexpr (SPLIT) {
    const int64_t row = ((int64_t)b * gridDim.z + blockIdx.z) * a.num_q_heads + hm.q0 + li;
    store_n<kF32, HD / 16>(reinterpret_cast<char*>(a.ws_acc + row * HD) + (HD / 4 * lg + HD / 16 * rr) * 4, O);
    if (rr == 0 && lg == 0) {
      a.ws_m[row] = M;
      a.ws_l[row] = Ls;
    }
    return;
  }
  const float inv = Ls > 0.0f ? vscale / Ls : 0.0f;
  char* op = a.out + (b * a.o_sb + (int64_t)(hm.q0 + li) * a.o_sh) * esize<QT>();
  float o[HD / 16];
#pragma unroll
  for (int dt = 0; dt < HD / 16; ++dt) o[dt] = O[dt] * inv;
  if (!PAD || HD / 4 * lg + HD / 16 * rr < a.head_dim)
    store_n<QT, HD / 16>(op + (HD / 4 * lg + HD / 16 * rr) * esize<QT>(), o);
}

// Merge of the split per-sequence layout's records: a.split = Z <= 64 records per (sequence b =
// blockIdx.x, query head h = blockIdx.y), one wave.  Every record load is issued at entry (in
// chunks of 16 records, each chunk taken only when Z reaches it, the index clamped into [0, Z)):
// lane z < Z reads record z's running max and sum and each lane HD / 64 accumulator elements of
// every record, so the call waits for one memory latency.  The wave then reduces the maxima and
// the weighted sums, and each lane combines its elements over the Z records.  A record without
// a finite maximum is weighted 1 when no record has one, so a NaN still reaches the output, as
// in merge_in.
template <int CACHE, int QT, int HD>
__global__ __launch_bounds__(64) void merge_split_kernel(DecodeArgs a) {
  constexpr int D = HD / 64;  // accumulator elements per lane
  constexpr int kChunk = 16, kChunks = 64 / kChunk;
  const int lane = threadIdx.x;
  const int64_t b = blockIdx.x;
  const int h = blockIdx.y;
  const int Z = a.split;
  char* op = a.out + (b * a.o_sb + (int64_t)h * a.o_sh + D * lane) * esize<QT>();
  float O[D];
#pragma unroll
  for (int j = 0; j < D; ++j) O[j] = 0.0f;
  float inv = 0.0f;
  if (seq_len_uniform(a, b) > 0) {  // uniform: an empty sequence left no records (zero rows)
    const float vscale = (CACHE == kI8) ? fmaxf(a.v_scale[h / a.group], 1e-6f) : 1.0f;
    const int64_t row0 = b * Z * a.num_q_heads + h;  // record z: row0 + z Hq
    const int64_t stride = (int64_t)a.num_q_heads * HD;
    const float* acc = a.ws_acc + row0 * HD + D * lane;
    float A[kChunks][kChunk][D];
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      if (c * kChunk < Z) {
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
          const int z = c * kChunk + k < Z ? c * kChunk + k : Z - 1;
#pragma unroll
          for (int j = 0; j < D; ++j) A[c][k][j] = acc[z * stride + j];
        }
      }
    }
    const int64_t rz = row0 + (int64_t)(lane < Z ? lane : 0) * a.num_q_heads;
    float m = a.ws_m[rz];
    float l = a.ws_l[rz];
    if (lane >= Z) {
      m = -INFINITY;
      l = 0.0f;
    }
    float M = m;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
    const float w = lane < Z ? (M == -INFINITY ? 1.0f : exp2_fast(m - M)) : 0.0f;
    float Lw = l * w;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) Lw += __shfl_xor(Lw, o);
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      if (c * kChunk < Z) {
#pragma unroll
        for (int k = 0; k < kChunk; ++k) {
          const float wk = __shfl(w, c * kChunk + k);
          if (c * kChunk + k < Z) {
#pragma unroll
            for (int j = 0; j < D; ++j) O[j] += wk * A[c][k][j];
          }
        }
      }
    }
    inv = Lw > 0.0f ? vscale / Lw : 0.0f;
  }
  if (D * lane >= a.head_dim) return;  // (head_dim below HD: the padded columns)
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const float v = O[j] * inv;
    if constexpr (QT == kF32)
      reinterpret_cast<float*>(op)[j] = v;
    else if constexpr (QT == kF16)
      reinterpret_cast<_Float16*>(op)[j] = (_Float16)v;
    else
      reinterpret_cast<__bf16*>(op)[j] = (__bf16)v;
  }
}

// Stores 4 consecutive fp32 values as DT (aligned to 4 elements).
template <int DT>
__device__ __forceinline__ void store4(char* p, f32x4 x) {
  if constexpr (DT == kF32) {
    *reinterpret_cast<f32x4*>(p) = x;
  } else if constexpr (DT == kF16) {
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
    f16x4 h = {(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]};
    *reinterpret_cast<f16x4*>(p) = h;
  } else {
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    bf16x4 h = {(__bf16)x[0], (__bf16)x[1], (__bf16)x[2], (__bf16)x[3]};
    *reinterpret_cast<bf16x4*>(p) = h;
  }
}

// Online-softmax merge of one more partial (m, l, acc) into a running (M, L, O).  A partial
// without a finite maximum is added unscaled, so non-finite scores (a NaN query) still reach the
// output as NaN, as they do in the reference.
__device__ __forceinline__ void merge_in(float& M, float& L, f32x4& O, float m, float l, f32x4 acc) {
  const float Mn = fmaxf(M, m);
  if (Mn == -INFINITY) {
    L += l;
    O += acc;
    return;
  }
  const float a = exp2_fast(M - Mn);
  const float c = exp2_fast(m - Mn);
  L = L * a + l * c;
  O = O * a + acc * c;
  M = Mn;
}

// Folds the partial records of query head h of a cut sequence b whose tiles lie in ranges
// r0 .. r0 + nr - 1 (range r0's slot-1 record, the later ranges' slot-0 records) and stores its
// output row; a workgroup of MW waves.  A wave's lanes are RS = 256 / HD range slots of HD / 4
// columns: lane (slot rs, column c4) of wave w owns head_dim elements [4 c4, 4 c4 + 4) of ranges
// RS w + rs, RS w + rs + RS MW, ... and folds them in with one online-softmax pass, FOLD ranges'
// loads in flight at a time (FOLD RS MW ranges per round for the workgroup); the RS MW running
// states per column are then merged through LDS.  About 1 + nr / (FOLD RS MW) dependent memory
// latencies.  Sixteen waves do not help a long sequence (one 32k-token sequence cut 256 ways: 7.2
// us with eight waves, 8.7 with 16: its workgroup streams nr x 512 bytes per query head on one
// compute unit).
template <int CACHE, int QT, int MW, int HD, int FOLD = 4>
__device__ __forceinline__ void merge_records(const DecodeArgs& a, int64_t b, int h, int64_t r0,
                                              int64_t nr) {
  constexpr int C4 = HD / 4;      // float4 columns of a head
  constexpr int RS = kWave / C4;  // range slots per wave
  __shared__ float s_m[RS * MW][C4];
  __shared__ float s_l[RS * MW][C4];
  __shared__ f32x4 s_o[RS * MW][C4];
  const int kvh = h / a.group;
  // Loaded at entry: after the barrier below it would add a memory latency to every merge.
  const float vscale = (CACHE == kI8) ? fmaxf(a.v_scale[kvh], 1e-6f) : 1.0f;
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int rs = lane / C4;  // range slot of this lane within the wave
  const int c4 = lane % C4;  // head_dim elements [4 c4, 4 c4 + 4)
  const int slot = RS * wave + rs;  // 0 .. RS MW - 1
  auto row_of = [&](int64_t c) -> int64_t {  // partial row of range r0 + c, head h
    return (2 * (r0 + c) + cut_slot(c)) * a.num_q_heads + h;  // tile 0 lies in range r0
  };

  constexpr int kStride = RS * MW;
  float M = -INFINITY, L = 0.0f;
  f32x4 O = (f32x4)(0.0f);
  for (int64_t cb = slot; cb < nr; cb += FOLD * kStride) {
    // All FOLD loads unconditionally (a slot past the last range reads the last range's record
    // again and is then ignored): a branch around each load made the compiler wait for the
    // previous ones before issuing the next, one memory latency per range instead of per round.
    float m[FOLD], l[FOLD];
    f32x4 v[FOLD];
#pragma unroll
    for (int u = 0; u < FOLD; ++u) {
      const int64_t c = cb + u * kStride;
      const int64_t row = row_of(c < nr ? c : nr - 1);
      m[u] = a.ws_m[row];
      l[u] = a.ws_l[row];
      v[u] = *reinterpret_cast<const f32x4*>(a.ws_acc + row * HD + 4 * c4);
    }
#pragma unroll
    for (int u = 0; u < FOLD; ++u) {
      const bool in = cb + u * kStride < nr;
      merge_in(M, L, O, in ? m[u] : -INFINITY, in ? l[u] : 0.0f, in ? v[u] : (f32x4)(0.0f));
    }
  }
  s_m[slot][c4] = M;
  s_l[slot][c4] = L;
  s_o[slot][c4] = O;
  __syncthreads();
  if (threadIdx.x >= C4) return;
  M = -INFINITY;
  L = 0.0f;
  O = (f32x4)(0.0f);
#pragma unroll
  for (int k = 0; k < kStride; ++k) merge_in(M, L, O, s_m[k][c4], s_l[k][c4], s_o[k][c4]);
  const float inv = L > 0.0f ? vscale / L : 0.0f;
  if (4 * c4 < a.head_dim)  // (head_dim below HD: the padded columns)
    store4<QT>(a.out + (b * a.o_sb + (int64_t)h * a.o_sh + 4 * c4) * esize<QT>(), O * inv);
}

// The merge indexed by sequence: grid (batch, num_q_heads), MW waves per query head; workgroup
// (b, h) finds b's ranges from the plan (every sequence's units before b, i.e. a scan of
// seq_lens[0 .. b]) and merges them if b is cut.  The host picks MW from the average number of
// ranges per sequence (one wave when a round covers them, up to eight for a few long sequences).
// Each wave's scan reads and sums all of the batch's lengths, so the cost grows with the batch
// (B x num_q_heads waves x B / 64 chunks): the host takes it for batches below half the range
// count, where its grid is also the smaller one.
constexpr int kMergeChunks = 8;  // 64-sequence chunks of seq_lens a merge wave requests at once

template <int CACHE, int QT, int MW, int HD, int FOLD>
__global__ __launch_bounds__(MW * 64) void merge_kernel(DecodeArgs a) {
  const int64_t b = blockIdx.x;
  const int h = blockIdx.y;
  const int lane = threadIdx.x % kWave;

  // The plan (units of the whole batch) and S, the units before sequence b.  Above 64 sequences
  // the lengths of the first kMergeChunks x 64 are requested at once instead of one 64-sequence
  // chunk after another (B = 256: merge 10.9 -> 9.6 us; B = 128: 6.5 -> 6.1 us).
  const int64_t nch = (a.batch + kWave - 1) / kWave;
  const int64_t cb = b / kWave;  // b's chunk
  const int bl = (int)(b - cb * kWave);
  int64_t U = 0, S = 0, n = 0;
  if (nch == 1) {
    const int64_t L0 = seq_len_of(a, lane);
    const int64_t u = units_of(a, tiles_of(a, L0));
    U = units_sum(a, u, lane);
    S = units_sum(a, lane < bl ? u : 0, lane);
    n = tiles_of(a, readlane64(L0, bl));
  } else {
    int64_t Lc[kMergeChunks];
    seq_len_chunks(a, 0, lane, Lc);
#pragma unroll
    for (int c = 0; c < kMergeChunks; ++c) {
      if (c >= nch) break;
      const int64_t u = units_of(a, tiles_of(a, Lc[c]));
      const int64_t chunk = units_sum(a, u, lane);
      U += chunk;
      if (c < cb) {
        S += chunk;
      } else if (c == cb) {
        S += units_sum(a, lane < bl ? u : 0, lane);
        n = tiles_of(a, readlane64(Lc[c], bl));
      }
    }
    for (int64_t c = kMergeChunks; c < nch; ++c) {  // batches above kMergeChunks x 64 sequences
      const int64_t u = units_of(a, tiles_of(a, seq_len_of(a, c * kWave + lane)));
      const int64_t chunk = units_sum(a, u, lane);
      U += chunk;
      if (c < cb) {
        S += chunk;
      } else if (c == cb) {
        S += units_sum(a, lane < bl ? u : 0, lane);
        n = tiles_of(a, seq_len_of(a, b));
      }
    }
  }
  const Plan plan = plan_of_units(a, U);
  if (n == 0) return;  // zeros written by decode_kernel
  const int64_t first = S + a.seq_cost;  // unit of tile 0
  const int64_t r0 = range_of(plan, first);
  const int64_t r1 = range_of(plan, first + n - 1);
  if (r0 == r1) return;  // finished inside one range by decode_kernel
  merge_records<CACHE, QT, MW, HD, FOLD>(a, b, h, r0, r1 - r0 + 1);
}

// The merge indexed by range: grid (max_ranges, num_q_heads), one wave per query head; workgroup
// (r0, h) merges the cut sequence that range r0 starts, named by the decode kernel's descriptor
// with the unit of its last tile, whose range under the plan is its last range r1 (ranges that
// start none return at once).  No scan of seq_lens: its
// cost does not grow with the batch (B = 256 x U[1, 2048]: 9.6 -> 5.0 us; B = 128 x U[1, 4096]:
// 6.2 -> 5.0 us), but every range costs a workgroup, which for batches below half the range
// count is the larger grid (B = 64 at 256 ranges: 4.6 -> 6.1 us).
template <int CACHE, int QT, int HD>
__global__ __launch_bounds__(64) void merge_by_range_kernel(DecodeArgs a) {
  const int64_t r0 = blockIdx.x;
  const int64_t b = a.ws_cut[4 * r0];
  const int64_t last = a.ws_cut[4 * r0 + 1];
  const Plan plan = unpack_plan(a.ws_cut[4 * r0 + 2], a.ws_cut[4 * r0 + 3]);
  // b < 0: range r0 starts no cut sequence.  The other bounds hold for every descriptor the
  // decode kernel writes (a MERGE call that does not follow MAIN on the same workspace reads
  // whatever is there; they keep it inside the buffers).  One test of all of them (no
  // short-circuit) has the kernel arguments read with the descriptor, not one dependent load
  // after another.
  const int64_t max_ranges = a.max_ranges;
  if ((b < 0) | (b >= a.batch) | (plan.U <= 0) | (plan.P <= 0) | (plan.P > max_ranges) |
      (last < 0) | (last >= plan.U) | ((int)blockIdx.y >= a.num_q_heads))
    return;
  const int64_t r1 = range_of(plan, last);
  if (r1 <= r0 || r1 >= max_ranges) return;
  merge_records<CACHE, QT, 1, HD>(a, b, (int)blockIdx.y, r0, r1 - r0 + 1);
}


// ------------------------------------------------------------------------ launchers
// kv heads per workgroup (one wave each per range it owns): the largest of 4, 3, 2, 1 dividing
// num_kv_heads.
inline int waves_per_wg(int32_t num_kv_heads) {
  for (int w = kMaxWavesPerWG; w > 1; --w)
    if (num_kv_heads % w == 0) return w;
  return 1;
}

template <int CACHE, int QT, bool NT, bool QQ, int HD, bool PAIR = false, bool PAD = false>
inline void launch_main(const DecodeArgs& a, dim3 grid, int W, hipStream_t s) {
  if constexpr (PAD) {  // head_dim below HD: one range per workgroup, two tiles (the plan's)
    hipLaunchKernelGGL((decode_kernel<CACHE, QT, NT, QQ, 1, HD, 2, false, true>), grid,
                       dim3(W * kWave), 0, s, a);
  } else {
    if constexpr (CACHE == kI8 && HD <= 128) {  // HD 256: one range per workgroup, two tiles
      if (a.halves == 2) {
        hipLaunchKernelGGL((decode_kernel<CACHE, QT, NT, QQ, 2, HD, 2, PAIR>), grid,
                           dim3(2 * W * kWave), 0, s, a);
        return;
      }
      // Four tiles in flight leave no registers for an fp32 query's lo operands: two for those.
      if (a.depth == 4 && QT != kF32) {
        hipLaunchKernelGGL((decode_kernel<CACHE, QT, NT, QQ, 1, HD, 4, PAIR>), grid,
                           dim3(W * kWave), 0, s, a);
        return;
      }
    }
    hipLaunchKernelGGL((decode_kernel<CACHE, QT, NT, QQ, 1, HD, 2, PAIR>), grid, dim3(W * kWave),
                       0, s, a);
  }
}

// The range decode kernel for one call: kv-head pairs at head_dim 64 run the HD = 128 kernel
// with PAIR (see DecodeArgs::kv_pair).
template <int CACHE, int QT, int HD, bool PAIR, bool PAD>
void launch_ranges(const DecodeArgs& a, dim3 grid, int W, bool nt, hipStream_t s) {
  constexpr int KH = PAIR ? 128 : HD;
  // INT8 caches: non-temporal loads for large pools, int8 scores for a quantised query.
  if constexpr (CACHE == kI8) {
    if (nt && a.quantize_q)
      launch_main<CACHE, QT, true, true, KH, PAIR, PAD>(a, grid, W, s);
    else if (nt)
      launch_main<CACHE, QT, true, false, KH, PAIR, PAD>(a, grid, W, s);
    else if (a.quantize_q)
      launch_main<CACHE, QT, false, true, KH, PAIR, PAD>(a, grid, W, s);
    else
      launch_main<CACHE, QT, false, false, KH, PAIR, PAD>(a, grid, W, s);
  } else {
    // 16-bit caches: non-temporal loads at head_dim 128 (plan_call decides), plain loads
    // elsewhere.
    if constexpr (HD == 128 && !PAIR && !PAD) {
      if (nt) {
        launch_main<CACHE, QT, true, false, KH, PAIR, PAD>(a, grid, W, s);
        return;
      }
    }
    launch_main<CACHE, QT, false, false, KH, PAIR, PAD>(a, grid, W, s);
  }
}

// Merge kernels a call can end with (HostPlan::merge).
enum MergeKind { kMergeNone = 0, kMergeBySequence = 1, kMergeByRange = 2, kMergeSplit = 3 };

// Everything the host decides for one call, from sizes, dtypes, flags and the CU count only
// (no device memory is read): int8kv_paged_decode launches from it and int8kv_decode_plan
// reports it.
struct HostPlan {
  int32_t num_ranges;   // range count upper bound (the workspace's records are sized by it)
  int32_t min_tiles;
  bool group_mode;      // per-sequence workgroups (split or not)
  int32_t split;        // split layout: workgroups per (sequence, kv head); 0 = not split
  bool kv_pair;
  int32_t halves;       // ranges per workgroup
  int32_t pair_min;
  int32_t depth;        // requested tiles in flight (the fp32-query INT8 kernel runs 2 of 4)
  int32_t seq_cost;
  bool scan32;
  bool cut_desc;        // range layout: the merge indexed by range (decode writes descriptors)
  bool nt;              // non-temporal INT8 K/V loads
  int32_t merge;        // MergeKind
  int32_t merge_waves;  // waves per merge workgroup
  int32_t merge_fold;   // merge by sequence: records per lane slot and round
  int32_t launch_depth; // tiles in flight of the kernel instance that runs
  int32_t hd;           // the kernels' head_dim (padded_head_dim)
  bool pad;             // the cache's head_dim is below hd
  int32_t grid_heads;   // kv heads x col_tiles
  int32_t col_tiles;    // MFMA column tiles of 16 query heads per kv head
  int64_t cus;
  size_t need;          // workspace bytes
};

// PAD: head_dim below HD (the kernels' padded instances; the plan keeps them to one range per
// workgroup with two tiles in flight and no kv-head pairs).
template <int CACHE, int QT, int HD, bool PAD>
int launch(const DecodeArgs& a, const HostPlan& hp, uint32_t flags, hipStream_t s) {
  const bool nt = hp.nt;
  const int32_t hv = a.kv_pair ? a.num_kv_heads / 2 : a.num_kv_heads;  // kv heads (pairs) per range
  const int W = waves_per_wg(a.group_mode ? a.num_kv_heads : hv);
  if (a.group_mode) {  // one kernel, plus merge_split_kernel when split
    if (flags & INT8KV_DECODE_MAIN) {
      dim3 grid((unsigned)a.batch, (unsigned)a.num_kv_heads, (unsigned)(a.split > 0 ? a.split : 1));
      const dim3 block(group_waves<HD>() * kWave);
      if (a.split > 0) {
        if (a.quantize_q)
          hipLaunchKernelGGL((group_kernel<CACHE, QT, true, HD, true, PAD>), grid, block, 0, s, a);
        else
          hipLaunchKernelGGL((group_kernel<CACHE, QT, false, HD, true, PAD>), grid, block, 0, s, a);
      } else {
        if (a.quantize_q)
          hipLaunchKernelGGL((group_kernel<CACHE, QT, true, HD, false, PAD>), grid, block, 0, s, a);
        else
          hipLaunchKernelGGL((group_kernel<CACHE, QT, false, HD, false, PAD>), grid, block, 0, s,
                             a);
      }
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return (int)e;
    }
    if (a.split > 0 && (flags & INT8KV_DECODE_MERGE)) {
      dim3 grid((unsigned)a.batch, (unsigned)a.num_q_heads);
      hipLaunchKernelGGL((merge_split_kernel<CACHE, QT, HD>), grid, dim3(kWave), 0, s, a);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return (int)e;
    }
    return INT8KV_OK;
  }
  if (flags & INT8KV_DECODE_MAIN) {
    dim3 grid((unsigned)((a.max_ranges + a.halves - 1) / a.halves), (unsigned)(hv / W));
    if constexpr (HD == 64 && !PAD) {
      if (a.kv_pair)
        launch_ranges<CACHE, QT, HD, true, false>(a, grid, W, nt, s);
      else
        launch_ranges<CACHE, QT, HD, false, false>(a, grid, W, nt, s);
    } else {
      launch_ranges<CACHE, QT, HD, false, PAD>(a, grid, W, nt, s);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  if (flags & INT8KV_DECODE_MERGE) {
    if (hp.merge == kMergeByRange) {  // the smaller grid, and no scan of seq_lens
      dim3 grid((unsigned)a.max_ranges, (unsigned)a.num_q_heads);
      hipLaunchKernelGGL((merge_by_range_kernel<CACHE, QT, HD>), grid, dim3(kWave), 0, s, a);
    } else {
      dim3 grid((unsigned)a.batch, (unsigned)a.num_q_heads);
      switch (hp.merge_waves * 16 + hp.merge_fold) {
        case 1 * 16 + 4:
          hipLaunchKernelGGL((merge_kernel<CACHE, QT, 1, HD, 4>), grid, dim3(kWave), 0, s, a);
          break;
        case 2 * 16 + 4:
          hipLaunchKernelGGL((merge_kernel<CACHE, QT, 2, HD, 4>), grid, dim3(2 * kWave), 0, s, a);
          break;
        case 4 * 16 + 4:
          hipLaunchKernelGGL((merge_kernel<CACHE, QT, 4, HD, 4>), grid, dim3(4 * kWave), 0, s, a);
          break;
        case 4 * 16 + 8:
          hipLaunchKernelGGL((merge_kernel<CACHE, QT, 4, HD, 8>), grid, dim3(4 * kWave), 0, s, a);
          break;
        default:
          hipLaunchKernelGGL((merge_kernel<CACHE, QT, 8, HD, 8>), grid, dim3(8 * kWave), 0, s, a);
          break;
      }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  return INT8KV_OK;
}

// The kernels' head_dim (HD) for a cache head_dim: the power of two 64, 128 or 256 at or above
// it; below it the padded instances run (elements at or past head_dim are never loaded into
// products that reach an output, nor stored).
inline int padded_head_dim(int head_dim) { return head_dim <= 64 ? 64 : head_dim <= 128 ? 128 : 256; }

template <int CACHE, bool PAD>
int launch_q(const DecodeArgs& a, const HostPlan& hp, int query_dtype, uint32_t flags,
             hipStream_t s) {
  const int hd = padded_head_dim(a.head_dim);
  switch (query_dtype) {
    case INT8KV_F32:
      return hd == 64    ? launch<CACHE, kF32, 64, PAD>(a, hp, flags, s)
             : hd == 128 ? launch<CACHE, kF32, 128, PAD>(a, hp, flags, s)
                         : launch<CACHE, kF32, 256, PAD>(a, hp, flags, s);
    case INT8KV_F16:
      return hd == 64    ? launch<CACHE, kF16, 64, PAD>(a, hp, flags, s)
             : hd == 128 ? launch<CACHE, kF16, 128, PAD>(a, hp, flags, s)
                         : launch<CACHE, kF16, 256, PAD>(a, hp, flags, s);
    default:
      return hd == 64    ? launch<CACHE, kBF16, 64, PAD>(a, hp, flags, s)
             : hd == 128 ? launch<CACHE, kBF16, 128, PAD>(a, hp, flags, s)
                         : launch<CACHE, kBF16, 256, PAD>(a, hp, flags, s);
  }
}


// One cache type's launcher (defined in paged_decode_<type>.hip), and the one for head_dims
// below the kernels' HD (paged_decode_<type>_pad.hip).
int launch_cache_int8(const DecodeArgs& a, const HostPlan& hp, int query_dtype, uint32_t flags,
                      hipStream_t s);
int launch_cache_bf16(const DecodeArgs& a, const HostPlan& hp, int query_dtype, uint32_t flags,
                      hipStream_t s);
int launch_cache_fp16(const DecodeArgs& a, const HostPlan& hp, int query_dtype, uint32_t flags,
                      hipStream_t s);
int launch_cache_int8_pad(const DecodeArgs& a, const HostPlan& hp, int query_dtype,
                          uint32_t flags, hipStream_t s);
int launch_cache_bf16_pad(const DecodeArgs& a, const HostPlan& hp, int query_dtype,
                          uint32_t flags, hipStream_t s);
int launch_cache_fp16_pad(const DecodeArgs& a, const HostPlan& hp, int query_dtype,
                          uint32_t flags, hipStream_t s);

}  // namespace int8kv

#endif  // INT8KV_PAGED_DECODE_KERNELS_H
