// Static per-head INT8 KV-cache write for gfx950.
//
// Replaces the Triton kernel src/triton_ops/int8_cache_write.py:6-82 and its wrapper :85-149.
// Numerics follow the reference's own oracle (src/quant.py:37-40 and the torch reference
// src/triton_ops/int8_cache_write.py:172-181): an IEEE fp32 quotient x / scale, rounded half to
// even (torch.round), clamped to [-127, 127].  The Triton kernel itself rounds half away from
// zero (:59-63); this kernel deliberately does not.  The scale is clamped to >= 1e-6 as the
// Triton kernel does (:50-51); calibrated scales already satisfy that (scripts/04 :55-65).
//
// Mapping (wide kernels, head_dim % 16 == 0 and 16-byte aligned cache rows): grid.y = kv head,
// one lane owns 16 consecutive head_dim elements of one (token, head) row of both K and V --
// 32-byte source loads, 16-byte cache stores, 8 lanes per 128-element row.  The slot is read
// first, so skipped rows cost no source bytes.  Sources are read and caches written with the
// non-temporal hint: both are streamed once (262k-token write on MI355X: 193 -> 166 us, 4.2 ->
// 4.9 TB/s).  Other layouts (head_dim % 16 == 8, or cache rows only 8-byte aligned) use the
// narrow kernels: one lane per 8 elements, 8-byte stores.
//
// Token-major map (the *_tm kernels): when a token's Hkv * head_dim / 16 lanes are a power of two
// that fits one wave, a token's kv heads sit in adjacent lanes of one wave, so one token's slot
// row (Hkv * head_dim contiguous bytes in a [blocks, block_size, Hkv, D] cache) is written by
// consecutive lanes, and the dynamic write gathers four heads' scales into one 16-byte store
// instead of four lone 4-byte stores (which cost a 32-byte write sector each: +23 % written
// bytes at 262,144 tokens).  The dynamic write always uses it; the static write only when its
// bytes exceed the Infinity Cache (static_token_major()).
//
// The quotient x / scale is not divided per element: quantise() (int8kv_common.h) multiplies by
// the correctly rounded reciprocal and divides only the elements whose quotient lies within
// 2^-20 relative of a half-integer, which provably gives the divide's codes (the divide is ~10
// VALU instructions per element and made the write VALU-bound: 262,144 tokens 158 -> 155.6 us
// static, 197 -> 175.6 us dynamic; 16,384 tokens 14.6 -> 12.1 us).

#include "int8kv_common.h"

namespace int8kv {

struct WriteArgs {
  const char* key;
  const char* value;
  int8_t* kc;
  int8_t* vc;
  const void* slots;
  const float* k_scale;
  const float* v_scale;
  int64_t k_st, k_sh;  // element strides of key (token, head)
  int64_t v_st, v_sh;
  int64_t kc_sb, kc_ss, kc_sh;  // element (= byte) strides of the int8 caches
  int64_t vc_sb, vc_ss, vc_sh;
  int64_t num_tokens;
  int64_t capacity;  // num_blocks * block_size
  int32_t num_kv_heads;
  int32_t vecs_per_row;  // head_dim / 8
  int32_t block_size;
  int32_t block_shift;  // log2(block_size) for a power of two, else -1
  int32_t slots_is64;
};

// A slot's block and row in it: a shift and a mask for a power-of-two block size (every paged
// cache in practice), a division otherwise (a 64-bit division is ~100 instructions per lane).
__device__ __forceinline__ void slot_block(const WriteArgs& a, int64_t slot, int64_t& blk,
                                           int64_t& off) {
  if (a.block_shift >= 0) {
    blk = slot >> a.block_shift;
    off = slot & ((1LL << a.block_shift) - 1);
  } else {
    blk = slot / a.block_size;
    off = slot - blk * a.block_size;
  }
}

// gid / n for a wave-uniform n >= 1: a shift when n is a power of two (head_dim / 16 lanes per
// row at head_dim 64, 128, 256), a division otherwise.
__device__ __forceinline__ uint32_t div_uniform(uint32_t gid, uint32_t n) {
  return (n & (n - 1)) == 0 ? gid >> __builtin_ctz(n) : gid / n;
}

template <int SRC>
__global__ __launch_bounds__(256) void cache_write_kernel(WriteArgs a) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t rows = a.num_tokens * a.num_kv_heads;
  const int64_t row = gid / a.vecs_per_row;
  if (row >= rows) return;
  const int dv = (int)(gid - row * a.vecs_per_row);
  const int h = (int)(row % a.num_kv_heads);
  const int64_t t = row / a.num_kv_heads;

  const int64_t slot = load_index(a.slots, t, a.slots_is64);
  if (slot < 0 || slot >= a.capacity) return;
  int64_t blk, off;
  slot_block(a, slot, blk, off);

  constexpr int esize = SRC == kF32 ? 4 : 2;
  const QuantScale ks = quant_scale(fmaxf(a.k_scale[h], 1e-6f));
  const QuantScale vs = quant_scale(fmaxf(a.v_scale[h], 1e-6f));

  float x[8];
  uint32_t w[2];
  load8_f32<SRC>(a.key + (t * a.k_st + h * a.k_sh + 8 * dv) * esize, x);
  quantise<8, false>(x, ks, w);
  const u32x2 kq = {w[0], w[1]};
  load8_f32<SRC>(a.value + (t * a.v_st + h * a.v_sh + 8 * dv) * esize, x);
  quantise<8, false>(x, vs, w);
  const u32x2 vq = {w[0], w[1]};

  *reinterpret_cast<u32x2*>(a.kc + blk * a.kc_sb + off * a.kc_ss + h * a.kc_sh + 8 * dv) = kq;
  *reinterpret_cast<u32x2*>(a.vc + blk * a.vc_sb + off * a.vc_ss + h * a.vc_sh + 8 * dv) = vq;
}


// ------------------------------------------------------------------ wide kernels (16 per lane)
template <bool NT>
__device__ __forceinline__ u32x4 ld16(const char* p) {
  if constexpr (NT)
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  else
    return *reinterpret_cast<const u32x4*>(p);
}

// 16 consecutive elements of type DT at p (16-byte aligned), widened to fp32, non-temporal.
template <int DT>
__device__ __forceinline__ void load16_f32(const char* p, float (&x)[16]) {
  if constexpr (DT == kF32) {
    // Typed f32x4 loads: element reads of a bit-cast u32x4 were miscompiled here (repeated
    // elements), as in the decode kernel's fp32 query path.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 w = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + 16 * j));
      x[4 * j + 0] = w[0];
      x[4 * j + 1] = w[1];
      x[4 * j + 2] = w[2];
      x[4 * j + 3] = w[3];
    }
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const u32x4 w = ld16<true>(p + 16 * j);
#pragma unroll
      for (int i = 0; i < 4; ++i) unpack2<DT>(w[i], x[8 * j + 2 * i], x[8 * j + 2 * i + 1]);
    }
  }
}

__device__ __forceinline__ void store16_nt(int8_t* p, const u32x4& v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// grid (ceil(num_tokens * vecs_per_row / 256), num_kv_heads); vecs_per_row = head_dim / 16.
template <int SRC>
__global__ __launch_bounds__(256) void cache_write16_kernel(WriteArgs a) {
  const int h = blockIdx.y;
  const uint32_t lpr = (uint32_t)a.vecs_per_row;
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  const uint32_t t = div_uniform(gid, lpr);
  if ((int64_t)t >= a.num_tokens) return;
  const int dv = (int)(gid - t * lpr);
  constexpr int esize = SRC == kF32 ? 4 : 2;
  // The slot and the row's source bytes are requested together (a skipped row, slot < 0 or past
  // the cache, then stores nothing): with every wave of a small write resident at once (config 1:
  // 16,384 tokens, 8,192 waves), a slot-first order put a second dependent memory latency on
  // each wave's path.
  const int64_t slot = load_index(a.slots, t, a.slots_is64);
  float x[16], y[16];
  load16_f32<SRC>(a.key + ((int64_t)t * a.k_st + h * a.k_sh + 16 * dv) * esize, x);
  load16_f32<SRC>(a.value + ((int64_t)t * a.v_st + h * a.v_sh + 16 * dv) * esize, y);
  if (slot < 0 || slot >= a.capacity) return;
  const QuantScale ks = quant_scale(fmaxf(a.k_scale[h], 1e-6f));
  const QuantScale vs = quant_scale(fmaxf(a.v_scale[h], 1e-6f));
  int64_t blk, off;
  slot_block(a, slot, blk, off);
  uint32_t wk[4], wv[4];
  quantise<16, false>(x, ks, wk);
  quantise<16, false>(y, vs, wv);
  const u32x4 kq = {wk[0], wk[1], wk[2], wk[3]};
  const u32x4 vq = {wv[0], wv[1], wv[2], wv[3]};
  store16_nt(a.kc + blk * a.kc_sb + off * a.kc_ss + h * a.kc_sh + 16 * dv, kq);
  store16_nt(a.vc + blk * a.vc_sb + off * a.vc_ss + h * a.vc_sh + 16 * dv, vq);
}

// ---------------------------------------------------------------------------------------------
// Dynamic per-(token, head) INT8 write (replaces the Triton kernel
// vllm_int8/vllm_int8_cache_ops.py:13-131): scale = max(absmax(x[t, h, :]) / 127, 1e-6),
// q = clamp(x / scale, -127, 127) rounded half away from zero, codes and the fp32 scale stored at
// the slot.  Same lane mapping as the static write: vecs_per_row lanes (a power of two) own one
// (token, head) row of K and V, 8 elements each; the row absmax is a butterfly over those lanes.
struct DynWriteArgs {
  WriteArgs w;
  float* ksc;
  float* vsc;
  int64_t ksc_sb, ksc_ss, ksc_sh;  // element strides of the [NB, BS, Hkv] scale caches
  int64_t vsc_sb, vsc_ss, vsc_sh;
  int32_t vec_scales;  // a slot's kv-head scales are 4-aligned contiguous runs: 16-byte stores
};

__device__ __forceinline__ float row_absmax(const float* x, int lanes_per_row) {
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(x[i]));
  for (int o = 1; o < lanes_per_row; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
  return m;
}

template <int SRC>
__global__ __launch_bounds__(256) void dynamic_write_kernel(DynWriteArgs d) {
  const WriteArgs& a = d.w;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t rows = a.num_tokens * a.num_kv_heads;
  const int64_t row = gid / a.vecs_per_row;
  // Whole rows share a wave (vecs_per_row divides 64), so a row's lanes agree on every branch
  // below and the butterfly only mixes lanes of one row.
  const bool in_range = row < rows;
  const int dv = (int)(gid - row * a.vecs_per_row);
  const int h = in_range ? (int)(row % a.num_kv_heads) : 0;
  const int64_t t = in_range ? row / a.num_kv_heads : 0;
  constexpr int esize = SRC == kF32 ? 4 : 2;

  float x[8], y[8];
  if (in_range) {
    load8_f32<SRC>(a.key + (t * a.k_st + h * a.k_sh + 8 * dv) * esize, x);
    load8_f32<SRC>(a.value + (t * a.v_st + h * a.v_sh + 8 * dv) * esize, y);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = y[i] = 0.0f;
  }
  const float ks = fmaxf(row_absmax(x, a.vecs_per_row) / 127.0f, 1e-6f);
  const float vs = fmaxf(row_absmax(y, a.vecs_per_row) / 127.0f, 1e-6f);
  if (!in_range) return;
  const int64_t slot = load_index(a.slots, t, a.slots_is64);
  if (slot < 0 || slot >= a.capacity) return;
  int64_t blk, off;
  slot_block(a, slot, blk, off);
  uint32_t wk[2], wv[2];
  quantise<8, true>(x, quant_scale(ks), wk);
  quantise<8, true>(y, quant_scale(vs), wv);
  const u32x2 kq = {wk[0], wk[1]};
  const u32x2 vq = {wv[0], wv[1]};
  *reinterpret_cast<u32x2*>(a.kc + blk * a.kc_sb + off * a.kc_ss + h * a.kc_sh + 8 * dv) = kq;
  *reinterpret_cast<u32x2*>(a.vc + blk * a.vc_sb + off * a.vc_ss + h * a.vc_sh + 8 * dv) = vq;
  if (dv == 0) {
    d.ksc[blk * d.ksc_sb + off * d.ksc_ss + h * d.ksc_sh] = ks;
    d.vsc[blk * d.vsc_sb + off * d.vsc_ss + h * d.vsc_sh] = vs;
  }
}


// Wide dynamic write: grid (ceil(num_tokens * vecs_per_row / 256), num_kv_heads), 16 elements
// per lane; vecs_per_row = head_dim / 16 is a power of two <= 64, so a row's lanes sit in one
// wave and the absmax butterfly stays inside the row.
template <int SRC>
__global__ __launch_bounds__(256) void dynamic_write16_kernel(DynWriteArgs d) {
  const WriteArgs& a = d.w;
  const int h = blockIdx.y;
  const uint32_t lpr = (uint32_t)a.vecs_per_row;
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  const uint32_t t = div_uniform(gid, lpr);
  const bool in_range = (int64_t)t < a.num_tokens;
  const int dv = (int)(gid - t * lpr);
  constexpr int esize = SRC == kF32 ? 4 : 2;
  float x[16], y[16];
  int64_t slot = -1;
  if (in_range) {
    slot = load_index(a.slots, t, a.slots_is64);
    load16_f32<SRC>(a.key + ((int64_t)t * a.k_st + h * a.k_sh + 16 * dv) * esize, x);
    load16_f32<SRC>(a.value + ((int64_t)t * a.v_st + h * a.v_sh + 16 * dv) * esize, y);
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = y[i] = 0.0f;
  }
  float km = 0.0f, vm = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    km = fmaxf(km, fabsf(x[i]));
    vm = fmaxf(vm, fabsf(y[i]));
  }
  for (uint32_t o = 1; o < lpr; o <<= 1) {
    km = fmaxf(km, __shfl_xor(km, (int)o));
    vm = fmaxf(vm, __shfl_xor(vm, (int)o));
  }
  const float ks = fmaxf(km / 127.0f, 1e-6f);
  const float vs = fmaxf(vm / 127.0f, 1e-6f);
  if (!in_range || slot < 0 || slot >= a.capacity) return;
  int64_t blk, off;
  slot_block(a, slot, blk, off);
  uint32_t wk[4], wv[4];
  quantise<16, true>(x, quant_scale(ks), wk);
  quantise<16, true>(y, quant_scale(vs), wv);
  const u32x4 kq = {wk[0], wk[1], wk[2], wk[3]};
  const u32x4 vq = {wv[0], wv[1], wv[2], wv[3]};
  store16_nt(a.kc + blk * a.kc_sb + off * a.kc_ss + h * a.kc_sh + 16 * dv, kq);
  store16_nt(a.vc + blk * a.vc_sb + off * a.vc_ss + h * a.vc_sh + 16 * dv, vq);
  if (dv == 0) {
    d.ksc[blk * d.ksc_sb + off * d.ksc_ss + h * d.ksc_sh] = ks;
    d.vsc[blk * d.vsc_sb + off * d.vsc_ss + h * d.vsc_sh] = vs;
  }
}

// ------------------------------------------------------------------ token-major wide kernels
// All kv heads of a token in adjacent lanes: lanes_per_token = Hkv * head_dim / 16 (a power of two
// dividing 64), head h in lanes [h * lpr, (h + 1) * lpr).  A token's K (and V) row is then read as
// one contiguous piece and its codes are written as one contiguous slot row (512 B for 4 x 128),
// and the dynamic write's per-head scales of a slot leave in 16-byte stores instead of one 4-byte
// store per (token, head) from different workgroups (which the write-sector granularity turned
// into 8x the bytes).  Grid: ceil(num_tokens * lanes_per_token / 256), 1-D.
struct TokenLane {
  uint32_t t;  // token
  int h;       // kv head
  int dv;      // 16-element piece of the head's row
};

__device__ __forceinline__ TokenLane token_lane(const WriteArgs& a, int lpr_shift, int lpt_shift) {
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  const uint32_t w = gid & ((1u << lpt_shift) - 1u);
  return {gid >> lpt_shift, (int)(w >> lpr_shift), (int)(w & ((1u << lpr_shift) - 1u))};
}

template <int SRC>
__global__ __launch_bounds__(256) void cache_write16_tm_kernel(WriteArgs a, int lpr_shift,
                                                               int lpt_shift) {
  const TokenLane L = token_lane(a, lpr_shift, lpt_shift);
  if ((int64_t)L.t >= a.num_tokens) return;
  const int64_t slot = load_index(a.slots, L.t, a.slots_is64);
  if (slot < 0 || slot >= a.capacity) return;  // skipped rows load nothing
  constexpr int esize = SRC == kF32 ? 4 : 2;
  float x[16], y[16];
  load16_f32<SRC>(a.key + ((int64_t)L.t * a.k_st + L.h * a.k_sh + 16 * L.dv) * esize, x);
  load16_f32<SRC>(a.value + ((int64_t)L.t * a.v_st + L.h * a.v_sh + 16 * L.dv) * esize, y);
  int64_t blk, off;
  slot_block(a, slot, blk, off);
  uint32_t wk[4], wv[4];
  quantise<16, false>(x, quant_scale(fmaxf(a.k_scale[L.h], 1e-6f)), wk);
  quantise<16, false>(y, quant_scale(fmaxf(a.v_scale[L.h], 1e-6f)), wv);
  store16_nt(a.kc + blk * a.kc_sb + off * a.kc_ss + L.h * a.kc_sh + 16 * L.dv,
             u32x4{wk[0], wk[1], wk[2], wk[3]});
  store16_nt(a.vc + blk * a.vc_sb + off * a.vc_ss + L.h * a.vc_sh + 16 * L.dv,
             u32x4{wv[0], wv[1], wv[2], wv[3]});
}

template <int SRC>
__global__ __launch_bounds__(256) void dynamic_write16_tm_kernel(DynWriteArgs d, int lpr_shift,
                                                                 int lpt_shift) {
  const WriteArgs& a = d.w;
  const TokenLane L = token_lane(a, lpr_shift, lpt_shift);
  // Whole tokens leave together, so every exchange below stays among one token's active lanes.
  if ((int64_t)L.t >= a.num_tokens) return;
  const int64_t slot = load_index(a.slots, L.t, a.slots_is64);
  if (slot < 0 || slot >= a.capacity) return;
  constexpr int esize = SRC == kF32 ? 4 : 2;
  float x[16], y[16];
  load16_f32<SRC>(a.key + ((int64_t)L.t * a.k_st + L.h * a.k_sh + 16 * L.dv) * esize, x);
  load16_f32<SRC>(a.value + ((int64_t)L.t * a.v_st + L.h * a.v_sh + 16 * L.dv) * esize, y);
  float km = 0.0f, vm = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    km = fmaxf(km, fabsf(x[i]));
    vm = fmaxf(vm, fabsf(y[i]));
  }
  const int lpr = 1 << lpr_shift;
  for (int o = 1; o < lpr; o <<= 1) {
    km = fmaxf(km, __shfl_xor(km, o));
    vm = fmaxf(vm, __shfl_xor(vm, o));
  }
  const float ks = fmaxf(km / 127.0f, 1e-6f);
  const float vs = fmaxf(vm / 127.0f, 1e-6f);
  int64_t blk, off;
  slot_block(a, slot, blk, off);
  uint32_t wk[4], wv[4];
  quantise<16, true>(x, quant_scale(ks), wk);
  quantise<16, true>(y, quant_scale(vs), wv);
  store16_nt(a.kc + blk * a.kc_sb + off * a.kc_ss + L.h * a.kc_sh + 16 * L.dv,
             u32x4{wk[0], wk[1], wk[2], wk[3]});
  store16_nt(a.vc + blk * a.vc_sb + off * a.vc_ss + L.h * a.vc_sh + 16 * L.dv,
             u32x4{wv[0], wv[1], wv[2], wv[3]});
  if (d.vec_scales) {
    // Lane (h, dv = 0) of a head h % 4 == 0 stores heads h .. h + 3; every lane of the token takes
    // part in the exchange (the reads stay inside the token's lanes).
    const int lane = threadIdx.x % kWave;
    f32x4 k4, v4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      k4[j] = __shfl(ks, lane + j * lpr);
      v4[j] = __shfl(vs, lane + j * lpr);
    }
    if (L.dv == 0 && (L.h & 3) == 0) {
      *reinterpret_cast<f32x4*>(d.ksc + blk * d.ksc_sb + off * d.ksc_ss + L.h) = k4;
      *reinterpret_cast<f32x4*>(d.vsc + blk * d.vsc_sb + off * d.vsc_ss + L.h) = v4;
    }
  } else if (L.dv == 0) {
    d.ksc[blk * d.ksc_sb + off * d.ksc_ss + L.h * d.ksc_sh] = ks;
    d.vsc[blk * d.vsc_sb + off * d.vsc_ss + L.h * d.vsc_sh] = vs;
  }
}

}  // namespace int8kv

using namespace int8kv;

static bool aligned(const void* p, int64_t stride_bytes, int64_t align) {
  return ((uintptr_t)p % align) == 0 && (stride_bytes % align) == 0;
}

namespace {

// The wide kernels need head_dim % 16 == 0, 16-byte aligned cache rows and a 32-bit lane index.
bool wide_ok(const void* key_cache, const void* value_cache, const int64_t kcs[4],
             const int64_t vcs[4], int64_t num_tokens, int32_t num_kv_heads, int32_t head_dim) {
  if (head_dim % 16 != 0 || num_kv_heads > 65535) return false;
  for (int i = 0; i < 3; ++i)
    if (!aligned(key_cache, kcs[i], 16) || !aligned(value_cache, vcs[i], 16)) return false;
  return num_tokens * (int64_t)(head_dim / 16) <= 0x7fffffffLL;
}

// log2(lanes per token) of the token-major kernels, or -1 when a token's lanes do not fit one wave
// as a power of two (kv heads not a power of two, or more than 64 lanes) or a lane index would
// overflow 32 bits.
int token_major_shift(int64_t num_tokens, int32_t num_kv_heads, int32_t vecs_per_row) {
  const int64_t lpt = (int64_t)num_kv_heads * vecs_per_row;
  if ((num_kv_heads & (num_kv_heads - 1)) != 0 || (vecs_per_row & (vecs_per_row - 1)) != 0 ||
      lpt > kWave || num_tokens * lpt > 0x7fffffffLL)
    return -1;
  return __builtin_ctzll((unsigned long long)lpt);
}

// The static write takes the token-major map only when it streams from HBM: its bytes exceed the
// 256 MB Infinity Cache.  MI355X, 262,144 tokens (805 MB): 153.3-153.6 vs 157.2 us; 16,896 rows
// (50 MB, cache-resident): 13.1-13.2 vs 12.2 us.  The dynamic write always takes it (its scale
// stores: 158-159 vs 175.7 us at 262,144 tokens, 13.7-14.0 vs 14.2-14.5 us at 16,896 rows).
constexpr double kInfinityCacheBytes = 256.0 * 1024 * 1024;

bool static_token_major(int64_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                        int64_t src_esize) {
  return (double)num_tokens * num_kv_heads * head_dim * (2.0 * src_esize + 2.0) > kInfinityCacheBytes;
}

// Validates the arguments shared by the static and the dynamic write and fills WriteArgs.
int prepare_write(WriteArgs& a, const void* key, const void* value, int src_dtype,
                  int64_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                  const int64_t key_strides[3], const int64_t value_strides[3], void* key_cache,
                  void* value_cache, int64_t num_blocks, int32_t block_size,
                  const int64_t key_cache_strides[4], const int64_t value_cache_strides[4],
                  const void* slot_mapping, int slot_dtype) {
  if (!key_strides || !value_strides || !key_cache_strides || !value_cache_strides)
    return INT8KV_E_NULL;
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || head_dim % 8 != 0 ||
      num_blocks < 0 || block_size <= 0)
    return INT8KV_E_SHAPE;
  if (src_dtype != INT8KV_F32 && src_dtype != INT8KV_F16 && src_dtype != INT8KV_BF16)
    return INT8KV_E_DTYPE;
  if (slot_dtype != INT8KV_I32 && slot_dtype != INT8KV_I64) return INT8KV_E_DTYPE;
  if (num_tokens == 0) return INT8KV_OK;
  if (!key || !value || !key_cache || !value_cache || !slot_mapping) return INT8KV_E_NULL;

  // Each lane loads 8 source elements with 16-byte vector loads.
  const int64_t esize = src_dtype == INT8KV_F32 ? 4 : 2;
  if (key_strides[2] != 1 || value_strides[2] != 1 || key_cache_strides[3] != 1 ||
      value_cache_strides[3] != 1)
    return INT8KV_E_STRIDE;
  if (!aligned(key, key_strides[0] * esize, 16) || !aligned(key, key_strides[1] * esize, 16) ||
      !aligned(value, value_strides[0] * esize, 16) ||
      !aligned(value, value_strides[1] * esize, 16))
    return INT8KV_E_STRIDE;
  for (int i = 0; i < 3; ++i) {
    if (!aligned(key_cache, key_cache_strides[i], 8) ||
        !aligned(value_cache, value_cache_strides[i], 8))
      return INT8KV_E_STRIDE;
  }
  a.key = static_cast<const char*>(key);
  a.value = static_cast<const char*>(value);
  a.kc = static_cast<int8_t*>(key_cache);
  a.vc = static_cast<int8_t*>(value_cache);
  a.slots = slot_mapping;
  a.k_scale = nullptr;
  a.v_scale = nullptr;
  a.k_st = key_strides[0];
  a.k_sh = key_strides[1];
  a.v_st = value_strides[0];
  a.v_sh = value_strides[1];
  a.kc_sb = key_cache_strides[0];
  a.kc_ss = key_cache_strides[1];
  a.kc_sh = key_cache_strides[2];
  a.vc_sb = value_cache_strides[0];
  a.vc_ss = value_cache_strides[1];
  a.vc_sh = value_cache_strides[2];
  a.num_tokens = num_tokens;
  a.capacity = num_blocks * (int64_t)block_size;
  a.num_kv_heads = num_kv_heads;
  a.vecs_per_row = head_dim / 8;
  a.block_size = block_size;
  a.block_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  a.slots_is64 = slot_dtype == INT8KV_I64;
  return 1;  // launch needed
}

}  // namespace

extern "C" int int8kv_cache_write(const void* key, const void* value, int src_dtype,
                                  int64_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                                  const int64_t key_strides[3], const int64_t value_strides[3],
                                  void* key_cache, void* value_cache, int64_t num_blocks,
                                  int32_t block_size, const int64_t key_cache_strides[4],
                                  const int64_t value_cache_strides[4], const void* slot_mapping,
                                  int slot_dtype, const float* k_scale, const float* v_scale,
                                  void* stream) {
  WriteArgs a;
  const int st = prepare_write(a, key, value, src_dtype, num_tokens, num_kv_heads, head_dim,
                               key_strides, value_strides, key_cache, value_cache, num_blocks,
                               block_size, key_cache_strides, value_cache_strides, slot_mapping,
                               slot_dtype);
  if (st <= 0) return st;
  if (!k_scale || !v_scale) return INT8KV_E_NULL;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  hipStream_t s = static_cast<hipStream_t>(stream);

  if (wide_ok(key_cache, value_cache, key_cache_strides, value_cache_strides, num_tokens,
              num_kv_heads, head_dim)) {
    a.vecs_per_row = head_dim / 16;
    const int lpt_shift = token_major_shift(num_tokens, num_kv_heads, a.vecs_per_row);
    const int64_t src_esize = src_dtype == INT8KV_F32 ? 4 : 2;
    if (lpt_shift >= 0 && static_token_major(num_tokens, num_kv_heads, head_dim, src_esize)) {
      const int lpr_shift = __builtin_ctz((unsigned)a.vecs_per_row);
      const dim3 grid((unsigned)(((num_tokens << lpt_shift) + 255) / 256));
      switch (src_dtype) {
        case INT8KV_F32:
          hipLaunchKernelGGL(cache_write16_tm_kernel<kF32>, grid, dim3(256), 0, s, a, lpr_shift, lpt_shift);
          break;
        case INT8KV_F16:
          hipLaunchKernelGGL(cache_write16_tm_kernel<kF16>, grid, dim3(256), 0, s, a, lpr_shift, lpt_shift);
          break;
        default:
          hipLaunchKernelGGL(cache_write16_tm_kernel<kBF16>, grid, dim3(256), 0, s, a, lpr_shift, lpt_shift);
          break;
      }
      return (int)hipGetLastError();
    }
    const int64_t blocks16 = (num_tokens * a.vecs_per_row + 255) / 256;
    const dim3 grid((unsigned)blocks16, (unsigned)num_kv_heads);
    switch (src_dtype) {
      case INT8KV_F32:
        hipLaunchKernelGGL(cache_write16_kernel<kF32>, grid, dim3(256), 0, s, a);
        break;
      case INT8KV_F16:
        hipLaunchKernelGGL(cache_write16_kernel<kF16>, grid, dim3(256), 0, s, a);
        break;
      default:
        hipLaunchKernelGGL(cache_write16_kernel<kBF16>, grid, dim3(256), 0, s, a);
        break;
    }
    return (int)hipGetLastError();
  }

  const int64_t lanes = num_tokens * num_kv_heads * (int64_t)a.vecs_per_row;
  const int threads = 256;
  const int64_t blocks = (lanes + threads - 1) / threads;
  if (blocks > 0x7fffffffLL) return INT8KV_E_SHAPE;
  switch (src_dtype) {
    case INT8KV_F32:
      hipLaunchKernelGGL(cache_write_kernel<kF32>, dim3((unsigned)blocks), dim3(threads), 0, s, a);
      break;
    case INT8KV_F16:
      hipLaunchKernelGGL(cache_write_kernel<kF16>, dim3((unsigned)blocks), dim3(threads), 0, s, a);
      break;
    default:
      hipLaunchKernelGGL(cache_write_kernel<kBF16>, dim3((unsigned)blocks), dim3(threads), 0, s, a);
      break;
  }
  return (int)hipGetLastError();
}

extern "C" int int8kv_dynamic_cache_write(
    const void* key, const void* value, int src_dtype, int64_t num_tokens, int32_t num_kv_heads,
    int32_t head_dim, const int64_t key_strides[3], const int64_t value_strides[3],
    void* key_cache, void* value_cache, int64_t num_blocks, int32_t block_size,
    const int64_t key_cache_strides[4], const int64_t value_cache_strides[4],
    float* k_scale_cache, float* v_scale_cache, const int64_t k_scale_cache_strides[3],
    const int64_t v_scale_cache_strides[3], const void* slot_mapping, int slot_dtype,
    void* stream) {
  if (!k_scale_cache_strides || !v_scale_cache_strides) return INT8KV_E_NULL;
  const int32_t vpr = head_dim / 8;
  if (head_dim <= 0 || head_dim % 8 != 0 || vpr > kWave || (vpr & (vpr - 1)) != 0)
    return INT8KV_E_SHAPE;  // a row's lanes must form a power-of-two group inside one wave
  DynWriteArgs d;
  d.vec_scales = 0;
  const int st = prepare_write(d.w, key, value, src_dtype, num_tokens, num_kv_heads, head_dim,
                               key_strides, value_strides, key_cache, value_cache, num_blocks,
                               block_size, key_cache_strides, value_cache_strides, slot_mapping,
                               slot_dtype);
  if (st <= 0) return st;
  if (!k_scale_cache || !v_scale_cache) return INT8KV_E_NULL;
  if (((uintptr_t)k_scale_cache % 4) || ((uintptr_t)v_scale_cache % 4)) return INT8KV_E_STRIDE;
  d.ksc = k_scale_cache;
  d.vsc = v_scale_cache;
  d.ksc_sb = k_scale_cache_strides[0];
  d.ksc_ss = k_scale_cache_strides[1];
  d.ksc_sh = k_scale_cache_strides[2];
  d.vsc_sb = v_scale_cache_strides[0];
  d.vsc_ss = v_scale_cache_strides[1];
  d.vsc_sh = v_scale_cache_strides[2];
  hipStream_t s = static_cast<hipStream_t>(stream);

  const int32_t vpr16 = head_dim / 16;
  if (wide_ok(key_cache, value_cache, key_cache_strides, value_cache_strides, num_tokens,
              num_kv_heads, head_dim) &&
      (vpr16 & (vpr16 - 1)) == 0) {
    d.w.vecs_per_row = vpr16;
    const int lpt_shift = token_major_shift(num_tokens, num_kv_heads, vpr16);
    if (lpt_shift >= 0) {
      const int lpr_shift = __builtin_ctz((unsigned)vpr16);
      d.vec_scales = k_scale_cache_strides[2] == 1 && v_scale_cache_strides[2] == 1 &&
                     num_kv_heads % 4 == 0 && aligned(k_scale_cache, k_scale_cache_strides[0] * 4, 16) &&
                     aligned(k_scale_cache, k_scale_cache_strides[1] * 4, 16) &&
                     aligned(v_scale_cache, v_scale_cache_strides[0] * 4, 16) &&
                     aligned(v_scale_cache, v_scale_cache_strides[1] * 4, 16);
      const dim3 grid((unsigned)(((num_tokens << lpt_shift) + 255) / 256));
      switch (src_dtype) {
        case INT8KV_F32:
          hipLaunchKernelGGL(dynamic_write16_tm_kernel<kF32>, grid, dim3(256), 0, s, d, lpr_shift, lpt_shift);
          break;
        case INT8KV_F16:
          hipLaunchKernelGGL(dynamic_write16_tm_kernel<kF16>, grid, dim3(256), 0, s, d, lpr_shift, lpt_shift);
          break;
        default:
          hipLaunchKernelGGL(dynamic_write16_tm_kernel<kBF16>, grid, dim3(256), 0, s, d, lpr_shift, lpt_shift);
          break;
      }
      return (int)hipGetLastError();
    }
    const int64_t blocks16 = (num_tokens * vpr16 + 255) / 256;
    const dim3 grid((unsigned)blocks16, (unsigned)num_kv_heads);
    switch (src_dtype) {
      case INT8KV_F32:
        hipLaunchKernelGGL(dynamic_write16_kernel<kF32>, grid, dim3(256), 0, s, d);
        break;
      case INT8KV_F16:
        hipLaunchKernelGGL(dynamic_write16_kernel<kF16>, grid, dim3(256), 0, s, d);
        break;
      default:
        hipLaunchKernelGGL(dynamic_write16_kernel<kBF16>, grid, dim3(256), 0, s, d);
        break;
    }
    return (int)hipGetLastError();
  }

  const int64_t lanes = num_tokens * num_kv_heads * (int64_t)vpr;
  const int threads = 256;
  const int64_t blocks = (lanes + threads - 1) / threads;
  if (blocks > 0x7fffffffLL) return INT8KV_E_SHAPE;
  switch (src_dtype) {
    case INT8KV_F32:
      hipLaunchKernelGGL(dynamic_write_kernel<kF32>, dim3((unsigned)blocks), dim3(threads), 0, s, d);
      break;
    case INT8KV_F16:
      hipLaunchKernelGGL(dynamic_write_kernel<kF16>, dim3((unsigned)blocks), dim3(threads), 0, s, d);
      break;
    default:
      hipLaunchKernelGGL(dynamic_write_kernel<kBF16>, dim3((unsigned)blocks), dim3(threads), 0, s, d);
      break;
  }
  return (int)hipGetLastError();
}

extern "C" const char* int8kv_version(void) { return "int8kv 0.1.0 gfx950"; }
