// PagedAttention decode for gfx950: one kernel family over INT8 and 16-bit paged caches.
//
// Replaces src/triton_ops/int8_paged_attention.py (V4 GQA kernel :61-327, split merge :330-388,
// dispatcher :683-769) and src/triton_ops/bf16_paged_attention.py:9-165.  The mathematics is
// the reference's (src/attention_ref.py:19-28 on the dequantised cache,
// src/triton_ops/int8_paged_attention.py:776-814): softmax over <q, k_t> * k_scale * sm_scale,
// weights times v_t * v_scale, with v_scale applied once at the end (:291-292).
//
// Work decomposition (MI355X-first, not the reference's grid):
//   * A work item is (sequence b, kv head g, chunk c of chunk_tokens tokens); the grid is
//     (max_chunks, num_kv_heads, batch) and items past the end of a sequence exit at once, so
//     ragged batches are balanced without reading seq_lens on the host.
//   * A workgroup is 4 waves; wave w takes the 32-token tiles w, w+4, ... of its chunk.  A tile
//     is two 16-token cache blocks of one kv head.  All query heads of the GQA group are
//     processed together on the matrix cores, so every K/V byte is read from HBM once.
//   * Per tile and wave:  S^T = K * Q^T  (2 x 4 MFMA 16x16x32; rows = tokens, cols = heads),
//     online softmax in the exp2 domain, then out^T += V^T * P^T (8 MFMA 16x16x32; rows =
//     head_dim, cols = heads).  The MFMA accumulator layout puts one head per lane column,
//     so the probabilities never leave registers.
//   * INT8 K/V are dequantised in registers to fp16 with the exact magic-number conversion
//     (0x6400 | (x ^ 0x80)) - 1152 = x, two elements per v_pk_add_f16; the per-head k_scale and
//     sm_scale * log2(e) are folded into Q once per work item, v_scale into the final output.
//   * A running max is only moved when a tile's max exceeds it by more than 8 (log2 units), so
//     most tiles skip the accumulator rescale; probabilities are then <= 2^8 (fits fp16/bf16).
//   * The 4 waves merge through LDS; a sequence that spans more than one chunk writes
//     (max, sum, accumulator) partials which merge_kernel combines.

#include "int8kv_common.h"

namespace int8kv {

constexpr int kHeadDim = 128;
constexpr int kBlock = 16;     // tokens per cache block
constexpr int kTile = 32;      // tokens per wave iteration
constexpr int kWaves = 4;      // waves per workgroup
constexpr int kMaxGroup = 16;  // query heads per kv head (MFMA column count)
constexpr float kLazyRescale = 8.0f;
constexpr float kLog2e = 1.4426950408889634f;

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
  float* ws_acc;
  float* ws_m;
  float* ws_l;
  int64_t num_blocks;
  int32_t num_kv_heads;
  int32_t group;
  int32_t width;        // block-table width in blocks
  int32_t chunk_tiles;  // 32-token tiles per work item
  int32_t max_chunks;
  int32_t bt_is64;
  int32_t sl_is64;
  float sm_scale_log2e;
};

// Registers holding one 32-token tile of K and V for one lane.
//   K: lane (i = lane % 16, g = lane / 16) holds token i of block s, head_dim elements
//      [32g, 32g + 32).
//   V: lane (i, g) holds tokens 4g + r (r = 0..3) of block s, head_dim elements [8i, 8i + 8).
template <int CACHE>
struct RawTile;
template <>
struct RawTile<kI8> {
  u32x4 k[2][2];
  u32x2 v[2][4];
};
template <int CACHE>
struct RawTile {
  u32x4 k[2][4];
  u32x4 v[2][4];
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
__device__ __forceinline__ void store_out(char* p, float x) {
  if constexpr (DT == kF32) {
    *reinterpret_cast<float*>(p) = x;
  } else if constexpr (DT == kF16) {
    *reinterpret_cast<_Float16*>(p) = (_Float16)x;
  } else {
    *reinterpret_cast<__bf16*>(p) = (__bf16)x;
  }
}

template <int DT>
constexpr int esize() {
  return DT == kF32 ? 4 : (DT == kI8 ? 1 : 2);
}

template <int CACHE>
__device__ __forceinline__ void issue_tile_loads(RawTile<CACHE>& r, const char* kb,
                                                 const char* vb, int64_t p0, int64_t p1,
                                                 const DecodeArgs& a, int li, int lg) {
  constexpr int E = esize<CACHE>();
  const int64_t ph[2] = {p0, p1};
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const char* kp = kb + ph[s] * a.kc_sb + li * a.kc_ss + lg * (32 * E);
    const u32x4* k4 = reinterpret_cast<const u32x4*>(kp);
    if constexpr (CACHE == kI8) {
      r.k[s][0] = k4[0];
      r.k[s][1] = k4[1];
    } else {
      r.k[s][0] = k4[0];
      r.k[s][1] = k4[1];
      r.k[s][2] = k4[2];
      r.k[s][3] = k4[3];
    }
    const char* vp = vb + ph[s] * a.vc_sb + (4 * lg) * a.vc_ss + li * (8 * E);
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      if constexpr (CACHE == kI8) {
        r.v[s][rr] = *reinterpret_cast<const u32x2*>(vp + rr * a.vc_ss);
      } else {
        r.v[s][rr] = *reinterpret_cast<const u32x4*>(vp + rr * a.vc_ss);
      }
    }
  }
}

// One 32-token tile: scores, online softmax update, P*V accumulation.
//   valid: number of tokens of this tile inside the sequence (1..32).
template <int CACHE>
__device__ __forceinline__ void compute_tile(RawTile<CACHE>& r,
                                             const typename MfmaOp<CACHE>::T (&qop)[4],
                                             f32x4 (&acc)[8], float& m_run, float& l_part,
                                             int valid, int lg, float s_scale) {
  typedef typename MfmaOp<CACHE>::T OpT;
  // ---- scores S^T[token][head] for the two blocks of the tile ----
  f32x4 S[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    S[s] = (f32x4)(0.0f);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      OpT kop;
      if constexpr (CACHE == kI8) {
        const uint32_t d0 = r.k[s][ks >> 1][(ks & 1) * 2] ^ kSignFlip;
        const uint32_t d1 = r.k[s][ks >> 1][(ks & 1) * 2 + 1] ^ kSignFlip;
        kop = i8x8_to_f16(d0, d1);
      } else {
        kop = __builtin_bit_cast(OpT, r.k[s][ks]);
      }
      S[s] = mfma(kop, qop[ks], S[s]);
    }
  }

  // ---- online softmax (exp2 domain); lane column = head, rows = tokens 16s + 4lg + r ----
  float sv[8];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) sv[4 * s + rr] = S[s][rr] * s_scale;
  if (valid < kTile) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        if (16 * s + 4 * lg + rr >= valid) sv[4 * s + rr] = -INFINITY;
    if constexpr (CACHE != kI8) {
      // 16-bit rows past the sequence end may hold non-finite garbage; 0 * NaN would leak.
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          if (16 * s + 4 * lg + rr >= valid) r.v[s][rr] = (u32x4)(0u);
    }
  }
  float mx = sv[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) mx = fmaxf(mx, sv[e]);
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const bool need = mx > m_run + kLazyRescale;
  if (__any(need)) {
    const float m_new = need ? mx : m_run;
    const float alpha = exp2_fast(m_run - m_new);
    m_run = m_new;
    l_part *= alpha;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;
  }
  float p[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    p[e] = exp2_fast(sv[e] - m_run);
    l_part += p[e];
  }
  OpT pop;
#pragma unroll
  for (int e = 0; e < 8; ++e) pop[e] = (typename MfmaOp<CACHE>::E)p[e];

  // ---- out^T[dim][head] += V^T[dim][token] * P^T[token][head] ----
  // MFMA row i of dim tile dt is head_dim element 8i + dt; k-slot e of lane group g is token
  // (block e / 4, row 4g + e % 4), matching the P^T operand built above.
  if constexpr (CACHE == kI8) {
    uint32_t pk[2][2][2][2];  // [block][token pair][lo/hi dword][byte pair 01/23]
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int rp = 0; rp < 2; ++rp)
#pragma unroll
        for (int hsel = 0; hsel < 2; ++hsel) {
          const uint32_t a0 = r.v[s][2 * rp][hsel] ^ kSignFlip;
          const uint32_t b0 = r.v[s][2 * rp + 1][hsel] ^ kSignFlip;
          pk[s][rp][hsel][0] = perm(a0, b0, 0x01050004u);  // [a.b0, b.b0, a.b1, b.b1]
          pk[s][rp][hsel][1] = perm(a0, b0, 0x03070206u);  // [a.b2, b.b2, a.b3, b.b3]
        }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int hsel = dt >> 2, bp = (dt >> 1) & 1;
      const uint32_t sel = (dt & 1) ? kSelHi : kSelLo;
      u32x4 w;
      w[0] = perm(kMagic, pk[0][0][hsel][bp], sel);
      w[1] = perm(kMagic, pk[0][1][hsel][bp], sel);
      w[2] = perm(kMagic, pk[1][0][hsel][bp], sel);
      w[3] = perm(kMagic, pk[1][1][hsel][bp], sel);
      const f16x8 vop = __builtin_bit_cast(f16x8, w) - (f16x8)(_Float16)1152.0f;
      acc[dt] = mfma(vop, pop, acc[dt]);
    }
  } else {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int wd = dt >> 1;
      const uint32_t sel = (dt & 1) ? 0x07060302u : 0x05040100u;
      u32x4 w;
      w[0] = perm(r.v[0][1][wd], r.v[0][0][wd], sel);
      w[1] = perm(r.v[0][3][wd], r.v[0][2][wd], sel);
      w[2] = perm(r.v[1][1][wd], r.v[1][0][wd], sel);
      w[3] = perm(r.v[1][3][wd], r.v[1][2][wd], sel);
      acc[dt] = mfma(__builtin_bit_cast(OpT, w), pop, acc[dt]);
    }
  }
}

template <int CACHE, int QT>
__global__ __launch_bounds__(256) void decode_kernel(DecodeArgs a) {
  typedef typename MfmaOp<CACHE>::T OpT;
  __shared__ float s_acc[kWaves][kMaxGroup][kHeadDim];
  __shared__ float s_m[kWaves][kMaxGroup];
  __shared__ float s_l[kWaves][kMaxGroup];

  const int c = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int G = a.group;

  int64_t L = load_index(a.sl, b, a.sl_is64);
  const int64_t cap = (int64_t)a.width * kBlock;
  L = L < 0 ? 0 : (L > cap ? cap : L);
  const int64_t CT = (int64_t)a.chunk_tiles * kTile;
  const int64_t nchunks = L > CT ? (L + CT - 1) / CT : 1;
  if (c >= nchunks) return;

  const int64_t tok0 = (int64_t)c * CT;
  const int64_t tok1 = (tok0 + CT < L) ? tok0 + CT : L;
  const int ntiles = tok1 > tok0 ? (int)((tok1 - tok0 + kTile - 1) / kTile) : 0;
  const int64_t nblk = (L + kBlock - 1) / kBlock;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int li = lane & 15;
  const int lg = lane >> 4;

  // ---- Q^T operand: lane (head li, group lg) holds q[li][32lg + 8ks + e] ----
  float qscale = 1.0f;
  float s_scale = a.sm_scale_log2e;
  if constexpr (CACHE == kI8) {
    qscale = fmaxf(a.k_scale[kvh], 1e-6f) * a.sm_scale_log2e;
    s_scale = 1.0f;
  }
  OpT qop[4];
  if (li < G) {
    constexpr int QE = esize<QT>();
    const char* qp = a.q + ((int64_t)b * a.q_sb + (int64_t)(kvh * G + li) * a.q_sh + 32 * lg) * QE;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      float x[8];
      load8_f32<QT>(qp + 8 * ks * QE, x);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        qop[ks][e] = (typename MfmaOp<CACHE>::E)(x[e] * qscale);
    }
  } else {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) qop[ks][e] = 0;
  }

  f32x4 acc[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) acc[dt] = (f32x4)(0.0f);
  float m_run = -INFINITY;
  float l_part = 0.0f;

  const char* kb = a.kc + (int64_t)kvh * a.kc_sh;
  const char* vb = a.vc + (int64_t)kvh * a.vc_sh;
  const int64_t bt_row = (int64_t)b * a.bt_sb;
  const int64_t nb_max = a.num_blocks - 1;

  auto phys = [&](int64_t lb) -> int64_t {
    int64_t p = load_index(a.bt, bt_row + lb * a.bt_sl, a.bt_is64);
    return p < 0 ? 0 : (p > nb_max ? nb_max : p);
  };
  auto load = [&](RawTile<CACHE>& r, int t) {
    const int64_t lb0 = (tok0 + (int64_t)t * kTile) / kBlock;
    const int64_t p0 = phys(lb0);
    const int64_t p1 = (lb0 + 1 < nblk) ? phys(lb0 + 1) : p0;
    issue_tile_loads<CACHE>(r, kb, vb, p0, p1, a, li, lg);
  };
  auto valid_of = [&](int t) -> int {
    const int64_t v = tok1 - (tok0 + (int64_t)t * kTile);
    return v >= kTile ? kTile : (int)v;
  };

  // Two register buffers: the next tile's loads are in flight while this one is computed.
  RawTile<CACHE> r0, r1;
  int t = wave;
  if (t < ntiles) load(r0, t);
  while (t < ntiles) {
    int tn = t + kWaves;
    if (tn < ntiles) load(r1, tn);
    compute_tile<CACHE>(r0, qop, acc, m_run, l_part, valid_of(t), lg, s_scale);
    t = tn;
    if (t >= ntiles) break;
    tn = t + kWaves;
    if (tn < ntiles) load(r0, tn);
    compute_tile<CACHE>(r1, qop, acc, m_run, l_part, valid_of(t), lg, s_scale);
    t = tn;
  }

  // ---- merge the 4 waves through LDS ----
  l_part += __shfl_xor(l_part, 16);
  l_part += __shfl_xor(l_part, 32);
  if (li < G) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) s_acc[wave][li][32 * lg + 8 * rr + dt] = acc[dt][rr];
    if (lg == 0) {
      s_m[wave][li] = m_run;
      s_l[wave][li] = l_part;
    }
  }
  __syncthreads();

  const float vscale = (CACHE == kI8) ? fmaxf(a.v_scale[kvh], 1e-6f) : 1.0f;
  const bool single = nchunks == 1;
  const int64_t item = ((int64_t)b * a.num_kv_heads + kvh) * a.max_chunks + c;
  for (int idx = threadIdx.x; idx < G * kHeadDim; idx += kWaves * kWave) {
    const int j = idx / kHeadDim;
    const int d = idx % kHeadDim;
    float M = s_m[0][j];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_m[w][j]);
    float Ls = 0.0f, O = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float wt = exp2_fast(s_m[w][j] - M);
        Ls += wt * s_l[w][j];
        O += wt * s_acc[w][j][d];
      }
    }
    if (single) {
      const float o = Ls > 0.0f ? O * vscale / Ls : 0.0f;
      store_out<QT>(a.out + ((int64_t)b * a.o_sb + (int64_t)(kvh * G + j) * a.o_sh + d) *
                                esize<QT>(),
                    o);
    } else {
      a.ws_acc[(item * G + j) * kHeadDim + d] = O;
      if (d == 0) {
        a.ws_m[item * G + j] = M;
        a.ws_l[item * G + j] = Ls;
      }
    }
  }
}

// Merges the chunk partials of every sequence that spans more than one chunk.
// grid (num_q_heads, batch), 128 threads (one per head_dim element).
template <int CACHE, int QT>
__global__ __launch_bounds__(128) void merge_kernel(DecodeArgs a) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int G = a.group;
  const int kvh = h / G;
  const int j = h % G;
  int64_t L = load_index(a.sl, b, a.sl_is64);
  const int64_t cap = (int64_t)a.width * kBlock;
  L = L < 0 ? 0 : (L > cap ? cap : L);
  const int64_t CT = (int64_t)a.chunk_tiles * kTile;
  const int64_t nchunks = L > CT ? (L + CT - 1) / CT : 1;
  if (nchunks <= 1) return;
  const int d = threadIdx.x;
  const int64_t item0 = ((int64_t)b * a.num_kv_heads + kvh) * a.max_chunks;
  float M = -INFINITY;
  for (int64_t c = 0; c < nchunks; ++c) M = fmaxf(M, a.ws_m[(item0 + c) * G + j]);
  float Ls = 0.0f, O = 0.0f;
  for (int64_t c = 0; c < nchunks; ++c) {
    const int64_t row = (item0 + c) * G + j;
    const float wt = exp2_fast(a.ws_m[row] - M);
    Ls += wt * a.ws_l[row];
    O += wt * a.ws_acc[row * kHeadDim + d];
  }
  const float vscale = (CACHE == kI8) ? fmaxf(a.v_scale[kvh], 1e-6f) : 1.0f;
  const float o = Ls > 0.0f ? O * vscale / Ls : 0.0f;
  store_out<QT>(a.out + ((int64_t)b * a.o_sb + (int64_t)h * a.o_sh + d) * esize<QT>(), o);
}

}  // namespace int8kv

using namespace int8kv;

namespace {

int64_t ceil_div(int64_t x, int64_t y) { return (x + y - 1) / y; }

int32_t auto_chunk_tokens(int64_t batch, int32_t num_kv_heads, int64_t table_width,
                          int32_t block_size) {
  const int64_t tokens = table_width * block_size;
  const int32_t cands[3] = {512, 256, 128};
  for (int i = 0; i < 3; ++i) {
    if (batch * num_kv_heads * ceil_div(tokens, cands[i]) >= 2048) return cands[i];
  }
  return 128;
}

size_t workspace_bytes(int64_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                       int64_t table_width, int32_t block_size, int32_t chunk_tokens) {
  const int64_t max_chunks = ceil_div(table_width * block_size, chunk_tokens);
  if (max_chunks <= 1) return 0;
  const int64_t rows = batch * (int64_t)num_q_heads * max_chunks;  // (item, head) rows
  return (size_t)(rows * (kHeadDim + 2) * (int64_t)sizeof(float));
}

bool aligned16(const void* p, int64_t stride_bytes) {
  return ((uintptr_t)p % 16) == 0 && (stride_bytes % 16) == 0;
}

template <int CACHE, int QT>
int launch(const DecodeArgs& a, int64_t batch, int32_t num_q_heads, uint32_t flags,
           hipStream_t s) {
  if (flags & INT8KV_DECODE_MAIN) {
    dim3 grid((unsigned)a.max_chunks, (unsigned)a.num_kv_heads, (unsigned)batch);
    hipLaunchKernelGGL((decode_kernel<CACHE, QT>), grid, dim3(kWaves * kWave), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  if ((flags & INT8KV_DECODE_MERGE) && a.max_chunks > 1) {
    dim3 grid((unsigned)num_q_heads, (unsigned)batch);
    hipLaunchKernelGGL((merge_kernel<CACHE, QT>), grid, dim3(kHeadDim), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  return INT8KV_OK;
}

template <int CACHE>
int launch_q(const DecodeArgs& a, int query_dtype, int64_t batch, int32_t num_q_heads,
             uint32_t flags, hipStream_t s) {
  switch (query_dtype) {
    case INT8KV_F32:
      return launch<CACHE, kF32>(a, batch, num_q_heads, flags, s);
    case INT8KV_F16:
      return launch<CACHE, kF16>(a, batch, num_q_heads, flags, s);
    default:
      return launch<CACHE, kBF16>(a, batch, num_q_heads, flags, s);
  }
}

}  // namespace

extern "C" int32_t int8kv_decode_auto_chunk_tokens(int64_t batch, int32_t num_kv_heads,
                                                   int64_t table_width, int32_t block_size) {
  if (batch <= 0 || num_kv_heads <= 0 || table_width <= 0 || block_size <= 0) return 128;
  return auto_chunk_tokens(batch, num_kv_heads, table_width, block_size);
}

extern "C" size_t int8kv_decode_workspace_bytes(int64_t batch, int32_t num_q_heads,
                                                int32_t num_kv_heads, int32_t head_dim,
                                                int64_t table_width, int32_t block_size,
                                                int32_t chunk_tokens) {
  if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim != kHeadDim ||
      block_size != kBlock || table_width <= 0 || num_q_heads % num_kv_heads != 0 ||
      num_q_heads / num_kv_heads > kMaxGroup || chunk_tokens < 0 || chunk_tokens % kTile != 0)
    return 0;
  if (chunk_tokens == 0)
    chunk_tokens = auto_chunk_tokens(batch, num_kv_heads, table_width, block_size);
  return workspace_bytes(batch, num_q_heads, num_kv_heads, table_width, block_size, chunk_tokens);
}

extern "C" int int8kv_paged_decode(
    const void* query, int query_dtype, int64_t batch, int32_t num_q_heads, int32_t head_dim,
    const int64_t query_strides[3], const void* key_cache, const void* value_cache,
    int cache_dtype, int64_t num_blocks, int32_t block_size, int32_t num_kv_heads,
    const int64_t key_cache_strides[4], const int64_t value_cache_strides[4],
    const void* block_tables, int table_dtype, int64_t table_width, const int64_t table_strides[2],
    const void* seq_lens, int seq_lens_dtype, const float* k_scale, const float* v_scale,
    float sm_scale, void* out, const int64_t out_strides[3], void* workspace,
    size_t workspace_bytes_given, int32_t chunk_tokens, uint32_t flags, void* stream) {
  if (!query_strides || !key_cache_strides || !value_cache_strides || !table_strides ||
      !out_strides)
    return INT8KV_E_NULL;
  if (query_dtype != INT8KV_F32 && query_dtype != INT8KV_F16 && query_dtype != INT8KV_BF16)
    return INT8KV_E_DTYPE;
  if (cache_dtype != INT8KV_I8 && cache_dtype != INT8KV_BF16 && cache_dtype != INT8KV_F16)
    return INT8KV_E_DTYPE;
  if (table_dtype != INT8KV_I32 && table_dtype != INT8KV_I64) return INT8KV_E_DTYPE;
  if (seq_lens_dtype != INT8KV_I32 && seq_lens_dtype != INT8KV_I64) return INT8KV_E_DTYPE;
  if (batch < 0 || num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
      num_q_heads / num_kv_heads > kMaxGroup || head_dim != kHeadDim || block_size != kBlock ||
      num_blocks <= 0 || table_width <= 0 || chunk_tokens < 0 || chunk_tokens % kTile != 0 ||
      batch > 65535 || num_kv_heads > 65535)
    return INT8KV_E_SHAPE;
  if (batch == 0) return INT8KV_OK;
  if (!query || !key_cache || !value_cache || !block_tables || !seq_lens || !out)
    return INT8KV_E_NULL;
  if (cache_dtype == INT8KV_I8 && (!k_scale || !v_scale)) return INT8KV_E_NULL;

  const int64_t qe = query_dtype == INT8KV_F32 ? 4 : 2;
  const int64_t ce = cache_dtype == INT8KV_I8 ? 1 : 2;
  if (query_strides[2] != 1 || out_strides[2] != 1 || key_cache_strides[3] != 1 ||
      value_cache_strides[3] != 1)
    return INT8KV_E_STRIDE;
  if (!aligned16(query, query_strides[0] * qe) || !aligned16(query, query_strides[1] * qe))
    return INT8KV_E_STRIDE;
  for (int i = 0; i < 3; ++i) {
    if (!aligned16(key_cache, key_cache_strides[i] * ce) ||
        !aligned16(value_cache, value_cache_strides[i] * ce))
      return INT8KV_E_STRIDE;
  }

  if (chunk_tokens == 0)
    chunk_tokens = auto_chunk_tokens(batch, num_kv_heads, table_width, block_size);
  const int64_t max_chunks = ceil_div(table_width * block_size, chunk_tokens);
  if (max_chunks > 0x7fffffffLL) return INT8KV_E_SHAPE;
  const size_t need =
      workspace_bytes(batch, num_q_heads, num_kv_heads, table_width, block_size, chunk_tokens);
  if (need > 0 && (workspace == nullptr || workspace_bytes_given < need ||
                   ((uintptr_t)workspace % 16) != 0))
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
  const int64_t rows = batch * (int64_t)num_q_heads * max_chunks;
  float* ws = static_cast<float*>(workspace);
  a.ws_acc = need ? ws : nullptr;
  a.ws_m = need ? ws + rows * kHeadDim : nullptr;
  a.ws_l = need ? ws + rows * (kHeadDim + 1) : nullptr;
  a.num_blocks = num_blocks;
  a.num_kv_heads = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.width = (int32_t)(table_width > 0x7fffffffLL ? 0x7fffffff : table_width);
  a.chunk_tiles = chunk_tokens / kTile;
  a.max_chunks = (int32_t)max_chunks;
  a.bt_is64 = table_dtype == INT8KV_I64;
  a.sl_is64 = seq_lens_dtype == INT8KV_I64;
  a.sm_scale_log2e = sm_scale * kLog2e;

  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (cache_dtype) {
    case INT8KV_I8:
      return launch_q<kI8>(a, query_dtype, batch, num_q_heads, flags, s);
    case INT8KV_BF16:
      return launch_q<kBF16>(a, query_dtype, batch, num_q_heads, flags, s);
    default:
      return launch_q<kF16>(a, query_dtype, batch, num_q_heads, flags, s);
  }
}
