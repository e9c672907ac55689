// Fused elementwise steps of the decode loop's transformer layers (bf16), for gfx950.
//
// Three HBM-bound kernels that replace chains of small framework kernels around the attention
// operators: residual add + RMSNorm, in-place rotary embedding of the q and k heads, and the
// SwiGLU activation.  Each moves every byte once with 16-byte accesses; in a decode step
// (32 rows) each is one launch of a few microseconds instead of five to ten launches.
//
// Rounding follows the unfused definitions step by step (fp32 arithmetic, a bf16 rounding
// wherever the unfused form stores bf16), so results match them up to the order of the fp32
// sum in the RMS statistic and the last bit of exp.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "int8kv_decode_loop.h"

namespace int8kv_loop {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float round_bf16(float f) {
  return static_cast<float>(static_cast<__bf16>(f));
}
__device__ __forceinline__ uint32_t pack(float a, float b) {
  const __bf16 x = static_cast<__bf16>(a), y = static_cast<__bf16>(b);
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, x)) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, y)) << 16);
}
__device__ __forceinline__ void unpack(const u32x4& v, float (&x)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = lo(v[i]);
    x[2 * i + 1] = hi(v[i]);
  }
}
__device__ __forceinline__ u32x4 pack8(const float (&x)[8]) {
  u32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = pack(x[2 * i], x[2 * i + 1]);
  return v;
}

constexpr int kNormThreads = 256;
constexpr int kNormMaxVec = 4;  // 4 x 256 x 8 = 8192 elements per row at most

template <bool ADD>
__global__ __launch_bounds__(kNormThreads) void add_rms_norm_kernel(
    uint16_t* __restrict__ residual, const uint16_t* __restrict__ delta,
    const uint16_t* __restrict__ weight, uint16_t* __restrict__ out, int hidden, int64_t rs,
    int64_t ds, int64_t os, float eps) {
  const int64_t row = blockIdx.x;
  const int nvec = hidden / 8;
  u32x4* r = reinterpret_cast<u32x4*>(residual + row * rs);
  const u32x4* d = reinterpret_cast<const u32x4*>(delta + (ADD ? row * ds : 0));
  float x[kNormMaxVec][8];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kNormMaxVec; ++j) {
    const int v = threadIdx.x + j * kNormThreads;
    if (v < nvec) {
      u32x4 a = r[v];
      unpack(a, x[j]);
      if (ADD) {
        float y[8];
        unpack(d[v], y);
#pragma unroll
        for (int i = 0; i < 8; ++i) x[j][i] = round_bf16(x[j][i] + y[i]);
        r[v] = pack8(x[j]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += x[j][i] * x[j][i];
    }
  }
  // Block sum of squares: wave butterfly, then one value per wave through LDS.
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
  __shared__ float part[kNormThreads / 64];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / 64; ++w) tot += part[w];
  const float inv = rsqrtf(tot / static_cast<float>(hidden) + eps);
  const u32x4* wv = reinterpret_cast<const u32x4*>(weight);
  u32x4* o = reinterpret_cast<u32x4*>(out + row * os);
#pragma unroll
  for (int j = 0; j < kNormMaxVec; ++j) {
    const int v = threadIdx.x + j * kNormThreads;
    if (v < nvec) {
      float w8[8];
      unpack(wv[v], w8);
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = w8[i] * round_bf16(x[j][i] * inv);
      o[v] = pack8(y);
    }
  }
}

constexpr int kRopeThreads = 256;

__global__ __launch_bounds__(kRopeThreads) void rotary_kernel(
    uint16_t* __restrict__ qkv, int64_t rows, int64_t row_stride, int num_heads, int head_dim,
    const int64_t* __restrict__ positions, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, int64_t max_pos) {
  const int chunks = head_dim / 16;  // 8 rotation pairs per thread
  const int64_t per_row = static_cast<int64_t>(num_heads) * chunks;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kRopeThreads + threadIdx.x;
  if (t >= rows * per_row) return;
  const int64_t row = t / per_row;
  const int rem = static_cast<int>(t - row * per_row);
  const int head = rem / chunks;
  const int c = rem - head * chunks;
  const int64_t p = positions[row];
  if (p < 0 || p >= max_pos) return;
  const int half = head_dim / 2;
  uint16_t* base = qkv + row * row_stride + static_cast<int64_t>(head) * head_dim + c * 8;
  u32x4* p1 = reinterpret_cast<u32x4*>(base);
  u32x4* p2 = reinterpret_cast<u32x4*>(base + half);
  float x1[8], x2[8];
  unpack(*p1, x1);
  unpack(*p2, x2);
  const float* cr = cos_t + p * head_dim + c * 8;
  const float* sr = sin_t + p * head_dim + c * 8;
  float o1[8], o2[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
#pragma clang fp contract(off)
    o1[i] = x1[i] * cr[i] + (-x2[i]) * sr[i];
    o2[i] = x2[i] * cr[half + i] + x1[i] * sr[half + i];
  }
  *p1 = pack8(o1);
  *p2 = pack8(o2);
}

constexpr int kActThreads = 256;

__global__ __launch_bounds__(kActThreads) void silu_mul_kernel(
    const uint16_t* __restrict__ gu, uint16_t* __restrict__ out, int64_t rows, int ffn,
    int64_t is, int64_t os) {
  const int per_row = ffn / 8;
  const int64_t total = rows * per_row;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * kActThreads + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * kActThreads) {
    const int64_t row = t / per_row;
    const int c = static_cast<int>(t - row * per_row);
    const uint16_t* src = gu + row * is + c * 8;
    float g[8], u[8], y[8];
    unpack(*reinterpret_cast<const u32x4*>(src), g);
    unpack(*reinterpret_cast<const u32x4*>(src + ffn), u);
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = round_bf16(g[i] / (1.0f + expf(-g[i]))) * u[i];
    *reinterpret_cast<u32x4*>(out + row * os + c * 8) = pack8(y);
  }
}

// Rotary embedding + KV-cache write of one decode token per row.  One thread per (row, head,
// 8-pair chunk): q heads are rotated in place; k heads are rotated in place and, like the
// v heads, written to the paged cache at the row's slot, block_tables[r, p / BS] * BS + p % BS
// for position p.  The cache value of a rotated k element is computed from its bf16-rounded
// rotation, exactly as when the rotated row is stored first and then written to the cache.
// INT8 caches: q = clamp(rint(x / max(scale, 1e-6)), -127, 127) with an IEEE fp32 divide.
struct RopeWriteArgs {
  uint16_t* qkv;
  int64_t row_stride;
  int64_t rows;
  int num_q_heads, num_kv_heads, head_dim;
  const int64_t* positions;
  const float* cos_t;
  const float* sin_t;
  int64_t max_pos;
  const int32_t* bt;
  int64_t bt_stride;
  int64_t table_width;
  int64_t num_blocks;
  int block_size;
  int block_shift;  // log2(block_size) for a power of two, else -1
  char* kc;
  char* vc;
  int64_t kc_sb, kc_ss, kc_sh;  // element strides
  int64_t vc_sb, vc_ss, vc_sh;
  const float* k_scale;
  const float* v_scale;
};

__device__ __forceinline__ uint32_t quant4_i8(const float* x, float s) {
  uint32_t w = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float q = rintf(x[i] / s);
    q = fminf(fmaxf(q, -127.0f), 127.0f);
    w |= (static_cast<uint32_t>(static_cast<int32_t>(q)) & 0xffu) << (8 * i);
  }
  return w;
}

template <bool I8>
__device__ __forceinline__ void store_cache8(char* base, int64_t elem_off, const float (&x)[8],
                                             float scale) {
  if constexpr (I8) {
    uint32_t w[2] = {quant4_i8(x, scale), quant4_i8(x + 4, scale)};
    *reinterpret_cast<uint64_t*>(base + elem_off) =
        static_cast<uint64_t>(w[0]) | (static_cast<uint64_t>(w[1]) << 32);
  } else {
    *reinterpret_cast<u32x4*>(base + 2 * elem_off) = pack8(x);
  }
}

template <bool I8>
__global__ __launch_bounds__(kRopeThreads) void rope_write_kernel(RopeWriteArgs a) {
  const int chunks = a.head_dim / 16;
  const int heads = a.num_q_heads + 2 * a.num_kv_heads;
  const int64_t per_row = static_cast<int64_t>(heads) * chunks;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kRopeThreads + threadIdx.x;
  if (t >= a.rows * per_row) return;
  const int64_t row = t / per_row;
  const int rem = static_cast<int>(t - row * per_row);
  const int head = rem / chunks;
  const int c = rem - head * chunks;
  const int64_t p = a.positions[row];
  if (p < 0 || p >= a.max_pos) return;
  const int half = a.head_dim / 2;
  uint16_t* base = a.qkv + row * a.row_stride + static_cast<int64_t>(head) * a.head_dim + c * 8;
  u32x4* p1 = reinterpret_cast<u32x4*>(base);
  u32x4* p2 = reinterpret_cast<u32x4*>(base + half);
  float x1[8], x2[8];
  unpack(*p1, x1);
  unpack(*p2, x2);
  const bool is_v = head >= a.num_q_heads + a.num_kv_heads;
  if (!is_v) {
    const float* cr = a.cos_t + p * a.head_dim + c * 8;
    const float* sr = a.sin_t + p * a.head_dim + c * 8;
    float o1[8], o2[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma clang fp contract(off)
      o1[i] = x1[i] * cr[i] + (-x2[i]) * sr[i];
      o2[i] = x2[i] * cr[half + i] + x1[i] * sr[half + i];
    }
    *p1 = pack8(o1);
    *p2 = pack8(o2);
    if (head < a.num_q_heads) return;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x1[i] = round_bf16(o1[i]);
      x2[i] = round_bf16(o2[i]);
    }
  }
  // k or v head: write both 8-element pieces to the cache row of this token.
  // (A shift for a power-of-two block size: a 64-bit division is ~100 instructions per lane.)
  const int64_t blk_idx = a.block_shift >= 0 ? p >> a.block_shift : p / a.block_size;
  if (blk_idx >= a.table_width) return;
  const int64_t blk = a.bt[row * a.bt_stride + blk_idx];
  if (blk < 0 || blk >= a.num_blocks) return;
  const int64_t off = p - blk_idx * a.block_size;
  const int kvh = is_v ? head - a.num_q_heads - a.num_kv_heads : head - a.num_q_heads;
  char* cache = is_v ? a.vc : a.kc;
  const int64_t row_off = is_v ? blk * a.vc_sb + off * a.vc_ss + kvh * a.vc_sh
                               : blk * a.kc_sb + off * a.kc_ss + kvh * a.kc_sh;
  float scale = 1.0f;
  if constexpr (I8) scale = fmaxf(is_v ? a.v_scale[kvh] : a.k_scale[kvh], 1e-6f);
  store_cache8<I8>(cache, row_off + c * 8, x1, scale);
  store_cache8<I8>(cache, row_off + half + c * 8, x2, scale);
}

// Greedy token of each row: the index of the first maximum (a NaN counts as the maximum, as in
// torch.argmax), one workgroup per row.  The row is read with 16-byte loads, kArgmaxUnroll of
// them in flight per thread, so that a row of a 150k vocabulary takes a handful of load
// latencies instead of one per element.
constexpr int kArgmaxThreads = 1024;
constexpr int kArgmaxUnroll = 4;

// (v, i) ranks before (bv, bi): NaN first, then larger value, then lower index.  bi < 0 = empty.
__device__ __forceinline__ bool better(float v, int32_t i, float bv, int32_t bi) {
  if (bi < 0) return i >= 0;
  if (i < 0) return false;
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ float bf16_at(uint32_t w, int hi) {
  return __uint_as_float(hi ? (w & 0xffff0000u) : (w << 16));
}

template <bool VEC>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const uint16_t* __restrict__ x,
                                                                int32_t vocab, int64_t stride,
                                                                int64_t* __restrict__ out) {
  const uint16_t* r = x + static_cast<int64_t>(blockIdx.x) * stride;
  const int32_t tid = threadIdx.x;
  float bv = 0.0f;
  int32_t bi = -1;
  int32_t tail = 0;  // first element left for the scalar loop
  if constexpr (VEC) {
    const u32x4* rv = reinterpret_cast<const u32x4*>(r);
    const int32_t nvec = vocab >> 3;
    for (int32_t i0 = tid; i0 < nvec; i0 += kArgmaxThreads * kArgmaxUnroll) {
      u32x4 w[kArgmaxUnroll];
#pragma unroll
      for (int j = 0; j < kArgmaxUnroll; ++j) {
        const int32_t i = i0 + j * kArgmaxThreads;
        w[j] = i < nvec ? rv[i] : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int j = 0; j < kArgmaxUnroll; ++j) {
        const int32_t i = i0 + j * kArgmaxThreads;
        if (i < nvec) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float v = bf16_at(w[j][e >> 1], e & 1);
            if (better(v, 8 * i + e, bv, bi)) {
              bv = v;
              bi = 8 * i + e;
            }
          }
        }
      }
    }
    tail = nvec << 3;
  }
  for (int32_t i = tail + tid; i < vocab; i += kArgmaxThreads) {
    const float v = __uint_as_float(static_cast<uint32_t>(r[i]) << 16);
    if (better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int32_t oi = __shfl_xor(bi, off, 64);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  __shared__ float sv[kArgmaxThreads / 64];
  __shared__ int32_t si[kArgmaxThreads / 64];
  if ((tid & 63) == 0) {
    sv[tid >> 6] = bv;
    si[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArgmaxThreads / 64; ++w)
      if (better(sv[w], si[w], bv, bi)) {
        bv = sv[w];
        bi = si[w];
      }
    out[blockIdx.x] = bi;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int status(hipError_t e) { return e == hipSuccess ? INT8KV_OK : static_cast<int>(e); }

}  // namespace int8kv_loop

using namespace int8kv_loop;

extern "C" int int8kv_add_rms_norm(void* residual, const void* delta, const void* weight,
                                   void* out, int64_t rows, int32_t hidden,
                                   int64_t residual_row_stride, int64_t delta_row_stride,
                                   int64_t out_row_stride, float eps, void* stream) {
  if (!residual || !weight || !out) return INT8KV_E_NULL;
  if (rows < 0 || rows > 0x7fffffff || hidden <= 0 || hidden % 8 ||
      hidden > kNormThreads * kNormMaxVec * 8)
    return INT8KV_E_SHAPE;
  if (!aligned16(residual) || !aligned16(weight) || !aligned16(out) ||
      (delta && !aligned16(delta)) || residual_row_stride % 8 || out_row_stride % 8 ||
      (delta && delta_row_stride % 8) || residual_row_stride < hidden || out_row_stride < hidden ||
      (delta && delta_row_stride < hidden))
    return INT8KV_E_STRIDE;
  if (rows == 0) return INT8KV_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto* r = static_cast<uint16_t*>(residual);
  auto* d = static_cast<const uint16_t*>(delta);
  auto* w = static_cast<const uint16_t*>(weight);
  auto* o = static_cast<uint16_t*>(out);
  if (d)
    hipLaunchKernelGGL(add_rms_norm_kernel<true>, dim3(static_cast<uint32_t>(rows)),
                       dim3(kNormThreads), 0, s, r, d, w, o, hidden, residual_row_stride,
                       delta_row_stride, out_row_stride, eps);
  else
    hipLaunchKernelGGL(add_rms_norm_kernel<false>, dim3(static_cast<uint32_t>(rows)),
                       dim3(kNormThreads), 0, s, r, d, w, o, hidden, residual_row_stride,
                       int64_t{0}, out_row_stride, eps);
  return status(hipGetLastError());
}

extern "C" int int8kv_rotary_inplace(void* qkv, int64_t rows, int64_t row_stride,
                                     int32_t num_heads, int32_t head_dim,
                                     const int64_t* positions, const float* cos_table,
                                     const float* sin_table, int64_t max_positions,
                                     void* stream) {
  if (!qkv || !positions || !cos_table || !sin_table) return INT8KV_E_NULL;
  if (rows < 0 || num_heads <= 0 || head_dim <= 0 || head_dim % 16 || max_positions <= 0)
    return INT8KV_E_SHAPE;
  if (!aligned16(qkv) || !aligned16(cos_table) || !aligned16(sin_table) || row_stride % 8 ||
      row_stride < static_cast<int64_t>(num_heads) * head_dim)
    return INT8KV_E_STRIDE;
  if (rows == 0) return INT8KV_OK;
  const int64_t threads = rows * num_heads * (head_dim / 16);
  const int64_t blocks = (threads + kRopeThreads - 1) / kRopeThreads;
  if (blocks > 0x7fffffff) return INT8KV_E_SHAPE;
  hipLaunchKernelGGL(rotary_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kRopeThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<uint16_t*>(qkv), rows,
                     row_stride, static_cast<int>(num_heads), static_cast<int>(head_dim),
                     positions, cos_table, sin_table, max_positions);
  return status(hipGetLastError());
}

extern "C" int int8kv_silu_mul(const void* gate_up, void* out, int64_t rows, int32_t ffn,
                               int64_t gate_up_row_stride, int64_t out_row_stride,
                               void* stream) {
  if (!gate_up || !out) return INT8KV_E_NULL;
  if (rows < 0 || ffn <= 0 || ffn % 8) return INT8KV_E_SHAPE;
  if (!aligned16(gate_up) || !aligned16(out) || gate_up_row_stride % 8 || out_row_stride % 8 ||
      gate_up_row_stride < 2 * static_cast<int64_t>(ffn) || out_row_stride < ffn)
    return INT8KV_E_STRIDE;
  if (rows == 0) return INT8KV_OK;
  const int64_t total = rows * (ffn / 8);
  int64_t blocks = (total + kActThreads - 1) / kActThreads;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kActThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(gate_up),
                     static_cast<uint16_t*>(out), rows, static_cast<int>(ffn),
                     gate_up_row_stride, out_row_stride);
  return status(hipGetLastError());
}

extern "C" int int8kv_rotary_cache_write(
    void* qkv, int64_t rows, int64_t row_stride, int32_t num_q_heads, int32_t num_kv_heads,
    int32_t head_dim, const int64_t* positions, const float* cos_table, const float* sin_table,
    int64_t max_positions, const int32_t* block_tables, int64_t table_width,
    int64_t table_row_stride, int64_t num_blocks, int32_t block_size, int cache_dtype,
    void* key_cache,
    void* value_cache, const int64_t key_cache_strides[4], const int64_t value_cache_strides[4],
    const float* k_scale, const float* v_scale, void* stream) {
  if (!qkv || !positions || !cos_table || !sin_table || !block_tables || !key_cache ||
      !value_cache || !key_cache_strides || !value_cache_strides)
    return INT8KV_E_NULL;
  if (cache_dtype != INT8KV_I8 && cache_dtype != INT8KV_BF16) return INT8KV_E_DTYPE;
  if (cache_dtype == INT8KV_I8 && (!k_scale || !v_scale)) return INT8KV_E_NULL;
  if (rows < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || head_dim % 16 ||
      max_positions <= 0 || table_width <= 0 || block_size <= 0 || num_blocks <= 0)
    return INT8KV_E_SHAPE;
  const int64_t e = cache_dtype == INT8KV_I8 ? 1 : 2;
  const int64_t need = e == 1 ? 8 : 16;  // bytes per 8-element piece of a cache row
  if (!aligned16(qkv) || !aligned16(cos_table) || !aligned16(sin_table) || row_stride % 8 ||
      row_stride < static_cast<int64_t>(num_q_heads + 2 * num_kv_heads) * head_dim ||
      key_cache_strides[3] != 1 || value_cache_strides[3] != 1 ||
      reinterpret_cast<uintptr_t>(key_cache) % need || reinterpret_cast<uintptr_t>(value_cache) % need)
    return INT8KV_E_STRIDE;
  for (int i = 0; i < 3; ++i)
    if ((key_cache_strides[i] * e) % need || (value_cache_strides[i] * e) % need)
      return INT8KV_E_STRIDE;
  if (rows == 0) return INT8KV_OK;
  RopeWriteArgs a;
  a.qkv = static_cast<uint16_t*>(qkv);
  a.row_stride = row_stride;
  a.rows = rows;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.head_dim = head_dim;
  a.positions = positions;
  a.cos_t = cos_table;
  a.sin_t = sin_table;
  a.max_pos = max_positions;
  a.bt = block_tables;
  a.bt_stride = table_row_stride;
  a.table_width = table_width;
  a.num_blocks = num_blocks;
  a.block_size = block_size;
  a.block_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  a.kc = static_cast<char*>(key_cache);
  a.vc = static_cast<char*>(value_cache);
  a.kc_sb = key_cache_strides[0];
  a.kc_ss = key_cache_strides[1];
  a.kc_sh = key_cache_strides[2];
  a.vc_sb = value_cache_strides[0];
  a.vc_ss = value_cache_strides[1];
  a.vc_sh = value_cache_strides[2];
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  const int64_t threads = rows * (num_q_heads + 2 * num_kv_heads) * (head_dim / 16);
  const int64_t blocks = (threads + kRopeThreads - 1) / kRopeThreads;
  if (blocks > 0x7fffffff) return INT8KV_E_SHAPE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (cache_dtype == INT8KV_I8)
    hipLaunchKernelGGL(rope_write_kernel<true>, dim3(static_cast<uint32_t>(blocks)),
                       dim3(kRopeThreads), 0, s, a);
  else
    hipLaunchKernelGGL(rope_write_kernel<false>, dim3(static_cast<uint32_t>(blocks)),
                       dim3(kRopeThreads), 0, s, a);
  return status(hipGetLastError());
}

extern "C" int int8kv_argmax_rows(const void* logits, int64_t rows, int64_t vocab,
                                  int64_t row_stride, int64_t* out, void* stream) {
  if (!logits || !out) return INT8KV_E_NULL;
  if (rows < 0 || rows > 0x7fffffff || vocab <= 0 || vocab > 0x7fffffff) return INT8KV_E_SHAPE;
  if (row_stride < vocab) return INT8KV_E_STRIDE;
  if (rows == 0) return INT8KV_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* x = static_cast<const uint16_t*>(logits);
  const int32_t v = static_cast<int32_t>(vocab);
  if (aligned16(logits) && row_stride % 8 == 0)
    hipLaunchKernelGGL(argmax_kernel<true>, dim3(static_cast<uint32_t>(rows)),
                       dim3(kArgmaxThreads), 0, s, x, v, row_stride, out);
  else
    hipLaunchKernelGGL(argmax_kernel<false>, dim3(static_cast<uint32_t>(rows)),
                       dim3(kArgmaxThreads), 0, s, x, v, row_stride, out);
  return status(hipGetLastError());
}
