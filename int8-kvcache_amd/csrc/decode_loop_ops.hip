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
