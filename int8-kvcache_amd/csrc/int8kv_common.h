// Shared device-side types and helpers of libint8kv.so (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/int8kv.h"

namespace int8kv {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Element type tags used as template parameters (values match enum int8kv_dtype).
enum Dt : int { kF32 = INT8KV_F32, kF16 = INT8KV_F16, kBF16 = INT8KV_BF16, kI8 = INT8KV_I8 };

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __builtin_bit_cast(float, h << 16);
}

// Unpacks the two 16-bit lanes of a dword into floats.
template <int DT>
__device__ __forceinline__ void unpack2(uint32_t w, float& lo, float& hi) {
  if constexpr (DT == kBF16) {
    lo = __builtin_bit_cast(float, w << 16);
    hi = __builtin_bit_cast(float, w & 0xffff0000u);
  } else {
    f16x2 h = __builtin_bit_cast(f16x2, w);
    lo = (float)h[0];
    hi = (float)h[1];
  }
}

// Loads 8 consecutive elements of type DT (16-byte aligned for 16-bit types, 32-byte for f32)
// and widens them to fp32.
template <int DT>
__device__ __forceinline__ void load8_f32(const void* p, float (&x)[8]) {
  if constexpr (DT == kF32) {
    const f32x4* q = reinterpret_cast<const f32x4*>(p);
    f32x4 a = q[0], b = q[1];
    x[0] = a[0]; x[1] = a[1]; x[2] = a[2]; x[3] = a[3];
    x[4] = b[0]; x[5] = b[1]; x[6] = b[2]; x[7] = b[3];
  } else {
    u32x4 w = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) unpack2<DT>(w[i], x[2 * i], x[2 * i + 1]);
  }
}

__device__ __forceinline__ int64_t load_index(const void* p, int64_t i, bool is64) {
  return is64 ? reinterpret_cast<const int64_t*>(p)[i]
              : (int64_t) reinterpret_cast<const int32_t*>(p)[i];
}

}  // namespace int8kv
