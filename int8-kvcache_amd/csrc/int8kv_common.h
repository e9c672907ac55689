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

// ------------------------------------------------------------------------ int8 quantisation
// The cache writes need code = clamp(round(RN(x / s)), -127, 127), RN the correctly rounded fp32
// divide (the reference's torch path divides a widened fp32 value by an fp32 scale), rounded to
// even (static scales) or half away from zero (dynamic scales).  A correctly rounded divide is
// about ten VALU instructions, so the kernels take a shortcut that provably gives the same code:
//   q0 = RN(x * r) with r = RN(1 / s):  |r - 1/s| <= 2^-24 / s, so with the rounding of the product
//   and of the divide  |q0 - RN(x/s)| <= 3.0000002 * 2^-24 |x/s|  (r normal: s < 2^100).
//   qc = q0 clamped to [-127, 127], n = rint(qc), and |qc - n| is exact (Sterbenz).
//   * |q0| > 127 (infinities included): qc = n = +-127, and RN(x/s) lies beyond +-126.5, so the
//     code is +-127 either way; a NaN gives -127 on both paths (fmaxf first returns the bound).
//   * |q0| <= 127: |q0 - RN(x/s)| <= 2.28e-5 < 127 * 2^-20.  When |qc - n| < 0.5 - 127 * 2^-20, qc
//     lies farther than that from every half-integer, so RN(x/s) lies in the same open interval
//     between half-integers and rounds to n under either rounding rule (they differ only at
//     half-integers).
// The rest (about 2.4e-4 of the elements, all of them when s >= 2^100) are divided.  Clamping
// before rounding and a constant window keep this to five VALU instructions per element before
// packing (the relative window 2^-20 |qc| and a second clamp after rounding took two more).  The
// argument and an exhaustive check over every bf16 and fp16 value: tests/test_quant_fast_path.py.
struct QuantScale {
  float s;    // the scale (already floored at 1e-6)
  float r;    // RN(1 / s)
  bool fast;  // r is normal, the bound above holds
};

__device__ __forceinline__ QuantScale quant_scale(float s) { return {s, 1.0f / s, s < 0x1p100f}; }

// Distance from rint(qc) below which the shortcut keeps it: 0.5 - 127 * 2^-20 (exact in fp32).
constexpr float kKeepBelow = 0.5f - 127.0f * 0x1p-20f;

// The shortcut code of x (as a float in [-127, 127]); sets `divide` when x needs the divide.
__device__ __forceinline__ float code_shortcut(float x, float r, bool& divide) {
#pragma clang fp contract(off)
  const float q0 = x * r;
  const float qc = fminf(fmaxf(q0, -127.0f), 127.0f);
  const float n = rintf(qc);
  divide = !(fabsf(qc - n) < kKeepBelow);
  return n;
}

// The codes through the correctly rounded divide (the definition the shortcut reproduces).
__device__ __forceinline__ float code_divide_even(float x, float s) {
  return fminf(fmaxf(rintf(x / s), -127.0f), 127.0f);
}
__device__ __forceinline__ float code_divide_half_away(float x, float s) {
  const float q = fminf(fmaxf(x / s, -127.0f), 127.0f);
  return q >= 0.0f ? floorf(q + 0.5f) : ceilf(q - 0.5f);
}

// Four codes (floats holding integers in [-127, 127]) packed as int8 bytes, first in the lowest:
// adding 1.5 * 2^23 leaves each integer's two's-complement low byte in the float's low byte.
__device__ __forceinline__ uint32_t pack_codes(float c0, float c1, float c2, float c3) {
  const uint32_t u0 = __builtin_bit_cast(uint32_t, c0 + 0x1.8p23f);
  const uint32_t u1 = __builtin_bit_cast(uint32_t, c1 + 0x1.8p23f);
  const uint32_t u2 = __builtin_bit_cast(uint32_t, c2 + 0x1.8p23f);
  const uint32_t u3 = __builtin_bit_cast(uint32_t, c3 + 0x1.8p23f);
  // v_perm_b32(hi, lo, sel): selector byte k < 4 picks byte k of lo, 4..7 byte k - 4 of hi,
  // 0x0c gives 0.
  const uint32_t lo = __builtin_amdgcn_perm(u1, u0, 0x0c0c0400u);  // [c0, c1, 0, 0]
  const uint32_t hi = __builtin_amdgcn_perm(u3, u2, 0x04000c0cu);  // [0, 0, c2, c3]
  return lo | hi;
}

// N codes of x with scale q; HALF_AWAY picks the dynamic write's rounding.  Returns the packed
// bytes (N / 4 dwords).
template <int N, bool HALF_AWAY>
__device__ __forceinline__ void quantise(const float (&x)[N], QuantScale q, uint32_t (&out)[N / 4]) {
  float c[N];
  bool dv[N];
  bool any = !q.fast;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    c[i] = code_shortcut(x[i], q.r, dv[i]);
    any |= dv[i];
  }
  if (any) {
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (dv[i] || !q.fast)
        c[i] = HALF_AWAY ? code_divide_half_away(x[i], q.s) : code_divide_even(x[i], q.s);
  }
#pragma unroll
  for (int i = 0; i < N / 4; ++i) out[i] = pack_codes(c[4 * i], c[4 * i + 1], c[4 * i + 2], c[4 * i + 3]);
}

__device__ __forceinline__ int64_t load_index(const void* p, int64_t i, bool is64) {
  return is64 ? reinterpret_cast<const int64_t*>(p)[i]
              : (int64_t) reinterpret_cast<const int32_t*>(p)[i];
}

}  // namespace int8kv
