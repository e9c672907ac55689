/*
 * int8kv_decode_loop.h -- fused elementwise steps of the decode loop's transformer layers,
 * exported by libint8kv.so next to the cache operators of int8kv.h.
 *
 * These entry points have no counterpart among the reference's own operators: in the
 * reference's end-to-end runs (bench/run_qwen_case_final.py of cjsmt/Int8-kvcache) the layers
 * around attention run inside vLLM, whose custom ops fused_add_rms_norm, rotary_embedding and
 * silu_and_mul (vLLM 0.16 / 0.26, csrc/layernorm_kernels.cu, csrc/pos_encoding_kernels.cu,
 * csrc/activation_kernels.cu -- third-party, not vendored) play this role.  They serve the
 * random-init Qwen2.5-7B-shaped decode loop of this library (config 4: TPOT and KV bytes).
 *
 * Conventions are those of int8kv.h: device pointers, element strides, a hipStream_t as void*,
 * 0 / negative INT8KV_E_* / positive hipError_t returns, no allocation, no synchronisation.
 * Every tensor here is bf16 (fp32 for the rotary tables); rows must be 16-byte aligned.
 */
#ifndef INT8KV_DECODE_LOOP_H
#define INT8KV_DECODE_LOOP_H

#include <stdint.h>

#include "int8kv.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Residual add + RMSNorm, per row r of `rows`:
 *   if delta != NULL: residual[r, :] = bf16(residual[r, :] + delta[r, :])     (in place)
 *   out[r, :] = bf16(weight * bf16(residual[r, :] * rsqrt(mean(residual[r, :]^2) + eps)))
 * (statistics in fp32).  hidden: a multiple of 8, at most 8192.  out may not alias residual.
 */
int int8kv_add_rms_norm(void* residual, const void* delta, const void* weight, void* out,
                        int64_t rows, int32_t hidden, int64_t residual_row_stride,
                        int64_t delta_row_stride, int64_t out_row_stride, float eps, void* stream);

/*
 * Rotary embedding (rotate-half form) in place on the first `num_heads` heads of each row:
 *   x = qkv[r, h*head_dim : (h+1)*head_dim], p = positions[r], half = head_dim / 2,
 *   x'[i]        = x[i] * cos[p, i] - x[i + half] * sin[p, i]
 *   x'[i + half] = x[i + half] * cos[p, i + half] + x[i] * sin[p, i + half]       (i < half)
 * with fp32 products and sum, each rounded (no fused multiply-add), then rounded to bf16.
 * cos/sin: fp32 [max_positions, head_dim], contiguous.  positions: int64 [rows].  A row whose
 * position lies outside [0, max_positions) is left unchanged.  head_dim: a multiple of 16.
 */
int int8kv_rotary_inplace(void* qkv, int64_t rows, int64_t row_stride, int32_t num_heads,
                          int32_t head_dim, const int64_t* positions, const float* cos_table,
                          const float* sin_table, int64_t max_positions, void* stream);

/*
 * SwiGLU activation: out[r, j] = bf16(bf16(silu(g)) * u), g = gate_up[r, j],
 * u = gate_up[r, ffn + j], silu(g) = g / (1 + exp(-g)) in fp32.  ffn: a multiple of 8.
 */
int int8kv_silu_mul(const void* gate_up, void* out, int64_t rows, int32_t ffn,
                    int64_t gate_up_row_stride, int64_t out_row_stride, void* stream);

/*
 * Rotary embedding plus KV-cache write of one decode token per row (the two steps of
 * int8kv_rotary_inplace and int8kv_cache_write fused, with the same results):
 *   qkv rows hold num_q_heads q heads, then num_kv_heads k heads, then num_kv_heads v heads;
 *   the q and k heads are rotated in place as in int8kv_rotary_inplace (positions[r], tables);
 *   the row's k (rotated, bf16-rounded) and v heads are written to the paged caches at the slot
 *   of position p = positions[r]: block block_tables[r, p / block_size], row p % block_size.
 *   INT8 caches (cache_dtype INT8KV_I8): clamp(rint(x / max(scale[h], 1e-6)), -127, 127) with
 *   an IEEE fp32 divide, as int8kv_cache_write; BF16 caches (INT8KV_BF16): the bf16 values.
 * block_tables: int32 [rows, table_width] with row stride table_row_stride.  Rows whose position
 * lies outside [0, max_positions), whose block index reaches table_width or whose block id is
 * negative or >= num_blocks write nothing to the caches.  Cache layout as int8kv.h:
 * [num_blocks, block_size, num_kv_heads, head_dim], element strides, innermost 1, rows 8-byte
 * (INT8) or 16-byte (BF16) aligned.  head_dim: a multiple of 16.
 */
int int8kv_rotary_cache_write(void* qkv, int64_t rows, int64_t row_stride, int32_t num_q_heads,
                              int32_t num_kv_heads, int32_t head_dim, const int64_t* positions,
                              const float* cos_table, const float* sin_table,
                              int64_t max_positions, const int32_t* block_tables,
                              int64_t table_width, int64_t table_row_stride, int64_t num_blocks,
                              int32_t block_size, int cache_dtype, void* key_cache,
                              void* value_cache, const int64_t key_cache_strides[4],
                              const int64_t value_cache_strides[4], const float* k_scale,
                              const float* v_scale, void* stream);

/*
 * Greedy decoding: out[r] = the index of the first maximum of the bf16 row logits[r, :vocab]
 * (a NaN counts as the largest value), as torch.argmax over the last dimension.
 * vocab in [1, 2^31 - 1]; row_stride >= vocab, in elements.  One workgroup per row; rows that
 * start 16-byte aligned (logits aligned, row_stride a multiple of 8) are read 16 bytes at a time.
 */
int int8kv_argmax_rows(const void* logits, int64_t rows, int64_t vocab, int64_t row_stride,
                       int64_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* INT8KV_DECODE_LOOP_H */
