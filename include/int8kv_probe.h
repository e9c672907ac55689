/*
 * Measurement probes of libint8kv.so: measurement only, no counterpart in the reference.
 *
 * bench.py --ceiling times the two read probes beside the INT8 decode to give the ceiling of the
 * decode's own K/V load pattern on the GPU it runs on (the decode kernel's achieved rate is read
 * against it as well as against the HBM peak).  They read device memory and write one word per
 * thread into `sink`; nothing else.  bench.py --cold uses the clock probe to read the shader
 * clock between the decode step's kernels.  Status codes as in int8kv.h (INT8KV_OK = 0).
 *
 * The measurement build libint8kv_stamps.so (never loaded by the operators) also exports
 * int8kv_stamps_read_<unit>(void* dst, size_t bytes) and int8kv_stamps_clear_<unit>(void) for
 * unit i8, bf16 and probe: the per-wave s_memrealtime stamps of paged_decode_kernels.h
 * (bench.py --stamps).  libint8kv.so has neither.
 */
#ifndef INT8KV_PROBE_H
#define INT8KV_PROBE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Streams `bytes` (a multiple of 16, 16-byte aligned) with 16-byte loads, four in flight per
 * lane, grid-stride over sink_words / 256 workgroups of 256 threads; non_temporal: the
 * non-temporal hint on every load.  sink: sink_words uint32 (a multiple of 256).
 */
int int8kv_probe_stream_read(const void* src, size_t bytes, int32_t non_temporal, uint32_t* sink,
                             int32_t sink_words, void* stream);

/*
 * The INT8 decode kernel's K/V loads at head_dim 128 without its arithmetic: caches int8
 * [num_blocks, 16, 4, 128] (contiguous), num_ranges workgroups of 4 waves (one per kv head),
 * range r streaming tiles_per_range 32-token tiles whose two 16-token blocks are
 * block_ids[r][2 t], block_ids[r][2 t + 1] (int32, block_id_count = 2 x num_ranges x
 * tiles_per_range entries, each clamped into [0, num_blocks)), four tiles in flight per wave, every
 * loaded dword consumed.  sink: at least num_ranges x 256 uint32.  num_kv_heads must be 4.
 */
int int8kv_probe_decode_loads(const void* key_cache, const void* value_cache, int64_t num_blocks,
                              int32_t num_kv_heads, const int32_t* block_ids,
                              int64_t block_id_count, int32_t num_ranges,
                              int32_t tiles_per_range, int32_t non_temporal, uint32_t* sink,
                              int64_t sink_words, void* stream);

/*
 * Shader clock: `workgroups` one-wave workgroups each spin for `ticks` ticks of the GPU's
 * constant 100 MHz real-time counter (s_memrealtime; at most 200,000 iterations) and store, in
 * out[2 w] and out[2 w + 1], the real-time ticks and the shader-clock cycles (s_memtime) that
 * elapsed meanwhile: cycles / (ticks x 10 ns) is the clock in cycles per ns.  workgroups in
 * [1, 65535], ticks in [1, 1000000] (10 ms); out holds 2 x workgroups uint64.
 */
int int8kv_probe_clock(uint64_t* out, int32_t workgroups, uint32_t ticks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* INT8KV_PROBE_H */
