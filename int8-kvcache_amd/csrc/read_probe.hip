// Measurement probes (include/int8kv_probe.h).  The read-ceiling probes give what this chip
// delivers for the INT8 decode's K/V stream with the arithmetic taken out, so that the decode
// kernel's rate can be read against the ceiling of its own load pattern rather than against the
// HBM peak alone; the clock probe reads the shader clock against the real-time counter.
//
//   probe_stream_kernel   a plain streaming read: 16-byte loads, four in flight per lane,
//                         grid-stride over a flat buffer (the best a simple reader gets).
//   probe_decode_kernel   the decode's loads exactly: one workgroup per range, one wave per kv
//                         head, 32-token tiles of two 16-token row groups whose block ids are
//                         staged in LDS, the same issue_k / issue_v functions as decode_kernel
//                         (INT8, head_dim 128: two 16-byte K loads and four 8-byte V loads per
//                         lane and row group), DEPTH tiles in flight with the same refill order
//                         (K after the tile's scores would run, V after its P*V), and every loaded
//                         dword consumed (xor) instead of the MFMA and softmax work.
#include "paged_decode_kernels.h"

#include "../../include/int8kv_probe.h"

namespace int8kv {
namespace {

constexpr int kProbeDepth = 4;  // tiles in flight per wave: the cfg3 INT8 decode's depth
constexpr int kProbeWaves = 4;  // kv heads (waves) per range

template <bool NT>
__global__ __launch_bounds__(256) void probe_stream_kernel(const u32x4* src, int64_t n16,
                                                           uint32_t* sink) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  uint32_t acc = 0;
  int64_t i = tid;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    u32x4 x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      x[j] = NT ? __builtin_nontemporal_load(src + i + j * stride) : src[i + j * stride];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc ^= x[j][0] ^ x[j][1] ^ x[j][2] ^ x[j][3];
  }
  for (; i < n16; i += stride) {
    const u32x4 x = NT ? __builtin_nontemporal_load(src + i) : src[i];
    acc ^= x[0] ^ x[1] ^ x[2] ^ x[3];
  }
  sink[tid] = acc;
}

template <bool NT>
__global__ __launch_bounds__(kProbeWaves * 64) __attribute__((amdgpu_waves_per_eu(1))) void
probe_decode_kernel(DecodeArgs a, int32_t tiles, uint32_t* sink) {
  constexpr int NB = tile_blocks<kI8>();
  constexpr int HD = 128;
  __shared__ int32_t s_ids[kProbeWaves][kChunkTiles * NB];
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int li = lane & 15, lg = lane >> 4;
  const int64_t r = blockIdx.x;  // range: row r of the block-id table, 2 x tiles entries
  INT8KV_STAMPS_DECL
  INT8KV_STAMP(0);
  const char* kb = a.kc + (int64_t)wave * a.kc_sh;
  const char* vb = a.vc + (int64_t)wave * a.vc_sh;
  int32_t* ids = s_ids[wave];
  KTile<kI8, NB, HD> kt[kProbeDepth];
  VTile<kI8, NB, HD> vt[kProbeDepth];
  TileRows<NB> ph[kProbeDepth];
  uint32_t acc = 0;
  const int64_t nblk = (int64_t)tiles * NB;
  for (int64_t c0 = 0; c0 < tiles; c0 += kChunkTiles) {
    const int64_t c1 = tiles - c0 > kChunkTiles ? c0 + kChunkTiles : tiles;
    stage_block_ids<NB>(a, ids, r, c0, c1, nblk, lane);
    auto blocks_of = [&](int64_t t, TileRows<NB>& p) {
#pragma unroll
      for (int s = 0; s < NB; ++s) {
        p.id[s] = __builtin_amdgcn_readfirstlane(ids[NB * (int)(t - c0) + s]);
        p.row[s] = 0;
      }
    };
#pragma unroll
    for (int d = 0; d < kProbeDepth; ++d) {
      blocks_of(c0 + d < c1 ? c0 + d : c1 - 1, ph[d]);
      issue_k<kI8, NB, NT, HD>(kt[d], kb, ph[d], a, li, lg);
      issue_v<kI8, NB, NT, HD>(vt[d], vb, ph[d], a, li, lg);
    }
    INT8KV_STAMP_ONCE(2);
    int64_t t = c0;
    for (; t + kProbeDepth - 1 < c1; t += kProbeDepth) {
#pragma unroll
      for (int d = 0; d < kProbeDepth; ++d) {
        const bool refill = t + d + kProbeDepth < c1;
#pragma unroll
        for (int s = 0; s < NB; ++s)
#pragma unroll
          for (int p = 0; p < k_pieces<kI8, HD>(); ++p)
            acc ^= kt[d].k[s][p][0] ^ kt[d].k[s][p][1] ^ kt[d].k[s][p][2] ^ kt[d].k[s][p][3];
        if (refill) {
          blocks_of(t + d + kProbeDepth, ph[d]);
          issue_k<kI8, NB, NT, HD>(kt[d], kb, ph[d], a, li, lg);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < NB; ++s)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
#pragma unroll
            for (int w = 0; w < v_dwords<kI8, HD>(); ++w) acc ^= vt[d].v[s][rr][w];
        if (refill) issue_v<kI8, NB, NT, HD>(vt[d], vb, ph[d], a, li, lg);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // The last (c1 - t) < kProbeDepth tiles sit in buffers 0, 1, ...
#pragma unroll
    for (int d = 0; d + 1 < kProbeDepth; ++d) {
      if (t + d < c1) {
#pragma unroll
        for (int s = 0; s < NB; ++s) {
#pragma unroll
          for (int p = 0; p < k_pieces<kI8, HD>(); ++p) acc ^= kt[d].k[s][p][0] ^ kt[d].k[s][p][3];
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) acc ^= vt[d].v[s][rr][0];
        }
      }
    }
    // Every buffer's loads have landed before the block ids are restaged.
#pragma unroll
    for (int d = 0; d < kProbeDepth; ++d) acc ^= kt[d].k[0][0][1] ^ vt[d].v[0][0][1];
  }
  sink[blockIdx.x * blockDim.x + threadIdx.x] = acc;
  INT8KV_STAMP(7);
  INT8KV_STAMPS_STORE(kProbeWaves, wave, lane);
}

// One wave per workgroup: shader-clock cycles (s_memtime) over a window of the 100 MHz real-time
// counter (s_memrealtime), the loop bounded by an iteration cap as well as by the window.
__global__ __launch_bounds__(64) void probe_clock_kernel(uint64_t* out, uint32_t ticks) {
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  const uint64_t c0 = __builtin_amdgcn_s_memtime();
  uint64_t r = r0, c = c0;
  for (int i = 0; i < 200000 && r - r0 < ticks; ++i) {
    r = __builtin_amdgcn_s_memrealtime();
    c = __builtin_amdgcn_s_memtime();
  }
  if (threadIdx.x == 0) {
    out[2 * blockIdx.x] = r - r0;
    out[2 * blockIdx.x + 1] = c - c0;
  }
}

}  // namespace
}  // namespace int8kv

using namespace int8kv;

INT8KV_STAMPS_ACCESSORS(probe)

extern "C" int int8kv_probe_stream_read(const void* src, size_t bytes, int32_t non_temporal,
                                        uint32_t* sink, int32_t sink_words, void* stream) {
  if (!src || !sink) return INT8KV_E_NULL;
  if (bytes % 16 != 0 || ((uintptr_t)src % 16) != 0) return INT8KV_E_STRIDE;
  constexpr int kThreads = 256;
  if (sink_words < kThreads || sink_words % kThreads != 0) return INT8KV_E_SHAPE;
  const dim3 grid((unsigned)(sink_words / kThreads));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n16 = (int64_t)(bytes / 16);
  if (non_temporal)
    hipLaunchKernelGGL((probe_stream_kernel<true>), grid, dim3(kThreads), 0, s,
                       static_cast<const u32x4*>(src), n16, sink);
  else
    hipLaunchKernelGGL((probe_stream_kernel<false>), grid, dim3(kThreads), 0, s,
                       static_cast<const u32x4*>(src), n16, sink);
  return (int)hipGetLastError();
}

extern "C" int int8kv_probe_decode_loads(const void* key_cache, const void* value_cache,
                                         int64_t num_blocks, int32_t num_kv_heads,
                                         const int32_t* block_ids, int64_t block_id_count,
                                         int32_t num_ranges, int32_t tiles_per_range,
                                         int32_t non_temporal, uint32_t* sink,
                                         int64_t sink_words, void* stream) {
  if (!key_cache || !value_cache || !block_ids || !sink) return INT8KV_E_NULL;
  if (num_kv_heads != kProbeWaves || num_ranges <= 0 || num_ranges > 65535 ||
      tiles_per_range <= 0 || num_blocks <= 0 ||
      block_id_count != 2LL * num_ranges * tiles_per_range ||
      sink_words < (int64_t)num_ranges * kProbeWaves * kWave)
    return INT8KV_E_SHAPE;
  if (((uintptr_t)key_cache % 16) != 0 || ((uintptr_t)value_cache % 16) != 0)
    return INT8KV_E_STRIDE;
  constexpr int HD = 128, kBlock = 16;
  DecodeArgs a{};
  a.kc = static_cast<const char*>(key_cache);
  a.vc = static_cast<const char*>(value_cache);
  a.kc_sh = a.vc_sh = HD;                              // [blocks, 16, Hkv, 128] int8
  a.kc_ss = a.vc_ss = (int64_t)num_kv_heads * HD;
  a.kc_sb = a.vc_sb = (int64_t)kBlock * num_kv_heads * HD;
  a.bt = block_ids;                                    // [num_ranges, 2 x tiles] int32
  a.bt_sb = 2LL * tiles_per_range;
  a.bt_sl = 1;
  a.bt_is64 = 0;
  a.num_blocks = num_blocks;
  a.block_shift = 4;
  a.head_dim = HD;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)num_ranges), block(kProbeWaves * kWave);
  if (non_temporal)
    hipLaunchKernelGGL((probe_decode_kernel<true>), grid, block, 0, s, a, tiles_per_range, sink);
  else
    hipLaunchKernelGGL((probe_decode_kernel<false>), grid, block, 0, s, a, tiles_per_range, sink);
  return (int)hipGetLastError();
}

extern "C" int int8kv_probe_clock(uint64_t* out, int32_t workgroups, uint32_t ticks,
                                  void* stream) {
  if (!out) return INT8KV_E_NULL;
  if (workgroups < 1 || workgroups > 65535 || ticks < 1 || ticks > 1000000) return INT8KV_E_SHAPE;
  if (((uintptr_t)out % 8) != 0) return INT8KV_E_STRIDE;
  hipLaunchKernelGGL(probe_clock_kernel, dim3((unsigned)workgroups), dim3(kWave), 0,
                     static_cast<hipStream_t>(stream), out, ticks);
  return (int)hipGetLastError();
}
