// The paged decode kernels for one cache type (bf16), instantiated here so that the cache types
// compile in parallel (see paged_decode_kernels.h).

#include "paged_decode_kernels.h"

namespace int8kv {

int launch_cache_bf16(const DecodeArgs& a, const HostPlan& hp, int query_dtype, uint32_t flags,
                      hipStream_t s) {
  return launch_q<kBF16, false>(a, hp, query_dtype, flags, s);
}

}  // namespace int8kv

// Measurement build only (empty otherwise): this unit's stamp buffer.
INT8KV_STAMPS_ACCESSORS(bf16)
