// The paged decode kernels for one cache type (bf16) at head_dims below the kernels' HD (a
// multiple of 16 other than 64, 128 and 256: 16-48, 80-112, 144-240), instantiated here so that
// they compile in parallel with the others (see paged_decode_kernels.h).

#include "paged_decode_kernels.h"

namespace int8kv {

int launch_cache_bf16_pad(const DecodeArgs& a, const HostPlan& hp, int query_dtype,
                          uint32_t flags, hipStream_t s) {
  return launch_q<kBF16, true>(a, hp, query_dtype, flags, s);
}

}  // namespace int8kv
