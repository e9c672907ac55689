"""Module-name alias of vllm_int8/vllm_int8_cache_ops.py: callers that import
``vllm_int8.vllm_int8_cache_ops`` (after ``int8kv.compat.install_reference_aliases(include_vllm_int8=True)``)
get the HIP write operations of ``int8kv.cache_ops`` under the reference's module path.  No code of
its own: the dynamic write, the runtime static write and the allocator live in ``int8kv.cache_ops``."""

from ..cache_ops import (  # noqa: F401
    allocate_int8_kv_cache,
    dequantize_int8_cache,
    print_int8_cache_memory,
    reshape_and_cache_int8,
    runtime_int8_cache_write,
    tensor_nbytes,
)
