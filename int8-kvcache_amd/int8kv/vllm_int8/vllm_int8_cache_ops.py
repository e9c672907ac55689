"""vllm_int8/vllm_int8_cache_ops.py counterpart: the write operations (HIP kernels)."""

from ..cache_ops import (  # noqa: F401
    allocate_int8_kv_cache,
    dequantize_int8_cache,
    print_int8_cache_memory,
    reshape_and_cache_int8,
    runtime_int8_cache_write,
    tensor_nbytes,
)
