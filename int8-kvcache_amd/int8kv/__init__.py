"""int8kv: MI355X-native static per-head INT8 KV cache (write + PagedAttention decode).

Drop-in counterparts of the reference operators (cjsmt/Int8-kvcache, src/triton_ops/):

    int8_kv_cache_write      src/triton_ops/int8_cache_write.py:85-149
    int8_paged_attention     src/triton_ops/int8_paged_attention.py:683-769
    bf16_paged_attention     src/triton_ops/bf16_paged_attention.py:118-165

All compute runs in libint8kv.so (hand-written HIP for gfx950); there is no other backend.
"""

from .bf16_paged_attention import bf16_paged_attention
from .int8_cache_write import dequantize_paged_cache_for_debug, int8_kv_cache_write
from .int8_paged_attention import int8_paged_attention

__all__ = [
    "int8_kv_cache_write",
    "dequantize_paged_cache_for_debug",
    "int8_paged_attention",
    "bf16_paged_attention",
]

__version__ = "0.1.0"
