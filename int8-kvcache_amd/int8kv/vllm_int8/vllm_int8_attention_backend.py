"""vLLM attention-backend form of the INT8 decode (vllm_int8/vllm_int8_attention_backend.py).

Like the reference module, this imports vLLM at the top.  The layer's cache comes from the
cache manager's pool (LayerInt8Cache) or, as in the reference's early patch, a dict with
"k", "v", "k_scale", "v_scale".
"""

from __future__ import annotations

from vllm.v1.attention.backend import AttentionImpl  # noqa: F401  (vLLM is required here)

from ..int8_paged_attention import int8_paged_attention
from .cache_manager import INT8_CACHE_POOL


class INT8AttentionMetadata:
    """Decode metadata: block_tables, seq_lens."""

    def __init__(self, block_tables, seq_lens):
        self.block_tables = block_tables
        self.seq_lens = seq_lens


class INT8PagedAttentionImpl(AttentionImpl):
    def __init__(self, layer_name, num_heads, head_size, num_kv_heads, scale, **kwargs):
        self.layer_name = layer_name
        self.num_heads = num_heads
        self.head_size = head_size
        self.num_kv_heads = num_kv_heads
        self.scale = scale

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output):
        """query [num_tokens, heads, dim]; decode only (vllm_int8_attention_backend.py:46-78)."""
        cache = INT8_CACHE_POOL[self.layer_name]
        if isinstance(cache, dict):
            k_cache, v_cache, k_scale, v_scale = cache["k"], cache["v"], cache["k_scale"], cache["v_scale"]
        else:
            k_cache, v_cache, k_scale, v_scale = cache.key_cache, cache.value_cache, cache.k_scale, cache.v_scale
        if query.ndim == 2:
            query = query.unsqueeze(0)
        out = int8_paged_attention(query, k_cache, v_cache, attn_metadata.block_tables,
                                   attn_metadata.seq_lens, k_scale, v_scale)
        output.copy_(out.reshape_as(output))
        return output
