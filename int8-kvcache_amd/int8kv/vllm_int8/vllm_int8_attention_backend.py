"""vLLM attention-backend form of the INT8 decode (counterpart of
vllm_int8/vllm_int8_attention_backend.py).

As in the reference module, vLLM is imported at the top.  ``INT8PagedAttentionBackend`` is what
a caller registers with vLLM (name "INT8_PAGED_ATTENTION", implementation class
``INT8PagedAttentionImpl``, :81-87); the implementation decodes with ``int8_paged_attention``
(HIP) on the layer's cache from the pool: a ``LayerInt8Cache`` of the cache manager, or, as the
reference's early patch stored it, a dict with "k", "v", "k_scale" and "v_scale".
"""

from __future__ import annotations

from vllm.v1.attention.backend import AttentionBackend, AttentionImpl

from ..int8_paged_attention import int8_paged_attention
from .cache_manager import INT8_CACHE_POOL


class INT8AttentionMetadata:
    """Decode metadata: block_tables [B, W] and seq_lens [B]."""

    def __init__(self, block_tables, seq_lens):
        self.block_tables = block_tables
        self.seq_lens = seq_lens


def _layer_cache(layer_name):
    entry = INT8_CACHE_POOL[layer_name]
    if isinstance(entry, dict):
        return entry["k"], entry["v"], entry["k_scale"], entry["v_scale"]
    return entry.key_cache, entry.value_cache, entry.k_scale, entry.v_scale


class INT8PagedAttentionImpl(AttentionImpl):
    """Decode-only attention over the layer's INT8 paged cache (:30-78)."""

    def __init__(self, layer_name, num_heads, head_size, num_kv_heads, scale, **kwargs):
        self.layer_name = layer_name
        self.num_heads = num_heads
        self.head_size = head_size
        self.num_kv_heads = num_kv_heads
        self.scale = scale

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output):
        """query [tokens, Hq, D] (a 2-D query is one token); ``output`` receives the result."""
        k_cache, v_cache, k_scale, v_scale = _layer_cache(self.layer_name)
        q = query.unsqueeze(0) if query.ndim == 2 else query
        out = int8_paged_attention(q, k_cache, v_cache, attn_metadata.block_tables,
                                   attn_metadata.seq_lens, k_scale, v_scale)
        output.copy_(out.reshape_as(output))
        return output


class INT8PagedAttentionBackend(AttentionBackend):
    """The backend a caller registers with vLLM for this implementation (:81-87)."""

    @staticmethod
    def get_name():
        return "INT8_PAGED_ATTENTION"

    @staticmethod
    def get_impl_cls():
        return INT8PagedAttentionImpl
