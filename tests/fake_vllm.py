"""A minimal stand-in for the parts of vLLM the integration layer touches (test infrastructure).

Registers ``vllm.v1.attention.backends.triton_attn.TritonAttentionImpl`` and
``vllm.v1.attention.backend.AttentionImpl`` in sys.modules.  The fake TritonAttentionImpl keeps a
native 16-bit KV cache in vLLM 0.16's split layout [num_blocks, 2, block_size, Hkv, D] and
computes decode attention over it in float32 torch -- it plays vLLM's BF16 path in the tests.
"""

from __future__ import annotations

import math
import sys
import types
from contextlib import contextmanager

import torch


class AttentionImpl:
    pass


class AttentionBackend:
    pass


class TritonAttentionImpl:
    def __init__(self, num_heads: int, head_size: int, num_kv_heads: int):
        self.num_heads = num_heads
        self.head_size = head_size
        self.num_kv_heads = num_kv_heads
        self.forward_calls = 0

    def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping):
        nb, two, bs, hkv, d = kv_cache.shape
        flat_k = kv_cache[:, 0].reshape(nb * bs, hkv, d)
        flat_v = kv_cache[:, 1].reshape(nb * bs, hkv, d)
        slots = slot_mapping.reshape(-1).long()
        ok = slots >= 0
        flat_k[slots[ok]] = key[ok].to(kv_cache.dtype)
        flat_v[slots[ok]] = value[ok].to(kv_cache.dtype)
        kv_cache[:, 0] = flat_k.view(nb, bs, hkv, d)
        kv_cache[:, 1] = flat_v.view(nb, bs, hkv, d)

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output,
                output_scale=None, output_block_scale=None):
        """Decode attention in float32 over the native cache (one query token per sequence)."""
        self.forward_calls += 1
        nb, _, bs, hkv, d = kv_cache.shape
        g = query.shape[1] // hkv
        bt = attn_metadata.block_table
        lens = attn_metadata.seq_lens.tolist()
        for b, L in enumerate(lens):
            n = (L + bs - 1) // bs
            blocks = bt[b, :n].long()
            k = kv_cache[blocks, 0].reshape(n * bs, hkv, d)[:L].float()
            v = kv_cache[blocks, 1].reshape(n * bs, hkv, d)[:L].float()
            k = k.repeat_interleave(g, dim=1)  # [L, Hq, D]
            v = v.repeat_interleave(g, dim=1)
            q = query[b].float()  # [Hq, D]
            s = (k * q[None]).sum(-1) / math.sqrt(d)  # [L, Hq]
            p = torch.softmax(s, dim=0)
            output[b] = (p[..., None] * v).sum(0).to(output.dtype)
        return output


@contextmanager
def installed():
    """Registers the fake modules for the duration of the block."""
    names = ["vllm", "vllm.v1", "vllm.v1.attention", "vllm.v1.attention.backends",
             "vllm.v1.attention.backends.triton_attn", "vllm.v1.attention.backend"]
    saved = {n: sys.modules.get(n) for n in names}
    mods = {n: types.ModuleType(n) for n in names}
    for n in names:
        mods[n].__path__ = []
    mods["vllm.v1.attention.backends.triton_attn"].TritonAttentionImpl = TritonAttentionImpl
    mods["vllm.v1.attention.backend"].AttentionImpl = AttentionImpl
    mods["vllm.v1.attention.backend"].AttentionBackend = AttentionBackend
    sys.modules.update(mods)
    original = (TritonAttentionImpl.do_kv_cache_update, TritonAttentionImpl.forward)
    try:
        yield mods
    finally:
        TritonAttentionImpl.do_kv_cache_update, TritonAttentionImpl.forward = original
        for n, m in saved.items():
            if m is None:
                sys.modules.pop(n, None)
            else:
                sys.modules[n] = m
