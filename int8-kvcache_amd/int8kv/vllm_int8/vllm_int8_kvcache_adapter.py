"""Whole-cache conversion helpers (vllm_int8/vllm_int8_kvcache_adapter.py of the reference).

Split a vLLM fused BF16 KV cache [blocks, Hkv, BS, 2*D] into INT8 K/V with per-head fp32 scales.
These are offline conversion/debug utilities, not the per-step hot path, and run as plain torch
on whatever device the tensors live on.
"""

from __future__ import annotations

import torch


def quantize_per_head(x: torch.Tensor):
    """Per-kv-head symmetric INT8: x [B, H, S, D] -> (int8, scale [H]) (:6-20).

    scale = clamp(absmax over (B, S, D) / 127, 1e-6); codes = clamp(round_half_even(x/scale)).
    """
    assert x.ndim == 4
    assert x.dtype in (torch.float16, torch.bfloat16, torch.float32)
    scale = x.float().abs().amax(dim=(0, 2, 3)) / 127.0
    scale = torch.clamp(scale, min=1e-6)
    x_int8 = torch.clamp(torch.round(x.float() / scale[None, :, None, None]), -127, 127)
    return x_int8.to(torch.int8), scale.to(torch.float32)


def convert_vllm_fused_kv_cache_to_int8(kv_cache: torch.Tensor):
    """Fused [blocks, Hkv, BS, 2*D] -> (k_int8, v_int8, k_scale [Hkv], v_scale [Hkv]) (:23-43)."""
    assert kv_cache.ndim == 4
    hidden = kv_cache.shape[3]
    assert hidden % 2 == 0, "vLLM fused KV cache last dimension must be 2*head_dim"
    head_dim = hidden // 2
    k_int8, k_scale = quantize_per_head(kv_cache[..., :head_dim])
    v_int8, v_scale = quantize_per_head(kv_cache[..., head_dim:])
    return k_int8, v_int8, k_scale, v_scale


def dequant_kv_cache(x_int8: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """Debug: INT8 -> fp32 with a per-head broadcast scale (:46-51)."""
    return x_int8.float() * scale[None, :, None, None]
