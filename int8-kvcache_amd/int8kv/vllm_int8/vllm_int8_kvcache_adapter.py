"""Whole-cache conversion helpers (counterpart of vllm_int8/vllm_int8_kvcache_adapter.py).

Offline conversion and debug utilities, not the per-step path: a vLLM fused 16-bit KV cache
[blocks, Hkv, BS, 2*D] becomes INT8 K and V caches with one fp32 scale per kv head
(absmax / 127 over the whole cache, floored at 1e-6; codes rounded half to even and clamped to
[-127, 127]).  Plain torch on whatever device the tensors live on.
"""

from __future__ import annotations

import torch

_SOURCE_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _per_head_int8(x: torch.Tensor, head_dim_axis: int = 1):
    """Symmetric INT8 codes and fp32 scales, one scale per index of ``head_dim_axis``."""
    xf = x.float()
    others = tuple(d for d in range(x.ndim) if d != head_dim_axis)
    scale = (xf.abs().amax(dim=others) / 127.0).clamp_min(1e-6)
    shape = [1] * x.ndim
    shape[head_dim_axis] = -1
    codes = torch.round(xf / scale.reshape(shape)).clamp(-127, 127)
    return codes.to(torch.int8), scale.to(torch.float32)


def quantize_per_head(x: torch.Tensor):
    """x [B, H, S, D] (fp16 / bf16 / fp32) -> (int8 codes, scale [H]) (:6-20)."""
    assert x.ndim == 4 and x.dtype in _SOURCE_DTYPES, "expected a 16/32-bit float [B, H, S, D] tensor"
    return _per_head_int8(x, 1)


def convert_vllm_fused_kv_cache_to_int8(kv_cache: torch.Tensor):
    """Fused [blocks, Hkv, BS, 2*D] -> (k_int8, v_int8, k_scale [Hkv], v_scale [Hkv]) (:23-43)."""
    assert kv_cache.ndim == 4, "expected vLLM's fused cache [blocks, kv heads, block size, 2*D]"
    width = kv_cache.shape[-1]
    assert width % 2 == 0, f"the fused cache's last dimension ({width}) must hold K and V halves"
    k_int8, k_scale = quantize_per_head(kv_cache[..., : width // 2])
    v_int8, v_scale = quantize_per_head(kv_cache[..., width // 2:])
    return k_int8, v_int8, k_scale, v_scale


def dequant_kv_cache(x_int8: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """Debug: INT8 [B, H, S, D] -> fp32 with the per-head scale (:46-51)."""
    return x_int8.float() * scale.float().reshape(1, -1, 1, 1)
