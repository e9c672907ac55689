"""Shadow INT8 cache write inside vLLM (vllm_int8/vllm_shadow_cache_patch.py of the reference).

Patches ``TritonAttentionImpl.do_kv_cache_update``: vLLM's own BF16 write runs unchanged, then the
same K/V rows are quantised into the layer's INT8 cache with the static scales by
``int8_kv_cache_write`` (HIP).  The INT8 cache is allocated on the layer's first call with the
page geometry of vLLM's native cache.
"""

from __future__ import annotations

import torch

from ..int8_cache_write import int8_kv_cache_write
from .cache_manager import allocate_layer_cache, get_layer_cache, has_layer_cache
from .static_scales import get_layer_scales

_PATCHED = False
WRITE_CALL_COUNT: dict[str, int] = {}
NATIVE_CACHE_BYTES_BY_LAYER: dict[str, int] = {}


def _infer_native_page_dims(kv_cache: torch.Tensor, num_kv_heads: int):
    """(num_blocks, block_size) of vLLM's native KV cache (:26-43).

    Layouts: v0.26 fused [NB, Hkv, BS, 2*D]; v0.16 split [NB, 2, BS, Hkv, D];
    older split [2, NB, BS, Hkv, D].
    """
    if kv_cache.ndim == 4 and kv_cache.shape[1] == num_kv_heads:
        return int(kv_cache.shape[0]), int(kv_cache.shape[2])
    if kv_cache.ndim == 5 and kv_cache.shape[1] == 2:
        return int(kv_cache.shape[0]), int(kv_cache.shape[2])
    if kv_cache.ndim == 5 and kv_cache.shape[0] == 2:
        return int(kv_cache.shape[1]), int(kv_cache.shape[2])
    raise ValueError(f"Unsupported vLLM kv_cache shape {tuple(kv_cache.shape)} for Hkv={num_kv_heads}")


def make_patched_do_kv_cache_update(original, verbose_layer: int = 0):
    """The patched method around ``original`` (kept separate so it can be tested on its own)."""

    def patched_do_kv_cache_update(self, layer, key: torch.Tensor, value: torch.Tensor,
                                   kv_cache: torch.Tensor, slot_mapping: torch.Tensor):
        original(self, layer, key, value, kv_cache, slot_mapping)
        layer_name = layer.layer_name
        if layer_name not in NATIVE_CACHE_BYTES_BY_LAYER:
            NATIVE_CACHE_BYTES_BY_LAYER[layer_name] = kv_cache.numel() * kv_cache.element_size()
        assert key.ndim == 3 and value.ndim == 3
        num_tokens, num_kv_heads, head_dim = key.shape
        num_blocks, block_size = _infer_native_page_dims(kv_cache, num_kv_heads)
        if not has_layer_cache(layer_name):
            k_scale, v_scale = get_layer_scales(layer_name, key.device)
            allocate_layer_cache(layer_name=layer_name, num_blocks=num_blocks,
                                 block_size=block_size, num_kv_heads=num_kv_heads,
                                 head_dim=head_dim, k_scale=k_scale, v_scale=v_scale,
                                 device=key.device)
            if f"layers.{verbose_layer}." in layer_name:
                print(f"[INT8 Shadow] allocate {layer_name}: INT8 K/V "
                      f"{(num_blocks, block_size, num_kv_heads, head_dim)} next to native "
                      f"{tuple(kv_cache.shape)} {kv_cache.dtype}")
        shadow = get_layer_cache(layer_name)
        runtime_slots = slot_mapping.reshape(-1).contiguous()
        assert runtime_slots.numel() == num_tokens, f"slot_mapping={runtime_slots.shape}, key={key.shape}"
        int8_kv_cache_write(key, value, shadow.key_cache, shadow.value_cache, runtime_slots,
                            shadow.k_scale, shadow.v_scale)
        WRITE_CALL_COUNT[layer_name] = WRITE_CALL_COUNT.get(layer_name, 0) + 1

    return patched_do_kv_cache_update


def apply_shadow_cache_patch(verbose_layer: int = 0) -> None:
    """Patches TritonAttentionImpl.do_kv_cache_update (vllm_shadow_cache_patch.py:46-191)."""
    global _PATCHED
    if _PATCHED:
        print("[INT8 Shadow] already patched")
        return
    from vllm.v1.attention.backends.triton_attn import TritonAttentionImpl

    TritonAttentionImpl.do_kv_cache_update = make_patched_do_kv_cache_update(
        TritonAttentionImpl.do_kv_cache_update, verbose_layer)
    _PATCHED = True
    print("[INT8 Shadow] TritonAttentionImpl.do_kv_cache_update patched.")
