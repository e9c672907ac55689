"""Shadow INT8 cache write inside vLLM: a patch of ``TritonAttentionImpl.do_kv_cache_update``.

Counterpart of the reference's vllm_int8/vllm_shadow_cache_patch.py:46-191; the public names its
drivers read are kept (``apply_shadow_cache_patch``, ``WRITE_CALL_COUNT``,
``NATIVE_CACHE_BYTES_BY_LAYER``, bench/run_qwen_case_final.py:133-204).  vLLM's own 16-bit write
runs unchanged; the same K/V rows then go through ``int8_kv_cache_write`` (HIP) into the layer's
INT8 cache, which is allocated on the layer's first call with the page geometry (number of
blocks, block size) of vLLM's native cache, so the two caches share block tables and slots.
"""

from __future__ import annotations

import torch

from ..int8_cache_write import int8_kv_cache_write
from .cache_manager import allocate_layer_cache, get_layer_cache, has_layer_cache
from .static_scales import get_layer_scales

_PATCHED = False
WRITE_CALL_COUNT: dict[str, int] = {}  # shadow writes per layer
NATIVE_CACHE_BYTES_BY_LAYER: dict[str, int] = {}  # bytes of vLLM's own cache per layer

# vLLM's native KV-cache layouts: (description, matches(shape, Hkv), (blocks axis, block-size axis)).
_NATIVE_LAYOUTS = (
    ("fused [NB, Hkv, BS, 2*D] (vLLM 0.26)", lambda s, h: len(s) == 4 and s[1] == h, (0, 2)),
    ("split [NB, 2, BS, Hkv, D] (vLLM 0.16)", lambda s, h: len(s) == 5 and s[1] == 2, (0, 2)),
    ("split [2, NB, BS, Hkv, D] (older vLLM)", lambda s, h: len(s) == 5 and s[0] == 2, (1, 2)),
)


def native_page_geometry(kv_cache: torch.Tensor, num_kv_heads: int) -> tuple:
    """(num_blocks, block_size) of vLLM's native cache for this layer."""
    shape = tuple(kv_cache.shape)
    for _, matches, (nb_axis, bs_axis) in _NATIVE_LAYOUTS:
        if matches(shape, num_kv_heads):
            return int(shape[nb_axis]), int(shape[bs_axis])
    known = "; ".join(desc for desc, _, _ in _NATIVE_LAYOUTS)
    raise ValueError(f"a vLLM KV cache of shape {shape} with {num_kv_heads} kv heads matches no "
                     f"known layout ({known})")


def _ensure_int8_cache(layer_name: str, key: torch.Tensor, kv_cache: torch.Tensor, loud: bool):
    if has_layer_cache(layer_name):
        return get_layer_cache(layer_name)
    _, num_kv_heads, head_dim = key.shape
    num_blocks, block_size = native_page_geometry(kv_cache, num_kv_heads)
    k_scale, v_scale = get_layer_scales(layer_name, key.device)
    cache = allocate_layer_cache(layer_name=layer_name, num_blocks=num_blocks,
                                 block_size=block_size, num_kv_heads=num_kv_heads,
                                 head_dim=head_dim, k_scale=k_scale, v_scale=v_scale,
                                 device=key.device)
    if loud:
        print(f"[int8kv shadow] {layer_name}: INT8 K/V caches "
              f"{tuple(cache.key_cache.shape)} beside vLLM's {tuple(kv_cache.shape)} "
              f"{kv_cache.dtype}")
    return cache


def make_patched_do_kv_cache_update(original, verbose_layer: int = 0):
    """A do_kv_cache_update that runs ``original`` (vLLM's write) and then the INT8 shadow write
    of the same rows.  ``verbose_layer``: the layer index whose cache allocation is printed."""
    watched = f"layers.{verbose_layer}."

    def patched_do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping):
        original(self, layer, key, value, kv_cache, slot_mapping)
        name = layer.layer_name
        NATIVE_CACHE_BYTES_BY_LAYER.setdefault(name, kv_cache.numel() * kv_cache.element_size())
        assert key.ndim == 3 and value.ndim == 3, "key/value must be [tokens, kv heads, head dim]"
        cache = _ensure_int8_cache(name, key, kv_cache, watched in name)
        slots = slot_mapping.reshape(-1).contiguous()
        assert slots.numel() == key.shape[0], \
            f"{slots.numel()} slots for {key.shape[0]} key rows"
        int8_kv_cache_write(key, value, cache.key_cache, cache.value_cache, slots, cache.k_scale,
                            cache.v_scale)
        WRITE_CALL_COUNT[name] = WRITE_CALL_COUNT.get(name, 0) + 1

    return patched_do_kv_cache_update


def apply_shadow_cache_patch(verbose_layer: int = 0) -> None:
    """Installs the shadow write on vLLM's TritonAttentionImpl; a second call changes nothing."""
    global _PATCHED
    if _PATCHED:
        return
    from vllm.v1.attention.backends.triton_attn import TritonAttentionImpl

    TritonAttentionImpl.do_kv_cache_update = make_patched_do_kv_cache_update(
        TritonAttentionImpl.do_kv_cache_update, verbose_layer)
    _PATCHED = True
    print("[int8kv shadow] vLLM cache writes now also fill the INT8 caches")
