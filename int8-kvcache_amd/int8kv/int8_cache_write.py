"""Static per-head INT8 KV-cache write (drop-in for src/triton_ops/int8_cache_write.py).

``int8_kv_cache_write`` keeps the reference signature and validation
(src/triton_ops/int8_cache_write.py:85-119) and launches the gfx950 kernel of libint8kv.so on
torch's current stream.  Numerics: ``clamp(rint(x / max(scale, 1e-6)), -127, 127)`` with an IEEE
fp32 quotient and round-half-to-even, i.e. bit-exact to the reference's torch path
(src/quant.py:37-40, src/triton_ops/int8_cache_write.py:172-181).
"""

from __future__ import annotations

import torch

from . import _decode, _ext, _lib
from .torch_reference import torch_int8_kv_cache_write_reference  # noqa: F401  (reference checker)

_SRC_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _aligned16(t: torch.Tensor) -> bool:
    e = t.element_size()
    return (
        t.data_ptr() % 16 == 0
        and t.stride(-1) == 1
        and (t.stride(0) * e) % 16 == 0
        and (t.stride(1) * e) % 16 == 0
    )


def int8_kv_cache_write(
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale: torch.Tensor,
    v_scale: torch.Tensor,
    num_warps: int = 4,
    num_stages: int = 2,
) -> None:
    """Quantise K/V [T, Hkv, D] with static per-head scales into the paged int8 caches.

    key/value: [T, Hkv, D] fp16/bf16/fp32; key_cache/value_cache: [num_blocks, BS, Hkv, D] int8;
    slot_mapping: [T] int32/int64 (slot = block * BS + offset; slot < 0 is skipped);
    k_scale/v_scale: [Hkv].  ``num_warps``/``num_stages`` are accepted for signature
    compatibility and ignored (the launch shape is fixed by the kernel design).
    """
    ext = _ext.module()
    if ext is not None and not _decode.DEBUG_CHECKS:
        # The same checks, conversions and launch in one call of the torch extension.
        ext.int8_kv_cache_write(key, value, key_cache, value_cache, slot_mapping, k_scale, v_scale)
        return None
    # Validation mirrors src/triton_ops/int8_cache_write.py:100-115.
    assert key.ndim == 3 and value.ndim == 3
    assert key_cache.ndim == 4 and value_cache.ndim == 4
    assert key.shape == value.shape and key_cache.shape == value_cache.shape
    assert key_cache.dtype == torch.int8 and value_cache.dtype == torch.int8
    assert key.dtype in _SRC_DTYPES
    assert value.dtype in _SRC_DTYPES
    num_tokens, num_kv_heads, head_dim = key.shape
    num_blocks, block_size, cache_num_kv_heads, cache_head_dim = key_cache.shape
    assert cache_num_kv_heads == num_kv_heads and cache_head_dim == head_dim
    assert slot_mapping.ndim == 1 and slot_mapping.numel() == num_tokens
    assert k_scale.ndim == 1 and v_scale.ndim == 1
    assert k_scale.numel() == num_kv_heads and v_scale.numel() == num_kv_heads
    assert slot_mapping.dtype in (torch.int32, torch.int64)
    dev = key.device
    assert key.is_cuda, "int8_kv_cache_write needs GPU tensors"
    assert (value.device == dev and key_cache.device == dev and value_cache.device == dev
            and slot_mapping.device == dev and k_scale.device == dev and v_scale.device == dev), \
        "all tensors must be on one device (the GPU)"
    assert key_cache.stride(-1) == 1 and value_cache.stride(-1) == 1

    if num_tokens == 0:
        return
    if _decode.DEBUG_CHECKS:
        _decode.debug_check_slots(slot_mapping, num_blocks, block_size)
    if value.dtype != key.dtype:
        # One source type per launch; widening to fp32 is exact, so the quotients are unchanged.
        key, value = key.float(), value.float()
    if not _aligned16(key):
        key = _lib.aligned_rows(key)
    if not _aligned16(value):
        value = _lib.aligned_rows(value)
    if k_scale.dtype != torch.float32 or not k_scale.is_contiguous():
        k_scale = k_scale.to(torch.float32).contiguous()
    if v_scale.dtype != torch.float32 or not v_scale.is_contiguous():
        v_scale = v_scale.to(torch.float32).contiguous()
    if not slot_mapping.is_contiguous():
        slot_mapping = slot_mapping.contiguous()

    lib = _lib.load()
    status = lib.int8kv_cache_write(
        key.data_ptr(),
        value.data_ptr(),
        _lib.DTYPE_CODE[key.dtype],
        num_tokens,
        num_kv_heads,
        head_dim,
        _lib.strides(key),
        _lib.strides(value),
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        num_blocks,
        block_size,
        _lib.strides(key_cache),
        _lib.strides(value_cache),
        slot_mapping.data_ptr(),
        _lib.DTYPE_CODE[slot_mapping.dtype],
        k_scale.data_ptr(),
        v_scale.data_ptr(),
        _lib.stream_handle(dev),
    )
    _lib.check(status, "int8kv_cache_write")


def dequantize_paged_cache_for_debug(cache: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """Debug helper: int8 cache [NB, BS, Hkv, D] * scale[Hkv] -> float32 (on the cache's device).

    Same contract as src/triton_ops/int8_cache_write.py:186-189.
    """
    assert cache.dtype == torch.int8
    return cache.float() * scale[None, None, :, None].float()
