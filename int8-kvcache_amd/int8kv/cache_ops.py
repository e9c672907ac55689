"""INT8 KV-cache write operations used by the vLLM integration layer.

Drop-in counterparts of vllm_int8/vllm_int8_cache_ops.py (cjsmt/Int8-kvcache):

    reshape_and_cache_int8    :134-210  dynamic per-(token, head) scales, HIP kernel
    allocate_int8_kv_cache    :213-247  int8 K/V caches + fp32 scale caches
    dequantize_int8_cache     :250-256  debug dequantisation
    tensor_nbytes / print_int8_cache_memory  :259-277
    runtime_int8_cache_write  :281-306  static per-head write (int8kv_cache_write)

The write kernels run in libint8kv.so; there is no other backend.
"""

from __future__ import annotations

import torch

from . import _decode, _lib
from .int8_cache_write import int8_kv_cache_write

_SRC_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _aligned16(t: torch.Tensor) -> bool:
    e = t.element_size()
    return (t.data_ptr() % 16 == 0 and t.stride(-1) == 1 and (t.stride(0) * e) % 16 == 0
            and (t.stride(1) * e) % 16 == 0)


def reshape_and_cache_int8(
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    k_scale_cache: torch.Tensor,
    v_scale_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
) -> None:
    """Dynamic INT8 quantisation of K/V [T, Hkv, D] into paged caches [NB, BS, Hkv, D] with one
    fp32 scale per (token, head) in k/v_scale_cache [NB, BS, Hkv].

    scale = max(absmax / 127, 1e-6); code = round_half_away(clamp(x / scale, -127, 127));
    slots < 0 are skipped (vllm_int8/vllm_int8_cache_ops.py:13-131).
    """
    # Validation mirrors vllm_int8/vllm_int8_cache_ops.py:143-170.
    assert key.is_cuda and value.is_cuda and key_cache.is_cuda and value_cache.is_cuda
    assert slot_mapping.is_cuda
    assert key.ndim == 3 and value.ndim == 3 and key.shape == value.shape
    num_tokens, num_kv_heads, head_dim = key.shape
    assert key_cache.ndim == 4 and value_cache.ndim == 4
    assert key_cache.dtype == torch.int8 and value_cache.dtype == torch.int8
    assert k_scale_cache.dtype == torch.float32 and v_scale_cache.dtype == torch.float32
    assert slot_mapping.numel() == num_tokens
    num_blocks, block_size, cache_heads, cache_dim = key_cache.shape
    assert cache_heads == num_kv_heads and cache_dim == head_dim
    assert value_cache.shape == key_cache.shape
    expected_scale_shape = (num_blocks, block_size, num_kv_heads)
    assert tuple(k_scale_cache.shape) == expected_scale_shape
    assert tuple(v_scale_cache.shape) == expected_scale_shape
    assert key.dtype in _SRC_DTYPES and value.dtype in _SRC_DTYPES
    assert slot_mapping.dtype in (torch.int32, torch.int64)
    assert key_cache.stride(-1) == 1 and value_cache.stride(-1) == 1
    dev = key.device
    assert all(t.device == dev for t in (value, key_cache, value_cache, k_scale_cache,
                                         v_scale_cache, slot_mapping))
    if num_tokens == 0:
        return
    if _decode.DEBUG_CHECKS:
        _decode.debug_check_slots(slot_mapping, num_blocks, block_size)
    if value.dtype != key.dtype:
        key, value = key.float(), value.float()
    if not _aligned16(key):
        key = _lib.aligned_rows(key)
    if not _aligned16(value):
        value = _lib.aligned_rows(value)
    slot_mapping = slot_mapping.contiguous()
    status = _lib.load().int8kv_dynamic_cache_write(
        key.data_ptr(), value.data_ptr(), _lib.DTYPE_CODE[key.dtype], num_tokens, num_kv_heads,
        head_dim, _lib.strides(key), _lib.strides(value), key_cache.data_ptr(),
        value_cache.data_ptr(), num_blocks, block_size, _lib.strides(key_cache),
        _lib.strides(value_cache), k_scale_cache.data_ptr(), v_scale_cache.data_ptr(),
        _lib.strides(k_scale_cache), _lib.strides(v_scale_cache), slot_mapping.data_ptr(),
        _lib.DTYPE_CODE[slot_mapping.dtype], _lib.stream_handle(dev))
    _lib.check(status, "int8kv_dynamic_cache_write")


def allocate_int8_kv_cache(num_blocks: int, block_size: int, num_kv_heads: int, head_dim: int,
                           device: torch.device | str = "cuda"):
    """int8 K/V caches [NB, BS, Hkv, D] and fp32 scale caches [NB, BS, Hkv] (uninitialised)."""
    key_cache = torch.empty((num_blocks, block_size, num_kv_heads, head_dim), device=device,
                            dtype=torch.int8)
    value_cache = torch.empty_like(key_cache)
    k_scale_cache = torch.empty((num_blocks, block_size, num_kv_heads), device=device,
                                dtype=torch.float32)
    v_scale_cache = torch.empty_like(k_scale_cache)
    return key_cache, value_cache, k_scale_cache, v_scale_cache


def dequantize_int8_cache(cache: torch.Tensor, scale_cache: torch.Tensor) -> torch.Tensor:
    """Debug: int8 cache * per-(slot, head) scale -> float32."""
    assert cache.dtype == torch.int8
    return cache.float() * scale_cache[..., None]


def tensor_nbytes(x: torch.Tensor) -> int:
    return x.numel() * x.element_size()


def print_int8_cache_memory(key_cache, value_cache, k_scale_cache, v_scale_cache) -> None:
    kv_bytes = tensor_nbytes(key_cache) + tensor_nbytes(value_cache)
    scale_bytes = tensor_nbytes(k_scale_cache) + tensor_nbytes(v_scale_cache)
    print(f"K/V INT8 : {kv_bytes / 1024**2:.3f} MB")
    print(f"Scales    : {scale_bytes / 1024**2:.3f} MB")
    print(f"Total     : {(kv_bytes + scale_bytes) / 1024**2:.3f} MB")


def runtime_int8_cache_write(key, value, key_cache, value_cache, slot_mapping, k_scale,
                             v_scale) -> None:
    """Static per-head write used by the vLLM patches (vllm_int8_cache_ops.py:281-306)."""
    assert key.ndim == 3 and value.shape == key.shape
    assert key_cache.dtype == torch.int8 and value_cache.dtype == torch.int8
    assert slot_mapping.ndim == 1 and slot_mapping.numel() == key.shape[0]
    assert k_scale.shape == (key.shape[1],) and v_scale.shape == (key.shape[1],)
    int8_kv_cache_write(key, value, key_cache, value_cache, slot_mapping, k_scale, v_scale)
