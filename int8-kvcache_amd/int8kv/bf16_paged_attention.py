"""BF16 PagedAttention decode (drop-in for src/triton_ops/bf16_paged_attention.py).

Same kernel family as the INT8 path with the dequantisation compiled out: the cache operands
feed the bf16 (or fp16) matrix cores directly.  Signature and output convention follow
src/triton_ops/bf16_paged_attention.py:118-165 (output shaped and typed like ``query``).
"""

from __future__ import annotations

import torch

from . import _decode, _ext, _lib


def bf16_paged_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    *,
    num_splits: int | None = None,
) -> torch.Tensor:
    """Paged decode on a 16-bit KV cache [num_blocks, BS, Hkv, D] (bf16 or fp16).

    ``num_splits`` (not in the reference's signature; keyword only) has int8_paged_attention's
    meaning: None automatic, 1 a single pass, S >= 2 S splits per sequence."""
    ext = _ext.module()
    if ext is not None and not _decode.DEBUG_CHECKS:
        return ext.bf16_paged_attention(query, key_cache, value_cache, block_tables, seq_lens,
                                        num_splits)
    assert query.ndim == 3 and key_cache.ndim == 4 and value_cache.ndim == 4
    assert block_tables.ndim == 2 and seq_lens.ndim == 1
    assert query.dtype in _decode.QUERY_DTYPES
    assert key_cache.dtype in (torch.bfloat16, torch.float16)
    assert value_cache.dtype == key_cache.dtype
    assert block_tables.dtype in (torch.int32, torch.int64)
    assert seq_lens.dtype in (torch.int32, torch.int64)
    B, Hq, D = query.shape
    num_blocks, block_size, Hkv, cache_D = key_cache.shape
    assert value_cache.shape == key_cache.shape
    assert cache_D == D and Hq % Hkv == 0
    assert _decode.head_dim_ok(D), _decode.HEAD_DIM_TEXT
    assert block_tables.shape[0] == B and seq_lens.numel() == B
    assert key_cache.stride(-1) == 1 and value_cache.stride(-1) == 1
    dev = query.device
    assert query.is_cuda, "bf16_paged_attention needs GPU tensors"
    assert (key_cache.device == dev and value_cache.device == dev and block_tables.device == dev
            and seq_lens.device == dev), "all tensors must be on one device (the GPU)"
    if _decode.DEBUG_CHECKS:
        _decode.debug_check(block_tables, seq_lens, num_blocks, block_size, False)
    ranges, split_flags = _decode.split_request(B, num_splits)
    output = torch.empty((B, Hq, D), device=query.device, dtype=query.dtype)
    return _decode.paged_decode(
        query, key_cache, value_cache, block_tables, seq_lens, None, None, output, ranges,
        _lib.DECODE_ALL | split_flags,
    )
