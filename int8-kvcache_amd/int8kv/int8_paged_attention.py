"""INT8 PagedAttention decode (drop-in for src/triton_ops/int8_paged_attention.py).

``int8_paged_attention`` keeps the reference signature, keyword semantics and validation
(src/triton_ops/int8_paged_attention.py:683-769) and runs the gfx950 kernel family of
libint8kv.so.  Differences that a caller can observe:

* No host synchronisation: the reference's ``seq_lens.min()/max().item()`` checks (:720-723)
  only run when the environment variable INT8KV_DEBUG=1 is set.  The kernel bounds every
  sequence by ``block_tables.shape[1] * block_size`` instead and writes 0 for empty sequences.
* Work split: the kernel cuts the batch's token stream (all sequences' 32-token tiles in batch
  order) into equal ranges, one workgroup each, so ragged batches are balanced; sequences cut
  by a range bound are combined by a merge pass.
* ``impl``: "v4" and "auto" run the group-shared kernels with the automatic layout; "v3" (one
  pass per query head and sequence in the reference, :393-504) runs a single pass: one
  workgroup per (sequence, kv head), whose waves share the sequence's tiles and combine their
  softmax states on chip (no partials, no merge kernel).  Any other value raises ValueError, as
  in the reference (:767-768).
* ``num_splits``: 1 is that single pass; S >= 2 runs S workgroups per (sequence, kv head), each
  over an equal share of the sequence's tiles, whose partials the merge kernel combines (the
  reference's grid (B, Hkv, S), :590-604; it splits the table's logical blocks, :156-162, this
  build the sequence's own tiles).  At most 64 splits are used.
* ``quantize_q=True`` quantises each (sequence, query head) row of q to int8 first, as the
  reference does (:137-146, :798-802): q_scale = max(absmax / 127, 1e-6),
  q8 = clamp(round_half_away_from_zero(q / q_scale), -127, 127), scores scaled by q_scale.
* ``num_warps`` is accepted and ignored.
"""

from __future__ import annotations

import torch

from . import _decode, _ext, _lib
from .torch_reference import torch_int8_paged_attention_reference  # noqa: F401  (reference checker)


def int8_paged_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    k_scale: torch.Tensor,
    v_scale: torch.Tensor,
    *,
    quantize_q: bool = False,
    num_warps: int = 4,
    impl: str = "auto",
    num_splits: int | None = None,
) -> torch.Tensor:
    """Paged decode on an INT8 KV cache.  Returns [B, Hq, D] in query.dtype."""
    ext = _ext.module()
    if ext is not None and not _decode.DEBUG_CHECKS:
        # The same checks, allocation and launch in one call of the torch extension.
        return ext.int8_paged_attention(query, key_cache, value_cache, block_tables, seq_lens,
                                        k_scale, v_scale, bool(quantize_q), impl, num_splits)
    # Validation mirrors src/triton_ops/int8_paged_attention.py:698-719.
    assert query.ndim == 3 and key_cache.ndim == 4 and value_cache.ndim == 4
    assert block_tables.ndim == 2 and seq_lens.ndim == 1
    assert query.dtype in _decode.QUERY_DTYPES
    assert key_cache.dtype == torch.int8 and value_cache.dtype == torch.int8
    assert block_tables.dtype in (torch.int32, torch.int64)
    assert seq_lens.dtype in (torch.int32, torch.int64)
    B, Hq, D = query.shape
    num_blocks, block_size, Hkv, cache_D = key_cache.shape
    assert value_cache.shape == key_cache.shape
    assert cache_D == D and Hq % Hkv == 0
    assert _decode.head_dim_ok(D), _decode.HEAD_DIM_TEXT
    assert block_tables.shape[0] == B and seq_lens.numel() == B
    assert k_scale.ndim == 1 and v_scale.ndim == 1
    assert k_scale.numel() == Hkv and v_scale.numel() == Hkv
    assert key_cache.stride(-1) == 1 and value_cache.stride(-1) == 1
    dev = query.device
    assert query.is_cuda, "int8_paged_attention needs GPU tensors"
    assert (key_cache.device == dev and value_cache.device == dev and block_tables.device == dev
            and seq_lens.device == dev and k_scale.device == dev and v_scale.device == dev), \
        "all tensors must be on one device (the GPU)"
    if impl not in ("auto", "v3", "v4"):
        raise ValueError(f"Unknown impl={impl!r}; expected 'auto', 'v3' or 'v4'")
    if _decode.DEBUG_CHECKS:
        _decode.debug_check(block_tables, seq_lens, num_blocks, block_size, True)

    if k_scale.dtype != torch.float32 or not k_scale.is_contiguous():
        k_scale = k_scale.to(torch.float32).contiguous()
    if v_scale.dtype != torch.float32 or not v_scale.is_contiguous():
        v_scale = v_scale.to(torch.float32).contiguous()
    if impl == "v3" and num_splits is None:
        num_splits = 1
    ranges, split_flags = _decode.split_request(B, num_splits)
    output = torch.empty((B, Hq, D), device=dev, dtype=query.dtype)
    flags = _lib.DECODE_ALL | split_flags | (_lib.DECODE_QUANTIZE_Q if quantize_q else 0)
    return _decode.paged_decode(
        query, key_cache, value_cache, block_tables, seq_lens, k_scale, v_scale, output, ranges,
        flags,
    )
