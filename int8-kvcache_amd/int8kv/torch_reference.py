"""The reference's pure-torch checking helpers, under their names (checkers, not operators).

The reference ships two torch implementations next to its Triton operators for its own
correctness tests: ``torch_int8_kv_cache_write_reference``
(src/triton_ops/int8_cache_write.py:150-181) and ``torch_int8_paged_attention_reference``
(src/triton_ops/int8_paged_attention.py:776-814).  Its tests import them from the operator
modules, so the drop-in modules re-export these restatements.  Same arguments, same arithmetic
(the write divides by the scale as given, without the operators' 1e-6 floor, and rounds half to
even; the attention dequantises K/V with the per-head scales, optionally quantises q per
(sequence, head) with half-away rounding, and returns ``query.dtype``), vectorised per sequence
instead of the reference's per-element loops.  They run on whatever device their inputs are on.

No operator of this package calls them: the operators run only on libint8kv.so.
"""

from __future__ import annotations

import math

import torch


def torch_int8_kv_cache_write_reference(
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale: torch.Tensor,
    v_scale: torch.Tensor,
) -> None:
    """In-place: caches[slot // BS, slot % BS] = clamp(round(x / scale), -127, 127) for slot >= 0."""
    assert key.ndim == 3
    num_tokens, num_kv_heads, head_dim = key.shape
    block_size = key_cache.shape[1]
    slots = slot_mapping.to(torch.int64)
    keep = slots >= 0
    if not bool(keep.any()):
        return
    slots = slots[keep]
    blk, off = slots // block_size, slots % block_size
    for x, scale, cache in ((key, k_scale, key_cache), (value, v_scale, value_cache)):
        q = torch.clamp(torch.round(x[keep].float() / scale.float()[None, :, None]), -127, 127)
        cache[blk, off] = q.to(torch.int8)


def _round_half_away_from_zero(x: torch.Tensor) -> torch.Tensor:
    return torch.where(x >= 0, torch.floor(x + 0.5), -torch.floor(-x + 0.5))


def torch_int8_paged_attention_reference(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    k_scale: torch.Tensor,
    v_scale: torch.Tensor,
    *,
    quantize_q: bool = False,
) -> torch.Tensor:
    """[B, Hq, D] decode attention over the paged int8 caches, in ``query.dtype``."""
    B, Hq, D = query.shape
    _, block_size, Hkv, _ = key_cache.shape
    assert Hq % Hkv == 0
    group = Hq // Hkv
    kv_of = torch.arange(Hq, device=query.device) // group
    ks = k_scale.float().to(query.device)
    vs = v_scale.float().to(query.device)
    lens = seq_lens.to("cpu", torch.int64).tolist()
    outputs = []
    for b in range(B):
        T = int(lens[b])
        q = query[b].float()  # [Hq, D]
        if quantize_q:
            q_scale = torch.clamp(q.abs().amax(dim=-1, keepdim=True) / 127.0, min=1e-6)
            q = torch.clamp(_round_half_away_from_zero(q / q_scale), -127, 127) * q_scale
        nblk = -(-T // block_size)
        ids = block_tables[b, :nblk].to(torch.int64)
        k = key_cache[ids].float().reshape(nblk * block_size, Hkv, D)[:T] * ks[None, :, None]
        v = value_cache[ids].float().reshape(nblk * block_size, Hkv, D)[:T] * vs[None, :, None]
        k = k[:, kv_of]  # [T, Hq, D]
        v = v[:, kv_of]
        score = (k * q[None]).sum(-1) / math.sqrt(D)  # [T, Hq]
        p = torch.softmax(score, dim=0)
        outputs.append((p[:, :, None] * v).sum(0))
    return torch.stack(outputs, dim=0).to(query.dtype)
