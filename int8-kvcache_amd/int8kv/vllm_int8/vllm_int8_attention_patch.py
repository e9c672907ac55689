"""INT8 decode attention inside vLLM (vllm_int8/vllm_int8_attention_patch.py of the reference).

Patches ``TritonAttentionImpl.forward``.  Pure decode steps of layers that have an INT8 shadow
cache run ``int8_paged_attention`` (HIP); prefill and chunked prefill fall back to vLLM.
Modes: "shadow" (vLLM output kept, INT8 compared), "takeover" (INT8 output, vLLM still run for
the comparison), "int8_only" (INT8 output only).
"""

from __future__ import annotations

from typing import Literal

import torch
import torch.nn.functional as F

from ..int8_paged_attention import int8_paged_attention
from .cache_manager import get_layer_cache, has_layer_cache

PatchMode = Literal["shadow", "takeover", "int8_only"]

_PATCHED = False
ATTN_COMPARE_COUNT: dict[str, int] = {}
ATTN_METRICS: dict[str, list] = {}
# Decode steps that actually ran int8_paged_attention (int8_only / takeover).
ATTN_INT8_HITS: dict[str, int] = {}
ATTN_INT8_STATS: dict[str, int] = {"last_batch": 0, "max_batch": 0}


def _relative_l2(x: torch.Tensor, y: torch.Tensor) -> float:
    x, y = x.float(), y.float()
    return ((x - y).norm() / y.norm().clamp_min(1e-12)).item()


def _cosine(x: torch.Tensor, y: torch.Tensor) -> float:
    return F.cosine_similarity(x.float().reshape(-1), y.float().reshape(-1), dim=0).item()


def _mae(x: torch.Tensor, y: torch.Tensor) -> float:
    return (x.float() - y.float()).abs().mean().item()


def _get_block_table(attn_metadata):
    """vLLM's Triton metadata has block_table; some wrappers use block_tables (:65-70)."""
    bt = getattr(attn_metadata, "block_table", None)
    if bt is None:
        bt = getattr(attn_metadata, "block_tables", None)
    return bt


def _is_supported_decode(query, attn_metadata) -> bool:
    """True for pure decode steps: one query token per sequence (:73-114)."""
    if attn_metadata is None or query.ndim != 3:
        return False
    seq_lens = getattr(attn_metadata, "seq_lens", None)
    block_table = _get_block_table(attn_metadata)
    if seq_lens is None or block_table is None or block_table.ndim != 2:
        return False
    batch = int(seq_lens.numel())
    if batch <= 0 or block_table.shape[0] != batch:
        return False
    num_tokens = getattr(attn_metadata, "num_actual_tokens", None)
    if num_tokens is None:
        num_tokens = query.shape[0]
    if int(num_tokens) != batch:
        return False
    max_query_len = getattr(attn_metadata, "max_query_len", None)
    if max_query_len is not None and int(max_query_len) != 1:
        return False
    return True


def _run_int8_attention(layer, query, attn_metadata):
    """int8_paged_attention on the layer's shadow cache (:117-137)."""
    shadow = get_layer_cache(layer.layer_name)
    seq_lens = attn_metadata.seq_lens.contiguous()
    block_table = _get_block_table(attn_metadata).contiguous()
    num_tokens = getattr(attn_metadata, "num_actual_tokens", query.shape[0])
    query = query[: int(num_tokens)]
    return int8_paged_attention(query, shadow.key_cache, shadow.value_cache, block_table, seq_lens,
                                shadow.k_scale, shadow.v_scale, quantize_q=False)


def make_patched_forward(original_forward, mode: PatchMode = "shadow", verbose_layer: int = 0,
                         max_compare_calls: int = 8):
    """The patched forward around ``original_forward`` (:160-321)."""
    if mode not in ("shadow", "takeover", "int8_only"):
        raise ValueError(f"Unknown mode: {mode}")

    def patched_forward(self, layer, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                        kv_cache: torch.Tensor, attn_metadata, output: torch.Tensor,
                        output_scale=None, output_block_scale=None):
        layer_name = getattr(layer, "layer_name", None)
        if (layer_name is None or not has_layer_cache(layer_name)
                or not _is_supported_decode(query, attn_metadata)):
            return original_forward(self, layer, query, key, value, kv_cache, attn_metadata,
                                    output, output_scale=output_scale,
                                    output_block_scale=output_block_scale)
        if mode in ("shadow", "takeover"):
            bf16_result = original_forward(self, layer, query, key, value, kv_cache,
                                           attn_metadata, output, output_scale=output_scale,
                                           output_block_scale=output_block_scale)
            bf16_out = output.detach().clone().reshape(query.shape[0], query.shape[1],
                                                       query.shape[2])
            int8_out = _run_int8_attention(layer, query, attn_metadata)
            n = int8_out.shape[0]
            metrics = {
                "cosine": _cosine(int8_out, bf16_out[:n]),
                "rel_l2": _relative_l2(int8_out, bf16_out[:n]),
                "mae": _mae(int8_out, bf16_out[:n]),
                "batch": int(attn_metadata.seq_lens.numel()),
                "seq_lens": [int(x) for x in attn_metadata.seq_lens.tolist()],
                "max_seq_len": int(attn_metadata.seq_lens.max().item()),
            }
            count = ATTN_COMPARE_COUNT.get(layer_name, 0)
            ATTN_COMPARE_COUNT[layer_name] = count + 1
            ATTN_METRICS.setdefault(layer_name, []).append(metrics)
            if f"layers.{verbose_layer}." in layer_name and count < max_compare_calls:
                print(f"[INT8 Attention / {mode}] {layer_name}: cosine={metrics['cosine']:.6f} "
                      f"relL2={metrics['rel_l2']:.3e} MAE={metrics['mae']:.3e}")
            if mode == "shadow":
                return bf16_result
            # the reference asserts here (vllm_int8_attention_patch.py:297-298)
            if torch.isnan(int8_out).any() or torch.isinf(int8_out).any():
                raise AssertionError(f"non-finite INT8 attention output: {layer_name}")
            output[:n].copy_(int8_out.reshape_as(output[:n]))
            return output
        int8_out = _run_int8_attention(layer, query, attn_metadata)
        if verbose_layer >= 0:
            if torch.isnan(int8_out).any():
                raise RuntimeError(f"NaN in INT8 attention: {layer_name}")
            if torch.isinf(int8_out).any():
                raise RuntimeError(f"Inf in INT8 attention: {layer_name}")
        ATTN_INT8_HITS[layer_name] = ATTN_INT8_HITS.get(layer_name, 0) + 1
        batch_now = int(attn_metadata.seq_lens.numel())
        ATTN_INT8_STATS["last_batch"] = batch_now
        ATTN_INT8_STATS["max_batch"] = max(ATTN_INT8_STATS.get("max_batch", 0), batch_now)
        n = int8_out.shape[0]
        output[:n].copy_(int8_out.reshape_as(output[:n]))
        return output

    return patched_forward


def apply_int8_attention_patch(*, mode: PatchMode = "shadow", verbose_layer: int = 0,
                               max_compare_calls: int = 8) -> None:
    """Patches TritonAttentionImpl.forward (vllm_int8_attention_patch.py:140-334)."""
    global _PATCHED
    if mode not in ("shadow", "takeover", "int8_only"):
        raise ValueError(f"Unknown mode: {mode}")
    if _PATCHED:
        raise RuntimeError("Attention has already been patched in this Python process.")
    from vllm.v1.attention.backends.triton_attn import TritonAttentionImpl

    TritonAttentionImpl.forward = make_patched_forward(TritonAttentionImpl.forward, mode,
                                                       verbose_layer, max_compare_calls)
    _PATCHED = True
    print(f"INT8 ATTENTION PATCH ENABLED (mode: {mode})")
