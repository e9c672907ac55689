"""INT8 decode attention inside vLLM: a patch of ``TritonAttentionImpl.forward``.

Counterpart of the reference's vllm_int8/vllm_int8_attention_patch.py:140-334.  The public names
its drivers use are kept: ``apply_int8_attention_patch``, ``PatchMode`` and the counters
``ATTN_COMPARE_COUNT``, ``ATTN_METRICS``, ``ATTN_INT8_HITS``, ``ATTN_INT8_STATS``
(bench/run_qwen_case_final.py:129-137, scripts/08-09 of the reference read them).

How one patched forward call is routed:
  * the layer owns no INT8 cache, or the call is not a pure decode step (prefill and chunked
    prefill have more query tokens than sequences, or max_query_len > 1): vLLM's own forward;
  * mode "int8_only": int8_paged_attention (HIP) on the layer's INT8 cache, nothing else;
  * mode "shadow": vLLM's forward, then the INT8 result, compared with it; vLLM's output stays;
  * mode "takeover": as "shadow", but the INT8 result replaces vLLM's output.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal, Optional

import torch

from ..int8_paged_attention import int8_paged_attention
from .cache_manager import get_layer_cache, has_layer_cache

PatchMode = Literal["shadow", "takeover", "int8_only"]
MODES = ("shadow", "takeover", "int8_only")

_PATCHED = False
# Comparisons recorded per layer (shadow / takeover) and the metrics of each.
ATTN_COMPARE_COUNT: dict[str, int] = {}
ATTN_METRICS: dict[str, list] = {}
# Decode calls answered by the INT8 op alone (int8_only), per layer, and the batch sizes seen.
ATTN_INT8_HITS: dict[str, int] = {}
ATTN_INT8_STATS: dict[str, int] = {"last_batch": 0, "max_batch": 0}


@dataclass(frozen=True)
class DecodeStep:
    """The inputs of one pure decode step: a query row per sequence."""

    query: torch.Tensor  # [B, Hq, D]: the first B rows of vLLM's (possibly padded) query
    block_table: torch.Tensor  # [B, W], contiguous
    seq_lens: torch.Tensor  # [B], contiguous


def decode_step_of(query: torch.Tensor, attn_metadata) -> Optional[DecodeStep]:
    """The decode inputs of this forward call, or None when it is not a pure decode step.

    vLLM's Triton backend names the table ``block_table``; some wrappers say ``block_tables``.
    vLLM 0.16 pads the query, so ``num_actual_tokens`` (when present) counts the real rows.
    """
    if attn_metadata is None or query.ndim != 3:
        return None
    lens = getattr(attn_metadata, "seq_lens", None)
    table = getattr(attn_metadata, "block_table", None)
    if table is None:
        table = getattr(attn_metadata, "block_tables", None)
    if lens is None or table is None or table.ndim != 2:
        return None
    batch = lens.numel()
    if batch == 0 or table.shape[0] != batch:
        return None
    rows = getattr(attn_metadata, "num_actual_tokens", None)
    rows = query.shape[0] if rows is None else int(rows)
    longest_query = getattr(attn_metadata, "max_query_len", None)
    if rows != batch or (longest_query is not None and int(longest_query) != 1):
        return None
    return DecodeStep(query[:batch], table.contiguous(), lens.contiguous())


def agreement(test: torch.Tensor, ref: torch.Tensor) -> dict:
    """Cosine, relative L2 and mean absolute difference of two outputs, in float64."""
    x = test.detach().double().reshape(-1)
    y = ref.detach().double().reshape(-1)
    d = x - y
    denom = float(x.norm() * y.norm())
    return {
        "cosine": float(x @ y) / denom if denom > 0 else 0.0,
        "rel_l2": float(d.norm()) / max(float(y.norm()), 1e-12),
        "mae": float(d.abs().mean()) if d.numel() else 0.0,
    }


def _int8_attention(layer_name: str, step: DecodeStep) -> torch.Tensor:
    cache = get_layer_cache(layer_name)
    return int8_paged_attention(step.query, cache.key_cache, cache.value_cache, step.block_table,
                                step.seq_lens, cache.k_scale, cache.v_scale, quantize_q=False)


def _require_finite(out: torch.Tensor, layer_name: str, error) -> None:
    for what, bad in (("NaN", torch.isnan), ("an infinity", torch.isinf)):
        if bool(bad(out).any()):
            raise error(f"{layer_name}: the INT8 decode output holds {what}")


def _write_rows(output: torch.Tensor, out8: torch.Tensor) -> None:
    n = out8.shape[0]
    output[:n].copy_(out8.reshape_as(output[:n]))


def _check_mode(mode) -> None:
    if mode not in MODES:
        raise ValueError(f"mode must be one of {MODES}, not {mode!r}")


def make_patched_forward(original_forward, mode: PatchMode = "shadow", verbose_layer: int = 0,
                         max_compare_calls: int = 8):
    """A forward method that routes decode steps as the module docstring describes and calls
    ``original_forward`` (vLLM's) otherwise.  ``verbose_layer``: the layer index whose first
    ``max_compare_calls`` comparisons are printed; in "int8_only" mode any value >= 0 also turns
    on the NaN / infinity check of the INT8 output (RuntimeError)."""
    _check_mode(mode)
    watched = f"layers.{verbose_layer}."

    def patched_forward(self, layer, query, key, value, kv_cache, attn_metadata, output,
                        output_scale=None, output_block_scale=None):
        name = getattr(layer, "layer_name", None)
        step = None
        if name is not None and has_layer_cache(name):
            step = decode_step_of(query, attn_metadata)
        if step is None:
            return original_forward(self, layer, query, key, value, kv_cache, attn_metadata,
                                    output, output_scale=output_scale,
                                    output_block_scale=output_block_scale)
        batch = step.seq_lens.numel()
        if mode == "int8_only":
            out8 = _int8_attention(name, step)
            if verbose_layer >= 0:
                _require_finite(out8, name, RuntimeError)
            ATTN_INT8_HITS[name] = ATTN_INT8_HITS.get(name, 0) + 1
            ATTN_INT8_STATS["last_batch"] = batch
            ATTN_INT8_STATS["max_batch"] = max(ATTN_INT8_STATS.get("max_batch", 0), batch)
            _write_rows(output, out8)
            return output

        vllm_result = original_forward(self, layer, query, key, value, kv_cache, attn_metadata,
                                       output, output_scale=output_scale,
                                       output_block_scale=output_block_scale)
        vllm_rows = output.detach().reshape(query.shape)[:batch].clone()
        out8 = _int8_attention(name, step)
        record = agreement(out8, vllm_rows)
        lens = [int(x) for x in step.seq_lens.tolist()]
        record.update(batch=batch, seq_lens=lens, max_seq_len=max(lens))
        seen = ATTN_COMPARE_COUNT.get(name, 0)
        ATTN_COMPARE_COUNT[name] = seen + 1
        ATTN_METRICS.setdefault(name, []).append(record)
        if watched in name and seen < max_compare_calls:
            print(f"[int8kv {mode}] {name} batch={batch} longest={record['max_seq_len']}: "
                  f"cos {record['cosine']:.6f}, rel-L2 {record['rel_l2']:.3e}, "
                  f"mean|d| {record['mae']:.3e} vs vLLM")
        if mode == "shadow":
            return vllm_result
        _require_finite(out8, name, AssertionError)
        _write_rows(output, out8)
        return output

    return patched_forward


def apply_int8_attention_patch(*, mode: PatchMode = "shadow", verbose_layer: int = 0,
                               max_compare_calls: int = 8) -> None:
    """Installs the patched forward on vLLM's TritonAttentionImpl (once per process)."""
    global _PATCHED
    _check_mode(mode)
    if _PATCHED:
        raise RuntimeError("apply_int8_attention_patch(): TritonAttentionImpl.forward is already "
                           "patched in this process")
    from vllm.v1.attention.backends.triton_attn import TritonAttentionImpl

    TritonAttentionImpl.forward = make_patched_forward(TritonAttentionImpl.forward, mode,
                                                       verbose_layer, max_compare_calls)
    _PATCHED = True
    answer = {"shadow": "vLLM's (INT8 compared beside it)",
              "takeover": "INT8 (vLLM still computed for the comparison)",
              "int8_only": "INT8 only"}[mode]
    print(f"[int8kv] decode attention patched, mode {mode}: decode output is {answer}")
