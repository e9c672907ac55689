"""Shared launcher of the paged decode kernel family (INT8 and 16-bit caches)."""

from __future__ import annotations

import math
import os
import threading

import torch

from . import _ext, _lib

QUERY_DTYPES = (torch.float16, torch.bfloat16, torch.float32)

# head_dims the decode kernels run: multiples of 16 up to 256 (the reference pads any head_dim to a
# power of two under a mask, src/triton_ops/int8_paged_attention.py:556-558,588-589).
HEAD_DIM_TEXT = "head_dim must be a multiple of 16 from 16 to 256 (this build's decode kernels)"


def head_dim_ok(d: int) -> bool:
    return 16 <= d <= 256 and d % 16 == 0

# When set, the op also runs the reference's host-synchronising input checks
# (src/triton_ops/int8_paged_attention.py:720-723) and checks block ids; off by default because
# each check is a device-to-host copy.
DEBUG_CHECKS = os.environ.get("INT8KV_DEBUG", "0") not in ("", "0")


def _aligned16(t: torch.Tensor, dims) -> bool:
    e = t.element_size()
    if t.data_ptr() % 16 or t.stride(-1) != 1:
        return False
    return all((t.stride(d) * e) % 16 == 0 for d in dims)


MAX_RANGES = 1 << 20

# Decode workspaces reused across calls, one per (host thread, device, stream).  A call is two
# launches (decode, then merge) that read and write its workspace; calls from one thread on one
# stream are enqueued whole, one after the other, so they never interleave.  Two threads that
# enqueue on one stream can interleave their launches (thread B's decode between thread A's
# decode and merge), so each thread keeps its own.  A call under HIP-graph capture gets its own
# (allocated from the graph's pool), so a graph never shares memory with eager calls.
_WORKSPACES = threading.local()
_WS_BYTES: dict = {}


def _workspace_bytes(lib, Hq, Hkv, D, block_size, num_ranges) -> int:
    key = (Hq, Hkv, D, block_size, num_ranges)
    need = _WS_BYTES.get(key)
    if need is None:
        need = _WS_BYTES[key] = lib.int8kv_decode_workspace_bytes(Hq, Hkv, D, block_size, num_ranges)
    return need


def _cached_workspace(dev, stream: int, need: int) -> torch.Tensor:
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
    cache = getattr(_WORKSPACES, "by_stream", None)
    if cache is None:
        cache = _WORKSPACES.by_stream = {}
    key = (dev.index, stream)
    ws = cache.get(key)
    if ws is None or ws.numel() < need:
        ws = cache[key] = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
    return ws


MAX_SPLITS = 64  # workgroups per (sequence, kv head) the split layout's merge combines


def split_request(batch: int, num_splits) -> tuple[int, int]:
    """(num_ranges, flags) of int8kv_paged_decode for the reference's ``num_splits``
    (src/triton_ops/int8_paged_attention.py:590-604: grid (B, Hkv, S), split s over logical
    blocks [s n / S, (s + 1) n / S)): None = the library's automatic choice; 1 = a single pass,
    one workgroup per (sequence, kv head) with no partials and no merge
    (INT8KV_DECODE_PER_SEQUENCE); S >= 2 = S workgroups per (sequence, kv head) over equal
    shares of its tiles, combined by the merge kernel (INT8KV_DECODE_SPLIT_SEQUENCES with
    num_ranges = S x batch; at most 64 splits)."""
    if num_splits is None:
        return 0, 0
    s = int(num_splits)
    if s <= 1:
        return 0, _lib.DECODE_PER_SEQUENCE
    s = min(s, MAX_SPLITS)
    return min(MAX_RANGES, s * max(1, int(batch))), _lib.DECODE_SPLIT_SEQUENCES


def debug_check_slots(slot_mapping, num_blocks: int, block_size: int) -> None:
    """Host-side check of a write's slot_mapping (INT8KV_DEBUG=1): every non-negative slot lies
    inside the cache and appears once.  The write kernels skip out-of-range slots and give each
    token its own lanes, so two tokens with one slot would race on that cache row."""
    s = slot_mapping.to("cpu", torch.int64)
    s = s[s >= 0]
    assert bool((s < num_blocks * block_size).all()), "slot_mapping holds a slot beyond the cache"
    assert int(torch.unique(s).numel()) == int(s.numel()), \
        "slot_mapping repeats a slot: two tokens would write one cache row concurrently"


def debug_check(block_tables, seq_lens, num_blocks, block_size, require_positive) -> None:
    lens = seq_lens.to("cpu", torch.int64)
    if require_positive:
        assert int(lens.min()) > 0
    need = -(-int(lens.max()) // block_size) if lens.numel() else 0
    assert block_tables.shape[1] >= need
    bt = block_tables.to("cpu", torch.int64)
    for b, n in enumerate(lens.tolist()):
        ids = bt[b, : -(-n // block_size)]
        assert bool(((ids >= 0) & (ids < num_blocks)).all()), f"block id out of range in row {b}"


def paged_decode(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    k_scale,
    v_scale,
    out: torch.Tensor,
    num_ranges: int = 0,
    flags: int = _lib.DECODE_ALL,
    workspace: torch.Tensor | None = None,
    min_tiles: int = 0,
) -> torch.Tensor:
    """Launches int8kv_paged_decode on torch's current stream; returns ``out``."""
    ext = _ext.module()
    if ext is not None:
        return ext.paged_decode(query, key_cache, value_cache, block_tables, seq_lens, k_scale,
                                v_scale, out, num_ranges, flags, workspace, min_tiles)
    B, Hq, D = query.shape
    num_blocks, block_size, Hkv, _ = key_cache.shape
    width = block_tables.shape[1]
    dev = query.device
    if B == 0:
        return out
    if not _aligned16(query, (0, 1)):
        query = _lib.aligned_rows(query)
    if not seq_lens.is_contiguous():
        seq_lens = seq_lens.contiguous()
    lib = _lib.load()
    stream = _lib.stream_handle(dev)
    need = _workspace_bytes(lib, Hq, Hkv, D, block_size, num_ranges)
    if workspace is None or workspace.numel() < need:
        workspace = _cached_workspace(dev, stream, need)
    status = lib.int8kv_paged_decode(
        query.data_ptr(),
        _lib.DTYPE_CODE[query.dtype],
        B,
        Hq,
        D,
        _lib.strides(query),
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        _lib.DTYPE_CODE[key_cache.dtype],
        num_blocks,
        block_size,
        Hkv,
        _lib.strides(key_cache),
        _lib.strides(value_cache),
        block_tables.data_ptr(),
        _lib.DTYPE_CODE[block_tables.dtype],
        width,
        _lib.strides(block_tables),
        seq_lens.data_ptr(),
        _lib.DTYPE_CODE[seq_lens.dtype],
        k_scale.data_ptr() if k_scale is not None else None,
        v_scale.data_ptr() if v_scale is not None else None,
        1.0 / math.sqrt(D),
        out.data_ptr(),
        _lib.strides(out),
        workspace.data_ptr(),
        workspace.numel(),
        num_ranges,
        min_tiles,
        flags,
        stream,
    )
    _lib.check(status, "int8kv_paged_decode")
    return out
