"""Algorithmic HBM bytes of the library's operators: what a call has to move at the least, the
numerator of the achieved-bandwidth figures the benchmark reports.

Decode (src/triton_ops/int8_paged_attention.py:683-769 and bf16_paged_attention.py:118-165, one
query token per sequence): every cached K and V element of each sequence's first L_b tokens read
once, the block-table entry of every block a sequence covers, the query read and the output
written once, one length per sequence, and for an INT8 cache its two per-kv-head scale vectors.

Cache write (src/triton_ops/int8_cache_write.py:85-149): every valid token's K and V rows read in
the source dtype and written as int8, the slot index of every row (valid or not), and the two
scale vectors; the dynamic per-(token, head) write (vllm_int8/vllm_int8_cache_ops.py) reads no
scales and writes one fp32 scale per (token, kv head) for K and for V instead.
"""

from __future__ import annotations

import numpy as np


def decode_bytes(seq_lens, num_kv_heads: int, head_dim: int, cache_elem: int, batch: int,
                 num_q_heads: int, q_elem: int = 2, block_size: int = 16) -> int:
    """Bytes of one decode call.  cache_elem: 1 (INT8 cache) or 2 (BF16/FP16); q_elem: bytes
    per query/output element."""
    lens = np.clip(np.asarray(seq_lens, dtype=np.int64), 0, None)
    tokens = int(lens.sum())
    blocks = int((-(-lens // block_size)).sum())
    per_token = 2 * num_kv_heads * head_dim * cache_elem  # K and V
    query_and_out = batch * num_q_heads * head_dim * q_elem * 2
    scales = 2 * num_kv_heads * 4 if cache_elem == 1 else 0
    return tokens * per_token + 4 * blocks + query_and_out + 4 * batch + scales


def write_bytes(valid_tokens: int, slot_rows: int, num_kv_heads: int, head_dim: int,
                src_elem: int = 2, slot_elem: int = 8, dynamic: bool = False) -> int:
    """Bytes of one cache write of ``valid_tokens`` tokens with ``slot_rows`` entries in the slot
    mapping (valid tokens plus the padding slots the write skips)."""
    row = num_kv_heads * head_dim
    kv = valid_tokens * row * 2 * (src_elem + 1)  # K and V: read in the source dtype, int8 out
    scales = valid_tokens * num_kv_heads * 4 * 2 if dynamic else 2 * num_kv_heads * 4
    return kv + slot_rows * slot_elem + scales
