"""PyTorch CPU restatement of the reference's decode path -- TEST INFRASTRUCTURE ONLY.

Only tests/ and bench.py's cpu_baseline leg may import this module: it is the CPU baseline
that the GPU kernels are reported against (timed on every host core) and a second checker.
The product (int8kv, libint8kv.so) never calls it.  It restates, in torch on CPU tensors:

    quant_kv_static_per_head   src/quant.py:37-40   round(x / scale) half to even, clamp
                                                    [-127, 127], int8
    write_paged                src/paged_cache.py:4-36 (the paged layout [NB, BS, Hkv, D];
                               here into a caller-given, shuffled block table, one sequence at
                               a time, as the benchmark harnesses place blocks)
    gather_sequence            src/paged_cache.py:39-59 (ragged: one sequence of its own length,
                               since the reference's gather stacks equal lengths only)
    expand_kv_for_gqa          src/attention_ref.py:11-16 (repeat_interleave over the kv heads)
    decode_attention_ref       src/attention_ref.py:19-28 (fp32 einsum scores / sqrt(D),
                               softmax, einsum with V)
    decode_step                the three above chained per sequence on the int8 cache, with the
                               per-head dequantisation of
                               src/triton_ops/int8_paged_attention.py:808-809

Pinned in tests/test_torch_cpu_path.py against the numpy oracle (oracle/int8kv_oracle.py, which
is itself pinned by known answers, brute force and float64 SDPA), plus its own known answers.
"""

from __future__ import annotations

import math

import torch


def quant_kv_static_per_head(x: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """int8 codes of ``x`` with a broadcastable fp32 ``scale`` (src/quant.py:37-40)."""
    return torch.round(x / scale).clamp(-127, 127).to(torch.int8)


def write_paged(k: torch.Tensor, v: torch.Tensor, key_cache: torch.Tensor,
                value_cache: torch.Tensor, table_row: torch.Tensor, k_scale: torch.Tensor,
                v_scale: torch.Tensor) -> None:
    """Quantises one sequence's K/V [T, Hkv, D] and places token t at block table_row[t // BS],
    row t % BS of the [NB, BS, Hkv, D] caches (src/paged_cache.py:24-32 with a given table)."""
    T, hkv, d = k.shape
    bs = key_cache.shape[1]
    n = (T + bs - 1) // bs
    slots = (table_row[:n].to(torch.int64)[:, None] * bs + torch.arange(bs)).reshape(-1)[:T]
    ks = k_scale.float().reshape(1, hkv, 1)
    vs = v_scale.float().reshape(1, hkv, 1)
    key_cache.view(-1, hkv, d)[slots] = quant_kv_static_per_head(k.float(), ks)
    value_cache.view(-1, hkv, d)[slots] = quant_kv_static_per_head(v.float(), vs)


def gather_sequence(cache: torch.Tensor, table_row: torch.Tensor, T: int) -> torch.Tensor:
    """[Hkv, T, D]: the sequence's tokens in logical order (src/paged_cache.py:45-58)."""
    bs = cache.shape[1]
    n = (T + bs - 1) // bs
    blocks = cache[table_row[:n].to(torch.int64)]  # [n, BS, Hkv, D]
    return blocks.reshape(n * bs, *cache.shape[2:])[:T].permute(1, 0, 2)


def expand_kv_for_gqa(x: torch.Tensor, num_query_heads: int) -> torch.Tensor:
    """[B, Hkv, T, D] -> [B, Hq, T, D] (src/attention_ref.py:11-16)."""
    hkv = x.shape[1]
    assert num_query_heads % hkv == 0
    return x.repeat_interleave(num_query_heads // hkv, dim=1)


def decode_attention_ref(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """q [B, Hq, D], k/v [B, Hkv, T, D] -> [B, Hq, D] fp32 (src/attention_ref.py:19-28)."""
    hq, d = q.shape[1], q.shape[2]
    k = expand_kv_for_gqa(k, hq)
    v = expand_kv_for_gqa(v, hq)
    scores = torch.einsum("bhd,bhtd->bht", q.float(), k.float()) / math.sqrt(d)
    p = torch.softmax(scores, dim=-1)
    return torch.einsum("bht,bhtd->bhd", p, v.float())


def decode_step(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                block_tables: torch.Tensor, seq_lens, k_scale: torch.Tensor,
                v_scale: torch.Tensor, sequences=None) -> torch.Tensor:
    """One decode step over the int8 paged caches -> [B, Hq, D] fp32 (rows of sequences not in
    ``sequences``, and of empty sequences, stay 0): per sequence, gather, dequantise with the
    per-head scales floored at 1e-6, then the reference attention."""
    B, hq, d = query.shape
    hkv = key_cache.shape[2]
    ks = k_scale.float().clamp_min(1e-6).reshape(1, hkv, 1, 1)
    vs = v_scale.float().clamp_min(1e-6).reshape(1, hkv, 1, 1)
    out = torch.zeros(B, hq, d, dtype=torch.float32)
    lens = [int(x) for x in seq_lens]
    for b in (range(B) if sequences is None else sequences):
        T = lens[b]
        if T <= 0:
            continue
        k = gather_sequence(key_cache, block_tables[b], T)[None].float() * ks
        v = gather_sequence(value_cache, block_tables[b], T)[None].float() * vs
        out[b] = decode_attention_ref(query[b:b + 1], k, v)[0]
    return out
