"""Seeded synthetic inputs shaped like Qwen2.5-7B attention (the benchmark configurations).

Shapes: 28 query heads, 4 kv heads, head_dim 128, cache block 16 tokens.
Distributions (as specified for the benchmark configurations):
  * Q ~ N(0, 1), bf16.
  * K ~ N(0, 1) with 4 of 128 channels per kv head scaled x8 (outlier channels, as the
    reference's K statistics show, outputs/kv_stats.csv) plus a per-(kv head, channel) mean
    offset ~ N(0, 0.5), bf16.
  * V ~ N(0, 0.5) (standard deviation 0.5), bf16.
  * Static scales: absmax / 127 per kv head over a separately seeded 4096-token sample,
    floored at 1e-6 (scripts/04_calibrate_static_scale.py:55-65 of the reference).
  * Block tables: a shuffled pool of physical blocks shared by all sequences
    (tests/test_int8_paged_attention.py:16-43 of the reference uses the same scheme).
Everything here is input generation; no operator is computed.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

HQ, HKV, HEAD_DIM, BLOCK = 28, 4, 128, 16


@dataclass
class KVDistribution:
    outlier_channels: torch.Tensor  # [Hkv, 4] int64
    k_offset: torch.Tensor  # [Hkv, D] float32


def make_distribution(seed: int = 0, hkv: int = HKV, d: int = HEAD_DIM) -> KVDistribution:
    g = torch.Generator().manual_seed(seed + 1000)
    chans = torch.stack([torch.randperm(d, generator=g)[:4] for _ in range(hkv)])
    offset = torch.randn(hkv, d, generator=g) * 0.5
    return KVDistribution(chans, offset)


def sample_kv(n_tokens: int, dist: KVDistribution, gen: torch.Generator, device="cpu"):
    """K, V of shape [n_tokens, Hkv, D] in bf16, drawn with ``gen`` on ``device``."""
    hkv, d = dist.k_offset.shape
    k = torch.randn(n_tokens, hkv, d, generator=gen, device=device)
    mult = torch.ones(hkv, d, device=device)
    mult.scatter_(1, dist.outlier_channels.to(device), 8.0)
    k.mul_(mult).add_(dist.k_offset.to(device))
    v = torch.randn(n_tokens, hkv, d, generator=gen, device=device).mul_(0.5)
    return k.to(torch.bfloat16), v.to(torch.bfloat16)


def calibrate_scales(dist: KVDistribution, seed: int = 1, n_tokens: int = 4096):
    """absmax/127 per kv head over a seeded sample -> (k_scale, v_scale) float32 [Hkv]."""
    g = torch.Generator().manual_seed(seed)
    k, v = sample_kv(n_tokens, dist, g)
    ks = (k.float().abs().amax(dim=(0, 2)) / 127.0).clamp_min(1e-6)
    vs = (v.float().abs().amax(dim=(0, 2)) / 127.0).clamp_min(1e-6)
    return ks, vs


def sample_query(batch: int, gen: torch.Generator, hq: int = HQ, d: int = HEAD_DIM, device="cpu"):
    return torch.randn(batch, hq, d, generator=gen, device=device).to(torch.bfloat16)


def random_block_tables(seq_lens, num_blocks: int, gen: torch.Generator, width: int | None = None,
                        block_size: int = BLOCK, fill: int = 0) -> torch.Tensor:
    """[B, width] int32 tables drawing distinct blocks from a shuffled pool of ``num_blocks``."""
    need = [(int(n) + block_size - 1) // block_size for n in seq_lens]
    width = max(max(need, default=1), 1) if width is None else width
    assert sum(need) <= num_blocks, "block pool too small"
    pool = torch.randperm(num_blocks, generator=gen)
    tables = torch.full((len(need), width), fill, dtype=torch.int32)
    ptr = 0
    for b, n in enumerate(need):
        tables[b, :n] = pool[ptr:ptr + n].to(torch.int32)
        ptr += n
    return tables


def slot_mapping_for(block_tables: torch.Tensor, seq_lens, block_size: int = BLOCK) -> torch.Tensor:
    """Token-order slots (physical_block * BS + offset) of every sequence, concatenated, int64."""
    out = []
    for b, n in enumerate(seq_lens):
        n = int(n)
        t = torch.arange(n, dtype=torch.int64)
        out.append(block_tables[b, t // block_size].to(torch.int64) * block_size + t % block_size)
    return torch.cat(out) if out else torch.zeros(0, dtype=torch.int64)


def ragged_lengths(batch: int, max_len: int, seed: int) -> torch.Tensor:
    """Uniform integer lengths in [1, max_len] (the large ragged decode batch)."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(1, max_len + 1, (batch,), generator=g, dtype=torch.int64)
