"""Seeded test cases shared by the GPU parity tests (inputs built on the CPU, then copied)."""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from int8kv import synthetic as syn
from oracle import int8kv_oracle as O


@dataclass
class DecodeCase:
    query: torch.Tensor  # CPU bf16 [B, Hq, D]
    key: torch.Tensor  # CPU bf16 [T_total, Hkv, D] (token order, sequences concatenated)
    value: torch.Tensor
    kc: np.ndarray  # oracle int8 caches [NB, BS, Hkv, D]
    vc: np.ndarray
    block_tables: torch.Tensor  # CPU int32 [B, width]
    seq_lens: torch.Tensor  # CPU int32 [B]
    slots: torch.Tensor  # CPU int64 [T_total]
    k_scale: torch.Tensor  # CPU fp32 [Hkv]
    v_scale: torch.Tensor
    num_blocks: int
    block_size: int = 16


def decode_case(lens, seed=0, hq=28, hkv=4, extra_blocks=17, width=None, randn_kv=False,
                fill=None, block_size=16, head_dim=128) -> DecodeCase:
    """Sequences of the given lengths written into a shuffled block pool.

    randn_kv=True uses the reference tests' inputs (K, V ~ N(0, 1), scales = absmax/127 of the
    data itself, tests/test_int8_paged_attention.py:121-150); otherwise the outlier-channel
    distribution of the benchmark configurations with separately calibrated scales.
    """
    g = torch.Generator().manual_seed(seed)
    lens = [int(n) for n in lens]
    total = sum(lens)
    if randn_kv:
        k = torch.randn(total, hkv, head_dim, generator=g).to(torch.bfloat16)
        v = torch.randn(total, hkv, head_dim, generator=g).to(torch.bfloat16)
        ks = (k.float().abs().amax(dim=(0, 2)) / 127.0).clamp_min(1e-6)
        vs = (v.float().abs().amax(dim=(0, 2)) / 127.0).clamp_min(1e-6)
    else:
        dist = syn.make_distribution(seed, hkv=hkv, d=head_dim)
        ks, vs = syn.calibrate_scales(dist, seed=seed + 1)
        k, v = syn.sample_kv(total, dist, g)
    q = torch.randn(len(lens), hq, head_dim, generator=g).to(torch.bfloat16)
    bs = block_size
    nblk = sum((n + bs - 1) // bs for n in lens)
    nb = nblk + extra_blocks
    if fill is None:
        fill = nb - 1
    bt = syn.random_block_tables(lens, nb, g, width=width, block_size=bs, fill=fill)
    slots = syn.slot_mapping_for(bt, lens, block_size=bs)
    kc = np.zeros((nb, bs, hkv, head_dim), np.int8)
    vc = np.zeros_like(kc)
    # Unwritten slots hold random bytes: the kernels must never read them into a result.
    rng = np.random.default_rng(seed + 7)
    kc[:] = rng.integers(-128, 128, kc.shape, dtype=np.int8)
    vc[:] = rng.integers(-128, 128, vc.shape, dtype=np.int8)
    O.int8_kv_cache_write(k.float().numpy(), v.float().numpy(), kc, vc, slots.numpy(),
                          ks.numpy(), vs.numpy())
    return DecodeCase(q, k, v, kc, vc, bt, torch.tensor(lens, dtype=torch.int32), slots, ks, vs, nb,
                      bs)


def oracle_int8(c: DecodeCase, query=None) -> np.ndarray:
    q = (c.query if query is None else query).float().numpy()
    return O.paged_attention_ref(q, c.kc, c.vc, c.block_tables.numpy(), c.seq_lens.numpy(),
                                 c.k_scale.numpy(), c.v_scale.numpy())


def bf16_caches(c: DecodeCase, dtype=torch.bfloat16):
    """16-bit paged caches holding the case's K/V (unwritten slots = random finite values)."""
    nb = c.num_blocks
    hkv = c.key.shape[1]
    g = torch.Generator().manual_seed(123)
    bs = c.block_size
    d = c.key.shape[2]
    kc = torch.randn(nb * bs, hkv, d, generator=g).to(dtype)
    vc = torch.randn(nb * bs, hkv, d, generator=g).to(dtype)
    kc[c.slots] = c.key.to(dtype)
    vc[c.slots] = c.value.to(dtype)
    return kc.view(nb, bs, hkv, d), vc.view(nb, bs, hkv, d)


def to_dev(c: DecodeCase, dev):
    return (c.query.to(dev), torch.from_numpy(c.kc).to(dev), torch.from_numpy(c.vc).to(dev),
            c.block_tables.to(dev), c.seq_lens.to(dev), c.k_scale.to(dev), c.v_scale.to(dev))


def ranges_call(case_or_tensors, dev, splits=None, quantize_q=False, out=None, min_tiles=0):
    """INT8 decode through the library's range layout with ``splits`` x batch explicit ranges
    (None: the automatic range count with ``min_tiles``, 2 if 0): int8kv_paged_decode called
    directly, so tests can pin the range layout and its range count (the drop-in operator's
    num_splits selects the per-sequence and split layouts).  ``case_or_tensors``: a DecodeCase
    or the tuple of to_dev."""
    from int8kv import _decode, _lib

    t = to_dev(case_or_tensors, dev) if isinstance(case_or_tensors, DecodeCase) else case_or_tensors
    q, kc, vc, bt, sl, ks, vs = t
    ranges = 0 if splits is None else max(1, int(splits) * q.shape[0])
    res = torch.empty_like(q) if out is None else out
    flags = _lib.DECODE_ALL | (_lib.DECODE_QUANTIZE_Q if quantize_q else 0)
    _decode.paged_decode(q, kc, vc, bt, sl, ks, vs, res, ranges, flags, None,
                         (min_tiles or 2) if splits is None else 0)
    torch.cuda.synchronize()
    return res
