"""Caches larger than 2 GiB, with every block a call touches past the 2^31-byte mark.

The kernels form cache addresses as 64-bit block id × byte stride products; a 32-bit product
would wrap for these blocks.  Each case runs the same inputs twice, once on a small cache and
once with the block ids (or slots) shifted to the top of a 2.4 GB cache, and requires the two
results to be identical (decode under one range per sequence, so that both calls use the same
layout; the automatic layout is checked against the oracle), and the written bytes of the
writes to match the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import int8kv
from cases import bf16_caches, decode_case, oracle_int8, to_dev
from conftest import MAX_ABS, MIN_COS, metrics
from int8kv import cache_ops
from oracle import int8kv_oracle as O

pytestmark = pytest.mark.gpu

GIB2 = 1 << 31


def _check(out, ref, what):
    err, cos, _ = metrics(out.float().cpu().numpy(), ref)
    assert err <= MAX_ABS and cos >= MIN_COS, f"{what}: max|diff|={err} cos={cos}"


def _shifted(cache: torch.Tensor, total_blocks: int):
    """A zeroed [total_blocks, ...] cache holding ``cache`` in its last blocks, and the id shift."""
    base = total_blocks - cache.shape[0]
    big = torch.zeros((total_blocks, *cache.shape[1:]), dtype=cache.dtype, device=cache.device)
    big[base:] = cache
    return big, base


def test_decode_reads_blocks_past_2gib(cuda):
    lens = [5, 700, 1234, 33, 4000, 0, 2049]
    c = decode_case(lens, seed=88, extra_blocks=3)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    row_bytes = kc[0].numel()  # bytes per block of the int8 cache
    kb, base = _shifted(kc, 300_000)
    vb, _ = _shifted(vc, 300_000)
    assert base * row_bytes > GIB2 and kb.numel() > GIB2
    btb = bt + base
    ref = oracle_int8(c)
    _check(int8kv.int8_paged_attention(q, kb, vb, btb, sl, ks, vs), ref, "int8 auto, shifted")
    for splits in (1, 3):
        small = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, num_splits=splits)
        big = int8kv.int8_paged_attention(q, kb, vb, btb, sl, ks, vs, num_splits=splits)
        torch.cuda.synchronize()
        _check(big, ref, f"int8 splits={splits}, shifted")
        if splits == 1:
            assert torch.equal(small, big)
    small_q = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, quantize_q=True, num_splits=1)
    big_q = int8kv.int8_paged_attention(q, kb, vb, btb, sl, ks, vs, quantize_q=True, num_splits=1)
    torch.cuda.synchronize()
    assert torch.equal(small_q, big_q)
    del kb, vb
    torch.cuda.empty_cache()

    k16, v16 = (x.to(cuda) for x in bf16_caches(c))
    kb16, base16 = _shifted(k16, 150_000)
    vb16, _ = _shifted(v16, 150_000)
    assert base16 * k16[0].numel() * 2 > GIB2
    ref16 = O.paged_attention_ref(c.query.float().numpy(), k16.float().cpu().numpy(),
                                  v16.float().cpu().numpy(), c.block_tables.numpy(), c.seq_lens.numpy())
    small16 = int8kv.bf16_paged_attention(q, k16, v16, bt, sl, num_splits=1)
    big16 = int8kv.bf16_paged_attention(q, kb16, vb16, bt + base16, sl, num_splits=1)
    auto16 = int8kv.bf16_paged_attention(q, kb16, vb16, bt + base16, sl)
    torch.cuda.synchronize()
    assert torch.equal(small16, big16)
    _check(auto16, ref16, "bf16 auto, shifted")


@pytest.mark.parametrize("T", [3000, 262_144])
def test_writes_land_past_2gib(cuda, T):
    """Static and dynamic writes into slots whose rows sit past 2^31 bytes.  262,144 bf16 tokens
    take the static write's token-major map (sources above 256 MB), 3000 the row map."""
    hkv, d, bs = 4, 128, 16
    g = torch.Generator().manual_seed(T)
    k = (torch.randn(T, hkv, d, generator=g) * 2).to(torch.bfloat16)
    v = torch.randn(T, hkv, d, generator=g).to(torch.bfloat16)
    nb_small = (T + bs - 1) // bs + 2
    slots = torch.randperm(nb_small * bs, generator=g)[:T]
    slots[torch.randperm(T, generator=g)[: T // 10]] = -1
    ks = (k.float().abs().amax(dim=(0, 2)) / 127).clamp_min(1e-6)
    vs = (v.float().abs().amax(dim=(0, 2)) / 127).clamp_min(1e-6)
    big_nb = 300_000
    base_blk = big_nb - nb_small
    assert base_blk * bs * hkv * d > GIB2
    shifted = torch.where(slots >= 0, slots + base_blk * bs, slots)
    kd, vd = k.to(cuda), v.to(cuda)

    kc = torch.zeros(big_nb, bs, hkv, d, dtype=torch.int8, device=cuda)
    vc = torch.zeros_like(kc)
    int8kv.int8_kv_cache_write(kd, vd, kc, vc, shifted.to(cuda), ks.to(cuda), vs.to(cuda))
    torch.cuda.synchronize()
    assert not kc[:base_blk].any() and not vc[:base_blk].any()  # nothing below the shifted rows
    kr = np.zeros((nb_small, bs, hkv, d), np.int8)
    vr = np.zeros_like(kr)
    kf, vf = k.float().numpy(), v.float().numpy()
    O.int8_kv_cache_write(kf, vf, kr, vr, slots.numpy(), ks.numpy(), vs.numpy())
    assert np.array_equal(kc[base_blk:].cpu().numpy(), kr), f"static K, T={T}"
    assert np.array_equal(vc[base_blk:].cpu().numpy(), vr), f"static V, T={T}"

    kc.zero_()
    vc.zero_()
    ksc = torch.zeros(big_nb, bs, hkv, device=cuda)
    vsc = torch.zeros_like(ksc)
    cache_ops.reshape_and_cache_int8(kd, vd, kc, vc, ksc, vsc, shifted.to(cuda))
    torch.cuda.synchronize()
    assert not kc[:base_blk].any() and not ksc[:base_blk].any()
    ref = [np.zeros((nb_small, bs, hkv, d), np.int8), np.zeros((nb_small, bs, hkv, d), np.int8),
           np.zeros((nb_small, bs, hkv), np.float32), np.zeros((nb_small, bs, hkv), np.float32)]
    O.reshape_and_cache_int8(kf, vf, *ref, slots.numpy())
    for name, got, want in zip(("K", "V", "K scale", "V scale"), (kc, vc, ksc, vsc), ref):
        assert np.array_equal(got[base_blk:].cpu().numpy(), want), f"dynamic {name}, T={T}"
