"""head_dim 64 with kv heads taken in pairs: a wave treats kv heads 2k and 2k + 1, whose 64-wide
rows sit side by side in the cache, as one 128-wide head, with the query block-diagonal over the
two halves (2 G <= 16 query heads in the MFMA columns).  The pairing applies to an even kv-head
count, GQA groups up to 8 and a head stride of head_dim; otherwise each wave takes one 64-wide
head.  Against the fp32 oracle: groups 4, 7 and 8 (paired), 9 and an odd kv-head count (not
paired), bf16 / fp16 / fp32 queries, quantize_q, forced splits, both merge grids, BF16 and FP16
caches, empty and one-token sequences, and a strided head layout that must fall back.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import int8kv
from cases import bf16_caches, decode_case, oracle_int8, ranges_call, to_dev
from conftest import MAX_ABS, MIN_COS, metrics
from oracle import int8kv_oracle as O

pytestmark = pytest.mark.gpu

LENS = [0, 1, 31, 33, 700, 2049, 4097, 9000, 16, 257]


def _check(out, ref, what):
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err, cos, _ = metrics(got, ref)
    print(f"{what}: max|diff|={err:.3e} cos={cos:.7f}", flush=True)
    assert err <= MAX_ABS and cos >= MIN_COS, f"{what}: max|diff|={err} cos={cos}"
    return err


@pytest.mark.parametrize("hq,hkv", [(32, 8), (14, 2), (16, 2), (18, 2), (12, 3)])
def test_int8_pairs_and_fallbacks(cuda, hq, hkv):
    c = decode_case(LENS, seed=hq * 10 + hkv, hq=hq, hkv=hkv, head_dim=64, extra_blocks=6)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    ref = oracle_int8(c)
    for splits in (None, 1, 2, 5):
        out = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, num_splits=splits)
        torch.cuda.synchronize()
        assert (out[0] == 0).all()
        _check(out, ref, f"int8 {hq}/{hkv} splits={splits}")
    for splits in (1, 2, 5):  # the range layout, where the kv heads go in pairs
        out = ranges_call((q, kc, vc, bt, sl, ks, vs), cuda, splits)
        assert (out[0] == 0).all()
        _check(out, ref, f"int8 {hq}/{hkv} {splits} ranges per sequence")
    for qdt in (torch.float16, torch.float32):
        out = int8kv.int8_paged_attention(q.to(qdt), kc, vc, bt, sl, ks, vs)
        torch.cuda.synchronize()
        err = _check(out, ref, f"int8 {hq}/{hkv} {qdt}")
        if qdt == torch.float32:
            assert err <= 1e-3, err
    ref_q = O.paged_attention_ref(c.query.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                  c.seq_lens.numpy(), c.k_scale.numpy(), c.v_scale.numpy(),
                                  quantize_q=True)
    out_q = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, quantize_q=True)
    torch.cuda.synchronize()
    _check(out_q, ref_q, f"int8 quantize_q {hq}/{hkv}")


@pytest.mark.parametrize("cache_dtype", [torch.bfloat16, torch.float16])
def test_16bit_cache_pairs(cuda, cache_dtype):
    c = decode_case(LENS, seed=7, hq=32, hkv=8, head_dim=64, extra_blocks=4)
    k16, v16 = bf16_caches(c, cache_dtype)
    ref = O.paged_attention_ref(c.query.float().numpy(), k16.float().numpy(), v16.float().numpy(),
                                c.block_tables.numpy(), c.seq_lens.numpy())
    q, bt, sl = c.query.to(cuda), c.block_tables.to(cuda), c.seq_lens.to(cuda)
    for qdt, splits in ((torch.bfloat16, None), (torch.float16, 3), (torch.float32, 1)):
        out = int8kv.bf16_paged_attention(q.to(qdt), k16.to(cuda), v16.to(cuda), bt, sl,
                                          num_splits=splits)
        torch.cuda.synchronize()
        _check(out, ref, f"{cache_dtype} cache {qdt} splits={splits}")


def test_strided_heads_fall_back_and_agree(cuda):
    """Caches whose head stride is twice head_dim (a [.., Hkv, 128] buffer viewed as [.., 64]):
    the pairs do not apply; the result matches the oracle and the contiguous (paired) call."""
    c = decode_case([5, 1500, 3000, 64, 0, 777], seed=17, hq=32, hkv=8, head_dim=64,
                    extra_blocks=3)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    kw = torch.zeros(*kc.shape[:3], 128, dtype=kc.dtype, device=cuda)
    vw = torch.zeros_like(kw)
    kw[..., :64] = kc
    vw[..., :64] = vc
    ks_, vs_ = kw[..., :64], vw[..., :64]
    assert ks_.stride(2) == 128
    ref = oracle_int8(c)
    strided = int8kv.int8_paged_attention(q, ks_, vs_, bt, sl, ks, vs)
    paired = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs)
    torch.cuda.synchronize()
    _check(strided, ref, "strided heads (one per wave)")
    _check(paired, ref, "contiguous heads (pairs)")
    diff = (strided.float() - paired.float()).abs().max().item()
    assert diff <= 4e-3, diff


def test_large_batch_merge_by_range(cuda):
    g = torch.Generator().manual_seed(64)
    lens = torch.randint(1, 800, (300,), generator=g).tolist()
    lens[3], lens[150] = 7000, 0
    c = decode_case(lens, seed=65, hq=32, hkv=8, head_dim=64, extra_blocks=5)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    out = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs)
    torch.cuda.synchronize()
    assert (out[150] == 0).all()
    _check(out, oracle_int8(c), "B=300 pairs")
