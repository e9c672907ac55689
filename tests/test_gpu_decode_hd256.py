"""head_dim 256 (the Gemma family's head size) on the decode kernels, against the fp32 oracle.

The reference's kernels take any head_dim (src/triton_ops/int8_paged_attention.py:112-129 pads it
to a power of two under a mask); this build runs 64, 128 and 256 on the matrix cores.  At 256 a
lane holds 64 K elements of its token (8 fp16 k-steps, 4 int8 ones) and 16 V elements of each of
its 4 token rows, the waves take one SIMD each with two tiles in flight, and the merge lanes are
one range slot of 64 float4 columns.  Cases: GQA groups 2, 1 and 8 (Gemma-2-9B 16/8, Gemma-7B
16/16, Gemma-2B 8/1), lengths at tile, block and chunk boundaries with empty and one-token
sequences, bf16 / fp16 / fp32 queries, quantize_q (int8 scores), forced splits, both merge grids,
BF16 and FP16 caches, the write-then-decode path, and the per-sequence layout (four waves per
workgroup at 256).
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

LENS = [0, 1, 17, 31, 32, 33, 255, 256, 257, 1000, 4097, 8200]


def _check(out, ref, what):
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err, cos, _ = metrics(got, ref)
    print(f"{what}: max|diff|={err:.3e} cos={cos:.7f}", flush=True)
    assert err <= MAX_ABS and cos >= MIN_COS, f"{what}: max|diff|={err} cos={cos}"
    return err


@pytest.mark.parametrize("hq,hkv", [(16, 8), (16, 16), (8, 1)])
def test_int8_cache(cuda, hq, hkv):
    c = decode_case(LENS, seed=hq + 3 * hkv, hq=hq, hkv=hkv, head_dim=256, extra_blocks=7)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    ref = oracle_int8(c)
    for splits in (None, 1, 3):
        out = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, num_splits=splits)
        torch.cuda.synchronize()
        assert out.shape == (len(LENS), hq, 256) and out.dtype == torch.bfloat16
        assert (out[0] == 0).all()
        _check(out, ref, f"int8 {hq}/{hkv} splits={splits}")
    for qdt in (torch.float16, torch.float32):
        out = int8kv.int8_paged_attention(q.to(qdt), kc, vc, bt, sl, ks, vs)
        torch.cuda.synchronize()
        err = _check(out, ref, f"int8 {hq}/{hkv} {qdt}")
        if qdt == torch.float32:
            assert err <= 1e-3, err  # q held as 16-bit hi + lo operands
    ref_q = O.paged_attention_ref(c.query.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                  c.seq_lens.numpy(), c.k_scale.numpy(), c.v_scale.numpy(),
                                  quantize_q=True)
    out_q = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, quantize_q=True)
    torch.cuda.synchronize()
    _check(out_q, ref_q, f"int8 quantize_q {hq}/{hkv}")


@pytest.mark.parametrize("cache_dtype", [torch.bfloat16, torch.float16])
def test_16bit_caches(cuda, cache_dtype):
    c = decode_case(LENS, seed=41, hq=16, hkv=8, head_dim=256, extra_blocks=5)
    k16, v16 = bf16_caches(c, cache_dtype)
    ref = O.paged_attention_ref(c.query.float().numpy(), k16.float().numpy(), v16.float().numpy(),
                                c.block_tables.numpy(), c.seq_lens.numpy())
    q = c.query.to(cuda)
    bt, sl = c.block_tables.to(cuda), c.seq_lens.to(cuda)
    kd, vd = k16.to(cuda), v16.to(cuda)
    for qdt, splits in ((torch.bfloat16, None), (torch.bfloat16, 3), (torch.float16, 1),
                        (torch.float32, None)):
        out = int8kv.bf16_paged_attention(q.to(qdt), kd, vd, bt, sl, num_splits=splits)
        torch.cuda.synchronize()
        assert (out[0] == 0).all()
        _check(out, ref, f"{cache_dtype} cache, {qdt} query, splits={splits}")


def test_merge_by_range_and_large_batch(cuda):
    """B = 96 at one range per sequence on average (2 B >= ranges: the merge indexed by range) and
    at 3 splits per sequence (the merge indexed by sequence), ragged with a few long ones."""
    g = torch.Generator().manual_seed(256)
    lens = torch.randint(1, 700, (96,), generator=g).tolist()
    lens[5], lens[50], lens[95] = 5000, 0, 3001
    c = decode_case(lens, seed=257, hq=16, hkv=8, head_dim=256, extra_blocks=5)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    ref = oracle_int8(c)
    for splits in (1, 2, 3):
        out = ranges_call((q, kc, vc, bt, sl, ks, vs), cuda, splits)
        assert (out[50] == 0).all()
        _check(out, ref, f"B=96 {splits} ranges per sequence")
        out = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, num_splits=splits)
        torch.cuda.synchronize()
        assert (out[50] == 0).all()
        _check(out, ref, f"B=96 splits={splits}")


def test_write_then_decode(cuda):
    """The static cache write and the decode at head_dim 256, end to end: the written cache is
    bit-exact to the oracle's and the decode over it matches the oracle."""
    lens = [3, 600, 129, 2048]
    c = decode_case(lens, seed=9, hq=8, hkv=2, head_dim=256, extra_blocks=3)
    kc = torch.zeros(c.kc.shape, dtype=torch.int8, device=cuda)
    vc = torch.zeros_like(kc)
    int8kv.int8_kv_cache_write(c.key.to(cuda), c.value.to(cuda), kc, vc, c.slots.to(cuda),
                               c.k_scale.to(cuda), c.v_scale.to(cuda))
    torch.cuda.synchronize()
    written = np.zeros(c.kc.shape, np.int8)
    written_v = np.zeros_like(written)
    O.int8_kv_cache_write(c.key.float().numpy(), c.value.float().numpy(), written, written_v,
                          c.slots.numpy(), c.k_scale.numpy(), c.v_scale.numpy())
    assert np.array_equal(kc.cpu().numpy(), written) and np.array_equal(vc.cpu().numpy(), written_v)
    out = int8kv.int8_paged_attention(c.query.to(cuda), kc, vc, c.block_tables.to(cuda),
                                      c.seq_lens.to(cuda), c.k_scale.to(cuda), c.v_scale.to(cuda))
    torch.cuda.synchronize()
    ref = O.paged_attention_ref(c.query.float().numpy(), written, written_v, c.block_tables.numpy(),
                                c.seq_lens.numpy(), c.k_scale.numpy(), c.v_scale.numpy())
    _check(out, ref, "write then decode")


def test_per_sequence_layout(cuda):
    """The per-sequence layout at 256 (four waves, one per SIMD, their states in 64 KB of LDS):
    forced, against the oracle for short and tile-boundary lengths, and the automatic choice on
    the same call agrees with it."""
    from int8kv import _decode, _lib

    c = decode_case([40, 7, 0, 32, 33, 129, 511], seed=3, hq=8, hkv=2, head_dim=256,
                    extra_blocks=2)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    ref = oracle_int8(c)
    out = torch.empty_like(q)
    _decode.paged_decode(q, kc, vc, bt, sl, ks, vs, out, 0,
                         _lib.DECODE_ALL | _lib.DECODE_PER_SEQUENCE)
    torch.cuda.synchronize()
    assert (out[2] == 0).all()
    _check(out, ref, "per-sequence layout")
    auto = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs)
    torch.cuda.synchronize()
    _check(auto, ref, "short call, automatic layout")
