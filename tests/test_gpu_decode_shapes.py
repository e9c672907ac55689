"""Head sizes between 64, 128 and 256 and GQA groups above 16 on the decode kernels, against the
fp32 oracle.

The reference's kernels take any head_dim (src/triton_ops/int8_paged_attention.py:112-129 pads it
to a power of two under a mask) and any group (the grid there is one program per query head).
This build runs head_dim 64, 128 and 256 on their own kernels; a head_dim in between (a multiple
of 16: 80 for Phi-2, 96 for Phi-3-mini, 112, 160, 192, ...) runs the next one with the elements
past head_dim read from inside the row but meeting zero query elements, and its output columns
past head_dim never stored.  A group above 16 (multi-query attention: Falcon-7B's 71 query heads
on one kv head, 64 query heads per kv head, group 24 ...) takes one wave or workgroup per 16 query
heads of a kv head.

Every case checks the oracle bar, that empty sequences give zero rows, and -- through an output
view whose rows are wider than head_dim, filled with NaN -- that nothing past head_dim is written.
Layouts: automatic (ranges, per-sequence, split), forced range counts with both merge grids,
forced splits; INT8 and BF16 caches, fp32 queries, quantize_q, and the write-then-decode path.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import int8kv
from cases import bf16_caches, decode_case, oracle_int8, ranges_call, to_dev
from conftest import MAX_ABS, MIN_COS, metrics
from int8kv import _decode, _lib
from oracle import int8kv_oracle as O

pytestmark = pytest.mark.gpu

LENS = [0, 1, 17, 31, 32, 33, 255, 256, 257, 1000, 4097, 2200]


def _check(out, ref, what):
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err, cos, _ = metrics(got, ref)
    print(f"{what}: max|diff|={err:.3e} cos={cos:.7f}", flush=True)
    assert err <= MAX_ABS and cos >= MIN_COS, f"{what}: max|diff|={err} cos={cos}"
    return err


def _wide_out(q):
    """An output view [B, Hq, D] inside NaN-filled rows of 256 elements: the columns past D must
    stay NaN."""
    B, Hq, D = q.shape
    full = torch.full((B, Hq, 256), float("nan"), dtype=q.dtype, device=q.device)
    return full, full[..., :D]


def _untouched(full, D, what):
    assert torch.isnan(full[..., D:]).all(), f"{what}: columns past head_dim were written"


def _decode_auto(q, kc, vc, bt, sl, ks, vs, flags=_lib.DECODE_ALL):
    full, out = _wide_out(q)
    _decode.paged_decode(q, kc, vc, bt, sl, ks, vs, out, 0, flags)
    torch.cuda.synchronize()
    return full, out


def _plan(q, kc, bt, num_ranges=0, flags=_lib.DECODE_ALL):
    B, Hq, D = q.shape
    nb, bs, hkv, _ = kc.shape
    return _lib.decode_plan(q.dtype, kc.dtype, B, Hq, hkv, D, nb, bs, bt.shape[1],
                            num_ranges=num_ranges, flags=flags)


@pytest.mark.parametrize("d", [80, 96, 112, 48, 160, 192])
def test_padded_head_dims_int8(cuda, d):
    hq, hkv = (32, 8) if d != 160 else (16, 4)
    c = decode_case(LENS, seed=d, hq=hq, hkv=hkv, head_dim=d, extra_blocks=7)
    t = to_dev(c, cuda)
    q, kc, vc, bt, sl, ks, vs = t
    ref = oracle_int8(c)
    full, out = _decode_auto(*t)
    print(f"d={d} auto plan: {_plan(q, kc, bt)['layout']}", flush=True)
    assert (out[0] == 0).all()
    _check(out, ref, f"int8 d={d} auto")
    _untouched(full, d, f"int8 d={d} auto")
    for splits in (1, 3):  # one range per sequence (by-range merge), three (by-sequence merge)
        full, out = _wide_out(q)
        ranges_call(t, cuda, splits=splits, out=out)
        _check(out, ref, f"int8 d={d} ranges x{splits}")
        _untouched(full, d, f"int8 d={d} ranges x{splits}")
    full, out = _wide_out(q)
    ranges_call(t, cuda, splits=None, out=out, min_tiles=2)
    _check(out, ref, f"int8 d={d} automatic ranges")
    for splits in (1, 4):  # per-sequence layout, split layout with 4 workgroups per sequence
        out = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, num_splits=splits)
        torch.cuda.synchronize()
        assert out.shape == (len(LENS), hq, d)
        _check(out, ref, f"int8 d={d} num_splits={splits}")
    out = int8kv.int8_paged_attention(q.float(), kc, vc, bt, sl, ks, vs)
    torch.cuda.synchronize()
    assert _check(out, ref, f"int8 d={d} fp32 query") <= 1e-3
    ref_q = O.paged_attention_ref(c.query.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                  c.seq_lens.numpy(), c.k_scale.numpy(), c.v_scale.numpy(),
                                  quantize_q=True)
    full, out = _wide_out(q)
    ranges_call(t, cuda, splits=2, quantize_q=True, out=out)
    _check(out, ref_q, f"int8 d={d} quantize_q")
    _untouched(full, d, f"int8 d={d} quantize_q")


@pytest.mark.parametrize("d", [80, 96, 192])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_padded_head_dims_16bit_cache(cuda, d, dtype):
    c = decode_case(LENS, seed=d + 1, hq=16, hkv=4, head_dim=d, extra_blocks=5)
    q = c.query.to(cuda)
    k_cpu, v_cpu = bf16_caches(c, dtype)
    ref = O.paged_attention_ref(c.query.float().numpy(), k_cpu.float().numpy(),
                                v_cpu.float().numpy(), c.block_tables.numpy(), c.seq_lens.numpy())
    k16, v16 = k_cpu.to(cuda), v_cpu.to(cuda)
    bt, sl = c.block_tables.to(cuda), c.seq_lens.to(cuda)
    full, out = _decode_auto(q, k16, v16, bt, sl, None, None)
    _check(out, ref, f"{dtype} d={d} auto")
    _untouched(full, d, f"{dtype} d={d} auto")
    for splits in (1, 4):
        out = int8kv.bf16_paged_attention(q, k16, v16, bt, sl, num_splits=splits)
        torch.cuda.synchronize()
        _check(out, ref, f"{dtype} d={d} num_splits={splits}")
    full, out = _wide_out(q)
    _decode.paged_decode(q, k16, v16, bt, sl, None, None, out, 3 * len(LENS))
    torch.cuda.synchronize()
    _check(out, ref, f"{dtype} d={d} ranges x3")
    _untouched(full, d, f"{dtype} d={d} ranges x3")


# (hq, hkv, head_dim): group 17 (two column tiles, the second one head), 24, 32 and 64 (MQA),
# Falcon-7B's 71 query heads on one kv head at head_dim 64, and a padded head_dim with group 20.
GROUPS = [(34, 2, 128), (48, 2, 128), (32, 1, 128), (64, 1, 128), (71, 1, 64), (40, 2, 96),
          (32, 1, 256)]


@pytest.mark.parametrize("hq,hkv,d", GROUPS)
def test_groups_above_16_int8(cuda, hq, hkv, d):
    c = decode_case(LENS, seed=hq + hkv, hq=hq, hkv=hkv, head_dim=d, extra_blocks=7)
    t = to_dev(c, cuda)
    q, kc, vc, bt, sl, ks, vs = t
    ref = oracle_int8(c)
    full, out = _decode_auto(*t)
    assert (out[0] == 0).all()
    _check(out, ref, f"int8 {hq}/{hkv} d={d} auto")
    _untouched(full, d, f"int8 {hq}/{hkv} d={d} auto")
    for splits in (1, 3):
        out = ranges_call(t, cuda, splits=splits)
        _check(out, ref, f"int8 {hq}/{hkv} d={d} ranges x{splits}")
    for splits in (1, 4):
        out = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, num_splits=splits)
        torch.cuda.synchronize()
        _check(out, ref, f"int8 {hq}/{hkv} d={d} num_splits={splits}")
    ref_q = O.paged_attention_ref(c.query.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                  c.seq_lens.numpy(), c.k_scale.numpy(), c.v_scale.numpy(),
                                  quantize_q=True)
    out = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, quantize_q=True)
    torch.cuda.synchronize()
    _check(out, ref_q, f"int8 {hq}/{hkv} d={d} quantize_q")


@pytest.mark.parametrize("hq,hkv,d", [(32, 1, 128), (71, 1, 64), (40, 2, 96)])
def test_groups_above_16_bf16_cache(cuda, hq, hkv, d):
    c = decode_case(LENS, seed=hq * 3 + hkv, hq=hq, hkv=hkv, head_dim=d, extra_blocks=5)
    q = c.query.to(cuda)
    k_cpu, v_cpu = bf16_caches(c)
    ref = O.paged_attention_ref(c.query.float().numpy(), k_cpu.float().numpy(),
                                v_cpu.float().numpy(), c.block_tables.numpy(), c.seq_lens.numpy())
    k16, v16 = k_cpu.to(cuda), v_cpu.to(cuda)
    bt, sl = c.block_tables.to(cuda), c.seq_lens.to(cuda)
    for splits in (None, 1, 4):
        out = int8kv.bf16_paged_attention(q, k16, v16, bt, sl, num_splits=splits)
        torch.cuda.synchronize()
        _check(out, ref, f"bf16 {hq}/{hkv} d={d} num_splits={splits}")


def test_short_and_long_batches_take_every_layout(cuda):
    """The automatic layouts at a padded head_dim with a group above 16: a short batch (per
    sequence), one long sequence (split) and a long batch (ranges), each against the oracle."""
    seen = set()
    for lens, seed in (([300, 12, 512, 0], 51), ([20000], 52), ([3000] * 24 + [0, 9000], 53)):
        c = decode_case(lens, seed=seed, hq=40, hkv=2, head_dim=80, extra_blocks=3)
        t = to_dev(c, cuda)
        q, kc, vc, bt = t[:4]
        seen.add(_plan(q, kc, bt)["layout"])
        full, out = _decode_auto(*t)
        _check(out, oracle_int8(c), f"lens={lens[:4]}... auto")
        _untouched(full, 80, "auto")
    assert seen == {"per_sequence", "split", "ranges"}, seen


def test_write_then_decode(cuda):
    """The cache-write kernel at head_dim 80 into a cache the padded decode reads."""
    lens = [700, 1, 0, 2500, 64]
    c = decode_case(lens, seed=61, hq=32, hkv=2, head_dim=80, extra_blocks=3)
    q, _, _, bt, sl, ks, vs = to_dev(c, cuda)
    kc = torch.zeros(c.kc.shape, dtype=torch.int8, device=cuda)
    vc = torch.zeros_like(kc)
    int8kv.int8_kv_cache_write(c.key.to(cuda), c.value.to(cuda), kc, vc, c.slots.to(cuda), ks, vs)
    torch.cuda.synchronize()
    written = c.slots.numpy()
    nb, bs = c.kc.shape[:2]
    flat = lambda x: x.reshape(nb * bs, *x.shape[2:])[written]
    assert np.array_equal(flat(kc.cpu().numpy()), flat(c.kc))
    assert np.array_equal(flat(vc.cpu().numpy()), flat(c.vc))
    out = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs)
    torch.cuda.synchronize()
    _check(out, oracle_int8(c), "write then decode d=80")
