"""Seeded random decode configurations against the oracle.

Each case draws a batch (1-47 sequences; lengths up to 64, 600, 3000 or 9000 tokens, some empty),
a GQA shape (group 1-16, including one kv head), head_dim 64 or 128, a cache block size of 16-256
tokens, the query dtype, the table and length dtypes, the split count, ``impl`` and
``quantize_q``, then checks ``int8_paged_attention`` (and, for a third of the cases,
``bf16_paged_attention`` on the same K/V in a 16-bit cache) against the fp32 oracle at the
usual bar (max |diff| <= 2e-2, cosine >= 0.9999; empty sequences exactly zero).  Three more sets
repeat the draws at head_dim 256, at head_dim 64, and forced into the split per-sequence layout.  The
seeds are fixed, so a failure names a reproducible case.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import int8kv
from cases import bf16_caches, decode_case, to_dev
from conftest import MAX_ABS, MIN_COS, metrics
from oracle import int8kv_oracle as O

pytestmark = pytest.mark.gpu

SHAPES = [(28, 4), (32, 8), (14, 2), (8, 8), (16, 1), (12, 4), (40, 8), (6, 1)]
QDTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _draw(seed: int) -> dict:
    rng = np.random.default_rng(1000 + seed)
    hq, hkv = SHAPES[rng.integers(len(SHAPES))]
    B = int(rng.integers(1, 48))
    maxlen = int(rng.choice([64, 600, 3000, 9000]))
    lens = rng.integers(1, maxlen + 1, B)
    lens[rng.random(B) < 0.1] = 0
    while lens.sum() > 60000:
        lens = lens // 2
    return dict(hq=int(hq), hkv=int(hkv), d=int(rng.choice([64, 128])),
                bs=int(rng.choice([16, 16, 32, 64, 256])), lens=[int(x) for x in lens],
                qdtype=QDTYPES[rng.integers(3)], bt64=bool(rng.random() < 0.3),
                sl64=bool(rng.random() < 0.3), splits=[None, None, 1, 2, 5][rng.integers(5)],
                impl=["auto", "auto", "v3", "v4"][rng.integers(4)], qq=bool(rng.random() < 0.25),
                randn=bool(rng.random() < 0.5), bf16=bool(rng.random() < 0.34))


def _check(out, ref, lens, what):
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    empty = [b for b, n in enumerate(lens) if n == 0]
    assert all((got[b] == 0).all() for b in empty), f"{what}: empty sequence not zero"
    if all(n == 0 for n in lens):
        return
    err, cos, _ = metrics(got, ref)
    assert err <= MAX_ABS and cos >= MIN_COS, f"{what}: max|diff|={err} cos={cos}"


def _run(cuda, p, seed):
    what = f"seed {seed}: {p}"
    c = decode_case(p["lens"], seed=seed, hq=p["hq"], hkv=p["hkv"], head_dim=p["d"],
                    block_size=p["bs"], randn_kv=p["randn"], extra_blocks=5)
    q = c.query.to(p["qdtype"])
    _, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    if p["bt64"]:
        bt = bt.to(torch.int64)
    if p["sl64"]:
        sl = sl.to(torch.int64)
    out = int8kv.int8_paged_attention(q.to(cuda), kc, vc, bt, sl, ks, vs, quantize_q=p["qq"],
                                      impl=p["impl"], num_splits=p["splits"])
    torch.cuda.synchronize()
    assert out.dtype == p["qdtype"] and tuple(out.shape) == tuple(q.shape), what
    ref = O.paged_attention_ref(q.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                c.seq_lens.numpy(), c.k_scale.numpy(), c.v_scale.numpy(),
                                quantize_q=p["qq"])
    _check(out, ref, p["lens"], "int8 " + what)
    if p["bf16"]:
        k16, v16 = bf16_caches(c)
        out16 = int8kv.bf16_paged_attention(q.to(cuda), k16.to(cuda), v16.to(cuda), bt, sl,
                                            num_splits=p["splits"])
        torch.cuda.synchronize()
        ref16 = O.paged_attention_ref(q.float().numpy(), k16.float().numpy(), v16.float().numpy(),
                                      c.block_tables.numpy(), c.seq_lens.numpy())
        _check(out16, ref16, p["lens"], "bf16 " + what)


@pytest.mark.parametrize("seed", range(24))
def test_random_configuration(cuda, seed):
    _run(cuda, _draw(seed), seed)


@pytest.mark.parametrize("seed", range(100, 110))
def test_random_configuration_head_dim_256(cuda, seed):
    """The same random draws at head_dim 256 (GQA groups 1-8 as the Gemma family uses; 16-bit
    caches with bf16/fp16 queries, the fp32 query being covered in tests/test_gpu_decode_hd256.py)."""
    p = _draw(seed)
    hq, hkv = [(16, 8), (16, 16), (8, 1), (8, 2), (32, 4)][seed % 5]
    p.update(hq=hq, hkv=hkv, d=256)
    if p["qdtype"] == torch.float32 and p["bf16"]:
        p["qdtype"] = torch.bfloat16
    p["lens"] = [min(n, 4000) for n in p["lens"]]
    _run(cuda, p, seed)


@pytest.mark.parametrize("seed", range(200, 212))
def test_random_configuration_head_dim_64(cuda, seed):
    """The random draws at head_dim 64: even kv-head counts with groups up to 8 take kv heads in
    pairs in the range layout (32/8 as Llama-3.2-1B, 24/8 as Llama-3.2-3B, 16/2, 8/8), odd ones
    and group 12 do not (12/3, 24/2); short calls take the per-sequence layout."""
    p = _draw(seed)
    hq, hkv = [(32, 8), (24, 8), (16, 2), (8, 8), (12, 3), (24, 2)][seed % 6]
    p.update(hq=hq, hkv=hkv, d=64)
    _run(cuda, p, seed)


@pytest.mark.parametrize("seed", range(300, 310))
def test_random_configuration_split_layout(cuda, seed):
    """The random draws forced into the split per-sequence layout (INT8KV_DECODE_SPLIT_SEQUENCES:
    several per-sequence workgroups per sequence and kv head, records merged per query head) at
    head_dim 64, 128 and 256, with the drawn block size, table / length dtypes, query dtype and
    quantize_q; a 16-bit cache for a third of them."""
    from int8kv import _decode, _lib

    p = _draw(seed)
    d = (64, 128, 256)[seed % 3]
    hq, hkv = [(28, 4), (32, 8), (16, 8), (8, 1), (14, 2)][seed % 5]
    p.update(hq=hq, hkv=hkv, d=d)
    lens = p["lens"][:6]
    c = decode_case(lens, seed=seed, hq=hq, hkv=hkv, head_dim=d, block_size=p["bs"],
                    randn_kv=p["randn"], extra_blocks=5)
    q = c.query.to(p["qdtype"]).to(cuda)
    _, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    if p["bt64"]:
        bt = bt.to(torch.int64)
    if p["sl64"]:
        sl = sl.to(torch.int64)
    flags = _lib.DECODE_ALL | _lib.DECODE_SPLIT_SEQUENCES | (_lib.DECODE_QUANTIZE_Q if p["qq"] else 0)
    out = torch.full_like(q, float("nan"))
    _decode.paged_decode(q, kc, vc, bt, sl, ks, vs, out, 0, flags)
    torch.cuda.synchronize()
    what = f"seed {seed}: d={d} {hq}/{hkv} lens={lens} bs={p['bs']} {p['qdtype']} qq={p['qq']}"
    ref = O.paged_attention_ref(q.float().cpu().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                c.seq_lens.numpy(), c.k_scale.numpy(), c.v_scale.numpy(),
                                quantize_q=p["qq"])
    _check(out, ref, lens, "split int8 " + what)
    if p["bf16"]:
        k16, v16 = bf16_caches(c)
        out16 = torch.full_like(q, float("nan"))
        _decode.paged_decode(q, k16.to(cuda), v16.to(cuda), bt, sl, None, None, out16, 0,
                             _lib.DECODE_ALL | _lib.DECODE_SPLIT_SEQUENCES)
        torch.cuda.synchronize()
        ref16 = O.paged_attention_ref(q.float().cpu().numpy(), k16.float().numpy(),
                                      v16.float().numpy(), c.block_tables.numpy(),
                                      c.seq_lens.numpy())
        _check(out16, ref16, lens, "split bf16 " + what)


@pytest.mark.parametrize("seed", range(400, 416))
def test_random_configuration_padded_head_dims_and_wide_groups(cuda, seed):
    """The random draws at head_dims between the kernels' 64 / 128 / 256 (any multiple of 16, run
    on the next kernel with the padding masked) and GQA groups above 16 (several MFMA column tiles
    per kv head), with the drawn block size, dtypes, split count, impl and quantize_q."""
    p = _draw(seed)
    d = [16, 32, 48, 80, 96, 112, 144, 160, 176, 192, 208, 224, 240][seed % 13]
    hq, hkv = [(28, 4), (34, 2), (20, 1), (48, 3), (71, 1), (40, 8), (16, 16), (64, 2)][seed % 8]
    p.update(hq=hq, hkv=hkv, d=d)
    p["lens"] = [min(n, 3000) for n in p["lens"]][:24]
    if d > 128 and p["qdtype"] == torch.float32 and p["bf16"]:
        p["qdtype"] = torch.bfloat16
    _run(cuda, p, seed)
