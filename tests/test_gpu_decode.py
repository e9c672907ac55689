"""GPU parity of INT8 / BF16 PagedAttention decode against the fp32 oracle.

Bar: max |out - oracle| <= 2e-2 and cosine >= 0.9999, where the oracle is
the reference's INT8 path run in fp32 (src/triton_ops/int8_paged_attention.py:776-814) on the
same int8 cache bytes.  Cases mirror the reference's tests (tests/test_int8_paged_attention.py:
108-323, tests/test_runtime_write_and_attention.py) plus the benchmark configurations, ragged
batches, block and chunk boundaries, strided views and every supported dtype.
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


def _check(out, ref, what=""):
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err, cos, rel = metrics(got, ref)
    print(f"{what}: max|diff|={err:.3e} cos={cos:.7f} relL2={rel:.3e}", flush=True)
    assert err <= MAX_ABS and cos >= MIN_COS, f"{what}: max|diff|={err} cos={cos}"
    return err, cos


def _int8(case, dev, **kw):
    q, kc, vc, bt, sl, ks, vs = to_dev(case, dev)
    out = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, **kw)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("lens,seed", [([127, 301], 0), ([97, 256], 1)])
@pytest.mark.parametrize("kw", [{}, {"impl": "v3"}, {"impl": "v4", "num_splits": 1},
                                {"impl": "v4", "num_splits": 4}, {"impl": "auto"}])
def test_reference_test_shapes(cuda, lens, seed, kw):
    """tests/test_int8_paged_attention.py:108-323 shapes and options (randn K/V)."""
    c = decode_case(lens, seed=seed, randn_kv=True, extra_blocks=20)
    _check(_int8(c, cuda, **kw), oracle_int8(c), f"{lens} {kw}")


def test_config0(cuda):
    c = decode_case([512], seed=0, extra_blocks=32)
    _check(_int8(c, cuda), oracle_int8(c), "cfg0")


@pytest.mark.parametrize("B", [1, 2, 4, 8])
@pytest.mark.parametrize("ctx", [512, 1024, 2048, 4096])
def test_config2_sweep(cuda, B, ctx):
    """Every config-2 point, INT8 (automatic layout and one range per sequence) and the BF16
    comparison kernel on the same K/V in a bf16 cache, each against the oracle."""
    c = decode_case([ctx] * B, seed=B * 7 + ctx)
    ref = oracle_int8(c)
    _check(_int8(c, cuda), ref, f"B={B} ctx={ctx} auto")
    _check(_int8(c, cuda, num_splits=1), ref, f"B={B} ctx={ctx} single-pass")
    kc, vc = bf16_caches(c)
    ref16 = O.paged_attention_ref(c.query.float().numpy(), kc.float().numpy(), vc.float().numpy(),
                                  c.block_tables.numpy(), c.seq_lens.numpy())
    for splits in (None, 1):
        out = int8kv.bf16_paged_attention(c.query.to(cuda), kc.to(cuda), vc.to(cuda),
                                          c.block_tables.to(cuda), c.seq_lens.to(cuda),
                                          num_splits=splits)
        torch.cuda.synchronize()
        _check(out, ref16, f"B={B} ctx={ctx} bf16 splits={splits}")


@pytest.mark.parametrize("lens", [
    [1], [2, 15, 16, 17], [31, 32, 33], [63, 64, 65], [127, 128, 129, 130],
    [511, 512, 513], [1, 4096, 3, 777], [1023, 1024, 1025, 2047, 2048, 2049],
])
def test_tile_block_chunk_boundaries(cuda, lens):
    c = decode_case(lens, seed=len(lens) * 31 + lens[0])
    ref = oracle_int8(c)
    for chunk in (None, 1, 3, 7):
        _check(_int8(c, cuda, num_splits=chunk), ref, f"{lens} splits={chunk}")
    for splits in (1, 3, 7):
        _check(ranges_call(c, cuda, splits), ref, f"{lens} {splits} ranges per sequence")


def test_one_token_sequences_return_v0(cuda):
    c = decode_case([1, 1, 1], seed=4)
    out = _int8(c, cuda).float().cpu().numpy()
    for b in range(3):
        blk = int(c.block_tables[b, 0])
        v0 = c.vc[blk, 0].astype(np.float32) * c.v_scale.numpy()[:, None]  # [Hkv, D]
        expect = np.repeat(v0, 7, axis=0)
        assert np.abs(out[b] - expect).max() <= 4e-3 * np.abs(expect).max()


def test_empty_sequence_gives_zeros(cuda):
    c = decode_case([300, 5], seed=5)
    sl = c.seq_lens.clone()
    sl[1] = 0
    q, kc, vc, bt, _, ks, vs = to_dev(c, cuda)
    out = int8kv.int8_paged_attention(q, kc, vc, bt, sl.to(cuda), ks, vs)
    torch.cuda.synchronize()
    ref = O.paged_attention_ref(c.query.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                sl.numpy(), c.k_scale.numpy(), c.v_scale.numpy())
    assert (out[1] == 0).all()
    _check(out, ref, "empty")


@pytest.mark.parametrize("qdtype", [torch.float16, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
def test_dtypes(cuda, qdtype, idx_dtype):
    c = decode_case([700, 33, 1500], seed=6)
    q = c.query.to(qdtype)
    q_d, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    out = int8kv.int8_paged_attention(q.to(cuda), kc, vc, bt.to(idx_dtype), sl.to(idx_dtype),
                                      ks, vs)
    torch.cuda.synchronize()
    assert out.dtype == qdtype and out.shape == q.shape
    _check(out, oracle_int8(c, query=q), f"q={qdtype} idx={idx_dtype}")


def test_strided_views(cuda):
    """Caches as views of the [num_blocks, 2, BS, Hkv, D] split layout, the query as a slice of a
    padded batch (vllm_int8_attention_patch.py:126-127) and a wider block table."""
    c = decode_case([400, 129, 1000], seed=8, width=80)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    kv = torch.empty((c.num_blocks, 2, 16, 4, 128), dtype=torch.int8, device=cuda)
    kv[:, 0] = kc
    kv[:, 1] = vc
    qpad = torch.zeros((5, 28, 128), dtype=q.dtype, device=cuda)
    qpad[:3] = q
    bt_wide = torch.zeros((3, 2 * bt.shape[1]), dtype=bt.dtype, device=cuda)
    bt_wide[:, ::2] = bt
    bt_view = bt_wide[:, ::2]  # non-unit column stride
    out = int8kv.int8_paged_attention(qpad[:3], kv[:, 0], kv[:, 1], bt_view, sl, ks, vs)
    torch.cuda.synchronize()
    _check(out, oracle_int8(c), "strided")


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 2), (32, 2), (12, 4)])
def test_group_sizes(cuda, hq, hkv):
    c = decode_case([333, 1200], seed=hq + hkv, hq=hq, hkv=hkv)
    _check(_int8(c, cuda), oracle_int8(c), f"Hq={hq} Hkv={hkv}")


def test_ragged_batch(cuda):
    lens = torch.randint(1, 4097, (16,), generator=torch.Generator().manual_seed(9)).tolist()
    c = decode_case(lens, seed=9)
    ref = oracle_int8(c)
    _check(_int8(c, cuda), ref, "ragged auto")
    _check(_int8(c, cuda, num_splits=2), ref, "ragged splits=2")


@pytest.mark.parametrize("cache_dtype", [torch.bfloat16, torch.float16])
def test_bf16_kernel(cuda, cache_dtype):
    lens = [127, 301, 1, 2048, 33]
    c = decode_case(lens, seed=10)
    kc, vc = bf16_caches(c, cache_dtype)
    ref = O.paged_attention_ref(c.query.float().numpy(), kc.float().numpy(), vc.float().numpy(),
                                c.block_tables.numpy(), c.seq_lens.numpy())
    dev = cuda
    for splits in (None, 1, 5):
        out = int8kv.bf16_paged_attention(c.query.to(dev), kc.to(dev), vc.to(dev),
                                          c.block_tables.to(dev), c.seq_lens.to(dev),
                                          num_splits=splits)
        torch.cuda.synchronize()
        _check(out, ref, f"{cache_dtype} splits={splits}")


def test_bf16_kernel_ignores_nonfinite_tail(cuda):
    """Cache rows past a sequence's end may hold NaN/Inf: they must not reach the output."""
    lens = [17, 40]
    c = decode_case(lens, seed=12)
    kc, vc = bf16_caches(c)
    written = torch.zeros(c.num_blocks * 16, dtype=torch.bool)
    written[c.slots] = True
    kf, vf = kc.view(-1, 4, 128).clone(), vc.view(-1, 4, 128).clone()
    kf[~written] = float("nan")
    vf[~written] = float("inf")
    kc, vc = kf.view_as(kc), vf.view_as(vc)
    ref = O.paged_attention_ref(c.query.float().numpy(), kc.float().numpy(), vc.float().numpy(),
                                c.block_tables.numpy(), c.seq_lens.numpy())
    out = int8kv.bf16_paged_attention(c.query.to(cuda), kc.to(cuda), vc.to(cuda),
                                      c.block_tables.to(cuda), c.seq_lens.to(cuda))
    torch.cuda.synchronize()
    _check(out, ref, "nan tail")


def test_int8_vs_bf16_quantisation_error(cuda):
    """INT8 path vs the BF16 kernel on the unquantised data: cos > 0.98
    (tests/test_int8_paged_attention.py:245-270)."""
    c = decode_case([127, 301], seed=0, randn_kv=True)
    kc, vc = bf16_caches(c)
    out8 = _int8(c, cuda).float().cpu().numpy()
    out16 = int8kv.bf16_paged_attention(c.query.to(cuda), kc.to(cuda), vc.to(cuda),
                                        c.block_tables.to(cuda), c.seq_lens.to(cuda))
    _, cos, _ = metrics(out8, out16.float().cpu().numpy())
    assert cos > 0.98


def test_write_then_decode_end_to_end(cuda):
    """runtime write -> decode (tests/test_runtime_write_and_attention.py:218-458)."""
    c = decode_case([127, 301], seed=0, randn_kv=True)
    kc = torch.zeros(c.num_blocks, 16, 4, 128, dtype=torch.int8, device=cuda)
    vc = torch.zeros_like(kc)
    int8kv.int8_kv_cache_write(c.key.to(cuda), c.value.to(cuda), kc, vc, c.slots.to(cuda),
                               c.k_scale.to(cuda), c.v_scale.to(cuda))
    out = int8kv.int8_paged_attention(c.query.to(cuda), kc, vc, c.block_tables.to(cuda),
                                      c.seq_lens.to(cuda), c.k_scale.to(cuda), c.v_scale.to(cuda))
    torch.cuda.synchronize()
    ref = O.paged_attention_ref(c.query.float().numpy(), kc.cpu().numpy(), vc.cpu().numpy(),
                                c.block_tables.numpy(), c.seq_lens.numpy(), c.k_scale.numpy(),
                                c.v_scale.numpy())
    _check(out, ref, "write->decode")


@pytest.mark.parametrize("lens", [[512], [1, 4096, 3, 777, 2048, 1500]])
def test_fp32_query_is_fp32_accurate(cuda, lens):
    """A genuine fp32 query (full 24-bit mantissas, not bf16 values) gives fp32 output within
    1e-4 of the fp32 oracle, for an INT8 and a BF16 cache: the kernel feeds the matrix cores the
    query as 16-bit hi + lo operands (two score MFMAs per k-step), and P as hi + lo for P*V.
    [512] runs the per-sequence layout, the ragged batch the range layout."""
    c = decode_case(lens, seed=21)
    q = torch.randn(c.query.shape, generator=torch.Generator().manual_seed(99))
    assert not torch.equal(q, q.bfloat16().float()), "the query must not be bf16-representable"
    _, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    out = int8kv.int8_paged_attention(q.to(cuda), kc, vc, bt, sl, ks, vs)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    err, cos, _ = metrics(out.cpu().numpy(), oracle_int8(c, query=q))
    print(f"fp32 int8 {lens}: max|diff|={err:.3e} cos={cos:.9f}", flush=True)
    assert err <= 1e-4 and cos >= 0.9999999
    k16, v16 = bf16_caches(c)
    ref16 = O.paged_attention_ref(q.numpy(), k16.float().numpy(), v16.float().numpy(),
                                  c.block_tables.numpy(), c.seq_lens.numpy())
    out16 = int8kv.bf16_paged_attention(q.to(cuda), k16.to(cuda), v16.to(cuda), bt, sl)
    torch.cuda.synchronize()
    err, cos, _ = metrics(out16.cpu().numpy(), ref16)
    print(f"fp32 bf16 {lens}: max|diff|={err:.3e} cos={cos:.9f}", flush=True)
    assert err <= 1e-4 and cos >= 0.9999999


@pytest.mark.parametrize("lens", [[127, 301], [1, 4096, 3, 777]])
@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float32])
def test_quantize_q(cuda, lens, qdtype):
    """quantize_q=True (src/triton_ops/int8_paged_attention.py:137-146, :798-802) against the
    oracle's quantise-dequantise of every query row."""
    c = decode_case(lens, seed=31)
    q = c.query.to(qdtype)
    q_d, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    out = int8kv.int8_paged_attention(q.to(cuda), kc, vc, bt, sl, ks, vs, quantize_q=True)
    torch.cuda.synchronize()
    ref = O.paged_attention_ref(q.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                c.seq_lens.numpy(), c.k_scale.numpy(), c.v_scale.numpy(),
                                quantize_q=True)
    _check(out, ref, f"quantize_q {lens} {qdtype}")
    if qdtype == torch.float32:
        err, _, _ = metrics(out.cpu().numpy(), ref)
        assert err <= 1e-4


def test_matches_reference_torch_checkers_on_device(cuda):
    """The reference's own test pattern: operator vs its torch checker, both on the GPU
    (tests/test_int8_paged_attention.py:108-323, tests/test_cache_write.py)."""
    from int8kv.torch_reference import (torch_int8_kv_cache_write_reference,
                                        torch_int8_paged_attention_reference)

    c = decode_case([33, 300, 1, 129], seed=21, randn_kv=True, extra_blocks=9)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    for quantize_q in (False, True):
        out = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, quantize_q=quantize_q)
        ref = torch_int8_paged_attention_reference(q.float(), kc, vc, bt, sl, ks, vs, quantize_q=quantize_q)
        _check(out, ref.cpu().numpy(), f"vs torch checker quantize_q={quantize_q}")
    # Cache write: operator and checker into two copies of the same sentinel-filled caches.
    k, v, slots = c.key.to(cuda), c.value.to(cuda), c.slots.to(cuda)
    a_k = torch.full_like(kc, 0x5A)
    a_v = torch.full_like(vc, 0x5A)
    b_k, b_v = a_k.clone(), a_v.clone()
    int8kv.int8_kv_cache_write(k, v, a_k, a_v, slots, ks, vs)
    torch_int8_kv_cache_write_reference(k, v, b_k, b_v, slots, ks, vs)
    torch.cuda.synchronize()
    assert torch.equal(a_k, b_k) and torch.equal(a_v, b_v)


def test_large_pool_streaming_path(cuda):
    """A pool whose reads can exceed 128 MB (half the Infinity Cache) takes the non-temporal
    streaming loads; results stay within the bar against the oracle, and equal the small-pool call
    on the same blocks when both use the same layout (one range per sequence: the automatic
    layout also depends on the table width, through the tiles in flight and the restart charge)."""
    c = decode_case([5, 700, 1234, 33], seed=41, extra_blocks=3)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    big_nb, width = 40000, 10000
    assert 4 * width * 16 * 4 * 128 * 2 > 128 << 20
    kb = torch.zeros(big_nb, 16, 4, 128, dtype=torch.int8, device=cuda)
    vb = torch.zeros_like(kb)
    kb[: kc.shape[0]] = kc
    vb[: vc.shape[0]] = vc
    btw = torch.zeros(bt.shape[0], width, dtype=bt.dtype, device=cuda)
    btw[:, : bt.shape[1]] = bt
    _check(int8kv.int8_paged_attention(q, kb, vb, btw, sl, ks, vs), oracle_int8(c), "large pool")
    small = ranges_call((q, kc, vc, bt, sl, ks, vs), cuda, 1)
    big = ranges_call((q, kb, vb, btw, sl, ks, vs), cuda, 1)
    _check(big, oracle_int8(c), "large pool, one range per sequence")
    assert torch.equal(small, big)
    # the int8-score kernel (quantize_q) on the streaming path as well
    small_q = ranges_call((q, kc, vc, bt, sl, ks, vs), cuda, 1, quantize_q=True)
    big_q = ranges_call((q, kb, vb, btw, sl, ks, vs), cuda, 1, quantize_q=True)
    ref_q = O.paged_attention_ref(c.query.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                  c.seq_lens.numpy(), c.k_scale.numpy(), c.v_scale.numpy(),
                                  quantize_q=True)
    _check(big_q, ref_q, "large pool quantize_q")
    assert torch.equal(small_q, big_q)


@pytest.mark.parametrize("block_size", [32, 64, 256])
def test_block_sizes(cuda, block_size):
    """Cache blocks of 32+ tokens (vLLM's other block sizes): oracle parity, INT8 and BF16, at
    block, tile and split boundaries."""
    lens = [1, 31, 32, 33, 63, 64, 65, 255, 256, 257, 1000, 2049]
    c = decode_case(lens, seed=block_size, block_size=block_size, extra_blocks=5)
    ref = oracle_int8(c)
    for splits in (None, 1, 3, 7):
        _check(_int8(c, cuda, num_splits=splits), ref, f"int8 bs={block_size} splits={splits}")
    for splits in (1, 3, 7):
        _check(ranges_call(c, cuda, splits), ref, f"int8 bs={block_size} {splits} ranges per seq")
    ref_q = O.paged_attention_ref(c.query.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                  c.seq_lens.numpy(), c.k_scale.numpy(), c.v_scale.numpy(),
                                  quantize_q=True)
    _check(_int8(c, cuda, quantize_q=True), ref_q, f"int8 quantize_q bs={block_size}")
    kc, vc = bf16_caches(c)
    ref16 = O.paged_attention_ref(c.query.float().numpy(), kc.float().numpy(), vc.float().numpy(),
                                  c.block_tables.numpy(), c.seq_lens.numpy())
    for splits in (None, 3):
        out = int8kv.bf16_paged_attention(c.query.to(cuda), kc.to(cuda), vc.to(cuda),
                                          c.block_tables.to(cuda), c.seq_lens.to(cuda),
                                          num_splits=splits)
        torch.cuda.synchronize()
        _check(out, ref16, f"bf16 bs={block_size} splits={splits}")


def test_block_size_relabelling_is_bit_exact(cuda):
    """A 32-token-block cache read as 16-token blocks (ids 2p, 2p + 1) is the same bytes in the
    same token order: the two calls must agree bit for bit, INT8 and BF16."""
    lens = [5, 32, 33, 700, 1, 4096, 95]
    c = decode_case(lens, seed=21, block_size=32, extra_blocks=3)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    nb = kc.shape[0]
    bt16 = torch.stack([2 * bt, 2 * bt + 1], dim=2).reshape(bt.shape[0], -1).contiguous()
    kc16, vc16 = kc.view(2 * nb, 16, 4, 128), vc.view(2 * nb, 16, 4, 128)
    for splits in (None, 1, 4):
        a = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, num_splits=splits)
        b = int8kv.int8_paged_attention(q, kc16, vc16, bt16, sl, ks, vs, num_splits=splits)
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"int8 splits={splits}"
        if splits is not None:
            a = ranges_call((q, kc, vc, bt, sl, ks, vs), cuda, splits)
            b = ranges_call((q, kc16, vc16, bt16, sl, ks, vs), cuda, splits)
            assert torch.equal(a, b), f"int8 {splits} ranges per sequence"
    k32, v32 = (x.to(cuda) for x in bf16_caches(c))
    a = int8kv.bf16_paged_attention(q, k32, v32, bt, sl)
    b = int8kv.bf16_paged_attention(q, k32.view(2 * nb, 16, 4, 128), v32.view(2 * nb, 16, 4, 128),
                                    bt16, sl)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_unsupported_block_sizes_raise(cuda):
    c = decode_case([40], seed=3)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    for bs in (8, 24, 48):
        kx = torch.zeros(64, bs, 4, 128, dtype=torch.int8, device=cuda)
        with pytest.raises(RuntimeError, match="E_SHAPE"):
            int8kv.int8_paged_attention(q, kx, kx.clone(), bt, sl, ks, vs)


def test_misaligned_query_is_copied(cuda):
    """A contiguous query at an odd storage offset (rows not 16-byte aligned) is read through an
    aligned copy; the result equals the aligned call bit for bit."""
    c = decode_case([77, 300], seed=12)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    buf = torch.empty(q.numel() + 1, dtype=q.dtype, device=cuda)
    q_odd = buf[1:].view(q.shape)
    q_odd.copy_(q)
    assert q_odd.data_ptr() % 16 != 0 and q_odd.is_contiguous()
    a = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs)
    b = int8kv.int8_paged_attention(q_odd, kc, vc, bt, sl, ks, vs)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def _pair_splits(hkv: int, batch: int) -> int:
    """Splits per sequence giving the range count of two waves per SIMD (twice the automatic
    count), the count at which INT8 workgroups take a pair of ranges."""
    from int8kv import _lib

    ranges = 2 * _lib.load().int8kv_decode_auto_ranges(hkv)
    assert ranges % batch == 0
    return ranges // batch


@pytest.mark.parametrize("hq,hkv,lens", [
    # 8485 stream units >= 16 x 512 ranges: paired workgroups for 4 kv heads
    (28, 4, [33000, 32768, 33001, 40000, 1, 33333, 32769, 34000]),
    # 4128 units >= 16 x 256 ranges (8 kv heads: two workgroups per range)
    (32, 8, [8192] * 15 + [8191]),
])
def test_paired_ranges_regime(cuda, hq, hkv, lens):
    """Two ranges per workgroup (the uneven first/second split) at the explicit range count of
    two waves per SIMD, against the oracle; the same inputs at the automatic count and with one
    range per sequence."""
    c = decode_case(lens, seed=hkv + len(lens), hq=hq, hkv=hkv)
    ref = oracle_int8(c)
    splits = _pair_splits(hkv, len(lens))
    _check(ranges_call(c, cuda, splits), ref, f"paired hq={hq} hkv={hkv}")
    _check(_int8(c, cuda), ref, f"automatic hq={hq} hkv={hkv}")
    _check(ranges_call(c, cuda, 1), ref, f"one range per sequence hq={hq} hkv={hkv}")
    _check(_int8(c, cuda, num_splits=1), ref, f"single pass hq={hq} hkv={hkv}")


@pytest.mark.parametrize("splits", [1, 2, None])
def test_four_tiles_in_flight(cuda, splits):
    """INT8 ranges of at least 32 stream units with at most one wave per SIMD keep four tiles of
    K/V loads in flight per wave (one or two ranges per sequence here; the automatic count cuts
    these short batches into short ranges, which keep two).  Tile counts leave 0-3 tiles after
    the last group of four (129, 258 = 256 + 2, 3, 4, 2, 1, 515 = 2 x 256 + 3 tiles); two
    sequences are longer than one 256-tile chunk of staged block ids; quantize_q as well."""
    lens = [4097, 8229, 65, 97, 33, 1, 16384 + 95, 640]
    c = decode_case(lens, seed=40 + (splits or 0), extra_blocks=5)
    ref = oracle_int8(c)

    def call(**kw):
        return _int8(c, cuda, **kw) if splits is None else ranges_call(c, cuda, splits, **kw)

    _check(call(), ref, f"splits={splits}")
    ref_q = O.paged_attention_ref(c.query.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                  c.seq_lens.numpy(), c.k_scale.numpy(), c.v_scale.numpy(),
                                  quantize_q=True)
    _check(call(quantize_q=True), ref_q, f"splits={splits} qq")


@pytest.mark.parametrize("how,splits", [("op", None), ("op", 1), ("op", 3), ("ranges", 1),
                                        ("ranges", 3)])
def test_batches_beyond_one_wave_of_sequences(cuda, how, splits):
    """B = 200 (four 64-sequence chunks in the kernels' batch walk) with ragged lengths, some
    empty sequences spread over the chunks, int64 lengths and tables."""
    g = torch.Generator().manual_seed(77)
    lens = torch.randint(1, 600, (200,), generator=g).tolist()
    c = decode_case(lens, seed=77, extra_blocks=11)
    sl = c.seq_lens.clone().to(torch.int64)
    for b in (0, 63, 64, 130, 199):
        sl[b] = 0
    q, kc, vc, bt, _, ks, vs = to_dev(c, cuda)
    if how == "op":
        out = int8kv.int8_paged_attention(q, kc, vc, bt.to(torch.int64), sl.to(cuda), ks, vs,
                                          num_splits=splits)
        torch.cuda.synchronize()
    else:
        out = ranges_call((q, kc, vc, bt.to(torch.int64), sl.to(cuda), ks, vs), cuda, splits)
    ref = O.paged_attention_ref(c.query.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                sl.numpy(), c.k_scale.numpy(), c.v_scale.numpy())
    for b in (0, 63, 64, 130, 199):
        assert (out[b] == 0).all(), b
    _check(out, ref, f"B=200 {how} splits={splits}")


@pytest.mark.parametrize("splits", [None, 3])
def test_batches_beyond_eight_chunks(cuda, splits):
    """B = 600: the merge kernel requests the lengths of the first 8 x 64 sequences at once and
    walks the rest chunk by chunk; sequences cut by range bounds on both sides of sequence 512,
    and empty ones in both parts, against the oracle."""
    g = torch.Generator().manual_seed(600)
    lens = torch.randint(1, 300, (600,), generator=g).tolist()
    lens[511], lens[512], lens[513] = 2000, 3000, 1500
    c = decode_case(lens, seed=600, extra_blocks=7)
    sl = c.seq_lens.clone()
    for b in (5, 300, 520, 599):
        sl[b] = 0
    q, kc, vc, bt, _, ks, vs = to_dev(c, cuda)
    # 3 ranges per sequence: the merge indexed by sequence (2 B < ranges)
    out = ranges_call((q, kc, vc, bt, sl.to(cuda), ks, vs), cuda, splits)
    ref = O.paged_attention_ref(c.query.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                sl.numpy(), c.k_scale.numpy(), c.v_scale.numpy())
    for b in (5, 300, 520, 599):
        assert (out[b] == 0).all(), b
    _check(out, ref, f"B=600 splits={splits}")


@pytest.mark.parametrize("how", ["auto", "single_pass", "ranges_auto", "ranges_512", "ranges_x2",
                                 "bf16"])
def test_thousands_of_short_sequences(cuda, how):
    """B = 5000 ragged sequences of 0-40 tokens (79 chunks of 64 in every batch walk, a fifth of
    them empty): the automatic call, the single pass (5000 x 4 per-sequence workgroups), the range
    layout at its automatic count, at 512 ranges (paired ranges) and at 2 ranges per sequence
    (10,000 ranges, the merge indexed by range), and the BF16 kernel, against the oracle."""
    g = torch.Generator().manual_seed(5000)
    lens = torch.randint(1, 41, (5000,), generator=g)
    lens[torch.rand(5000, generator=g) < 0.2] = 0
    lens = lens.tolist()
    c = decode_case(lens, seed=5000, extra_blocks=9)
    t = to_dev(c, cuda)
    q, kc, vc, bt, sl, ks, vs = t
    if how == "bf16":
        k16, v16 = (x.to(cuda) for x in bf16_caches(c))
        out = int8kv.bf16_paged_attention(q, k16, v16, bt, sl)
        torch.cuda.synchronize()
        ref = O.paged_attention_ref(c.query.float().numpy(), k16.float().cpu().numpy(),
                                    v16.float().cpu().numpy(), c.block_tables.numpy(),
                                    c.seq_lens.numpy())
    else:
        if how == "auto":
            out = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs)
        elif how == "single_pass":
            out = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, num_splits=1)
        elif how == "ranges_auto":
            out = ranges_call(t, cuda)
        elif how == "ranges_512":
            from int8kv import _decode
            out = torch.full_like(q, float("nan"))
            _decode.paged_decode(q, kc, vc, bt, sl, ks, vs, out, 512)
        else:
            out = ranges_call(t, cuda, 2)
        torch.cuda.synchronize()
        ref = oracle_int8(c)
    empty = [b for b, n in enumerate(lens) if n == 0]
    assert (out[empty] == 0).all()
    _check(out, ref, f"B=5000 {how}")


@pytest.mark.parametrize("lens", [[300_000], [200_000, 70_000, 0, 5]])
def test_sequences_beyond_the_range_cap(cuda, lens):
    """Sequences longer than the automatic range count can cut finely (300,000 tokens: ~9,400
    tiles, 37 per range at 256 ranges): the automatic call, the single pass (one workgroup per
    kv head streams the whole sequence), 64 split workgroups per (sequence, kv head), the range
    layout at its automatic count, and the BF16 kernel, against the oracle."""
    c = decode_case(lens, seed=len(lens), extra_blocks=3)
    t = to_dev(c, cuda)
    q, kc, vc, bt, sl, ks, vs = t
    ref = oracle_int8(c)
    for what, fn in (
            ("auto", lambda: int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs)),
            ("single pass", lambda: int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs,
                                                                num_splits=1)),
            ("64 splits", lambda: int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs,
                                                              num_splits=64)),
            ("ranges", lambda: ranges_call(t, cuda))):
        out = fn()
        torch.cuda.synchronize()
        if 0 in lens:
            assert (out[lens.index(0)] == 0).all(), what
        _check(out, ref, f"lens={lens} {what}")
    k16, v16 = (x.to(cuda) for x in bf16_caches(c))
    out16 = int8kv.bf16_paged_attention(q, k16, v16, bt, sl)
    torch.cuda.synchronize()
    ref16 = O.paged_attention_ref(c.query.float().numpy(), k16.float().cpu().numpy(),
                                  v16.float().cpu().numpy(), c.block_tables.numpy(),
                                  c.seq_lens.numpy())
    _check(out16, ref16, f"lens={lens} bf16")


@pytest.mark.parametrize("splits", [None, 3])
def test_wide_tables_take_the_64bit_unit_scan(cuda, splits):
    """A table wide enough that one sequence could hold 2^25 tiles (4096-token blocks, 2^18
    table entries per row) makes the kernels count stream units with 64-bit wave scans instead
    of the 32-bit DPP scan: oracle parity over B = 70 (two 64-sequence chunks), one empty
    sequence in each chunk."""
    g = torch.Generator().manual_seed(5)
    lens = torch.randint(1, 600, (70,), generator=g).tolist()
    lens[3], lens[66] = 9000, 4097
    c = decode_case(lens, seed=5, block_size=4096, width=1 << 18, extra_blocks=3)
    sl = c.seq_lens.clone()
    sl[10] = sl[65] = 0
    q, kc, vc, bt, _, ks, vs = to_dev(c, cuda)
    out = ranges_call((q, kc, vc, bt, sl.to(cuda), ks, vs), cuda, splits)
    ref = O.paged_attention_ref(c.query.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                sl.numpy(), c.k_scale.numpy(), c.v_scale.numpy())
    assert (out[10] == 0).all() and (out[65] == 0).all()
    _check(out, ref, f"64-bit unit scan splits={splits}")


HD64_SHAPES = [(32, 8), (14, 2), (8, 8)]  # Llama-3.2-1B, Qwen2.5-0.5B, multi-head


@pytest.mark.parametrize("hq,hkv", HD64_SHAPES)
def test_head_dim_64(cuda, hq, hkv):
    """head_dim 64 (GQA models with 64-wide heads): INT8 and BF16 parity at tile, block and split
    boundaries, quantize_q, and an fp32 query."""
    lens = [1, 15, 16, 17, 31, 32, 33, 300, 1025, 2048]
    c = decode_case(lens, seed=hq + hkv, hq=hq, hkv=hkv, head_dim=64, extra_blocks=7)
    ref = oracle_int8(c)
    for splits in (None, 1, 3):
        _check(_int8(c, cuda, num_splits=splits), ref, f"d64 {hq}/{hkv} splits={splits}")
    for splits in (1, 3):
        _check(ranges_call(c, cuda, splits), ref, f"d64 {hq}/{hkv} {splits} ranges per seq")
    ref_q = O.paged_attention_ref(c.query.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                  c.seq_lens.numpy(), c.k_scale.numpy(), c.v_scale.numpy(),
                                  quantize_q=True)
    _check(_int8(c, cuda, quantize_q=True), ref_q, f"d64 {hq}/{hkv} quantize_q")
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    out32 = int8kv.int8_paged_attention(q.float(), kc, vc, bt, sl, ks, vs)
    torch.cuda.synchronize()
    err, _, _ = metrics(out32.cpu().numpy(), ref)
    assert err <= 1e-3, err
    k16, v16 = bf16_caches(c)
    ref16 = O.paged_attention_ref(c.query.float().numpy(), k16.float().numpy(), v16.float().numpy(),
                                  c.block_tables.numpy(), c.seq_lens.numpy())
    out16 = int8kv.bf16_paged_attention(q, k16.to(cuda), v16.to(cuda), bt, sl)
    torch.cuda.synchronize()
    _check(out16, ref16, f"d64 {hq}/{hkv} bf16")


def test_head_dim_64_paired_regime(cuda):
    """head_dim 64 at the range count of two waves per SIMD: 16 x 8192 tokens pair the ranges
    (32 q / 8 kv heads); 15 x 8192 + 77 tokens take the same grid with unpaired ranges (the
    device-side check on the actual units).  The automatic count and one range per sequence
    (four tiles in flight) as well."""
    for lens in ([8192] * 16, [8192] * 15 + [77]):
        c = decode_case(lens, seed=64 + len(lens), hq=32, hkv=8, head_dim=64, extra_blocks=3)
        ref = oracle_int8(c)
        _check(ranges_call(c, cuda, _pair_splits(8, len(lens))), ref, f"d64 large {lens[-1]}")
        _check(_int8(c, cuda), ref, f"d64 automatic {lens[-1]}")
        _check(ranges_call(c, cuda, 1), ref, f"d64 one range per sequence {lens[-1]}")
        _check(_int8(c, cuda, num_splits=1), ref, f"d64 single pass {lens[-1]}")


def test_unsupported_head_dims_raise(cuda):
    """head_dims the kernels do not run (not a multiple of 16, or above 256) fail before the C ABI
    with an AssertionError naming the supported set, on both operators and both host paths; the
    C ABI itself returns INT8KV_E_SHAPE."""
    from int8kv import _decode, _ext

    c = decode_case([40], seed=3)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    for d in (8, 72, 200, 272, 512):
        kx = torch.zeros(kc.shape[0], 16, 4, d, dtype=torch.int8, device=cuda)
        qx = torch.zeros(q.shape[0], q.shape[1], d, dtype=q.dtype, device=cuda)
        for debug in (False, True):  # the extension, then the ctypes path
            old = _decode.DEBUG_CHECKS
            _decode.DEBUG_CHECKS = debug
            try:
                with pytest.raises(AssertionError, match="multiple of 16"):
                    int8kv.int8_paged_attention(qx, kx, kx.clone(), bt, sl, ks, vs)
                with pytest.raises(AssertionError, match="multiple of 16"):
                    int8kv.bf16_paged_attention(qx, kx.bfloat16(), kx.bfloat16(), bt, sl)
            finally:
                _decode.DEBUG_CHECKS = old
        out = torch.empty_like(qx)
        with pytest.raises(RuntimeError, match="E_SHAPE"):
            _decode.paged_decode(qx, kx, kx.clone(), bt, sl, ks, vs, out)
    assert _ext.module() is not None


def _group(q, kc, vc, bt, sl, ks, vs, extra_flags=0):
    from int8kv import _decode, _lib

    out = torch.empty_like(q)
    _decode.paged_decode(q, kc, vc, bt, sl, ks, vs, out, 0,
                         _lib.DECODE_ALL | _lib.DECODE_PER_SEQUENCE | extra_flags)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("hq,hkv,d", [(28, 4, 128), (14, 2, 64), (8, 8, 128), (16, 8, 256),
                                    (8, 1, 256)])
def test_per_sequence_mode(cuda, hq, hkv, d):
    """One workgroup per (sequence, kv head) whose waves merge their states in LDS
    (INT8KV_DECODE_PER_SEQUENCE): against the oracle for INT8 (fp32 query too) and quantize_q,
    and for a BF16 cache; empty and one-token sequences, fewer tiles than waves (waves with no
    tiles), tile counts that do not divide evenly, a sequence longer than one 256-tile chunk."""
    from int8kv import _lib

    lens = [0, 1, 17, 33, 95, 257, 511, 4096, 8229, 300]
    c = decode_case(lens, seed=hq + d, hq=hq, hkv=hkv, head_dim=d, extra_blocks=9)
    ref = oracle_int8(c)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    out = _group(q, kc, vc, bt, sl, ks, vs)
    assert (out[0] == 0).all()
    _check(out, ref, f"per-sequence int8 {hq}/{hkv}/{d}")
    out32 = _group(q.float(), kc, vc, bt, sl, ks, vs)
    err, _, _ = metrics(out32.cpu().numpy(), ref)
    assert err <= 1e-3, err
    ref_q = O.paged_attention_ref(c.query.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                  c.seq_lens.numpy(), c.k_scale.numpy(), c.v_scale.numpy(),
                                  quantize_q=True)
    _check(_group(q, kc, vc, bt, sl, ks, vs, _lib.DECODE_QUANTIZE_Q), ref_q,
           f"per-sequence quantize_q {hq}/{hkv}/{d}")
    k16, v16 = bf16_caches(c)
    ref16 = O.paged_attention_ref(c.query.float().numpy(), k16.float().numpy(), v16.float().numpy(),
                                  c.block_tables.numpy(), c.seq_lens.numpy())
    _check(_group(q, k16.to(cuda), v16.to(cuda), bt, sl, None, None), ref16,
           f"per-sequence bf16 {hq}/{hkv}/{d}")


@pytest.mark.parametrize("block_size,table64,qdtype", [(64, True, torch.float32),
                                                      (32, True, torch.bfloat16),
                                                      (256, False, torch.float16)])
def test_per_sequence_mode_first_chunk_forms(cuda, block_size, table64, qdtype):
    """The per-sequence layout's first chunk: its waves load the first round of block ids as raw
    32-bit words (the high word of a 64-bit table too), build the query operand before those
    loads' wait, then stage any further rounds (a 9000-token sequence gives a wave 35 tiles,
    70 row groups: one more round).  Oracle parity with 64-bit and 32-bit tables, 32-256-token
    blocks (several row groups per block id), empty, one-token and block-boundary lengths."""
    lens = [0, 1, 9000, block_size, block_size + 1, 700]
    c = decode_case(lens, seed=block_size + 7, extra_blocks=7, block_size=block_size)
    ref = O.paged_attention_ref(c.query.to(qdtype).float().numpy(), c.kc, c.vc,
                                c.block_tables.numpy(), c.seq_lens.numpy(), c.k_scale.numpy(),
                                c.v_scale.numpy())
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    if table64:
        bt = bt.to(torch.int64)
    out = _group(q.to(qdtype), kc, vc, bt, sl, ks, vs)
    assert (out[0] == 0).all()
    _check(out, ref, f"per-sequence bs={block_size} table64={table64} {qdtype}")


@pytest.mark.parametrize("cache_dtype", [torch.bfloat16, torch.float16])
def test_sixteen_bit_cache_non_temporal_path(cuda, cache_dtype):
    """16-bit caches above the 128 MiB bound (8 sequences, 600-block tables over a pool of ~4,570
    blocks: ~150 MB of possible K/V reads) take the range kernel with non-temporal loads and K in
    the k_spread order (the plan reports it).  Oracle parity for a BF16 and an fp32 query, ragged lengths, one empty
    sequence and one sequence at the table's full width."""
    from int8kv import _lib

    lens = [9000, 0, 4097, 9600, 31, 7000, 2500, 8191]
    c = decode_case(lens, seed=77, width=600, extra_blocks=2000)
    k16, v16 = (x.to(cuda) for x in bf16_caches(c, cache_dtype))
    q, _, _, bt, sl, _, _ = to_dev(c, cuda)
    plan = _lib.decode_plan(q.dtype, cache_dtype, len(lens), 28, 4, 128, k16.shape[0], 16,
                            bt.shape[1])
    assert plan["layout"] == "ranges" and plan["non_temporal"] == 1, plan
    ref = O.paged_attention_ref(c.query.float().numpy(), k16.float().cpu().numpy(),
                                v16.float().cpu().numpy(), c.block_tables.numpy(),
                                c.seq_lens.numpy())
    op = int8kv.bf16_paged_attention
    out = op(q, k16, v16, bt, sl)
    torch.cuda.synchronize()
    assert (out[1] == 0).all()
    _check(out, ref, f"{cache_dtype} cache, bf16 query, non-temporal")
    out32 = op(q.float(), k16, v16, bt, sl)
    torch.cuda.synchronize()
    err, _, _ = metrics(out32.cpu().numpy(), ref)
    assert err <= 1e-3, err


@pytest.mark.parametrize("ranges", [100, 200, 201, 640])
def test_merge_grids_on_both_sides_of_the_rule(cuda, ranges):
    """The merge indexed by range (one workgroup per range, from the decode kernel's cut-sequence
    descriptors; taken when 2 x batch >= ranges: 100 and 200 ranges for B = 100) and the merge
    indexed by sequence (a scan of seq_lens; 201 and 640 ranges): oracle parity with sequences
    cut once, cut many ways (one 6000-token sequence), uncut and empty, INT8 with a bf16 and an
    fp32 query, quantize_q, and a BF16 cache."""
    from int8kv import _decode, _lib

    g = torch.Generator().manual_seed(100)
    lens = torch.randint(1, 400, (100,), generator=g).tolist()
    lens[50], lens[0], lens[99] = 6000, 2500, 1200
    for b in (3, 51, 98):
        lens[b] = 0
    c = decode_case(lens, seed=101, extra_blocks=5)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)

    def run(qq, k, v, kscale, vscale, flags=_lib.DECODE_ALL):
        out = torch.empty_like(qq)
        _decode.paged_decode(qq, k, v, bt, sl, kscale, vscale, out, ranges, flags, None, 2)
        torch.cuda.synchronize()
        return out

    ref = oracle_int8(c)
    out = run(q, kc, vc, ks, vs)
    for b in (3, 51, 98):
        assert (out[b] == 0).all(), b
    _check(out, ref, f"int8 ranges={ranges}")
    err, _, _ = metrics(run(q.float(), kc, vc, ks, vs).cpu().numpy(), ref)
    assert err <= 1e-3, f"fp32 query ranges={ranges}: {err}"
    ref_q = O.paged_attention_ref(c.query.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                  c.seq_lens.numpy(), c.k_scale.numpy(), c.v_scale.numpy(),
                                  quantize_q=True)
    _check(run(q, kc, vc, ks, vs, _lib.DECODE_ALL | _lib.DECODE_QUANTIZE_Q), ref_q,
           f"int8 quantize_q ranges={ranges}")
    k16, v16 = bf16_caches(c)
    ref16 = O.paged_attention_ref(c.query.float().numpy(), k16.float().numpy(), v16.float().numpy(),
                                  c.block_tables.numpy(), c.seq_lens.numpy())
    _check(run(q, k16.to(cuda), v16.to(cuda), None, None), ref16, f"bf16 ranges={ranges}")


def test_paired_ranges_with_the_range_indexed_merge(cuda):
    """B = 256 at two waves per SIMD (512 ranges for 4 kv heads): the ranges come in pairs (every
    range holds more than 16 stream units) and 2 x batch = ranges takes the merge indexed by range,
    whose descriptors carry the paired plan; against the oracle, INT8 with and without quantize_q,
    with empty sequences at both ends."""
    g = torch.Generator().manual_seed(256)
    lens = torch.randint(600, 1500, (256,), generator=g).tolist()
    lens[0] = lens[255] = lens[128] = 0
    lens[7] = 9000
    splits = _pair_splits(4, len(lens))
    assert splits == 2
    c = decode_case(lens, seed=256, extra_blocks=5)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    out = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, num_splits=splits)
    torch.cuda.synchronize()
    for b in (0, 128, 255):
        assert (out[b] == 0).all(), b
    _check(out, oracle_int8(c), "paired, merge by range")
    ref_q = O.paged_attention_ref(c.query.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                  c.seq_lens.numpy(), c.k_scale.numpy(), c.v_scale.numpy(),
                                  quantize_q=True)
    out_q = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, num_splits=splits, quantize_q=True)
    torch.cuda.synchronize()
    _check(out_q, ref_q, "paired quantize_q, merge by range")


# (head_dim, q heads, kv heads, cache, batch, table width in 16-token blocks, per-sequence?) on a
# 256-CU MI355X: the automatic choice's thresholds on both sides.
AUTO_LAYOUT_POINTS = [
    (64, 32, 8, "int8", 96, 64, True),      # 3 workgroups per CU, 4 tiles per wave
    (64, 32, 8, "int8", 160, 64, False),    # 5 per CU: past the 4-per-CU cap
    (64, 32, 8, "int8", 1, 96, True),       # 6 tiles per wave at any count
    (64, 32, 8, "int8", 2, 128, False),     # 8 tiles per wave: needs CUs / 8 = 32 workgroups
    (64, 32, 8, "int8", 4, 128, True),
    (64, 32, 8, "int8", 64, 160, False),    # 10 tiles per wave
    (64, 32, 8, "bf16", 8, 64, True),       # 16-bit cache: up to 4 tiles per wave
    (64, 32, 8, "bf16", 8, 96, False),
    (128, 28, 4, "bf16", 128, 32, True),    # 16-bit cache at 128: up to 3 workgroups per CU
    (128, 28, 4, "bf16", 200, 32, False),
    (128, 28, 4, "int8", 96, 32, False),    # INT8 at 128: at most one workgroup per CU
    (128, 28, 4, "int8", 48, 32, True),
    (128, 28, 4, "int8", 8, 64, False),     # few workgroups, 4 tiles per wave: the split layout
    (128, 28, 4, "int8", 1, 48, True),      # under a tile per split workgroup: per-sequence
    (256, 16, 8, "int8", 32, 32, True),     # 256: four waves per workgroup, 4 tiles per wave
    (256, 16, 8, "int8", 2, 32, False),     # few workgroups with 4 tiles per wave: the split layout
    (256, 16, 8, "int8", 128, 16, False),   # 4 workgroups per CU: past the 3-per-CU cap
    (256, 16, 8, "int8", 8, 64, False),     # 8 tiles per wave: needs CUs / 2 workgroups
    (256, 16, 8, "int8", 32, 64, True),
    (256, 16, 8, "bf16", 1, 16, True),      # 16-bit cache: 2 tiles per wave at any count
    (256, 16, 8, "bf16", 4, 32, False),     # 4 tiles per wave: needs CUs / 2 workgroups
    (256, 16, 8, "bf16", 16, 32, True),
]


def _forced_like(plan, q, kc, vc, bt, sl, ks, vs):
    """The call forced into the layout a plan names (flags, or the plan's explicit range count
    and minimum range for the range layout), which runs the same kernels as the automatic call
    the plan describes."""
    from int8kv import _decode, _lib

    out = torch.empty_like(q)
    if plan["layout"] == "per_sequence":
        args = (0, _lib.DECODE_ALL | _lib.DECODE_PER_SEQUENCE, None, 0)
    elif plan["layout"] == "split":
        args = (0, _lib.DECODE_ALL | _lib.DECODE_SPLIT_SEQUENCES, None, 0)
    else:
        args = (plan["num_ranges"], _lib.DECODE_ALL, None, plan["min_tiles"])
    _decode.paged_decode(q, kc, vc, bt, sl, ks, vs, out, *args)
    torch.cuda.synchronize()
    return out


def _plan_of(q, kc, bt, cus=0):
    from int8kv import _lib

    return _lib.decode_plan(q.dtype, kc.dtype, q.shape[0], q.shape[1], kc.shape[2], q.shape[2],
                            kc.shape[0], kc.shape[1], bt.shape[1], kc.stride(2), kc.stride(2),
                            compute_units=cus)


@pytest.mark.parametrize("d,hq,hkv,cache,batch,width,per_seq", AUTO_LAYOUT_POINTS)
def test_automatic_layout_choice(cuda, d, hq, hkv, cache, batch, width, per_seq):
    """The automatic call (num_ranges = 0, min_tiles = 0) runs the layout int8kv_decode_plan
    reports for this device: its output is bit-identical to the call forced into that layout,
    and both match the oracle.  At 256 compute units the plan is the rule's choice on each side
    of its thresholds (the CPU tests check the rule itself, for other CU counts too).  Ragged
    lengths up to the table width, one empty sequence."""
    g = torch.Generator().manual_seed(batch * width + d)
    lens = torch.randint(1, width * 16 + 1, (batch,), generator=g).tolist()
    lens[0] = width * 16
    if batch > 2:
        lens[batch // 2] = 0
    c = decode_case(lens, seed=batch + width, hq=hq, hkv=hkv, head_dim=d, width=width,
                    extra_blocks=3)
    assert c.block_tables.shape[1] == width
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    q = q.float()  # fp32 outputs: a bf16 rounding could hide a different summation order
    if cache == "int8":
        ref = oracle_int8(c)
        auto = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs)
    else:
        k16, v16 = bf16_caches(c)
        ref = O.paged_attention_ref(c.query.float().numpy(), k16.float().numpy(),
                                    v16.float().numpy(), c.block_tables.numpy(), c.seq_lens.numpy())
        kc, vc, ks, vs = k16.to(cuda), v16.to(cuda), None, None
        auto = int8kv.bf16_paged_attention(q, kc, vc, bt, sl)
    plan = _plan_of(q, kc, bt)
    assert (_plan_of(q, kc, bt, 256)["layout"] == "per_sequence") == per_seq
    forced = _forced_like(plan, q, kc, vc, bt, sl, ks, vs)
    torch.cuda.synchronize()
    _check(auto, ref, f"automatic {cache} d={d} B={batch} width={width} ({plan['layout']})")
    _check(forced, ref, f"forced {plan['layout']} {cache} d={d} B={batch} width={width}")
    assert torch.equal(auto, forced)


@pytest.mark.parametrize("hq,hkv,d", [(28, 4, 128), (32, 8, 64), (16, 8, 256), (8, 1, 128)])
def test_split_sequences_layout(cuda, hq, hkv, d):
    """INT8KV_DECODE_SPLIT_SEQUENCES: several per-sequence workgroups per (sequence, kv head),
    each leaving one record per query head, combined by merge_split_kernel.  Few long sequences
    with an empty one and one shorter than the split count (workgroups without tiles leave
    neutral records); INT8 with bf16 and fp32 queries, quantize_q, a BF16 cache."""
    from int8kv import _decode, _lib

    lens = [9000, 0, 5, 30000] if d < 256 else [9000, 0, 5, 12000]
    c = decode_case(lens, seed=hq + d + 5, hq=hq, hkv=hkv, head_dim=d, extra_blocks=4)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    flags = _lib.DECODE_ALL | _lib.DECODE_SPLIT_SEQUENCES

    def run(qq, k, v, kscale, vscale, extra=0):
        out = torch.full_like(qq, float("nan"))
        _decode.paged_decode(qq, k, v, bt, sl, kscale, vscale, out, 0, flags | extra)
        torch.cuda.synchronize()
        return out

    ref = oracle_int8(c)
    out = run(q, kc, vc, ks, vs)
    assert (out[1] == 0).all()
    _check(out, ref, f"split int8 {hq}/{hkv}/{d}")
    err, _, _ = metrics(run(q.float(), kc, vc, ks, vs).cpu().numpy(), ref)
    assert err <= 1e-3, err
    ref_q = O.paged_attention_ref(c.query.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                  c.seq_lens.numpy(), c.k_scale.numpy(), c.v_scale.numpy(),
                                  quantize_q=True)
    _check(run(q, kc, vc, ks, vs, _lib.DECODE_QUANTIZE_Q), ref_q, f"split quantize_q {hq}/{hkv}/{d}")
    k16, v16 = bf16_caches(c)
    ref16 = O.paged_attention_ref(c.query.float().numpy(), k16.float().numpy(), v16.float().numpy(),
                                  c.block_tables.numpy(), c.seq_lens.numpy())
    _check(run(q, k16.to(cuda), v16.to(cuda), None, None), ref16, f"split bf16 {hq}/{hkv}/{d}")


# (head_dim, q heads, kv heads, batch, table width in 16-token blocks, split?) on 256 CUs.
AUTO_SPLIT_POINTS = [
    (128, 28, 4, 1, 2048, True),     # 64 workgroups per kv head, 2 tiles per wave
    (128, 28, 4, 8, 2048, False),    # 8 workgroups per kv head, 16 tiles per wave
    (64, 32, 8, 1, 256, True),       # head_dim 64: 32 workgroups, under one tile per wave
    (64, 32, 8, 4, 1024, False),     # head_dim 64: 8 tiles per wave (paired range layout)
    (256, 16, 8, 1, 1024, True),     # head_dim 256: four waves, 4 tiles per wave
    (128, 28, 4, 16, 512, False),    # 4 workgroups per (sequence, kv head)
    (128, 28, 4, 8, 64, True),       # preferred to the per-sequence layout: 4 tiles per wave there
    (128, 28, 4, 1, 48, False),      # per-sequence layout: under a tile per split workgroup
    (256, 16, 8, 2, 32, True),       # preferred to the four-wave per-sequence layout at 256
]


@pytest.mark.parametrize("d,hq,hkv,batch,width,split", AUTO_SPLIT_POINTS)
def test_automatic_split_choice(cuda, d, hq, hkv, batch, width, split):
    """The automatic call runs the layout the plan reports for this device (bit-identical to the
    call forced into it, both against the oracle); at 256 compute units that is the split layout
    exactly where the rule says."""
    g = torch.Generator().manual_seed(batch * width + d + 1)
    lens = torch.randint(1, width * 16 + 1, (batch,), generator=g).tolist()
    lens[0] = width * 16
    c = decode_case(lens, seed=batch + width + 1, hq=hq, hkv=hkv, head_dim=d, width=width,
                    extra_blocks=3)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    q = q.float()  # fp32 outputs: a bf16 rounding could hide a different summation order
    auto = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs)
    plan = _plan_of(q, kc, bt)
    assert (_plan_of(q, kc, bt, 256)["layout"] == "split") == split
    forced = _forced_like(plan, q, kc, vc, bt, sl, ks, vs)
    ref = oracle_int8(c)
    _check(auto, ref, f"automatic d={d} B={batch} width={width} ({plan['layout']})")
    _check(forced, ref, f"forced {plan['layout']} d={d} B={batch} width={width}")
    assert torch.equal(auto, forced)
