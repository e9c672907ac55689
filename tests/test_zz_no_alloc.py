"""The no-allocation decode entry point, int8kv_paged_decode_noalloc, called through the C ABI.

It must give exactly what int8kv_paged_decode gives with a caller's workspace (same kernels,
same plan, partials in the library's fixed scratch array instead).  Two calls in a row on the
same GPU, the second with a smaller input, both bit-identical to the workspace entry point and
within the oracle bar; then the INT8 x BF16-cache and forced-range variants, a BF16 cache above the
non-temporal bound, the merge indexed by range, head_dim 256, head_dim 64 (kv-head pairs,
per-sequence layout) and the split per-sequence layout, a padded head_dim and a group above 16.
"""

from __future__ import annotations

import math

import pytest
import torch

from cases import bf16_caches, decode_case, oracle_int8, to_dev
from conftest import MAX_ABS, MIN_COS, metrics
from int8kv import _decode, _lib

pytestmark = pytest.mark.gpu


def _noalloc(q, kc, vc, bt, sl, ks, vs, out, num_ranges=0, flags=_lib.DECODE_ALL):
    lib = _lib.load()
    B, Hq, D = q.shape
    nb, bs, hkv, _ = kc.shape
    status = lib.int8kv_paged_decode_noalloc(
        q.data_ptr(), _lib.DTYPE_CODE[q.dtype], B, Hq, D, _lib.strides(q), kc.data_ptr(),
        vc.data_ptr(), _lib.DTYPE_CODE[kc.dtype], nb, bs, hkv, _lib.strides(kc), _lib.strides(vc),
        bt.data_ptr(), _lib.DTYPE_CODE[bt.dtype], bt.shape[1], _lib.strides(bt), sl.data_ptr(),
        _lib.DTYPE_CODE[sl.dtype], ks.data_ptr() if ks is not None else None,
        vs.data_ptr() if vs is not None else None, 1.0 / math.sqrt(D), out.data_ptr(),
        _lib.strides(out), num_ranges, 0, flags, _lib.stream_handle(q.device))
    _lib.check(status, "int8kv_paged_decode_noalloc")
    return out


def _with_workspace(q, kc, vc, bt, sl, ks, vs, num_ranges=0):
    out = torch.full_like(q, float("nan"))
    need = _lib.load().int8kv_decode_workspace_bytes(q.shape[1], kc.shape[2], q.shape[2],
                                                     kc.shape[1], num_ranges)
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=q.device)
    return _decode.paged_decode(q, kc, vc, bt, sl, ks, vs, out, num_ranges, workspace=ws)


# (lengths, seed, forced range count): the first call is the larger one.
CALLS = [
    ([4096, 1, 777, 2048, 3000, 15, 4096, 1500], 31, 0),
    ([300, 3, 150], 32, 6),
]


def test_two_calls_match_the_workspace_entry_point(cuda):
    for lens, seed, ranges in CALLS:
        print(f"noalloc: lens={lens} ranges={ranges}", flush=True)
        c = decode_case(lens, seed=seed)
        q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
        want = _with_workspace(q, kc, vc, bt, sl, ks, vs, ranges)
        got = _noalloc(q, kc, vc, bt, sl, ks, vs, torch.full_like(q, float("nan")), ranges)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"lens={lens}: outputs differ from int8kv_paged_decode"
        err, cos, _ = metrics(got.float().cpu().numpy(), oracle_int8(c))
        assert err <= MAX_ABS and cos >= MIN_COS, (lens, err, cos)


def test_bf16_cache_and_paired_ranges(cuda):
    c = decode_case([4096, 1, 2500, 4096, 333, 4096, 2048, 4000], seed=33)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    for ranges in (512, 0):  # 512: two ranges per workgroup (INT8); 0: automatic
        want = _with_workspace(q, kc, vc, bt, sl, ks, vs, ranges)
        got = _noalloc(q, kc, vc, bt, sl, ks, vs, torch.full_like(q, float("nan")), ranges)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"int8, ranges={ranges}"
    k16, v16 = (t.to(cuda) for t in bf16_caches(c))
    want = _with_workspace(q, k16, v16, bt, sl, None, None)
    got = _noalloc(q, k16, v16, bt, sl, None, None, torch.full_like(q, float("nan")))
    torch.cuda.synchronize()
    assert torch.equal(got, want), "bf16 cache"


def test_bf16_cache_above_the_non_temporal_bound(cuda):
    """A BF16 cache whose call may read ~150 MB (600-block tables over a ~4,570-block pool): the
    range kernel with non-temporal loads, the same from both entry points."""
    c = decode_case([9000, 0, 4097, 9600, 31, 7000, 2500, 8191], seed=78, width=600,
                    extra_blocks=2000)
    q, _, _, bt, sl, _, _ = to_dev(c, cuda)
    k16, v16 = (t.to(cuda) for t in bf16_caches(c))
    plan = _lib.decode_plan(q.dtype, k16.dtype, q.shape[0], 28, 4, 128, k16.shape[0], 16,
                            bt.shape[1], no_alloc=True)
    assert plan["non_temporal"] == 1, plan
    want = _with_workspace(q, k16, v16, bt, sl, None, None)
    got = _noalloc(q, k16, v16, bt, sl, None, None, torch.full_like(q, float("nan")))
    torch.cuda.synchronize()
    assert torch.equal(got, want), "bf16 cache, non-temporal"


def test_range_indexed_merge_and_head_dim_256(cuda):
    """A batch of at least half the range count (the merge indexed by range, whose per-range
    descriptors then live in the scratch array too), followed by a smaller head_dim-256 call."""
    g = torch.Generator().manual_seed(35)
    lens = torch.randint(1, 900, (160,), generator=g).tolist()
    lens[7], lens[80] = 6000, 0
    for case, what in ((decode_case(lens, seed=35, extra_blocks=4), "B=160 range merge"),
                       (decode_case([700, 3, 2500, 64], seed=36, hq=16, hkv=8, head_dim=256,
                                    extra_blocks=3), "head_dim 256")):
        print(f"noalloc: {what}", flush=True)
        q, kc, vc, bt, sl, ks, vs = to_dev(case, cuda)
        want = _with_workspace(q, kc, vc, bt, sl, ks, vs)
        got = _noalloc(q, kc, vc, bt, sl, ks, vs, torch.full_like(q, float("nan")))
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{what}: outputs differ from int8kv_paged_decode"
        err, cos, _ = metrics(got.float().cpu().numpy(), oracle_int8(case))
        assert err <= MAX_ABS and cos >= MIN_COS, (what, err, cos)


def test_head_dim_64_and_split_layouts(cuda):
    """head_dim 64 with kv heads taken in pairs (twice the automatic range count, sized by the
    entry point from the pairs), a short call that takes the per-sequence layout, then one long
    sequence in the split per-sequence layout (its records in the scratch array)."""
    for lens, seed, hq, hkv, d, what in (
            ([5000, 1, 3000, 0, 4100, 77], 37, 32, 8, 64, "head_dim 64 pairs"),
            ([300, 12, 512], 38, 32, 8, 64, "head_dim 64 per-sequence"),
            ([30000], 39, 28, 4, 128, "one long sequence, split per-sequence layout")):
        print(f"noalloc: {what}", flush=True)
        case = decode_case(lens, seed=seed, hq=hq, hkv=hkv, head_dim=d, extra_blocks=3)
        q, kc, vc, bt, sl, ks, vs = to_dev(case, cuda)
        want = _with_workspace(q, kc, vc, bt, sl, ks, vs)
        got = _noalloc(q, kc, vc, bt, sl, ks, vs, torch.full_like(q, float("nan")))
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{what}: outputs differ from int8kv_paged_decode"
        err, cos, _ = metrics(got.float().cpu().numpy(), oracle_int8(case))
        assert err <= MAX_ABS and cos >= MIN_COS, (what, err, cos)


def test_large_group_fits_the_scratch_with_fewer_ranges(cuda):
    """A GQA group whose automatic range count's partials exceed the 16 MiB array (32 query
    heads per 2 kv heads at head_dim 128: 512 ranges would need 17.1 MB) runs with the most
    ranges the array holds (int8kv_decode_plan reports the count) instead of being refused: the
    same bits as the workspace entry point at that range count, within the oracle bar."""
    g = torch.Generator().manual_seed(41)
    lens = torch.randint(1, 3000, (64,), generator=g).tolist()
    c = decode_case(lens, seed=41, hq=32, hkv=2, extra_blocks=3)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    args = (q.dtype, kc.dtype, 64, 32, 2, 128, kc.shape[0], 16, bt.shape[1])
    small = _lib.decode_plan(*args, no_alloc=True)
    full = _lib.decode_plan(*args)
    assert small["layout"] == full["layout"] == "ranges"
    assert small["num_ranges"] < full["num_ranges"] and small["workspace_bytes"] <= 16 << 20
    got = _noalloc(q, kc, vc, bt, sl, ks, vs, torch.full_like(q, float("nan")))
    want = _with_workspace(q, kc, vc, bt, sl, ks, vs, small["num_ranges"])
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    err, cos, _ = metrics(got.float().cpu().numpy(), oracle_int8(c))
    assert err <= MAX_ABS and cos >= MIN_COS, (err, cos)


def test_padded_head_dim_and_groups_above_16(cuda):
    """A head_dim of 80 (records of the 128-wide kernels in the scratch array), then a smaller
    call with 71 query heads on one kv head (five column tiles of the same kv head)."""
    for lens, seed, hq, hkv, d, what in (
            ([5000, 1, 3000, 0, 4100, 77, 900, 2600], 42, 16, 2, 80, "head_dim 80, group 8"),
            ([700, 3, 1500], 43, 71, 1, 64, "71 query heads, one kv head")):
        print(f"noalloc: {what}", flush=True)
        case = decode_case(lens, seed=seed, hq=hq, hkv=hkv, head_dim=d, extra_blocks=3)
        q, kc, vc, bt, sl, ks, vs = to_dev(case, cuda)
        for ranges in (0, 2 * len(lens)):
            want = _with_workspace(q, kc, vc, bt, sl, ks, vs, ranges)
            got = _noalloc(q, kc, vc, bt, sl, ks, vs, torch.full_like(q, float("nan")), ranges)
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"{what}, ranges={ranges}"
        err, cos, _ = metrics(got.float().cpu().numpy(), oracle_int8(case))
        assert err <= MAX_ABS and cos >= MIN_COS, (what, err, cos)


def test_oversized_request_is_refused(cuda):
    c = decode_case([64], seed=34)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    out = torch.zeros_like(q)
    per_range = _lib.load().int8kv_decode_workspace_bytes(28, 4, 128, 16, 1)
    with pytest.raises(_lib.Int8KVError, match="INT8KV_E_SCRATCH"):
        _noalloc(q, kc, vc, bt, sl, ks, vs, out, (16 << 20) // per_range + 1)
    torch.cuda.synchronize()
    assert not out.any()  # nothing was launched
