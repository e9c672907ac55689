"""CPU tests of the decode planner (int8kv_decode_plan): the host-side choices of
int8kv_paged_decode -- layout, range count, minimum range, tiles in flight, range pairs, kv-head
pairs, merge kernel, non-temporal loads, workspace -- on both sides of every threshold, for
MI355X's 256 compute units and for other CU counts.  The query launches nothing and reads no
device memory, so it runs without a GPU (compute_units given explicitly).

The reference decides its split count and kernel on the host as well
(src/triton_ops/int8_paged_attention.py:39-58): these tests are the counterpart of reading those
two functions' outputs for given sizes.
"""

from __future__ import annotations

import pytest
import torch

from int8kv import _lib

I8, BF16, F16 = torch.int8, torch.bfloat16, torch.float16
Q = torch.bfloat16


@pytest.fixture(scope="module", autouse=True)
def _library():
    if not _lib.LIB_PATH.exists():
        pytest.fail("libint8kv.so is not built (run __graft_entry__.build())")
    _lib.load()


def plan(cache=I8, batch=1, hq=28, hkv=4, d=128, width=32, cus=256, nb=None, bs=16, query=Q,
         ranges=0, min_tiles=0, flags=_lib.DECODE_ALL, head_stride=None, no_alloc=False):
    nb = batch * width + 16 if nb is None else nb
    return _lib.decode_plan(query, cache, batch, hq, hkv, d, nb, bs, width,
                            head_stride, head_stride, ranges, min_tiles, flags, cus, no_alloc)


def layout(**kw):
    return plan(**kw)["layout"]


# ------------------------------------------------------------------ per-sequence layout rule
@pytest.mark.parametrize("cus", [256, 304, 80])
def test_int8_head_dim_128_one_workgroup_per_cu(cus):
    """INT8 at head_dim 128: short sequences (<= 3 tiles per wave of the 8-wave workgroup) take
    the per-sequence layout up to one workgroup per CU (4 kv heads: batch = CUs / 4)."""
    b = cus // 4
    assert layout(batch=b, width=32, cus=cus) == "per_sequence"      # 512 tokens, 2 per wave
    assert layout(batch=b + 1, width=32, cus=cus) == "ranges"
    assert layout(batch=b, width=48, cus=cus) == "per_sequence"      # 768 tokens, 3 per wave


@pytest.mark.parametrize("cus", [256, 304])
def test_int8_head_dim_128_longer_sequences_need_workgroups(cus):
    """4-8 tiles per wave: per-sequence only from (tiles per wave - 3) x CUs / 8 workgroups (at
    most CUs / 2)."""
    for per_wave, width in ((6, 96), (8, 128)):
        need = min((per_wave - 3) * cus // 8, cus // 2)
        b = -(-need // 4)  # smallest batch with 4 b >= need
        assert layout(batch=b, width=width, cus=cus) == "per_sequence", (per_wave, b)
        assert layout(batch=b - 1, width=width, cus=cus) == "ranges", (per_wave, b - 1)
    # 9 tiles per wave: never
    assert layout(batch=cus // 4, width=144, cus=cus) == "ranges"


@pytest.mark.parametrize("cus", [256, 304, 80])
def test_16bit_head_dim_128(cus):
    """16-bit caches at head_dim 128: the split layout for up to CUs / 8 workgroups once each of
    its workgroups gets a tile; otherwise the per-sequence layout up to 2 tiles per wave at any
    count, 4 from CUs / 2 workgroups, at most 3 workgroups per CU."""
    bmax = cus // 32                                   # 8 x (4 b) <= CUs
    assert layout(cache=BF16, batch=1, width=32, cus=cus) == "split"       # 16 tiles, Z = 16
    assert layout(cache=BF16, batch=bmax, width=32, cus=cus) == "split"
    assert layout(cache=BF16, batch=bmax + 1, width=32, cus=cus) == "per_sequence"
    assert layout(cache=BF16, batch=1, width=16, cus=cus) == "per_sequence"  # 8 tiles < Z = 16
    assert layout(cache=BF16, batch=3 * cus // 4, width=32, cus=cus) == "per_sequence"
    assert layout(cache=BF16, batch=3 * cus // 4 + 1, width=32, cus=cus) == "ranges"
    half = cus // 2
    assert layout(cache=BF16, batch=-(-half // 4), width=64, cus=cus) == "per_sequence"
    assert layout(cache=BF16, batch=-(-half // 4) - 1, width=64, cus=cus) != "per_sequence"


@pytest.mark.parametrize("cus", [256, 304])
def test_head_dim_64_rule(cus):
    """head_dim 64 (32 q / 8 kv heads): INT8 up to 6 tiles per wave at any count, 8 from CUs / 8
    workgroups, at most 4 workgroups per CU; 16-bit caches up to 4 tiles per wave."""
    kw = dict(hq=32, hkv=8, d=64, cus=cus)
    assert layout(batch=1, width=96, **kw) == "per_sequence"                 # 6 tiles per wave
    assert layout(batch=cus // 2, width=64, **kw) == "per_sequence"          # 4 per CU
    assert layout(batch=cus // 2 + 1, width=64, **kw) == "ranges"
    b = -(-(cus // 8) // 8)
    assert layout(batch=b, width=128, **kw) == "per_sequence"                # 8 tiles per wave
    assert layout(batch=b - 1, width=128, **kw) != "per_sequence"
    assert layout(cache=BF16, batch=8, width=64, **kw) == "per_sequence"     # 4 tiles per wave
    assert layout(cache=BF16, batch=8, width=96, **kw) != "per_sequence"


@pytest.mark.parametrize("cus", [256, 304])
def test_head_dim_256_rule(cus):
    """head_dim 256 (16 q / 8 kv heads, four-wave workgroups): INT8 up to 4 tiles per wave at up
    to 3 workgroups per CU (few workgroups with 3+ tiles per wave: the split layout); 8 tiles per
    wave from CUs / 2 to CUs workgroups."""
    kw = dict(hq=16, hkv=8, d=256, cus=cus)
    b = 3 * cus // 8
    assert layout(batch=b, width=32, **kw) == "per_sequence"
    assert layout(batch=b + 1, width=32, **kw) == "ranges"
    assert layout(batch=1, width=16, **kw) == "per_sequence"                 # 2 tiles per wave
    assert layout(batch=2, width=32, **kw) == "split"                        # few, 4 per wave
    lo = -(-(cus // 2) // 8)
    assert layout(batch=lo, width=64, **kw) == "per_sequence"
    assert layout(batch=lo - 1, width=64, **kw) != "per_sequence"
    assert layout(cache=BF16, batch=1, width=16, **kw) == "per_sequence"
    assert layout(cache=BF16, batch=4, width=32, **kw) != "per_sequence"


# ------------------------------------------------------------------ split layout rule
@pytest.mark.parametrize("cus", [256, 304, 80])
def test_split_rule(cus):
    """Few long sequences: at most CUs / 8 workgroups per kv-head grid and at most 4 tiles per wave
    of Z = min(CUs / workgroups, 64) workgroups of 8 waves."""
    p = plan(batch=1, width=2048, cus=cus)       # one 32k-token sequence
    z = min(cus // 4, 64)
    assert p["layout"] == ("split" if 1024 / (z * 8) <= 4 else "ranges")
    if p["layout"] == "split":
        assert p["split"] == z and p["kernels"] == 2 and p["merge"] == "split"
    bmax = cus // 32                              # 8 x (4 b) <= CUs
    assert layout(batch=bmax, width=256, cus=cus) == "split"
    assert layout(batch=bmax + 1, width=256, cus=cus) == "ranges"


def test_split_rule_at_256():
    """The thresholds as stated for MI355X (one 32k sequence splits 64 ways; 16 tiles per wave of
    8 sequences x 8 workgroups stays in the range layout)."""
    p = plan(batch=1, width=2048)
    assert (p["layout"], p["split"], p["merge_waves"]) == ("split", 64, 1)
    # At head_dim 128 at most max(16, tiles / 4) workgroups per sequence and kv head.
    for cache in (I8, BF16):
        for width, z in ((64, 16), (128, 16), (256, 32), (512, 64)):   # 1024-8192 tokens
            p = plan(cache=cache, batch=1, width=width)
            assert (p["layout"], p["split"]) == ("split", z), (cache, width, p)
        assert plan(cache=cache, batch=2, width=64)["split"] == 16
        assert plan(cache=cache, batch=2, width=256)["split"] == 32
    assert plan(hq=32, hkv=8, d=64, batch=1, width=256)["split"] == 32  # (no cap at 64)
    assert layout(batch=8, width=2048) == "ranges"
    assert layout(hq=32, hkv=8, d=64, batch=1, width=256) == "split"
    assert layout(hq=32, hkv=8, d=64, batch=4, width=1024) == "ranges"


def test_gpu_rule_points_at_256_cus():
    """The points the GPU layout tests run: the plan at 256 CUs is the rule's choice."""
    from test_gpu_decode import AUTO_LAYOUT_POINTS, AUTO_SPLIT_POINTS

    for d, hq, hkv, cache, batch, width, per_seq in AUTO_LAYOUT_POINTS:
        got = layout(cache=I8 if cache == "int8" else BF16, batch=batch, hq=hq, hkv=hkv, d=d,
                     width=width)
        assert (got == "per_sequence") == per_seq, (d, hq, hkv, cache, batch, width, got)
    for d, hq, hkv, batch, width, split in AUTO_SPLIT_POINTS:
        got = layout(batch=batch, hq=hq, hkv=hkv, d=d, width=width)
        assert (got == "split") == split, (d, hq, hkv, batch, width, got)


# ------------------------------------------------------------------ forced layouts
def test_forced_layouts():
    p = plan(batch=64, width=2048, flags=_lib.DECODE_ALL | _lib.DECODE_PER_SEQUENCE)
    assert (p["layout"], p["kernels"], p["merge"], p["non_temporal"]) == ("per_sequence", 1, "none", 0)
    # the reference's num_splits = S: S workgroups per (sequence, kv head), at most 64
    for s in (2, 3, 7, 64):
        p = plan(batch=5, width=512, ranges=5 * s, flags=_lib.DECODE_ALL | _lib.DECODE_SPLIT_SEQUENCES)
        assert (p["layout"], p["split"], p["kernels"], p["merge"]) == ("split", s, 2, "split")
        assert p["workspace_bytes"] == 5 * s * (2 * 28 * 130 * 4 + 32)
    p = plan(batch=5, width=512, ranges=5 * 100, flags=_lib.DECODE_ALL | _lib.DECODE_SPLIT_SEQUENCES)
    assert p["split"] == 64
    # the automatic split count fills the chip: min(CUs / (batch x kv heads), 64)
    p = plan(batch=2, width=512, flags=_lib.DECODE_ALL | _lib.DECODE_SPLIT_SEQUENCES)
    assert p["split"] == 32
    p = plan(batch=64, width=512, flags=_lib.DECODE_ALL | _lib.DECODE_SPLIT_SEQUENCES)
    assert (p["layout"], p["split"]) == ("per_sequence", 0)  # one workgroup per CU already
    assert plan(batch=0)["kernels"] == 0


# ------------------------------------------------------------------ range layout details
def test_min_tiles_rule():
    """2-tile minimum ranges unless that could cut one sequence into more than 128 ranges."""
    assert plan(batch=2, width=2048, ranges=256)["min_tiles"] == 2
    p = plan(batch=1, width=2048, ranges=256)
    assert p["min_tiles"] == 4 and p["layout"] == "ranges"
    assert plan(batch=1, width=508, ranges=256)["min_tiles"] == 2    # 256 units: 128 ranges
    assert plan(batch=1, width=512, ranges=256)["min_tiles"] == 4    # 258 units: 129 ranges


@pytest.mark.parametrize("cus", [256, 304])
def test_depth_and_start_charge(cus):
    """INT8 range layouts keep four tiles in flight when the longest possible batch holds at least
    32 units per range (and one wave per SIMD); the start charge follows (6 vs 4 units); an fp32
    query runs two; 16-bit caches two with a 2-unit charge."""
    ranges = 4 * cus // 4
    width = 252  # 126 tiles + 2 units per sequence
    need_b = -(-(32 * ranges) // 128)
    p = plan(batch=need_b, width=width, cus=cus)
    assert p["layout"] == "ranges" and p["num_ranges"] == ranges
    assert (p["depth"], p["seq_cost"]) == (4, 6)
    p = plan(batch=need_b - 1, width=width, cus=cus)
    assert (p["layout"], p["depth"], p["seq_cost"]) == ("ranges", 2, 4)
    assert plan(batch=need_b, width=width, cus=cus, query=torch.float32)["depth"] == 2
    p = plan(cache=BF16, batch=need_b, width=width, cus=cus)
    assert (p["depth"], p["seq_cost"]) == (2, 2)


def test_range_pairs():
    """Twice the automatic range count (two waves per SIMD) pairs the ranges of an INT8 call that
    can give every CU a pair of at least 16 units each."""
    p = plan(batch=64, width=2048, ranges=512)
    assert (p["ranges_per_workgroup"], p["depth"]) == (2, 2)
    p = plan(batch=2, width=1024, ranges=512)    # 2 x 514 units < 512 x 16
    assert p["ranges_per_workgroup"] == 1
    assert plan(cache=BF16, batch=64, width=2048, ranges=512)["ranges_per_workgroup"] == 1
    assert plan(batch=64, width=2048, ranges=256)["ranges_per_workgroup"] == 1


def test_merge_kernel_choice():
    """The range layout's second kernel: the merge indexed by range when 2 x batch >= ranges,
    else by sequence with waves and records per round from the ranges per sequence (bounded by
    the table width); the per-sequence layout has none, the split layout its own."""
    p = plan(batch=128, width=256)
    assert (p["layout"], p["merge"], p["merge_waves"], p["kernels"]) == ("ranges", "by_range", 1, 2)
    p = plan(batch=127, width=256)
    assert (p["merge"], p["merge_waves"], p["merge_fold"]) == ("by_sequence", 1, 4)
    p = plan(batch=8, width=2048, ranges=256)                     # 32 ranges per sequence
    assert (p["merge"], p["merge_waves"], p["merge_fold"]) == ("by_sequence", 4, 4)
    p = plan(batch=8, width=2048, ranges=8 * 100, min_tiles=2)    # 100 per sequence
    assert (p["merge_waves"], p["merge_fold"]) == (4, 8)
    p = plan(batch=1, width=2048, ranges=256, min_tiles=2)        # 256 per sequence
    assert (p["merge_waves"], p["merge_fold"]) == (8, 8)
    p = plan(batch=1, width=64, ranges=256, min_tiles=2)          # the table bounds it: 19
    assert (p["merge_waves"], p["merge_fold"]) == (4, 4)
    p = plan(batch=4, width=2048, ranges=64)                      # 16 per sequence
    assert (p["merge_waves"], p["merge_fold"]) == (2, 4)
    assert plan(batch=1, width=32)["merge"] == "none"
    assert plan(batch=1, width=2048)["merge"] == "split"


def test_non_temporal_threshold():
    """Non-temporal K/V loads when the call can read more than 128 MiB of K and V (min(pool,
    batch x width) blocks), range layout only: INT8 caches at every head_dim, 16-bit caches at
    head_dim 128 without padding or kv-head pairs (their K loads in the k_spread order)."""
    per_block = 16 * 4 * 128 * 2
    n = (128 << 20) // per_block  # 8192 blocks
    kw = dict(batch=64, ranges=256)  # the range layout at every width
    assert plan(width=n // 64, nb=n + 1000, **kw)["non_temporal"] == 0
    assert plan(width=n // 64 + 1, nb=n + 1000, **kw)["non_temporal"] == 1
    assert plan(width=4096, nb=n, **kw)["non_temporal"] == 0         # the pool bounds it
    # 16-bit caches: twice the bytes per block, so half the blocks reach the bound.
    assert plan(cache=BF16, width=n // 128, nb=n + 1000, **kw)["non_temporal"] == 0
    assert plan(cache=BF16, width=n // 128 + 1, nb=n + 1000, **kw)["non_temporal"] == 1
    assert plan(cache=F16, width=4096, nb=10 * n, **kw)["non_temporal"] == 1
    big = dict(width=4096, nb=10 * n, **kw)
    assert plan(cache=BF16, d=256, hq=16, hkv=8, **big)["non_temporal"] == 0   # head_dim 256
    assert plan(cache=BF16, d=96, **big)["non_temporal"] == 0                  # padded
    assert plan(cache=BF16, d=64, hq=32, hkv=8, **big)["non_temporal"] == 0    # kv-head pairs
    assert plan(cache=BF16, d=64, hq=12, hkv=3, **big)["non_temporal"] == 0    # head_dim 64
    assert plan(d=256, hq=16, hkv=8, **big)["non_temporal"] == 1               # INT8: all
    assert plan(cache=BF16, batch=1, width=256, nb=10 * n)["non_temporal"] == 0  # per-sequence


def test_kv_head_pairs():
    """head_dim 64: kv heads in pairs for an even kv-head count, groups up to 8 and a head stride
    of head_dim, in the range layout (its automatic count is that of the pairs)."""
    kw = dict(d=64, batch=64, width=2048)
    p = plan(hq=32, hkv=8, **kw)
    assert (p["layout"], p["kv_pair"], p["num_ranges"]) == ("ranges", 1, 256)
    strided = plan(hq=32, hkv=8, head_stride=128, **kw)
    assert (strided["kv_pair"], strided["num_ranges"]) == (0, 128)
    assert plan(hq=36, hkv=4, **kw)["kv_pair"] == 0    # group 9
    assert plan(hq=24, hkv=3, **kw)["kv_pair"] == 0    # odd kv-head count
    assert plan(hq=32, hkv=8, d=64, batch=1, width=64)["kv_pair"] == 0  # per-sequence layout


@pytest.mark.parametrize("cus", [256, 304, 80])
def test_automatic_range_count(cus):
    """One wave per SIMD: 4 x CUs / kv heads ranges (of kv-head pairs at head_dim 64)."""
    assert plan(batch=64, width=2048, cus=cus)["num_ranges"] == cus
    assert plan(batch=64, width=2048, cus=cus, hq=64, hkv=8)["num_ranges"] == cus // 2
    assert plan(batch=64, width=2048, cus=cus, hq=8, hkv=1)["num_ranges"] == 4 * cus


# ------------------------------------------------------------------ no-allocation entry point
def test_noalloc_lowers_the_automatic_range_count():
    """The no-allocation entry point's 16 MiB scratch: an automatic count whose partials do not
    fit is lowered to the most ranges that do; a given count that does not fit is refused."""
    cap = 16 << 20

    def per_range(hq, d):
        return 2 * hq * (d + 2) * 4 + 32

    for hq, hkv, d in ((32, 2, 128), (16, 1, 128), (64, 4, 128), (32, 4, 256)):
        full = plan(batch=64, width=2048, hq=hq, hkv=hkv, d=d)
        p = plan(batch=64, width=2048, hq=hq, hkv=hkv, d=d, no_alloc=True)
        assert full["workspace_bytes"] > cap
        assert p["num_ranges"] == cap // per_range(hq, d) < full["num_ranges"]
        assert p["workspace_bytes"] <= cap
    for hq, hkv, d in ((28, 4, 128), (60, 4, 128), (16, 8, 256)):
        full = plan(batch=64, width=2048, hq=hq, hkv=hkv, d=d)
        p = plan(batch=64, width=2048, hq=hq, hkv=hkv, d=d, no_alloc=True)
        assert p["num_ranges"] == full["num_ranges"] and p["workspace_bytes"] <= cap
    too_many = cap // per_range(28, 128) + 1
    with pytest.raises(_lib.Int8KVError, match="E_SCRATCH"):
        plan(batch=64, width=2048, ranges=too_many, no_alloc=True)
    assert plan(batch=64, width=2048, ranges=too_many)["num_ranges"] == too_many


# ------------------------------------------------------------------ widened shapes
def _per_range(hq, d):
    return 2 * hq * (d + 2) * 4 + 32


@pytest.mark.parametrize("d, hd", [(16, 64), (48, 64), (80, 128), (96, 128), (112, 128),
                                   (160, 256), (192, 256), (240, 256)])
def test_padded_head_dims(d, hd):
    """A head_dim below 64, 128 or 256 runs the next of those kernels: its records are that wide,
    the layout rules are those of the padded width, and the range layout keeps one range per
    workgroup with two tiles in flight (no pairs, no four-deep pipeline, no kv-head pairs)."""
    for kw in (dict(batch=64, width=2048), dict(batch=64, width=2048, ranges=512),
               dict(batch=64, width=252)):
        p = plan(d=d, **kw)
        ref = plan(d=hd, head_stride=hd + 16, **kw)  # (no kv-head pairs at 64)
        assert p["layout"] == ref["layout"] == "ranges"
        assert p["num_ranges"] == ref["num_ranges"]
        assert p["workspace_bytes"] == p["num_ranges"] * _per_range(28, hd)
        assert (p["ranges_per_workgroup"], p["depth"], p["kv_pair"]) == (1, 2, 0)
    for kw in (dict(batch=4, width=32), dict(batch=1, width=2048), dict(batch=64, width=16)):
        assert layout(d=d, **kw) == layout(d=hd, **kw)
    assert plan(d=d, hq=32, hkv=8, batch=64, width=2048)["kv_pair"] == 0


def test_groups_above_16_take_column_tiles():
    """More than 16 query heads per kv head: ceil(group / 16) waves per kv head, so the range
    count, the per-sequence and split rules and the workspace are those of kv heads x tiles."""
    for hq, hkv, tiles in ((34, 2, 2), (64, 1, 4), (71, 1, 5), (48, 2, 3), (128, 8, 1 * 8)):
        t = -(-(hq // hkv) // 16)
        grid = hkv * t
        for kw in (dict(batch=64, width=2048), dict(batch=2, width=32), dict(batch=1, width=4096)):
            p = plan(hq=hq, hkv=hkv, **kw)
            # the kv-head count with the same grid heads and group <= 16 takes the same layout
            ref = plan(hq=grid, hkv=grid, **kw)
            assert p["layout"] == ref["layout"], (hq, hkv, kw)
            assert p["num_ranges"] == ref["num_ranges"]
            assert p["workspace_bytes"] == p["num_ranges"] * _per_range(hq, 128)
    # MQA with 64 query heads: 4 grid heads, the automatic count of 4 kv heads
    assert plan(hq=64, hkv=1, batch=64, width=2048)["num_ranges"] == \
        plan(hq=28, hkv=4, batch=64, width=2048)["num_ranges"]


def test_plan_rejects_what_the_decode_rejects():
    for d in (8, 72, 100, 272, 512):  # head_dim: a multiple of 16 in [16, 256]
        with pytest.raises(_lib.Int8KVError, match="E_SHAPE"):
            plan(d=d)
    with pytest.raises(_lib.Int8KVError, match="E_SHAPE"):
        plan(bs=8)
    with pytest.raises(_lib.Int8KVError, match="E_SHAPE"):
        plan(hq=30, hkv=4)  # not a whole group
    with pytest.raises(_lib.Int8KVError, match="E_SHAPE"):
        plan(hq=65535 * 17, hkv=65535)  # 131070 grid heads
    with pytest.raises(_lib.Int8KVError, match="E_SHAPE"):
        plan(cus=-1)
    with pytest.raises(_lib.Int8KVError, match="E_DTYPE"):
        plan(cache=torch.float32)
