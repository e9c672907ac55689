"""CPU checks of the C ABI: the library loads, exports every declared symbol, and rejects bad
arguments before touching the GPU."""

from __future__ import annotations

import ctypes
import re

import pytest

from conftest import REPO

HEADERS = sorted((REPO / "include").glob("*.h"))


def _declared_functions():
    names = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names.update(re.findall(r"\b(int8kv_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    from int8kv import _lib

    if not _lib.LIB_PATH.exists():
        pytest.fail("libint8kv.so is not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_declares_expected_entry_points():
    assert [h.name for h in HEADERS] == ["int8kv.h", "int8kv_decode_loop.h", "int8kv_probe.h"]
    assert _declared_functions() == [
        "int8kv_add_rms_norm",
        "int8kv_argmax_rows",
        "int8kv_cache_write",
        "int8kv_decode_auto_ranges",
        "int8kv_decode_plan",
        "int8kv_decode_workspace_bytes",
        "int8kv_dynamic_cache_write",
        "int8kv_paged_decode",
        "int8kv_paged_decode_noalloc",
        "int8kv_probe_clock",
        "int8kv_probe_decode_loads",
        "int8kv_probe_stream_read",
        "int8kv_rotary_cache_write",
        "int8kv_rotary_inplace",
        "int8kv_silu_mul",
        "int8kv_version",
    ]


def test_library_exports_every_declared_symbol(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} missing from libint8kv.so"
    assert lib.int8kv_version().decode().startswith("int8kv ")


def test_workspace_bytes(lib):
    # per range: 2 slots x 28 query heads x (128 accumulators + max + sum) fp32, and the range's
    # 32-byte cut-sequence descriptor (sequence id, unit of its last tile, the batch's units)
    def per_range(hq, d):
        return 2 * hq * (d + 2) * 4 + 32

    assert lib.int8kv_decode_workspace_bytes(28, 4, 128, 16, 512) == 512 * per_range(28, 128)
    assert lib.int8kv_decode_workspace_bytes(28, 4, 128, 16, 1) == per_range(28, 128)
    assert per_range(28, 128) % 16 == 0 and per_range(7, 64) % 16 == 0
    # head_dims below 64, 128 or 256 keep records of that width
    for d, hd in ((16, 64), (32, 64), (96, 128), (80, 128), (192, 256)):
        assert lib.int8kv_decode_workspace_bytes(28, 4, d, 16, 9) == 9 * per_range(28, hd)
    # unsupported sizes -> 0
    for d in (0, 8, 24, 72, 272, 512):  # head_dim: a multiple of 16 in [16, 256]
        assert lib.int8kv_decode_workspace_bytes(28, 4, d, 16, 0) == 0
    assert lib.int8kv_decode_workspace_bytes(16, 8, 256, 16, 5) == 5 * per_range(16, 256)
    assert lib.int8kv_decode_workspace_bytes(28, 4, 64, 16, 3) == 3 * per_range(28, 64)
    for bs in (8, 24, 48, 1 << 17):  # block size: a power of two in [16, 65536]
        assert lib.int8kv_decode_workspace_bytes(28, 4, 128, bs, 0) == 0
    for bs in (16, 32, 64, 1 << 16):  # the partials do not depend on the block size
        assert lib.int8kv_decode_workspace_bytes(28, 4, 128, bs, 7) == 7 * per_range(28, 128)
    assert lib.int8kv_decode_workspace_bytes(30, 4, 128, 16, 0) == 0  # not a whole group
    # group 17: two column tiles per kv head, the automatic count of 4 grid heads
    assert lib.int8kv_decode_workspace_bytes(34, 2, 128, 16, 0) == \
        lib.int8kv_decode_auto_ranges(4) * per_range(34, 128)
    assert lib.int8kv_decode_workspace_bytes(28, 4, 128, 16, -1) == 0
    assert lib.int8kv_decode_workspace_bytes(28, 4, 128, 16, (1 << 20) + 1) == 0
    # automatic: a few workgroups per compute unit (no GPU here: the library assumes 256 CUs)
    auto = lib.int8kv_decode_auto_ranges(4)
    assert auto >= 1
    assert lib.int8kv_decode_workspace_bytes(28, 4, 128, 16, 0) == \
        lib.int8kv_decode_workspace_bytes(28, 4, 128, 16, auto)
    assert lib.int8kv_decode_auto_ranges(8) * 2 == auto


def _decode_call(lib, **over):
    st3 = (ctypes.c_int64 * 3)(28 * 128, 128, 1)
    st4 = (ctypes.c_int64 * 4)(16 * 4 * 128, 4 * 128, 128, 1)
    st2 = (ctypes.c_int64 * 2)(8, 1)
    args = dict(query=16, query_dtype=2, batch=1, num_q_heads=28, head_dim=128, qs=st3,
                kc=16, vc=16, cache_dtype=3, num_blocks=8, block_size=16, num_kv_heads=4,
                kcs=st4, vcs=st4, bt=16, table_dtype=4, width=8, bts=st2, sl=16, sl_dtype=4,
                ks=16, vs=16, sm=0.088, out=16, os=st3, ws=16, wsb=1 << 30, ranges=0,
                min_tiles=0, flags=3, stream=None)
    args.update(over)
    return lib.int8kv_paged_decode(*args.values())


def test_probes_reject_bad_arguments_without_launching(lib):
    P = 16  # fake device pointers: every call fails validation first
    sink = 1 << 20
    assert lib.int8kv_probe_stream_read(None, 1024, 0, P, 256, None) == -1
    assert lib.int8kv_probe_stream_read(P, 1000, 0, P, 256, None) == -4   # not whole 16 B
    assert lib.int8kv_probe_stream_read(P, 1024, 0, P, 100, None) == -3   # sink of 256s
    probe = lambda **o: lib.int8kv_probe_decode_loads(*{**dict(
        kc=P, vc=P, nb=1024, hkv=4, ids=P, nids=2 * 8 * 16, ranges=8, tiles=16, nt=0, sink=P,
        words=sink, stream=None), **o}.values())
    assert probe(hkv=8) == -3 and probe(nids=10) == -3 and probe(words=100) == -3
    assert probe(ranges=0) == -3 and probe(kc=None) == -1 and probe(kc=24) == -4
    assert lib.int8kv_probe_clock(None, 4, 100, None) == -1
    assert lib.int8kv_probe_clock(P, 0, 100, None) == -3 and lib.int8kv_probe_clock(P, 65536, 100, None) == -3
    assert lib.int8kv_probe_clock(P, 4, 0, None) == -3 and lib.int8kv_probe_clock(P, 4, 1000001, None) == -3
    assert lib.int8kv_probe_clock(P + 4, 4, 100, None) == -4


def test_decode_rejects_bad_arguments_without_launching(lib):
    # Fake (never dereferenced) device pointers: every call below fails validation first.
    assert _decode_call(lib, query_dtype=3) == -2
    assert _decode_call(lib, cache_dtype=4) == -2
    assert _decode_call(lib, table_dtype=2) == -2
    assert _decode_call(lib, head_dim=72) == -3
    assert _decode_call(lib, head_dim=272) == -3
    assert _decode_call(lib, block_size=8) == -3
    assert _decode_call(lib, block_size=48) == -3
    assert _decode_call(lib, num_q_heads=30) == -3
    assert _decode_call(lib, ranges=-1) == -3
    assert _decode_call(lib, min_tiles=-1) == -3
    assert _decode_call(lib, query=None) == -1
    assert _decode_call(lib, ks=None) == -1
    st3 = (ctypes.c_int64 * 3)(28 * 128, 128, 2)
    assert _decode_call(lib, qs=st3) == -4
    assert _decode_call(lib, query=24) == -4  # misaligned
    assert _decode_call(lib, out=40) == -4  # misaligned output
    # the partial workspace is always required
    assert _decode_call(lib, ws=None) == -5
    assert _decode_call(lib, wsb=1000) == -5
    assert _decode_call(lib, ws=24) == -5
    assert _decode_call(lib, batch=0) == 0  # nothing to do


def test_noalloc_decode_rejects_without_touching_the_device(lib):
    """int8kv_paged_decode_noalloc validates like int8kv_paged_decode, then refuses a call whose
    partials exceed the fixed scratch array (INT8KV_E_SCRATCH) -- before any device call."""

    def call(**over):
        args = dict(query=16, query_dtype=2, batch=1, num_q_heads=28, head_dim=128,
                    qs=(ctypes.c_int64 * 3)(28 * 128, 128, 1), kc=16, vc=16, cache_dtype=3,
                    num_blocks=8, block_size=16, num_kv_heads=4,
                    kcs=(ctypes.c_int64 * 4)(16 * 4 * 128, 4 * 128, 128, 1),
                    vcs=(ctypes.c_int64 * 4)(16 * 4 * 128, 4 * 128, 128, 1), bt=16,
                    table_dtype=4, width=8, bts=(ctypes.c_int64 * 2)(8, 1), sl=16, sl_dtype=4,
                    ks=16, vs=16, sm=0.088, out=16, os=(ctypes.c_int64 * 3)(28 * 128, 128, 1),
                    ranges=0, min_tiles=0, flags=3, stream=None)
        args.update(over)
        return lib.int8kv_paged_decode_noalloc(*args.values())

    limit = 16 << 20  # INT8KV_DECODE_SCRATCH_BYTES
    per_range = lib.int8kv_decode_workspace_bytes(28, 4, 128, 16, 1)
    too_many = limit // per_range + 1
    assert call(ranges=too_many) == -6
    assert call(ranges=too_many, num_q_heads=56) == -6
    assert call(query_dtype=3) == -2 and call(head_dim=72) == -3 and call(query=None) == -1
    assert call(query=24) == -4
    assert call(batch=0) == 0


def test_write_rejects_bad_arguments_without_launching(lib):
    st3 = (ctypes.c_int64 * 3)(512, 128, 1)
    st4 = (ctypes.c_int64 * 4)(16 * 512, 512, 128, 1)

    def call(**over):
        a = dict(key=16, value=16, src=2, T=4, hkv=4, d=128, ks_=st3, vs_=st3, kc=16, vc=16,
                 nb=4, bs=16, kcs=st4, vcs=st4, slots=16, sdt=5, k_scale=16, v_scale=16,
                 stream=None)
        a.update(over)
        return lib.int8kv_cache_write(*a.values())

    assert call(src=3) == -2
    assert call(sdt=2) == -2
    assert call(d=100) == -3
    assert call(key=None) == -1
    assert call(kcs=(ctypes.c_int64 * 4)(16 * 512, 512, 128, 2)) == -4
    assert call(key=8) == -4
    assert call(T=0) == 0


def test_dynamic_write_rejects_bad_arguments_without_launching(lib):
    st3 = (ctypes.c_int64 * 3)(512, 128, 1)
    st4 = (ctypes.c_int64 * 4)(16 * 512, 512, 128, 1)
    sc3 = (ctypes.c_int64 * 3)(64, 4, 1)

    def call(**over):
        a = dict(key=16, value=16, src=2, T=4, hkv=4, d=128, ks_=st3, vs_=st3, kc=16, vc=16,
                 nb=4, bs=16, kcs=st4, vcs=st4, ksc=16, vsc=16, kscs=sc3, vscs=sc3, slots=16,
                 sdt=5, stream=None)
        a.update(over)
        return lib.int8kv_dynamic_cache_write(*a.values())

    assert call(src=3) == -2
    assert call(d=96) == -3  # 12 lanes per row: not a power of two
    assert call(d=1024) == -3  # more than one wave per row
    assert call(ksc=None) == -1
    assert call(kscs=None) == -1
    assert call(ksc=18) == -4  # misaligned fp32 scale cache
    assert call(key=8) == -4
    assert call(T=0) == 0


def test_loop_ops_reject_bad_arguments_without_launching(lib):
    """Fake device pointers; every call below fails validation before any launch."""
    E_NULL, E_SHAPE, E_STRIDE = -1, -3, -4
    P = 256  # 16-byte aligned fake pointer
    # add_rms_norm(residual, delta, weight, out, rows, hidden, rs, ds, os, eps, stream)
    ok = dict(r=P, d=P, w=P, o=P, rows=4, hidden=512, rs=512, ds=512, os=512, eps=1e-6, s=None)

    def norm(**kw):
        a = dict(ok, **kw)
        return lib.int8kv_add_rms_norm(*a.values())

    assert norm(r=None) == E_NULL and norm(w=None) == E_NULL and norm(o=None) == E_NULL
    assert norm(hidden=12) == E_SHAPE and norm(hidden=8200) == E_SHAPE and norm(rows=-1) == E_SHAPE
    assert norm(r=P + 2) == E_STRIDE and norm(rs=500) == E_STRIDE and norm(ds=4) == E_STRIDE
    assert norm(rows=0) == 0  # nothing to do, nothing launched
    # rotary_inplace(qkv, rows, row_stride, num_heads, head_dim, positions, cos, sin, max_pos, stream)
    rot = dict(q=P, rows=4, rs=4608, heads=32, d=128, pos=P, c=P, s=P, maxp=10, st=None)

    def rope(**kw):
        a = dict(rot, **kw)
        return lib.int8kv_rotary_inplace(*a.values())

    assert rope(pos=None) == E_NULL and rope(c=None) == E_NULL
    assert rope(d=120) == E_SHAPE and rope(maxp=0) == E_SHAPE and rope(heads=0) == E_SHAPE
    assert rope(rs=4000) == E_STRIDE and rope(c=P + 4) == E_STRIDE
    assert rope(rows=0) == 0
    # silu_mul(gate_up, out, rows, ffn, in_stride, out_stride, stream)
    assert lib.int8kv_silu_mul(None, P, 4, 64, 128, 64, None) == E_NULL
    assert lib.int8kv_silu_mul(P, P, 4, 60, 120, 60, None) == E_SHAPE
    assert lib.int8kv_silu_mul(P, P, 4, 64, 64, 64, None) == E_STRIDE
    assert lib.int8kv_silu_mul(P, P, 0, 64, 128, 64, None) == 0
    # rotary_cache_write(qkv, rows, rs, hq, hkv, d, pos, cos, sin, maxp, bt, width, bts, nb, bs,
    #                    dtype, kc, vc, kcs, vcs, ks, vs, stream)
    st4 = (ctypes.c_int64 * 4)(16 * 4 * 128, 4 * 128, 128, 1)
    bad4 = (ctypes.c_int64 * 4)(16 * 4 * 128, 4 * 128, 128, 2)
    rw = dict(q=P, rows=4, rs=4608, hq=28, hkv=4, d=128, pos=P, c=P, s=P, maxp=10, bt=P, width=8,
              bts=8, nb=64, bs=16, dt=3, kc=P, vc=P, kcs=st4, vcs=st4, ks=P, vs=P, st=None)

    def rope_write(**kw):
        a = dict(rw, **kw)
        return lib.int8kv_rotary_cache_write(*a.values())

    assert rope_write(bt=None) == E_NULL and rope_write(ks=None) == E_NULL
    assert rope_write(dt=0) == -2  # fp32 caches are not a decode-loop format
    assert rope_write(ks=None, vs=None, dt=2, rows=0) == 0  # bf16 caches need no scales
    assert rope_write(d=120) == E_SHAPE and rope_write(nb=0) == E_SHAPE and rope_write(bs=0) == E_SHAPE
    assert rope_write(rs=4000) == E_STRIDE and rope_write(kcs=bad4) == E_STRIDE
    assert rope_write(kc=P + 4) == E_STRIDE
    assert rope_write(rows=0) == 0
    # argmax_rows(logits, rows, vocab, row_stride, out, stream)
    assert lib.int8kv_argmax_rows(None, 4, 100, 100, P, None) == E_NULL
    assert lib.int8kv_argmax_rows(P, 4, 0, 100, P, None) == E_SHAPE
    assert lib.int8kv_argmax_rows(P, 4, 1 << 31, 1 << 31, P, None) == E_SHAPE
    assert lib.int8kv_argmax_rows(P, 4, 100, 99, P, None) == E_STRIDE
    assert lib.int8kv_argmax_rows(P, 0, 100, 100, P, None) == 0
