"""CPU checks of the C ABI: the library loads, exports every declared symbol, and rejects bad
arguments before touching the GPU."""

from __future__ import annotations

import ctypes
import re

import pytest

from conftest import REPO

HEADER = REPO / "include" / "int8kv.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(int8kv_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from int8kv import _lib

    if not _lib.LIB_PATH.exists():
        pytest.fail("libint8kv.so is not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_declares_expected_entry_points():
    assert _declared_functions() == [
        "int8kv_cache_write",
        "int8kv_decode_auto_chunk_tokens",
        "int8kv_decode_workspace_bytes",
        "int8kv_paged_decode",
        "int8kv_version",
    ]


def test_library_exports_every_declared_symbol(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} missing from libint8kv.so"
    assert lib.int8kv_version().decode().startswith("int8kv ")


def test_workspace_bytes(lib):
    # B=64, Hq=28, Hkv=4, D=128, width 2048 blocks, chunk 512 -> 64 chunks of partials
    n = lib.int8kv_decode_workspace_bytes(64, 28, 4, 128, 2048, 16, 512)
    assert n == 64 * 28 * 64 * (128 + 2) * 4
    # a single chunk per sequence needs no workspace
    assert lib.int8kv_decode_workspace_bytes(8, 28, 4, 128, 32, 16, 512) == 0
    # unsupported sizes -> 0
    assert lib.int8kv_decode_workspace_bytes(8, 28, 4, 64, 32, 16, 0) == 0
    assert lib.int8kv_decode_workspace_bytes(8, 28, 4, 128, 32, 32, 0) == 0
    assert lib.int8kv_decode_workspace_bytes(8, 34, 2, 128, 32, 16, 0) == 0  # group 17
    assert lib.int8kv_decode_workspace_bytes(8, 28, 4, 128, 32, 16, 48) == 0  # not /32
    auto = lib.int8kv_decode_auto_chunk_tokens(64, 4, 2048, 16)
    assert auto % 32 == 0 and 128 <= auto <= 4096
    assert lib.int8kv_decode_workspace_bytes(64, 28, 4, 128, 2048, 16, 0) == \
        lib.int8kv_decode_workspace_bytes(64, 28, 4, 128, 2048, 16, auto)


def _decode_call(lib, **over):
    st3 = (ctypes.c_int64 * 3)(28 * 128, 128, 1)
    st4 = (ctypes.c_int64 * 4)(16 * 4 * 128, 4 * 128, 128, 1)
    st2 = (ctypes.c_int64 * 2)(8, 1)
    args = dict(query=16, query_dtype=2, batch=1, num_q_heads=28, head_dim=128, qs=st3,
                kc=16, vc=16, cache_dtype=3, num_blocks=8, block_size=16, num_kv_heads=4,
                kcs=st4, vcs=st4, bt=16, table_dtype=4, width=8, bts=st2, sl=16, sl_dtype=4,
                ks=16, vs=16, sm=0.088, out=16, os=st3, ws=None, wsb=0, chunk=0, flags=3,
                stream=None)
    args.update(over)
    return lib.int8kv_paged_decode(*args.values())


def test_decode_rejects_bad_arguments_without_launching(lib):
    # Fake (never dereferenced) device pointers: every call below fails validation first.
    assert _decode_call(lib, query_dtype=3) == -2
    assert _decode_call(lib, cache_dtype=4) == -2
    assert _decode_call(lib, table_dtype=2) == -2
    assert _decode_call(lib, head_dim=64) == -3
    assert _decode_call(lib, block_size=32) == -3
    assert _decode_call(lib, num_q_heads=30) == -3
    assert _decode_call(lib, chunk=40) == -3
    assert _decode_call(lib, query=None) == -1
    assert _decode_call(lib, ks=None) == -1
    st3 = (ctypes.c_int64 * 3)(28 * 128, 128, 2)
    assert _decode_call(lib, qs=st3) == -4
    assert _decode_call(lib, query=24) == -4  # misaligned
    # needs partials (width 64 blocks = 1024 tokens > chunk 128) but no workspace
    st2 = (ctypes.c_int64 * 2)(64, 1)
    assert _decode_call(lib, width=64, bts=st2, chunk=128) == -5
    assert _decode_call(lib, batch=0) == 0  # nothing to do


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
