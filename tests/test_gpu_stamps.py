"""The measurement build libint8kv_stamps.so (bench.py --stamps): the same kernels with per-wave
s_memrealtime stamps.  Its outputs must be bit-identical to the product library's (the stamps only
read a clock and store at each wave's end), and every stored timeline must be ordered: entry <=
plan / sequence length <= first segment entered <= block ids staged <= query built <= first
scores <= first P*V <= segment done <= end (the per-sequence layout requests the query at entry
and builds it while the block ids are in flight: query built <= block ids staged there).
Covered: the INT8 range layout (several segments per wave), the INT8 per-sequence layout, the
BF16 split per-sequence layout, and the load-only probe."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from cases import bf16_caches, decode_case, to_dev
from int8kv import _build, _decode, _lib

pytestmark = pytest.mark.gpu

SLOTS = 10


@pytest.fixture(scope="module")
def slib():
    assert _build.STAMPS_LIB_PATH.exists(), "libint8kv_stamps.so is not built (__graft_entry__.build())"
    return _lib.bind(_build.STAMPS_LIB_PATH)


def _read(lib, unit):
    buf = np.zeros(16384 * SLOTS, np.uint64)
    _lib.check(getattr(lib, f"int8kv_stamps_read_{unit}")(buf.ctypes.data, buf.nbytes), "read")
    st = buf.reshape(-1, SLOTS).astype(np.int64)
    return st[st[:, 7] > 0]


def _noalloc(lib, q, kc, vc, bt, sl, ks, vs, num_ranges=0, flags=_lib.DECODE_ALL):
    out = torch.full_like(q, float("nan"))
    B, Hq, D = q.shape
    nb, bs, hkv, _ = kc.shape
    _lib.check(lib.int8kv_paged_decode_noalloc(
        q.data_ptr(), _lib.DTYPE_CODE[q.dtype], B, Hq, D, _lib.strides(q), kc.data_ptr(),
        vc.data_ptr(), _lib.DTYPE_CODE[kc.dtype], nb, bs, hkv, _lib.strides(kc), _lib.strides(vc),
        bt.data_ptr(), _lib.DTYPE_CODE[bt.dtype], bt.shape[1], _lib.strides(bt), sl.data_ptr(),
        _lib.DTYPE_CODE[sl.dtype], ks.data_ptr() if ks is not None else None,
        vs.data_ptr() if vs is not None else None, 1.0 / math.sqrt(D), out.data_ptr(),
        _lib.strides(out), num_ranges, 0, flags, _lib.stream_handle(q.device)), "stamps decode")
    torch.cuda.synchronize()
    return out


def _product(q, kc, vc, bt, sl, ks, vs, num_ranges=0, flags=_lib.DECODE_ALL):
    out = torch.full_like(q, float("nan"))
    need = _lib.load().int8kv_decode_workspace_bytes(q.shape[1], kc.shape[2], q.shape[2],
                                                     kc.shape[1], num_ranges)
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=q.device)
    _decode.paged_decode(q, kc, vc, bt, sl, ks, vs, out, num_ranges, flags, ws)
    torch.cuda.synchronize()
    return out


def _ordered(st, chain):
    d = np.diff(st[:, chain], axis=1)
    return bool((d >= 0).all())


def test_range_layout_int8(cuda, slib):
    c = decode_case([4096, 1, 777, 2048, 3000, 15, 4096, 1500, 0, 333], seed=71)
    t = to_dev(c, cuda)
    _lib.check(slib.int8kv_stamps_clear_i8(), "clear")
    got = _noalloc(slib, *t, num_ranges=24)  # a few ranges per sequence: cut sequences, merge
    want = _product(*t, num_ranges=24)
    assert torch.equal(got, want)
    st = _read(slib, "i8")
    print(f"range layout: {len(st)} waves stored", flush=True)
    assert 0 < len(st) <= 24 * 4
    assert (st[:, 8] < 8).all()  # XCD ids
    assert _ordered(st, [0, 1, 7])
    seg = st[st[:, 9] > 0]
    assert len(seg) > 0 and _ordered(seg, [0, 1, 9, 2, 3, 4, 5, 6, 7])


def test_split_layout_bf16(cuda, slib):
    c = decode_case([512, 300], seed=72)
    q, _, _, bt, sl, _, _ = to_dev(c, cuda)
    k16, v16 = (x.to(cuda) for x in bf16_caches(c))
    flags = _lib.DECODE_ALL | _lib.DECODE_SPLIT_SEQUENCES
    _lib.check(slib.int8kv_stamps_clear_bf16(), "clear")
    got = _noalloc(slib, q, k16, v16, bt, sl, None, None, num_ranges=16 * 2, flags=flags)
    want = _product(q, k16, v16, bt, sl, None, None, num_ranges=16 * 2, flags=flags)
    assert torch.equal(got, want)
    st = _read(slib, "bf16")
    seg = st[st[:, 9] > 0]
    print(f"split layout: {len(st)} waves stored, {len(seg)} with tiles", flush=True)
    assert len(seg) > 0 and _ordered(seg, [0, 1, 9, 2, 3, 4, 5, 6, 7])


def test_per_sequence_layout_int8(cuda, slib):
    c = decode_case([512, 300, 0, 1000], seed=73)
    t = to_dev(c, cuda)
    flags = _lib.DECODE_ALL | _lib.DECODE_PER_SEQUENCE
    _lib.check(slib.int8kv_stamps_clear_i8(), "clear")
    got = _noalloc(slib, *t, flags=flags)
    want = _product(*t, flags=flags)
    assert torch.equal(got, want)
    st = _read(slib, "i8")
    seg = st[st[:, 9] > 0]
    print(f"per-sequence layout: {len(st)} waves stored, {len(seg)} with tiles", flush=True)
    assert len(seg) > 0 and _ordered(seg, [0, 1, 9, 3, 2, 4, 5, 6, 7])


def test_load_probe(cuda, slib):
    R, T, NB = 8, 20, 2 * 8 * 20 + 5
    g = torch.Generator().manual_seed(3)
    kc = torch.randint(-127, 128, (NB, 16, 4, 128), dtype=torch.int8, generator=g).to(cuda)
    vc = torch.randint(-127, 128, (NB, 16, 4, 128), dtype=torch.int8, generator=g).to(cuda)
    ids = torch.randperm(NB, generator=g)[: 2 * R * T].to(torch.int32).to(cuda)
    sink = torch.zeros(R * 256, dtype=torch.int32, device=cuda)
    _lib.check(slib.int8kv_stamps_clear_probe(), "clear")
    _lib.check(slib.int8kv_probe_decode_loads(kc.data_ptr(), vc.data_ptr(), NB, 4, ids.data_ptr(),
                                              ids.numel(), R, T, 1, sink.data_ptr(), sink.numel(),
                                              _lib.stream_handle(cuda)), "probe")
    torch.cuda.synchronize()
    st = _read(slib, "probe")
    assert len(st) == R * 4
    assert _ordered(st, [0, 2, 7])
