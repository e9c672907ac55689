"""The probes of include/int8kv_probe.h (measurement only, bench.py --ceiling and --cold) on small
inputs: the read probes run, every word of the sink they own is written, and the decode-load
probe's result depends only on the bytes it reads (the xor of every loaded dword per lane is
recomputed on the CPU for the ordinary and the non-temporal variant); the clock probe reports a
window at least as long as asked and a shader clock in a plausible range."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from int8kv import _lib

pytestmark = pytest.mark.gpu


def _xor_reduce(a: np.ndarray) -> np.ndarray:
    out = np.zeros(a.shape[:-1], np.uint32)
    for i in range(a.shape[-1]):
        out ^= a[..., i]
    return out


def test_stream_probe(cuda):
    lib = _lib.load()
    n = 1 << 20  # bytes
    src = torch.randint(-2**31, 2**31 - 1, (n // 4,), dtype=torch.int32, device=cuda)
    words = 4 * 256
    sink = torch.full((words,), -1, dtype=torch.int32, device=cuda)
    stream = _lib.stream_handle(cuda)
    for nt in (0, 1):
        _lib.check(lib.int8kv_probe_stream_read(src.data_ptr(), n, nt, sink.data_ptr(), words,
                                                stream), "int8kv_probe_stream_read")
        torch.cuda.synchronize()
        # thread i xors the 16-byte pieces i, i + words, i + 2 words, ... of the buffer
        pieces = src.cpu().numpy().view(np.uint32).reshape(-1, 4)
        want = np.zeros(words, np.uint32)
        for i in range(0, pieces.shape[0], words):
            want ^= _xor_reduce(pieces[i:i + words])
        assert np.array_equal(sink.cpu().numpy().view(np.uint32), want), nt


def test_decode_load_probe(cuda):
    lib = _lib.load()
    R, T = 8, 20  # ranges, tiles per range (a chunk of 20 tiles: 5 rounds of four)
    NB = 2 * R * T + 5
    g = torch.Generator().manual_seed(3)
    kc = torch.randint(-127, 128, (NB, 16, 4, 128), dtype=torch.int8, generator=g)
    vc = torch.randint(-127, 128, (NB, 16, 4, 128), dtype=torch.int8, generator=g)
    ids = torch.randperm(NB, generator=g)[: 2 * R * T].to(torch.int32)
    sink = torch.full((R * 256,), -1, dtype=torch.int32, device=cuda)
    kd, vd, idd = kc.to(cuda), vc.to(cuda), ids.to(cuda)
    stream = _lib.stream_handle(cuda)
    outs = []
    for nt in (0, 1):
        _lib.check(lib.int8kv_probe_decode_loads(kd.data_ptr(), vd.data_ptr(), NB, 4, idd.data_ptr(),
                                                 ids.numel(), R, T, nt, sink.data_ptr(),
                                                 sink.numel(), stream),
                   "int8kv_probe_decode_loads")
        torch.cuda.synchronize()
        outs.append(sink.cpu().clone())
    assert torch.equal(outs[0], outs[1])  # the hint changes nothing but the caching
    assert (outs[0] != -1).any()
    # Shuffling the pool's contents outside the blocks the probe reads changes nothing.
    unused = torch.ones(NB, dtype=torch.bool)
    unused[ids.long()] = False
    kd[unused.to(cuda)] = 0
    _lib.check(lib.int8kv_probe_decode_loads(kd.data_ptr(), vd.data_ptr(), NB, 4, idd.data_ptr(),
                                             ids.numel(), R, T, 0, sink.data_ptr(), sink.numel(),
                                             stream), "int8kv_probe_decode_loads")
    torch.cuda.synchronize()
    assert torch.equal(sink.cpu(), outs[0])


def test_clock_probe(cuda):
    lib = _lib.load()
    W, ticks = 64, 300  # 3 us windows
    out = torch.zeros(2 * W, dtype=torch.int64, device=cuda)
    _lib.check(lib.int8kv_probe_clock(out.data_ptr(), W, ticks, _lib.stream_handle(cuda)),
               "int8kv_probe_clock")
    torch.cuda.synchronize()
    o = out.cpu().numpy().reshape(W, 2)
    assert (o[:, 0] >= ticks).all() and (o[:, 0] < 100 * ticks).all(), o[:4]
    mhz = o[:, 1] / (o[:, 0] * 0.01)  # cycles per microsecond
    print(f"clock probe: {np.median(mhz):.1f} MHz (min {mhz.min():.1f}, max {mhz.max():.1f})", flush=True)
    assert ((mhz > 100) & (mhz < 5000)).all(), mhz
