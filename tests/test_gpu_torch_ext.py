"""The torch extension path (int8kv/_int8kv_torch.so) against the ctypes path of the same C ABI.

Both call the same kernels with the same arguments, so outputs and caches must be bit-identical:
INT8 attention (automatic, v3, forced splits, quantize_q, fp32 query, int64 tables), BF16
attention, the static cache write (bf16 and mixed fp16/fp32 sources, strided and misaligned
views), and the decode launcher under HIP-graph capture (the workspace then comes from the
graph's pool), replayed several times with eager work between the replays.
"""

from __future__ import annotations

import pytest
import torch

import int8kv
from cases import bf16_caches, decode_case, oracle_int8, to_dev
from conftest import MAX_ABS, MIN_COS, metrics
from int8kv import _decode, _ext, _lib

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ext(cuda):
    m = _ext.module()
    assert m is not None, "the torch extension is not built"
    return m


def _both(fn):
    a = fn()
    torch.cuda.synchronize()
    with _ext.use_ctypes():
        b = fn()
    torch.cuda.synchronize()
    return a, b


@pytest.mark.parametrize("kw", [{}, {"impl": "v3"}, {"num_splits": 3}, {"quantize_q": True},
                                {"impl": "v4", "num_splits": 1}])
def test_int8_attention_paths_identical(ext, cuda, kw):
    c = decode_case([4096, 1, 777, 0, 2048, 33], seed=41)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    a, b = _both(lambda: int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, **kw))
    assert torch.equal(a, b), kw
    if not kw.get("quantize_q"):
        err, cos, _ = metrics(a.float().cpu().numpy(), oracle_int8(c))
        assert err <= MAX_ABS and cos >= MIN_COS


def test_int8_attention_fp32_query_int64_tables(ext, cuda):
    c = decode_case([300, 1500, 64], seed=42)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    q32, bt64, sl64 = q.float(), bt.long(), sl.long()
    a, b = _both(lambda: int8kv.int8_paged_attention(q32, kc, vc, bt64, sl64, ks.double(), vs))
    assert a.dtype == torch.float32 and torch.equal(a, b)


def test_bf16_attention_paths_identical(ext, cuda):
    c = decode_case([1024, 5, 3000], seed=43)
    k16, v16 = (t.to(cuda) for t in bf16_caches(c))
    q, _, _, bt, sl, _, _ = to_dev(c, cuda)
    for splits in (None, 2):
        a, b = _both(lambda: int8kv.bf16_paged_attention(q, k16, v16, bt, sl, num_splits=splits))
        assert torch.equal(a, b)


def test_cache_write_paths_identical(ext, cuda):
    g = torch.Generator(device=cuda).manual_seed(44)
    T, nb = 1000, 96
    k = torch.randn(T, 4, 128, generator=g, device=cuda).to(torch.bfloat16)
    v = torch.randn(T, 4, 128, generator=g, device=cuda).to(torch.bfloat16)
    slots = torch.randperm(nb * 16, generator=g, device=cuda)[:T]
    slots[::7] = -1
    ks = torch.rand(4, generator=g, device=cuda) * 0.05 + 0.01
    vs = torch.rand(4, generator=g, device=cuda) * 0.05 + 0.01
    wide = torch.randn(T, 4, 136, generator=g, device=cuda).to(torch.float16)[..., 4:132]  # misaligned
    cases = [(k, v), (k.half(), v.float()), (wide, v)]
    for kk, vv in cases:
        out = []
        for ctypes_path in (False, True):
            kc = torch.zeros(nb, 16, 4, 128, dtype=torch.int8, device=cuda)
            vc = torch.zeros_like(kc)
            if ctypes_path:
                with _ext.use_ctypes():
                    int8kv.int8_kv_cache_write(kk, vv, kc, vc, slots, ks, vs)
            else:
                assert int8kv.int8_kv_cache_write(kk, vv, kc, vc, slots, ks, vs) is None
            torch.cuda.synchronize()
            out.append((kc, vc))
        assert torch.equal(out[0][0], out[1][0]) and torch.equal(out[0][1], out[1][1])


def test_library_errors_raise_int8kv_error(ext, cuda):
    c = decode_case([64], seed=45)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    bad = torch.zeros(kc.shape[0], 8, 4, 128, dtype=torch.int8, device=cuda)  # block size 8
    with pytest.raises(_lib.Int8KVError, match="E_SHAPE"):
        int8kv.int8_paged_attention(q, bad, bad, bt, sl, ks, vs)
    with pytest.raises(ValueError, match="impl"):
        int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs, impl="v5")


def test_graph_capture_through_the_extension(ext, cuda):
    c = decode_case([2048, 700, 4096, 1], seed=46)
    q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
    eager = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs)
    out = torch.empty_like(q)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _decode.paged_decode(q, kc, vc, bt, sl, ks, vs, out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs)
    for i in range(4):
        captured.zero_()
        graph.replay()
        torch.cuda.synchronize()
        _ = (eager.float() * 2).sum().item()  # eager work between replays
        assert torch.equal(captured, eager), f"replay {i} differs from the eager call"
