"""The operators under concurrent host use: two host threads on their own streams, two threads on
one shared stream, and HIP-graph replays interleaved with eager calls on one stream (also for the
merge indexed by range, whose per-range descriptors live in the workspace).

The host paths keep state across calls: the ctypes path caches a decode workspace per (host thread,
device, stream) and ctypes stride arrays per stride tuple; the extension allocates outputs and workspaces
through torch's stream-ordered caching allocator.  Every output must equal the same call made
alone on the default stream, bit for bit (the kernels are deterministic for given inputs).
"""

from __future__ import annotations

import threading

import pytest
import torch

import int8kv
from cases import bf16_caches, decode_case, to_dev
from int8kv import _ext

pytestmark = pytest.mark.gpu

SENTINEL = 0x5A


@pytest.fixture(params=["extension", "ctypes"])
def host_path(request, cuda):
    if request.param == "ctypes":
        with _ext.use_ctypes():
            yield request.param
    else:
        assert _ext.module() is not None, "the torch extension is not built"
        yield request.param


def _jobs(dev):
    """Calls with inputs built once; each call allocates its own outputs (and, for the write,
    its own sentinel-filled caches), so concurrent calls share only read-only inputs."""
    a = decode_case([4096, 1, 777, 2048, 33], seed=61)
    qa, kca, vca, bta, sla, ksa, vsa = to_dev(a, dev)
    b = decode_case([1500, 3000, 64], seed=62)
    qb, kcb, vcb, btb, slb, ksb, vsb = to_dev(b, dev)
    kb16, vb16 = (t.to(dev) for t in bf16_caches(b))
    g = torch.Generator().manual_seed(63)
    T, nb = 700, 64
    key = (torch.randn(T, 4, 128, generator=g) * 2).to(torch.bfloat16).to(dev)
    val = torch.randn(T, 4, 128, generator=g).to(torch.bfloat16).to(dev)
    slots = torch.randperm(nb * 16, generator=g)[:T].to(dev)
    ks = (key.float().abs().amax(dim=(0, 2)) / 127).clamp_min(1e-6)
    vs = (val.float().abs().amax(dim=(0, 2)) / 127).clamp_min(1e-6)

    def int8_decode():
        return (int8kv.int8_paged_attention(qa, kca, vca, bta, sla, ksa, vsa),)

    def int8_quantize_q_and_bf16():
        return (int8kv.int8_paged_attention(qb, kcb, vcb, btb, slb, ksb, vsb, quantize_q=True),
                int8kv.bf16_paged_attention(qb, kb16, vb16, btb, slb))

    def write():
        kc = torch.full((nb, 16, 4, 128), SENTINEL, dtype=torch.int8, device=dev)
        vc = torch.full_like(kc, SENTINEL)
        int8kv.int8_kv_cache_write(key, val, kc, vc, slots, ks, vs)
        return kc, vc

    jobs = [int8_decode, int8_quantize_q_and_bf16, write]
    refs = [job() for job in jobs]
    torch.cuda.synchronize()
    return jobs, refs


def _check(got, want, what):
    for i, (x, y) in enumerate(zip(got, want)):
        assert torch.equal(x, y), f"{what}: output {i} differs from the call made alone"


def _run_threads(jobs, refs, streams, reps=24):
    errors = []
    barrier = threading.Barrier(len(streams))

    def worker(ti):
        try:
            s = streams[ti]
            barrier.wait()
            outs = []
            with torch.cuda.stream(s):
                for r in range(reps):
                    j = (ti + r) % len(jobs)
                    outs.append((r, j, jobs[j]()))
            s.synchronize()
            for r, j, o in outs:
                for i, (x, y) in enumerate(zip(o, refs[j])):
                    if not torch.equal(x, y):
                        errors.append(f"thread {ti}, call {r} (job {j}), output {i} differs")
        except Exception as e:  # reported by the main thread
            errors.append(f"thread {ti}: {e!r}")

    threads = [threading.Thread(target=worker, args=(ti,)) for ti in range(len(streams))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors[:5]


def test_two_threads_on_their_own_streams(cuda, host_path):
    jobs, refs = _jobs(cuda)
    _run_threads(jobs, refs, [torch.cuda.Stream(), torch.cuda.Stream()])


def test_two_threads_on_one_stream(cuda, host_path):
    jobs, refs = _jobs(cuda)
    s = torch.cuda.Stream()
    _run_threads(jobs, refs, [s, s])


def test_graph_replays_interleaved_with_eager_calls(cuda, host_path):
    """A graph holding a decode and a cache write, replayed on the stream it was captured on
    between eager calls of the same operators there (the ctypes path's per-stream workspace is
    in use by the eager calls; the captured decode got its own from the graph's pool)."""
    jobs, refs = _jobs(cuda)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for job in jobs:  # eager calls on s first: the ctypes path caches a workspace for s
            _check(job(), refs[jobs.index(job)], "eager warm-up")
    s.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        captured = jobs[0]() + jobs[2]()
    want = refs[0] + refs[2]
    with torch.cuda.stream(s):
        for rep in range(5):
            for t in captured:
                t.zero_()
            before = jobs[1]()
            graph.replay()
            after = jobs[0]()
            s.synchronize()
            _check(captured, want, f"replay {rep}")
            _check(before, refs[1], f"eager call before replay {rep}")
            _check(after, refs[0], f"eager call after replay {rep}")
            _ = (after[0].float() * 2).sum().item()  # eager work and a sync between replays


def test_graph_replays_of_the_range_indexed_merge(cuda, host_path):
    """B = 256 decodes (the merge indexed by range, which reads the per-range descriptors the
    decode kernel leaves in the workspace): one captured in a graph and replayed between eager
    calls of another B = 256 decode and of a B = 5 decode (the merge indexed by sequence) on the
    same stream; every replay and every eager output bit-identical to the call made alone."""
    g = torch.Generator().manual_seed(77)
    cases = []
    for seed, B in ((71, 256), (72, 256), (73, 5)):
        lens = torch.randint(1, 1200, (B,), generator=g).tolist()
        lens[B // 2] = 0
        c = decode_case(lens, seed=seed, extra_blocks=3)
        q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
        cases.append(lambda q=q, kc=kc, vc=vc, bt=bt, sl=sl, ks=ks, vs=vs:
                     (int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs),))
    refs = [job() for job in cases]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for job, ref in zip(cases, refs):
            _check(job(), ref, "eager warm-up")
    s.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        captured = cases[0]()
    with torch.cuda.stream(s):
        for rep in range(5):
            captured[0].zero_()
            before = cases[1]()
            graph.replay()
            between = cases[2]()
            after = cases[1]()
            s.synchronize()
            _check(captured, refs[0], f"replay {rep}")
            _check(before, refs[1], f"eager B=256 before replay {rep}")
            _check(between, refs[2], f"eager B=5 after replay {rep}")
            _check(after, refs[1], f"eager B=256 after replay {rep}")
            _ = (after[0].float() * 2).sum().item()  # eager work and a sync between replays


def test_graph_replays_at_head_dims_64_and_256(cuda, host_path):
    """Graphs holding the head_dim-64 paired range decode (kv heads two per wave, merge), the
    head_dim-256 per-sequence decode (four-wave workgroups, one kernel) and the split
    per-sequence decode of one long sequence (records and merge_split_kernel), each replayed
    between eager calls of another on the same stream; every output bit-identical to the call
    made alone."""
    cases = []
    for lens, seed, hq, hkv, d in (([4000, 17, 2600, 0, 900], 81, 32, 8, 64),
                                   ([300, 5, 512, 64], 82, 16, 8, 256),
                                   ([20000, 0], 83, 28, 4, 128)):
        c = decode_case(lens, seed=seed, hq=hq, hkv=hkv, head_dim=d, extra_blocks=3)
        q, kc, vc, bt, sl, ks, vs = to_dev(c, cuda)
        cases.append(lambda q=q, kc=kc, vc=vc, bt=bt, sl=sl, ks=ks, vs=vs:
                     (int8kv.int8_paged_attention(q, kc, vc, bt, sl, ks, vs),))
    refs = [job() for job in cases]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for job, ref in zip(cases, refs):
            _check(job(), ref, "eager warm-up")
    s.synchronize()
    graphs, captured = [], []
    for job in cases:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            captured.append(job())
        graphs.append(g)
    with torch.cuda.stream(s):
        for rep in range(4):
            for i, (g, out) in enumerate(zip(graphs, captured)):
                out[0].zero_()
                j = (i + 1) % len(cases)
                other = cases[j]()
                g.replay()
                s.synchronize()
                _check(out, refs[i], f"graph {i} replay {rep}")
                _check(other, refs[j], f"eager call beside graph {i}, replay {rep}")
                _ = (other[0].float() * 2).sum().item()  # eager work and a sync between replays
