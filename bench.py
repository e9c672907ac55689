#!/usr/bin/env python3
"""Headline benchmark: INT8 PagedAttention decode on one MI355X (the large ragged batch).

Workload (the configuration the headline metric is quoted on): one decode step of one layer,
Qwen2.5-7B attention shape (28 query heads, 4 kv heads, head_dim 128, 16-token cache blocks),
B = 64 sequences with context lengths drawn uniformly from [1, 32768], block tables shuffled
over a shared pool of ~73k physical blocks (~1.2 GB of int8 K+V).  Inputs are synthetic
(seeded), written into the int8 cache by this library's own cache-write kernel, and resident
in HBM before the timed region starts.

A "step" is one int8_paged_attention call (decode kernel + split merge).  Reported:
  * value: whole-call algorithmic HBM GB/s (K+V bytes once, block-table entries, q, out,
    seq_lens, scales) over the measured step time;
  * settle: before the first timed loop the op runs back to back until the device has been
    busy for at least 100 ms and two consecutive event-timed batches agree within 1 % (the
    device slows down for ~10 ms a few ms into a sustained load, then recovers; a timed loop
    inside that dip measures the power controller, not the kernel).  Untimed; reported;
  * roofline: the decode kernel alone, timed with one HIP event pair around back-to-back
    launches on the launch stream, against the 8 TB/s HBM peak; ``traffic`` comes from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary when it describes this same workload;
  * the same-kernel BF16 path on the same data (bf16 cache), for the INT8-vs-BF16 comparison;
  * writes: the prefill cache write of config 1 (16,384 tokens + 512 padding slots) and an
    HBM-sized 262,144-token write, static and dynamic scales, beside a same-mix ceiling (torch's
    bf16 -> int8 conversion over the same elements: 2 bytes read, 1 written per element);
  * cpu_baseline: the reference's decode path restated in torch (oracle/torch_cpu_path.py:
    gather, dequantise, GQA-expanded fp32 attention) on every host core, median of 3 passes over
    a bounded sample of the workload's sequences; the single-thread numpy oracle rate beside it.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (REPO, REPO / "int8-kvcache_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "INT8 paged decode attn µs/call + achieved HBM GB/s (% peak), B=64 ctx≤32k"
HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = REPO / "profiles" / "decode_int8_cfg3_traffic.json"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def build_workload(dev, batch=64, max_len=32768, seed=0):
    """Seeded cfg3 inputs on ``dev``: int8 + bf16 caches holding the same K/V, tables, lens."""
    import torch

    import int8kv
    from int8kv import synthetic as syn

    lens = syn.ragged_lengths(batch, max_len, seed + 2)
    width = (max_len + 15) // 16
    need = int(((lens + 15) // 16).sum())
    num_blocks = need + 64
    g_cpu = torch.Generator().manual_seed(seed + 2)
    bt = syn.random_block_tables(lens.tolist(), num_blocks, g_cpu, width=width, fill=0)
    slots = syn.slot_mapping_for(bt, lens.tolist())
    dist = syn.make_distribution(seed)
    ks, vs = syn.calibrate_scales(dist, seed=seed + 1)

    kc = torch.zeros(num_blocks, 16, 4, 128, dtype=torch.int8, device=dev)
    vc = torch.zeros_like(kc)
    kc16 = torch.zeros(num_blocks, 16, 4, 128, dtype=torch.bfloat16, device=dev)
    vc16 = torch.zeros_like(kc16)
    ks_d, vs_d = ks.to(dev), vs.to(dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    slots_d = slots.to(dev)
    step = 1 << 17
    for s0 in range(0, slots.numel(), step):
        sl = slots_d[s0:s0 + step]
        k, v = syn.sample_kv(sl.numel(), dist, g, device=dev)
        int8kv.int8_kv_cache_write(k, v, kc, vc, sl, ks_d, vs_d)
        kc16.view(-1, 4, 128)[sl] = k
        vc16.view(-1, 4, 128)[sl] = v
    q = syn.sample_query(batch, torch.Generator().manual_seed(seed + 3)).to(dev)
    torch.cuda.synchronize()
    return dict(q=q, kc=kc, vc=vc, kc16=kc16, vc16=vc16, bt=bt.to(dev), sl=lens.to(torch.int32).to(dev),
                ks=ks_d, vs=vs_d, lens=lens, bt_cpu=bt, num_blocks=num_blocks, seed=seed)


def time_loop(fn, steps: int, warmup: int) -> float:
    """ms per call of ``fn`` over ``steps`` back-to-back calls (synchronised on both sides)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def time_events(fn, steps: int, warmup: int) -> float:
    """Average device duration (ms) of one ``fn`` launch: one HIP event pair around ``steps``
    back-to-back launches, recorded on torch's current stream (the stream the library launches
    on).  A pair around every single launch would add the event-to-dispatch gap (~3-4 us on
    MI355X) to each sample; back to back, consecutive launches leave almost no gap, so the
    average agrees with rocprofv3's kernel durations."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def time_graph(fn, calls: int = 20, replays: int = 10, settle_ms: float = 30.0) -> float:
    """Device time per call (ms) of ``fn`` captured ``calls`` times in one HIP graph and replayed:
    removes the host's per-call launch cost, which dominates calls of a few microseconds.  The
    replays are timed after a settle phase of replays (``settle``): capturing leaves the device
    idle for a few ms, and the start-up transient that follows would otherwise fall on the timed
    replays (B=32 x 8256 tokens: 56.7 us per decode + merge call inside it, ~53 us after it)."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            fn()
    torch.cuda.synchronize()
    settle(graph.replay, batch=2, min_ms=settle_ms, max_ms=4 * settle_ms)
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(replays):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / (replays * calls)


def settle(fn, batch: int = 20, min_ms: float = 100.0, tol: float = 0.01,
           max_ms: float = 4000.0) -> dict:
    """Runs ``fn`` back to back in event-timed batches of ``batch`` calls until the device has
    been busy with it for at least ``min_ms`` and the last three batches agree within ``tol``
    (or ``max_ms`` have passed).  Batches are enqueued eight at a time between host
    synchronisations, so the load is continuous.

    Why: on MI355X the first few ms of a sustained HBM-bound load run at full speed, then every
    launch slows by up to ~25 % for about 10 ms and recovers (rocprofv3 traces of this bench:
    calls 11-65 after the workload build, while the earlier calls and everything after run at
    the steady-state duration); on some boxes the recovery takes longer (the headline call was
    still at 199 us after 129 ms busy, then ran at 190 us).  A short warm-up leaves the timed loop
    inside that dip.  The figures returned describe it: the first, slowest and last batch
    averages in microseconds, and every eighth batch's."""
    import torch

    means, busy, calls = [], 0.0, 0
    while True:
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(9)]
        ev[0].record()
        for i in range(8):
            for _ in range(batch):
                fn()
            ev[i + 1].record()
        ev[-1].synchronize()
        for i in range(8):
            ms = ev[i].elapsed_time(ev[i + 1])
            busy += ms
            calls += batch
            means.append(ms / batch)
        last = means[-3:]
        settled = busy >= min_ms and max(last) - min(last) <= tol * min(last)
        if settled or busy >= max_ms:
            break
    return {"calls": calls, "busy_ms": round(busy, 2), "settled": bool(settled),
            "first_batch_us": round(means[0] * 1e3, 2), "slowest_batch_us": round(max(means) * 1e3, 2),
            "last_batch_us": round(means[-1] * 1e3, 2),
            "every_8th_batch_us": [round(m * 1e3, 1) for m in means[7::8]]}


def write_legs(dev, cfg1_graph: bool = True) -> dict:
    """The cache writes beside the headline (config 1 and an HBM-sized write), each beside two
    plain streaming kernels over the same bytes, without the slot scatter: a device-to-device
    copy (hipMemcpyAsync) of the same byte count (half read, half written), and an elementwise
    kernel with the write's 2:1 read/write mix (torch.ne on the bf16 K/V into a bool tensor: 2
    bytes read, 1 written per element).  The faster of the two is the copy ceiling the write is
    compared with.  Config 1 (16,384 tokens + 512
    padding slots into a 2048-block cache, ~50 MB) fits the 256 MB Infinity Cache, so its rate is
    cache-resident; it is timed as HIP-graph replays (the host's launch cost exceeds the kernel).
    The 262,144-token write (805 MB moved) streams from HBM and is timed with events around
    back-to-back launches after a settle."""
    import torch

    import int8kv
    from int8kv import cache_ops, roofline
    from int8kv import synthetic as syn

    res = {}
    g = torch.Generator().manual_seed(11)
    dist = syn.make_distribution(11)
    ks, vs = syn.calibrate_scales(dist, seed=12)
    ks_d, vs_d = ks.to(dev), vs.to(dev)

    def leg(n_tok, n_pad, nb, gen, graph: bool):
        k, v = syn.sample_kv(n_tok + n_pad, dist, gen)
        slots = torch.randperm(nb * 16, generator=gen)[: n_tok + n_pad].to(torch.int64)
        if n_pad:
            slots[torch.randperm(n_tok + n_pad, generator=gen)[:n_pad]] = -1
        k, v, sd = k.to(dev), v.to(dev), slots.to(dev)
        kc = torch.zeros(nb, 16, 4, 128, dtype=torch.int8, device=dev)
        vc = torch.zeros_like(kc)
        ksc = torch.zeros(nb, 16, 4, dtype=torch.float32, device=dev)
        vsc = torch.zeros_like(ksc)
        kd = torch.empty(k.shape, dtype=torch.bool, device=dev)
        vd = torch.empty_like(kd)
        moved = (n_tok + n_pad) * 4 * 128 * 6  # K/V bf16 read + int8 written, every row
        src = torch.empty(moved // 2, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)

        def static():
            int8kv.int8_kv_cache_write(k, v, kc, vc, sd, ks_d, vs_d)

        def dynamic():
            cache_ops.reshape_and_cache_int8(k, v, kc, vc, ksc, vsc, sd)

        def mix21():
            torch.ne(k, 0, out=kd)
            torch.ne(v, 0, out=vd)

        def copy():
            dst.copy_(src)

        if graph:
            timer = time_graph
        else:
            settle(static, batch=10, min_ms=50.0)
            timer = lambda fn: time_events(fn, 40, 10)  # noqa: E731
        ms_s, ms_d = timer(static), timer(dynamic)
        ms_m, ms_c = timer(mix21), timer(copy)
        sbytes = roofline.write_bytes(n_tok, n_tok + n_pad, 4, 128)
        dbytes = roofline.write_bytes(n_tok, n_tok + n_pad, 4, 128, dynamic=True)
        ceiling = moved / min(ms_m, ms_c) / 1e6
        out = {"tokens": n_tok, "padding_slots": n_pad, "cache_blocks": nb,
               "static_us": round(ms_s * 1e3, 2), "static_bytes": sbytes,
               "static_GBps": round(sbytes / ms_s / 1e6, 1),
               "dynamic_us": round(ms_d * 1e3, 2), "dynamic_bytes": dbytes,
               "dynamic_GBps": round(dbytes / ms_d / 1e6, 1),
               "copy_same_bytes_us": round(ms_c * 1e3, 2),
               "copy_same_bytes_GBps": round(moved / ms_c / 1e6, 1),
               "mix_2to1_elementwise_us": round(ms_m * 1e3, 2),
               "mix_2to1_elementwise_GBps": round(moved / ms_m / 1e6, 1),
               "static_frac_of_copy_ceiling": round(sbytes / ms_s / 1e6 / ceiling, 3),
               "timing": "HIP-graph replays" if graph else "HIP events, back-to-back launches"}
        return out

    res["cfg1"] = leg(16384, 512, 2048, g, graph=cfg1_graph)
    log(f"cfg1 write: {json.dumps(res['cfg1'])}")
    res["hbm_262k"] = leg(262144, 0, 32768, torch.Generator().manual_seed(13), graph=False)
    log(f"262k write: {json.dumps(res['hbm_262k'])}")
    torch.cuda.empty_cache()
    return res


def cpu_threads() -> int:
    """Host threads for the CPU baseline: the cores this process may run on, capped by
    OMP_NUM_THREADS when the environment sets it (the GPU box sets it to its CPU share)."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_baseline(w, out_gpu, target_s: float = 4.0, runs: int = 3):
    """The reference's decode path on the CPU: oracle/torch_cpu_path.decode_step (gather through
    the block table, dequantise, GQA-expanded fp32 einsum attention) on every host core.  The
    sample is the workload's first sequences in batch order, as many as one pass of ``target_s``
    seconds covers; it is then run ``runs`` more times and the median pass is reported.  Also
    returns the agreement of the GPU output with this CPU result on the sample."""
    import torch

    from int8kv import roofline
    from oracle import torch_cpu_path as TP

    threads = cpu_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        kc, vc = w["kc"].cpu(), w["vc"].cpu()
        q = w["q"].cpu()
        bt, lens = w["bt_cpu"], w["lens"]
        ks, vs = w["ks"].cpu(), w["vs"].cpu()
        sample, t_cal = [], 0.0
        ref = torch.zeros(q.shape, dtype=torch.float32)
        for b in range(len(lens)):
            t0 = time.perf_counter()
            part = TP.decode_step(q, kc, vc, bt, lens, ks, vs, sequences=[b])
            t_cal += time.perf_counter() - t0
            ref[b] = part[b]
            sample.append(b)
            if t_cal >= target_s:
                break
        times = []
        for _ in range(runs):
            t0 = time.perf_counter()
            TP.decode_step(q, kc, vc, bt, lens, ks, vs, sequences=sample)
            times.append(time.perf_counter() - t0)
        med = statistics.median(times)
        s_lens = lens[sample].numpy()
        nbytes = roofline.decode_bytes(s_lens, 4, 128, 1, len(sample), 28)
        got = out_gpu.float().cpu()[sample].double()
        r = ref[sample].double()
        check = {"sequences": len(sample), "max_abs": round(float((got - r).abs().max()), 6),
                 "cos": round(float((got * r).sum() / (got.norm() * r.norm())), 7)}
        cb = {
            "value": round(nbytes / med / 1e9, 4),
            "unit": "GB/s",
            "cores": threads,
            "kind": "port",
            "sample": f"{len(sample)} of the workload's {len(lens)} sequences ({int(s_lens.sum())} "
                      f"tokens, {nbytes} algorithmic bytes): torch restatement of the reference's "
                      f"paged gather -> dequantise -> GQA attention (oracle/torch_cpu_path.py), "
                      f"median of {runs} passes ({', '.join(f'{t:.2f}' for t in times)} s)",
            "torch_num_threads": torch.get_num_threads(),
            "sched_affinity_cores": len(os.sched_getaffinity(0)),
            "ms_per_pass_median": round(med * 1e3, 1),
            "us_per_call_extrapolated": round(med / max(int(s_lens.sum()), 1) * int(lens.sum()) * 1e6, 1),
        }
    finally:
        torch.set_num_threads(prev)
    return cb, check


def cpu_oracle_single_thread(w, budget_s: float = 3.0) -> dict:
    """The numpy oracle on one thread over the workload's sequences until ``budget_s`` seconds
    of work (a secondary figure beside the all-core torch baseline)."""
    from int8kv import roofline
    from oracle import int8kv_oracle as O

    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    kc, vc = w["kc"].cpu().numpy(), w["vc"].cpu().numpy()
    q = w["q"].float().cpu().numpy()
    bt, lens = w["bt_cpu"].numpy(), w["lens"].numpy()
    ks, vs = w["ks"].cpu().numpy(), w["vs"].cpu().numpy()
    ctx = threadpool_limits(limits=1) if threadpool_limits else None
    t_total, nbytes, calls = 0.0, 0, 0
    try:
        if ctx:
            ctx.__enter__()
        for b in range(len(lens)):
            t0 = time.perf_counter()
            O.paged_attention_ref(q[b:b + 1], kc, vc, bt[b:b + 1], lens[b:b + 1], ks, vs)
            t_total += time.perf_counter() - t0
            nbytes += roofline.decode_bytes(lens[b:b + 1], 4, 128, 1, 1, 28)
            calls += 1
            if t_total >= budget_s:
                break
    finally:
        if ctx:
            ctx.__exit__(None, None, None)
    return {"value": round(nbytes / t_total / 1e9, 4), "unit": "GB/s", "cores": 1,
            "sample": f"{calls} single-sequence numpy-oracle calls, {t_total:.1f} s"}


def read_traffic(w, nbytes8: int):
    """HBM bytes per decode launch from the committed rocprofv3 counter summary, when it was
    measured on this same workload (seed, token count and algorithmic bytes all match); else
    None."""
    if not TRAFFIC_FILE.exists():
        return None
    try:
        d = json.loads(TRAFFIC_FILE.read_text())
        same = (int(d["seed"]) == int(w["seed"]) and int(d["tokens"]) == int(w["lens"].sum())
                and int(d["algorithmic_bytes_per_launch"]) == int(nbytes8))
        return int(d["traffic_bytes_per_launch"]) if same else None
    except (ValueError, KeyError, TypeError):
        return None


def sweep_configs(dev, out_path: str | None) -> dict:
    """INT8 and BF16 decode at B in {1, 2, 4, 8} x uniform ctx in {512, 1024, 2048, 4096}
    (config 2), automatic layout vs the single pass (num_splits=1: one workgroup per sequence
    and kv head, no merge).  The working sets fit the 256 MB
    Infinity Cache, so their GB/s are cache-resident rates and µs/call is the meaningful figure.
    Times are device times per call from HIP-graph replays (a few-microsecond call is otherwise
    dominated by the host's launch cost)."""
    import torch

    import int8kv
    from int8kv import roofline
    from int8kv import synthetic as syn

    res = {}
    dist = syn.make_distribution(11)
    ks, vs = syn.calibrate_scales(dist, seed=12)
    ks_d, vs_d = ks.to(dev), vs.to(dev)
    rows = []
    for B in (1, 2, 4, 8):
        for ctx in (512, 1024, 2048, 4096):
            gq = torch.Generator().manual_seed(B * 7 + ctx)
            nblk = B * ctx // 16
            pool = nblk * 2
            bt = syn.random_block_tables([ctx] * B, pool, gq)
            sl = syn.slot_mapping_for(bt, [ctx] * B)
            kk, vv = syn.sample_kv(B * ctx, dist, gq)
            q = syn.sample_query(B, gq).to(dev)
            kc8 = torch.zeros(pool, 16, 4, 128, dtype=torch.int8, device=dev)
            vc8 = torch.zeros_like(kc8)
            int8kv.int8_kv_cache_write(kk.to(dev), vv.to(dev), kc8, vc8, sl.to(dev), ks_d, vs_d)
            kc16 = torch.zeros(pool * 16, 4, 128, dtype=torch.bfloat16, device=dev)
            vc16 = torch.zeros_like(kc16)
            kc16[sl.to(dev)] = kk.to(dev)
            vc16[sl.to(dev)] = vv.to(dev)
            kc16, vc16 = kc16.view(pool, 16, 4, 128), vc16.view(pool, 16, 4, 128)
            btd = bt.to(dev)
            lens = torch.full((B,), ctx, dtype=torch.int32, device=dev)
            row = {"B": B, "ctx": ctx}
            for name, fn in (
                ("int8_auto", lambda: int8kv.int8_paged_attention(q, kc8, vc8, btd, lens, ks_d, vs_d)),
                ("int8_single_pass", lambda: int8kv.int8_paged_attention(q, kc8, vc8, btd, lens, ks_d, vs_d,
                                                                         num_splits=1)),
                ("bf16_auto", lambda: int8kv.bf16_paged_attention(q, kc16, vc16, btd, lens)),
                ("bf16_single_pass", lambda: int8kv.bf16_paged_attention(q, kc16, vc16, btd, lens,
                                                                         num_splits=1)),
            ):
                ms = time_graph(fn)
                e = 2 if name.startswith("bf16") else 1
                nbytes = roofline.decode_bytes([ctx] * B, 4, 128, e, B, 28)
                row[name + "_us"] = round(ms * 1e3, 2)
                row[name + "_GBps"] = round(nbytes / ms / 1e6, 1)
            rows.append(row)
            log(f"cfg2 B={B} ctx={ctx}: int8 {row['int8_auto_us']} us (single pass "
                f"{row['int8_single_pass_us']}), bf16 {row['bf16_auto_us']} us (single pass "
                f"{row['bf16_single_pass_us']})")
    res["cfg2_sweep"] = rows
    if out_path:
        Path(out_path).parent.mkdir(parents=True, exist_ok=True)
        Path(out_path).write_text(json.dumps(res, indent=1))
    return res


# Decode calls between config 2 and config 3 (0.03-0.27 GB of INT8 K/V per call): config 4's
# attention shape (B=32 x ~8.2k tokens) and its neighbours.  (name, batch, length, ragged):
# ragged batches draw lengths uniformly from [1, length].
MIDSIZE_CASES = (("B32x8256", 32, 8256, False), ("B32xU16k", 32, 16384, True),
                 ("B128xU4k", 128, 4096, True), ("B16x16k", 16, 16384, False),
                 ("B8x32k", 8, 32768, False), ("B1x32k", 1, 32768, False),
                 ("B256xU2k", 256, 2048, True))


# Short and few-sequence decode calls across head_dim and cache type, for the host's choice of
# layout: (head_dim, q heads, kv heads, cache, batch, uniform length).  Qwen2.5-7B (28/4) at 128,
# Llama-3.2-1B (32/8) at 64, Gemma-2-9B (16/8) at 256.
LAYOUT_CASES = (
    (128, 28, 4, "int8", 1, 512), (128, 28, 4, "int8", 8, 1024), (128, 28, 4, "int8", 4, 768),
    (128, 28, 4, "int8", 1, 32768), (128, 28, 4, "int8", 2, 8192), (128, 28, 4, "int8", 16, 8192),
    (128, 28, 4, "bf16", 1, 8192), (128, 28, 4, "bf16", 128, 512),
    (64, 32, 8, "int8", 1, 1024), (64, 32, 8, "int8", 128, 2048), (64, 32, 8, "int8", 1, 8192),
    (64, 32, 8, "int8", 4, 16384), (64, 32, 8, "bf16", 8, 1024),
    (256, 16, 8, "int8", 1, 256), (256, 16, 8, "int8", 2, 512), (256, 16, 8, "int8", 32, 512),
    (256, 16, 8, "int8", 1, 16384), (256, 16, 8, "bf16", 16, 512),
)


def layout_legs(dev, out_path: str | None) -> dict:
    """Per case: the automatic call against each layout forced (per-sequence, split per-sequence,
    and the range layout with the automatic range count and 2-tile minimum), op time per call from
    HIP-graph replays (median of three); random K/V in a shuffled pool of exactly the needed
    blocks plus 16."""
    import torch

    from int8kv import _decode, _lib

    lib = _lib.load()
    rows = []
    for d, hq, hkv, cache, B, ctx in LAYOUT_CASES:
        per = 2 * hq * (d + 2) * 4 + 32
        ws_bytes = lib.int8kv_decode_workspace_bytes(hq, hkv, d, 16, 0)
        auto_ranges = ws_bytes // per
        ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
        g = torch.Generator().manual_seed(B * ctx + d)
        width = (ctx + 15) // 16
        nb = B * width + 16
        bt = torch.randperm(nb, generator=g)[: B * width].view(B, width).to(torch.int32).to(dev)
        sl = torch.full((B,), ctx, dtype=torch.int32, device=dev)
        if cache == "int8":
            kc = torch.randint(-127, 128, (nb, 16, hkv, d), dtype=torch.int8, device=dev)
            vc = torch.randint(-127, 128, (nb, 16, hkv, d), dtype=torch.int8, device=dev)
            ks = torch.full((hkv,), 0.05, device=dev)
            vs = torch.full((hkv,), 0.01, device=dev)
        else:
            kc = torch.randn(nb, 16, hkv, d, device=dev).to(torch.bfloat16)
            vc = torch.randn(nb, 16, hkv, d, device=dev).to(torch.bfloat16)
            ks = vs = None
        q = torch.randn(B, hq, d, device=dev).to(torch.bfloat16)
        out = torch.empty_like(q)
        row = {"head_dim": d, "heads": f"{hq}/{hkv}", "cache": cache, "B": B, "ctx": ctx}
        for name, ranges, min_tiles, flags in (
                ("auto", 0, 0, _lib.DECODE_ALL),
                ("per_sequence", 0, 0, _lib.DECODE_ALL | _lib.DECODE_PER_SEQUENCE),
                ("split", 0, 0, _lib.DECODE_ALL | _lib.DECODE_SPLIT_SEQUENCES),
                ("range", int(auto_ranges), 2, _lib.DECODE_ALL)):
            def call():
                _decode.paged_decode(q, kc, vc, bt, sl, ks, vs, out, ranges, flags, ws, min_tiles)
            if d > 128 and name == "per_sequence" and ctx > 4096:
                row[name + "_us"] = None  # a whole long sequence on one four-wave workgroup
                continue
            call()
            torch.cuda.synchronize()
            row[name + "_us"] = round(sorted(time_graph(call, settle_ms=10.0) * 1e3
                                             for _ in range(3))[1], 2)
        rows.append(row)
        log(f"layouts d={d} {hq}/{hkv} {cache} B={B} ctx={ctx}: " +
            ", ".join(f"{k[:-3]} {v}" for k, v in row.items() if k.endswith("_us")))
        del kc, vc, q, out, ws
    res = {"layouts": rows}
    if out_path:
        Path(out_path).parent.mkdir(parents=True, exist_ok=True)
        Path(out_path).write_text(json.dumps(res, indent=1))
    return res


def midsize_legs(dev, out_path: str | None) -> dict:
    """INT8 decode at the mid sizes above (random int8 K/V in a pool just larger than the batch
    needs, shuffled block tables, Qwen2.5-7B attention shape).  Per case: the decode kernel alone
    (HIP events over back-to-back launches after a settle phase), the merge kernel alone and the
    whole op (HIP-graph replays), and GB/s of algorithmic bytes for the kernel and the op."""
    import torch

    from int8kv import _decode, _lib, roofline
    from int8kv import synthetic as syn

    rows = []
    for i, (name, B, ctx, ragged) in enumerate(MIDSIZE_CASES):
        lens = syn.ragged_lengths(B, ctx, 5 + i) if ragged else torch.full((B,), ctx, dtype=torch.int64)
        need = int(((lens + 15) // 16).sum())
        nb = need + 64
        g = torch.Generator().manual_seed(100 + i)
        bt = syn.random_block_tables(lens.tolist(), nb, g).to(dev)
        kc = torch.randint(-127, 128, (nb, 16, 4, 128), dtype=torch.int8, generator=g).to(dev)
        vc = torch.randint(-127, 128, (nb, 16, 4, 128), dtype=torch.int8, generator=g).to(dev)
        q = torch.randn(B, 28, 128, generator=g).to(torch.bfloat16).to(dev)
        ks = torch.full((4,), 0.02, device=dev)
        vs = torch.full((4,), 0.01, device=dev)
        sl = lens.to(torch.int32).to(dev)
        out = torch.empty_like(q)
        ws = torch.zeros(_lib.load().int8kv_decode_workspace_bytes(28, 4, 128, 16, 0),
                         dtype=torch.uint8, device=dev)

        def call(flags):
            return lambda: _decode.paged_decode(q, kc, vc, bt, sl, ks, vs, out, 0, flags, ws, 0)

        plan = _lib.decode_plan(q.dtype, kc.dtype, B, 28, 4, 128, nb, 16, bt.shape[1])
        settle(call(_lib.DECODE_ALL), batch=20, min_ms=30.0)
        ms_main = time_events(call(_lib.DECODE_MAIN), 50, 10)
        ms_op = time_graph(call(_lib.DECODE_ALL))
        # A second (merge) kernel only in the layouts that have one.
        ms_merge = time_graph(call(_lib.DECODE_MERGE)) if plan["kernels"] == 2 else None
        nbytes = roofline.decode_bytes(lens.numpy(), 4, 128, 1, B, 28)
        row = {"case": name, "batch": B, "tokens": int(lens.sum()), "bytes": nbytes,
               "layout": plan["layout"], "merge": plan["merge"], "kernels": plan["kernels"],
               "decode_kernel_us": round(ms_main * 1e3, 2),
               "decode_kernel_TBps": round(nbytes / ms_main / 1e9, 3),
               "merge_graph_us": None if ms_merge is None else round(ms_merge * 1e3, 2),
               "op_graph_us": round(ms_op * 1e3, 2), "op_TBps": round(nbytes / ms_op / 1e9, 3)}
        rows.append(row)
        log(f"midsize {name}: first kernel {row['decode_kernel_us']} us "
            f"({row['decode_kernel_TBps']} TB/s), op {row['op_graph_us']} us ({row['op_TBps']} TB/s), "
            f"{plan['layout']} layout, merge {plan['merge']} {row['merge_graph_us']}")
        del kc, vc
    res = {"midsize": rows}
    if out_path:
        Path(out_path).parent.mkdir(parents=True, exist_ok=True)
        Path(out_path).write_text(json.dumps(res, indent=1))
    return res


def capture_graph(fns):
    """A HIP graph that captures ``fns`` once each, in order (after one eager warm-up pass on a
    side stream)."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for fn in fns:
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for fn in fns:
            fn()
    torch.cuda.synchronize()
    return graph


def graph_us(fns, replays: int = 10, settle_ms: float = 30.0) -> float:
    """Device time (us) of one replay of a HIP graph that captures ``fns`` once each, in order."""
    import torch

    graph = capture_graph(fns)
    settle(graph.replay, batch=1, min_ms=settle_ms, max_ms=4 * settle_ms)
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(replays):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / replays


# Config 4's attention call as the decode loop makes it: B = 32 sequences at one decode step of
# the 8192-token prompts (8193 tokens), each sequence owning its blocks of a shuffled pool of
# B x 520 blocks (tables 520 wide), one pool per layer in one [layers, blocks, 16, 4, 128] tensor.
COLD_CASE = dict(batch=32, length=8193, width=520, layers=28)


class ColdSetup:
    """Config 4's per-layer attention inputs (28 layer pools of random int8 K/V) and, for the
    "between layers" traffic, the decode step's four per-layer GEMMs on random bf16 weights of
    Qwen2.5-7B's shapes (qkv 3584 -> 4608, o 3584 -> 3584, gate_up 3584 -> 37888, down 18944 ->
    3584; 0.5 GB per layer, 13.9 GB in all) with M = 32 rows, as the decode step runs them."""

    def __init__(self, dev):
        import torch

        from int8kv import _lib, roofline

        c = COLD_CASE
        B, L, W, NL = c["batch"], c["length"], c["width"], c["layers"]
        self.B, self.L, self.NL = B, L, NL
        nb = B * W
        g = torch.Generator().manual_seed(2)
        self.bt = torch.randperm(nb, generator=g).to(torch.int32).view(B, W).to(dev)
        gd = torch.Generator(device=dev).manual_seed(3)
        self.kc = torch.randint(-127, 128, (NL, nb, 16, 4, 128), dtype=torch.int8, device=dev, generator=gd)
        self.vc = torch.randint(-127, 128, (NL, nb, 16, 4, 128), dtype=torch.int8, device=dev, generator=gd)
        self.q = torch.randn(B, 28, 128, device=dev, generator=gd).to(torch.bfloat16)
        self.ks = torch.full((NL, 4), 0.02, device=dev)
        self.vs = torch.full((NL, 4), 0.01, device=dev)
        self.sl = torch.full((B,), L, dtype=torch.int32, device=dev)
        self.out = torch.empty_like(self.q)
        self.ws = torch.zeros(_lib.load().int8kv_decode_workspace_bytes(28, 4, 128, 16, 0),
                              dtype=torch.uint8, device=dev)
        self.nbytes = roofline.decode_bytes([L] * B, 4, 128, 1, B, 28)

        def w(n, k):
            return (torch.randn(NL, n, k, device=dev, generator=gd) * 0.02).to(torch.bfloat16)

        self.wqkv, self.wo, self.wgu, self.wdown = w(4608, 3584), w(3584, 3584), w(37888, 3584), w(3584, 18944)
        self.x = torch.randn(B, 3584, device=dev, generator=gd).to(torch.bfloat16)
        self.act = torch.randn(B, 18944, device=dev, generator=gd).to(torch.bfloat16)
        self.y = [torch.empty(B, n, device=dev, dtype=torch.bfloat16) for n in (4608, 3584, 37888, 3584)]
        self.weight_bytes = sum(t[0].numel() * 2 for t in (self.wqkv, self.wo, self.wgu, self.wdown))

    def op(self, layer, flags=None):
        from int8kv import _decode, _lib

        fl = _lib.DECODE_ALL if flags is None else flags
        return lambda: _decode.paged_decode(self.q, self.kc[layer], self.vc[layer], self.bt, self.sl,
                                            self.ks[layer], self.vs[layer], self.out, 0, fl, self.ws, 0)

    def gemms(self, layer):
        import torch

        def run():
            torch.mm(self.x, self.wqkv[layer].t(), out=self.y[0])
            torch.mm(self.x, self.wo[layer].t(), out=self.y[1])
            torch.mm(self.x, self.wgu[layer].t(), out=self.y[2])
            torch.mm(self.act, self.wdown[layer].t(), out=self.y[3])
        return run

    def read_weights(self, layer, non_temporal):
        """The layer's four weight matrices read by the stream probe (16-byte loads, ordinary or
        non-temporal) instead of multiplied: the GEMMs' bytes without their arithmetic."""
        import torch

        from int8kv import _lib

        lib = _lib.load()
        if not hasattr(self, "sink"):
            self.sink = torch.empty(256 * 8 * 256, dtype=torch.int32, device=self.x.device)
        ws = [w[layer] for w in (self.wqkv, self.wo, self.wgu, self.wdown)]

        def run():
            s = torch.cuda.current_stream().cuda_stream
            for w in ws:
                _lib.check(lib.int8kv_probe_stream_read(w.data_ptr(), w.numel() * 2, non_temporal,
                                                        self.sink.data_ptr(), self.sink.numel(), s),
                           "int8kv_probe_stream_read")
        return run

    def clock(self, out, ticks):
        """The clock probe over 1,024 one-wave workgroups (one per SIMD) into out[1024, 2]."""
        import torch

        from int8kv import _lib

        lib = _lib.load()
        return lambda: _lib.check(lib.int8kv_probe_clock(out.data_ptr(), 1024, ticks,
                                                         torch.cuda.current_stream().cuda_stream),
                                  "int8kv_probe_clock")

    def separator(self):
        """A one-workgroup stream-probe launch that marks leg boundaries in a kernel trace."""
        import torch

        from int8kv import _lib

        lib = _lib.load()
        if not hasattr(self, "sep"):
            self.sep = torch.zeros(2 * 4096, dtype=torch.int32, device=self.x.device)
        _lib.check(lib.int8kv_probe_stream_read(self.sep.data_ptr(), 16384, 0,
                                                self.sep.data_ptr() + 16384, 256,
                                                torch.cuda.current_stream().cuda_stream),
                   "separator")


def cold_legs(dev, out_path: str | None) -> dict:
    """The decode op (decode + merge) at config 4's per-layer shape with warm and cold caches.

    * rotate_N: one HIP graph of 28 calls over N distinct layer pools (layer i % N), per call.
      N = 1 repeats one 272 MB pool (the midsize figure), N = 28 touches each pool once per
      replay, as the decode step does.
    * between_gemms: 28 x (layer i's four GEMMs, then the call on layer i's pool), minus the same
      graph without the calls: the attention call in the decode step's traffic (0.5 GB of
      weights streamed between two layers' calls).  Also for the decode kernel alone.
    * after_<predecessor>: the same difference with other work in the GEMMs' place: the GEMMs on
      layer 0's weights every time (the same 466 MB), the layer's weights read by the stream
      probe with ordinary or non-temporal loads, a 200 us spin of the clock probe.
    * clock_after_<leg>: the shader clock (MHz, clock probe over a 5 us window, median over
      1,024 waves and the 28 positions) right after the call alone, the GEMMs, the GEMMs + call.
    * trace legs: graphs of 28 x (GEMMs, call), 28 x GEMMs and 28 x call, replayed 12 times each
      between two separator launches, for a kernel trace (`--trace-table` summarises it)."""
    import numpy as np
    import torch

    from int8kv import _lib

    cs = ColdSetup(dev)
    NL, nbytes = cs.NL, cs.nbytes
    res = {"case": {**COLD_CASE, "tokens": cs.B * cs.L, "bytes_per_call": nbytes,
                    "weight_bytes_per_layer": cs.weight_bytes}}
    for n in (1, 28):
        us = graph_us([cs.op(i % n) for i in range(NL)]) / NL
        res[f"rotate_{n}_op_us"] = round(us, 2)
        res[f"rotate_{n}_op_TBps"] = round(nbytes / us / 1e6, 3)
        log(f"cold: rotate over {n} pools: op {us:.2f} us ({nbytes / us / 1e6:.2f} TB/s)")
    base = graph_us([cs.gemms(i) for i in range(NL)])
    for name, flags in (("op", _lib.DECODE_ALL), ("decode", _lib.DECODE_MAIN)):
        fns = []
        for i in range(NL):
            fns += [cs.gemms(i), cs.op(i, flags)]
        us = (graph_us(fns) - base) / NL
        res[f"between_gemms_{name}_us"] = round(us, 2)
        res[f"between_gemms_{name}_TBps"] = round(nbytes / us / 1e6, 3)
        log(f"cold: between the GEMMs: {name} {us:.2f} us ({nbytes / us / 1e6:.2f} TB/s)")
    res["gemms_per_layer_us"] = round(base / NL, 2)
    spin_out = torch.zeros(1024, 2, dtype=torch.int64, device=dev)
    preds = {
        "gemms_same_weights": lambda i: cs.gemms(0),
        "read_weights": lambda i: cs.read_weights(i, 0),
        "read_weights_nt": lambda i: cs.read_weights(i, 1),
        "spin_200us": lambda i: cs.clock(spin_out, 20000),
    }
    for name, mk in preds.items():
        pre = [mk(i) for i in range(NL)]
        without = graph_us(pre)
        us = (graph_us([f for i in range(NL) for f in (pre[i], cs.op(i))]) - without) / NL
        res[f"after_{name}_op_us"] = round(us, 2)
        log(f"cold: after {name}: op {us:.2f} us")
    clk = torch.zeros(NL, 1024, 2, dtype=torch.int64, device=dev)
    for name, mk in (("op", lambda i: [cs.op(i)]), ("gemms", lambda i: [cs.gemms(i)]),
                     ("gemms_op", lambda i: [cs.gemms(i), cs.op(i)])):
        graph_us([f for i in range(NL) for f in (*mk(i), cs.clock(clk[i], 500))], replays=1,
                 settle_ms=100.0)
        o = clk.cpu().numpy().astype(np.float64)
        mhz = float(np.median(o[..., 1] / (o[..., 0] * 0.01)))
        res[f"clock_after_{name}_mhz"] = round(mhz, 1)
        log(f"cold: shader clock after {name}: {mhz:.1f} MHz")
    for name, fns in (("gemms_op", [f for i in range(NL) for f in (cs.gemms(i), cs.op(i))]),
                      ("gemms", [cs.gemms(i) for i in range(NL)]),
                      ("op", [cs.op(i) for i in range(NL)])):
        g = capture_graph(fns)
        settle(g.replay, batch=1, min_ms=30.0, max_ms=120.0)
        cs.separator()
        for _ in range(12):
            g.replay()
        cs.separator()
        torch.cuda.synchronize()
        del g
    res["trace_legs"] = ["gemms_op", "gemms", "op"]
    del cs
    torch.cuda.empty_cache()
    if out_path:
        Path(out_path).parent.mkdir(parents=True, exist_ok=True)
        Path(out_path).write_text(json.dumps({"cold": res}, indent=1))
    return res


def trace_table(csv_path: str, out_path: str | None) -> dict:
    """Summarises a rocprofv3 kernel trace (``--kernel-trace --output-format csv``) of ``--cold``:
    the dispatches between each pair of separator launches (one-workgroup stream probes, the
    last six of the run) are the 12 replays of one trace leg (28 x (GEMMs, call), 28 x GEMMs,
    28 x call).  Per leg: the span per replay and each kernel class's mean duration (the GEMMs by
    their position in the layer: qkv, o_proj, gate_up, down).  In a graph each dispatch starts
    when the previous one ends, so a duration includes the kernel's start-up after it."""
    import csv

    rows = sorted(csv.DictReader(open(csv_path)), key=lambda r: int(r["Start_Timestamp"]))
    seps = [i for i, r in enumerate(rows)
            if "probe_stream_kernel" in r["Kernel_Name"] and int(r["Grid_Size_X"]) == 256][-6:]
    gemm_names = ("qkv", "o_proj", "gate_up", "down")
    res = {"csv": csv_path}
    for k, leg in enumerate(("gemms_op", "gemms", "op")):
        win = rows[seps[2 * k] + 1: seps[2 * k + 1]]
        dur: dict = {}
        n_gemm = 0
        for r in win:
            name = r["Kernel_Name"]
            us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            if "decode_kernel" in name:
                c = "decode"
            elif "merge" in name:
                c = "merge"
            else:
                c = "gemm_" + gemm_names[n_gemm % 4]
                n_gemm += 1
            dur.setdefault(c, []).append(us)
        span = (int(win[-1]["End_Timestamp"]) - int(win[0]["Start_Timestamp"])) / 1e3 / 12
        res[leg] = {"dispatches": len(win), "span_per_replay_us": round(span, 1),
                    **{c: round(sum(v) / len(v), 2) for c, v in sorted(dur.items())}}
        log(f"trace {leg}: {res[leg]}")
    if out_path:
        Path(out_path).parent.mkdir(parents=True, exist_ok=True)
        Path(out_path).write_text(json.dumps({"trace_table": res}, indent=1))
    return res


def step_table(csv_path: str, out_path: str | None) -> dict:
    """Summarises a rocprofv3 kernel trace of ``--tpot-only``: the dispatches of the INT8 run's
    last eight graph-replayed decode steps (each step ends with the library's argmax kernel), per
    kernel: dispatches per step, µs per step and mean duration (template arguments dropped).  In
    a graph each dispatch starts when the previous one ends, so a duration includes its start-up;
    the smallest ones show the per-dispatch floor."""
    import csv
    import re

    rows = sorted(csv.DictReader(open(csv_path)), key=lambda r: int(r["Start_Timestamp"]))
    dec = [i for i, r in enumerate(rows)
           if "decode_kernel" in r["Kernel_Name"] and "true" in r["Kernel_Name"].split(",")[2]]
    ends = [i for i, r in enumerate(rows)
            if "argmax_kernel" in r["Kernel_Name"] and dec[0] < i <= dec[-1] + 64]
    steps = list(zip(ends[:-1], ends[1:]))[-8:]
    per: dict = {}
    span = 0.0
    for a, b in steps:
        win = rows[a + 1: b + 1]
        span += (int(win[-1]["End_Timestamp"]) - int(win[0]["Start_Timestamp"])) / 1e3
        for r in win:
            name = re.sub(r"\(.*", "", r["Kernel_Name"]).replace("void ", "")
            name = re.sub(r"<.*", "", name)[:80]
            d = per.setdefault(name, [0, 0.0])
            d[0] += 1
            d[1] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    n = len(steps)
    table = sorted(({"kernel": k, "per_step": round(c / n, 1), "us_per_step": round(t / n, 1),
                     "mean_us": round(t / c, 2)} for k, (c, t) in per.items()),
                   key=lambda e: -e["us_per_step"])
    res = {"csv": csv_path, "steps": n, "span_per_step_us": round(span / n, 1),
           "dispatches_per_step": round(sum(c for c, _ in per.values()) / n, 1), "kernels": table}
    log(f"steps {n}: span {res['span_per_step_us']} us, {res['dispatches_per_step']} dispatches")
    for e in table:
        log(f"  {e['per_step']:6.1f} x {e['us_per_step']:9.1f} us/step  mean {e['mean_us']:7.2f}  {e['kernel']}")
    if out_path:
        Path(out_path).parent.mkdir(parents=True, exist_ok=True)
        Path(out_path).write_text(json.dumps({"step_table": res}, indent=1))
    return res


def stamps_legs(dev, out_path: str | None) -> dict:
    """Per-wave timelines from the measurement build (libint8kv_stamps.so, -DINT8KV_STAMPS; main()
    points the ctypes binding at it): s_memrealtime stamps (10 ns ticks) at fixed points of each
    wave (entry, plan or sequence length, first segment's block ids + first requests, query
    operand, first tile's scores and P*V, segment done, end), read back after single calls.
    Each figure is the median over 10 calls of a per-call statistic over the waves, in ns from the
    median entry of the wave's XCD unless it is a phase length.  Legs:
    * cfg3: the headline INT8 call (range layout): dispatch spread, plan, first tile, exits (by
      XCD, and their call-to-call correlation); and with a caller's 512 ranges (two per
      workgroup), the exits of each workgroup's first and second range;
    * ceiling: the load-only decode probe and the INT8 decode on the read-ceiling pool (256
      equal ranges x 128 tiles; 64 sequences of 16,384 tokens): their exit spreads;
    * cfg4 call: config 4's per-layer call, the last of 28 in a HIP graph, alone (pools
      rotated) and after its layer's GEMMs;
    * cfg2 B=1 x 512: the INT8 and BF16 split layout at 16 workgroups per (sequence, kv head)
      and INT8's single-pass per-sequence layout: the phases of a one-tile wave.
    The stamps change each kernel's schedule a little; they show where time goes, not the
    product build's durations."""
    import ctypes

    import numpy as np
    import torch

    import int8kv
    from int8kv import _decode, _lib
    from int8kv import synthetic as syn

    lib = _lib.load()
    buf = np.zeros(16384 * 10, np.uint64)

    def collect(unit, run, reps=10):
        out = []
        for _ in range(reps):
            _lib.check(getattr(lib, f"int8kv_stamps_clear_{unit}")(), "stamps_clear")
            run()
            torch.cuda.synchronize()
            _lib.check(getattr(lib, f"int8kv_stamps_read_{unit}")(
                buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes), "stamps_read")
            st = buf.reshape(-1, 10).astype(np.int64)
            st = np.concatenate([st, np.arange(len(st))[:, None]], axis=1)  # column 10: slot
            out.append(st[st[:, 7] > 0].copy())
        return out

    def med(calls, fn):
        return round(float(np.median([fn(st) for st in calls])), 0)

    def timeline(calls, halves=False):
        """Range layout / probe: spreads and exits in ns.  The XCDs' real-time counters are
        offset from each other by up to ~2 us, so cross-wave times are taken from the median
        entry of the wave's own XCD (all XCDs receive their first workgroups within a few hundred
        ns of each other); the offsets' spread is reported as xcd_entry_median_spread."""
        def rel(st, i):
            origin = np.zeros(len(st), np.int64)
            for x in np.unique(st[:, 8]):
                sel = st[:, 8] == x
                origin[sel] = int(np.median(st[sel, 0]))
            return (st[:, i] - origin) * 10
        r = {"waves": med(calls, len),
             "entry_first": med(calls, lambda st: rel(st, 0).min()),
             "entry_last": med(calls, lambda st: rel(st, 0).max()),
             "exit_first": med(calls, lambda st: rel(st, 7).min()),
             "exit_p50": med(calls, lambda st: np.percentile(rel(st, 7), 50)),
             "exit_last": med(calls, lambda st: rel(st, 7).max())}
        r["finish_spread"] = r["exit_last"] - r["exit_p50"]
        if calls[0][:, 1].any():
            r["plan"] = med(calls, lambda st: np.median((st[:, 1] - st[:, 0]) * 10))
        seg = [st[st[:, 9] > 0] for st in calls]
        if len(seg[0]):
            r["first_segment_entered"] = med(seg, lambda st: np.median((st[:, 9] - st[:, 0]) * 10))
            r["first_scores_done"] = med(seg, lambda st: np.median((st[:, 4] - st[:, 0]) * 10))
            r["body_p50"] = med(seg, lambda st: np.median((st[:, 7] - st[:, 9]) * 10))
        # Entry per XCD (median over its waves, relative to the earliest XCD's): the XCDs' clock
        # offsets and dispatch order.
        def xcd(st):
            m = [np.median(st[st[:, 8] == x, 0]) for x in range(8) if (st[:, 8] == x).any()]
            return (max(m) - min(m)) * 10
        r["xcd_entry_median_spread"] = med(calls, xcd)
        # Exit (ns from the XCD's median entry) by XCD, and how well one call's per-wave exits
        # predict the next call's (Pearson correlation over the waves both stored).
        r["exit_median_by_xcd"] = [med(calls, lambda st, x=x: np.median(rel(st, 7)[st[:, 8] == x]))
                                   for x in range(8)]
        corr = []
        for a, b in zip(calls[:-1], calls[1:]):
            ea = dict(zip(a[:, 10], rel(a, 7)))
            eb = dict(zip(b[:, 10], rel(b, 7)))
            both = sorted(set(ea) & set(eb))
            corr.append(np.corrcoef([ea[k] for k in both], [eb[k] for k in both])[0, 1])
        r["exit_call_to_call_corr"] = round(float(np.median(corr)), 3)
        if halves:
            # Two ranges per workgroup (waves 0-3: the first, 4-7: the second, which holds the
            # pair's smaller share): median exit of each.
            for h, name in ((0, "exit_p50_first_range"), (1, "exit_p50_second_range")):
                r[name] = med(calls, lambda st, h=h: np.median(rel(st, 7)[(st[:, 10] % 8 >= 4) == bool(h)]))
        return r

    def phases(calls, query_first=False):
        """Per-sequence / split layout: the phases of the median wave (ns).  query_first: the
        per-sequence layout, which requests the query at entry and builds it while the first
        block ids are in flight (stamp 3 before stamp 2)."""
        seg = [st[st[:, 9] > 0] for st in calls]
        if query_first:
            names = (("sequence_length", 1, 0), ("ids_requested_query_built", 3, 9),
                     ("ids_staged_and_issue", 2, 3), ("k_scores_softmax", 4, 2))
        else:
            names = (("sequence_length", 1, 0), ("stage_and_issue", 2, 9), ("query", 3, 2),
                     ("k_scores_softmax", 4, 3))
        names += (("v_pv", 5, 4), ("rest_of_segment", 6, 5), ("state_to_barrier", 7, 6),
                  ("entry_to_barrier", 7, 0))
        return {n: med(seg, lambda st, a=a, b=b: np.median((st[:, a] - st[:, b]) * 10))
                for n, a, b in names}

    res = {"library": str(_lib.LIB_PATH.name)}
    # cfg3
    w = build_workload(dev)
    call = lambda: int8kv.int8_paged_attention(w["q"], w["kc"], w["vc"], w["bt"], w["sl"], w["ks"], w["vs"])
    settle(call, batch=5, min_ms=50.0)
    res["cfg3_int8"] = timeline(collect("i8", call))
    log(f"stamps cfg3: {res['cfg3_int8']}")
    # The paired layout (a caller's 512 ranges: two ranges per 8-wave workgroup, the first taking
    # 62.5 % of the pair's units): how the pair's two ranges finish.
    out = torch.empty_like(w["q"])
    ws = torch.empty(lib.int8kv_decode_workspace_bytes(28, 4, 128, 16, 512), dtype=torch.uint8,
                     device=dev)
    pcall = lambda: _decode.paged_decode(w["q"], w["kc"], w["vc"], w["bt"], w["sl"], w["ks"],
                                         w["vs"], out, 512, _lib.DECODE_ALL, ws)
    settle(pcall, batch=5, min_ms=50.0)
    res["cfg3_int8_paired_512"] = timeline(collect("i8", pcall), halves=True)
    log(f"stamps cfg3 paired: {res['cfg3_int8_paired_512']}")
    del out, ws
    del w
    torch.cuda.empty_cache()
    # ceiling pool: load-only probe and the decode over the same blocks
    R, T = 256, 128
    NB = R * T * 2
    pool = torch.empty(2, NB, 16, 4, 128, dtype=torch.int8, device=dev)
    pool.view(-1).copy_(torch.randint(-127, 128, (pool.numel(),), device=dev, dtype=torch.int8,
                                      generator=torch.Generator(device=dev).manual_seed(5)))
    ids = torch.randperm(NB, generator=torch.Generator().manual_seed(6)).to(torch.int32).to(dev)
    sink = torch.empty(1 << 20, dtype=torch.int32, device=dev)
    stream = _lib.stream_handle(dev)
    probe = lambda: _lib.check(lib.int8kv_probe_decode_loads(
        pool[0].data_ptr(), pool[1].data_ptr(), NB, 4, ids.data_ptr(), ids.numel(), R, T, 1,
        sink.data_ptr(), sink.numel(), stream), "probe_decode_loads")
    settle(probe, batch=5, min_ms=30.0)
    res["ceiling_probe"] = timeline(collect("probe", probe))
    B, L = 64, 16384
    bt = ids[: B * (L // 16)].view(B, L // 16).contiguous()
    sl = torch.full((B,), L, dtype=torch.int32, device=dev)
    q = torch.randn(B, 28, 128, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16).to(dev)
    sc = torch.full((4,), 0.02, device=dev)
    dec = lambda: int8kv.int8_paged_attention(q, pool[0], pool[1], bt, sl, sc, sc)
    settle(dec, batch=5, min_ms=30.0)
    res["ceiling_decode"] = timeline(collect("i8", dec))
    log(f"stamps ceiling: probe {res['ceiling_probe']}, decode {res['ceiling_decode']}")
    del pool, ids, sink, bt
    torch.cuda.empty_cache()
    # config 4's call, the last of 28 in a graph, alone and after its layer's GEMMs
    cs = ColdSetup(dev)
    for name, fns in (("cfg4_call_alone", [cs.op(i) for i in range(cs.NL)]),
                      ("cfg4_call_after_gemms",
                       [f for i in range(cs.NL) for f in (cs.gemms(i), cs.op(i))])):
        g = capture_graph(fns)
        settle(g.replay, batch=1, min_ms=30.0, max_ms=120.0)
        res[name] = timeline(collect("i8", g.replay))
        log(f"stamps {name}: {res[name]}")
        del g
    del cs
    torch.cuda.empty_cache()
    # config 2, B=1 x 512: one tile per wave
    dist = syn.make_distribution(11)
    ks, vs = syn.calibrate_scales(dist, seed=12)
    ks_d, vs_d = ks.to(dev), vs.to(dev)
    B, ctx = 1, 512
    gq = torch.Generator().manual_seed(B * 7 + ctx)
    pool_n = 2 * B * ctx // 16
    bt = syn.random_block_tables([ctx] * B, pool_n, gq)
    slots = syn.slot_mapping_for(bt, [ctx] * B)
    kk, vv = syn.sample_kv(B * ctx, dist, gq)
    q = syn.sample_query(B, gq).to(dev)
    kc8 = torch.zeros(pool_n, 16, 4, 128, dtype=torch.int8, device=dev)
    vc8 = torch.zeros_like(kc8)
    int8kv.int8_kv_cache_write(kk.to(dev), vv.to(dev), kc8, vc8, slots.to(dev), ks_d, vs_d)
    kc16 = torch.zeros(pool_n * 16, 4, 128, dtype=torch.bfloat16, device=dev)
    vc16 = torch.zeros_like(kc16)
    kc16[slots.to(dev)] = kk.to(dev)
    vc16[slots.to(dev)] = vv.to(dev)
    kc16, vc16 = kc16.view(pool_n, 16, 4, 128), vc16.view(pool_n, 16, 4, 128)
    btd = bt.to(dev)
    lens = torch.full((B,), ctx, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    ws = torch.empty(lib.int8kv_decode_workspace_bytes(28, 4, 128, 16, 64), dtype=torch.uint8,
                     device=dev)
    split = _lib.DECODE_ALL | _lib.DECODE_SPLIT_SEQUENCES
    for name, unit, kc, vc, ksc, vsc, fl in (
            ("cfg2_b1x512_int8_split16", "i8", kc8, vc8, ks_d, vs_d, split),
            ("cfg2_b1x512_bf16_split16", "bf16", kc16, vc16, None, None, split)):
        run = lambda: _decode.paged_decode(q, kc, vc, btd, lens, ksc, vsc, out, 16 * B, fl, ws, 0)
        settle(run, batch=20, min_ms=20.0)
        res[name] = phases(collect(unit, run))
        log(f"stamps {name}: {res[name]}")
    run = lambda: int8kv.int8_paged_attention(q, kc8, vc8, btd, lens, ks_d, vs_d)
    settle(run, batch=20, min_ms=20.0)
    res["cfg2_b1x512_int8_per_sequence"] = phases(collect("i8", run), query_first=True)
    log(f"stamps cfg2_b1x512_int8_per_sequence: {res['cfg2_b1x512_int8_per_sequence']}")
    if out_path:
        Path(out_path).parent.mkdir(parents=True, exist_ok=True)
        Path(out_path).write_text(json.dumps({"stamps": res}, indent=1))
    return res


def ceiling_legs(dev, out_path: str | None) -> dict:
    """Read ceilings of the INT8 decode's K/V stream on this GPU (include/int8kv_probe.h), next to
    the decode itself, all on one 1 GiB shuffled pool (65,536 INT8 blocks of 16 tokens x 4 kv
    heads x 128 for K and as many for V, 256 ranges x 128 tiles): a plain streaming read of the
    pool (ordinary and non-temporal loads), the decode's own per-lane K/V loads without its
    arithmetic (ordinary and non-temporal), and the INT8 decode kernel over the same blocks
    (64 sequences of 16,384 tokens, its automatic plan: the range layout, non-temporal loads).
    Event-timed back-to-back launches; TB/s of the pool's bytes (the decode: its algorithmic
    bytes)."""
    import torch

    import int8kv
    from int8kv import _decode, _lib, roofline

    lib = _lib.load()
    R, T = 256, 128                      # ranges, tiles per range
    NB = R * T * 2                       # 16-token blocks
    pool = torch.empty(2, NB, 16, 4, 128, dtype=torch.int8, device=dev)
    g = torch.Generator(device=dev).manual_seed(5)
    pool.view(-1).copy_(torch.randint(-127, 128, (pool.numel(),), generator=g, device=dev,
                                      dtype=torch.int8))
    kc, vc = pool[0], pool[1]
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(6)).to(torch.int32)
    ids = perm.to(dev)
    nbytes = pool.numel()
    stream = _lib.stream_handle(dev)
    sink = torch.empty(1 << 20, dtype=torch.int32, device=dev)
    res = {"pool_bytes": nbytes, "ranges": R, "tiles_per_range": T}

    def probe_stream(nt):
        def fn():
            _lib.check(lib.int8kv_probe_stream_read(pool.data_ptr(), nbytes, nt, sink.data_ptr(),
                                                    256 * 8 * 256, stream), "probe_stream_read")
        return fn

    def probe_decode(nt):
        def fn():
            _lib.check(lib.int8kv_probe_decode_loads(kc.data_ptr(), vc.data_ptr(), NB, 4,
                                                     ids.data_ptr(), ids.numel(), R, T, nt,
                                                     sink.data_ptr(), sink.numel(), stream),
                       "probe_decode_loads")
        return fn

    for name, fn in (("stream_read", probe_stream(0)), ("stream_read_nt", probe_stream(1)),
                     ("decode_loads", probe_decode(0)), ("decode_loads_nt", probe_decode(1))):
        settle(fn, batch=5, min_ms=30.0)
        ms = time_events(fn, 20, 5)
        res[name + "_us"] = round(ms * 1e3, 2)
        res[name + "_TBps"] = round(nbytes / ms / 1e9, 3)
        log(f"ceiling: {name}: {ms * 1e3:.2f} us, {nbytes / ms / 1e9:.3f} TB/s")
    # The decode over the same blocks: 64 sequences of 16,384 tokens, sequence b owning blocks
    # perm[1024 b .. 1024 b + 1023] of the K and V pools (every block once, as in the probes).
    B, L = 64, 16384
    bt = ids[: B * (L // 16)].view(B, L // 16).contiguous()
    sl = torch.full((B,), L, dtype=torch.int32, device=dev)
    q = torch.randn(B, 28, 128, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16).to(dev)
    ks = torch.full((4,), 0.02, device=dev)
    vs = torch.full((4,), 0.02, device=dev)
    out = torch.empty_like(q)
    ws = torch.empty(lib.int8kv_decode_workspace_bytes(28, 4, 128, 16, 0), dtype=torch.uint8,
                     device=dev)
    dbytes = roofline.decode_bytes(sl.cpu().numpy(), 4, 128, 1, B, 28)
    plan = _lib.decode_plan(q.dtype, kc.dtype, B, 28, 4, 128, NB, 16, L // 16)
    for name, flags in (("decode_kernel", _lib.DECODE_MAIN), ("decode_op", _lib.DECODE_ALL)):
        fn = lambda flags=flags: _decode.paged_decode(q, kc, vc, bt, sl, ks, vs, out, 0, flags, ws)
        settle(fn, batch=5, min_ms=30.0)
        ms = time_events(fn, 20, 5)
        res[name + "_us"] = round(ms * 1e3, 2)
        res[name + "_TBps"] = round(dbytes / ms / 1e9, 3)
        log(f"ceiling: {name} (B={B} x {L}, {plan['layout']}, nt={plan['non_temporal']}): "
            f"{ms * 1e3:.2f} us, {dbytes / ms / 1e9:.3f} TB/s")
    res["decode_bytes"] = dbytes
    res["decode_plan"] = plan
    res["decode_kernel_of_pattern_ceiling"] = round(res["decode_kernel_TBps"] / res["decode_loads_nt_TBps"], 3)
    del pool
    torch.cuda.empty_cache()
    if out_path:
        Path(out_path).parent.mkdir(parents=True, exist_ok=True)
        Path(out_path).write_text(json.dumps({"ceiling": res}, indent=1))
    return res


def counter_run(dev, mode: str) -> None:
    """Eager calls for a rocprofv3 counter pass (the profiler serialises counted dispatches, so
    graphs are not used): "warm" = 40 calls on one layer pool; "cold" = 2 x 28 layers of (the
    layer's GEMMs, the call on its pool); "cfg3" = 10 INT8 and 10 BF16 calls of the headline
    workload."""
    import torch

    if mode == "cfg3":
        import int8kv

        w = build_workload(dev)
        for _ in range(10):
            int8kv.int8_paged_attention(w["q"], w["kc"], w["vc"], w["bt"], w["sl"], w["ks"], w["vs"])
        for _ in range(10):
            int8kv.bf16_paged_attention(w["q"], w["kc16"], w["vc16"], w["bt"], w["sl"])
        torch.cuda.synchronize()
        return
    cs = ColdSetup(dev)
    if mode == "warm":
        for _ in range(40):
            cs.op(0)()
    else:
        for _ in range(2):
            for i in range(cs.NL):
                cs.gemms(i)()
                cs.op(i)()
    torch.cuda.synchronize()
    log(f"counter run {mode}: done")


def tpot_config4(dev, out_path: str | None, batch: int = 32, context: int = 8192,
                 new_tokens: int = 128, layers: int = 28, gemm_tuning: str = "use",
                 tuning_file: str | None = None) -> dict:
    """Config 4: greedy decode of a random-init Qwen2.5-7B-shaped bf16 model, INT8 vs BF16 KV.

    B sequences of ``context`` random prompt ids, ``new_tokens`` greedy tokens each; attention
    runs on this library (INT8: static per-head write + INT8 decode; BF16: bf16 cache + BF16
    decode), the rest on torch (hipBLASLt GEMMs, SDPA for the prefill).  Each decode step is one
    HIP-graph replay.  TPOT = (T128 - T1) / 127 as in the reference's
    bench/benchmark_decode_tpot.py:64-68; KV bytes are the paged caches of all layers.
    """
    import dataclasses

    import torch

    from int8kv import decode_loop as DL

    shape = dataclasses.replace(DL.QWEN25_7B, layers=layers)
    tuned = DL.configure_gemm_tuning(gemm_tuning, tuning_file or DL.GEMM_TUNING_FILE)
    torch.zeros(1, device=dev)  # initialises the allocator before its statistics are reset
    torch.cuda.reset_peak_memory_stats(dev)
    t0 = time.perf_counter()
    weights = DL.random_weights(shape, dev, seed=0)
    torch.cuda.synchronize(dev)
    log(f"cfg4: weights {weights.nbytes() / 1e9:.2f} GB in {time.perf_counter() - t0:.1f} s")
    calib = torch.randint(0, shape.vocab, (4, 512), generator=torch.Generator().manual_seed(3))
    scales = DL.calibrate_static_scales(weights, calib)
    res = {"config": {"model": "random-init Qwen2.5-7B shape (bf16)", **dataclasses.asdict(shape),
                      "batch": batch, "context": context, "new_tokens": new_tokens,
                      "calibration": "4 x 512 random ids, absmax/127 of post-rotary K and V",
                      "gemm_tuning": gemm_tuning if tuned else "off"},
           "runs": []}
    gens, step1, first = {}, {}, {}
    for mode in DL.MODES:
        rec = DL.run_tpot(weights, batch, context, new_tokens, mode,
                          scales=scales if mode == "int8" else None, log=lambda m, **k: log(m))
        loop = rec.pop("_loop")
        gens[mode] = rec.pop("_generated").cpu()
        step1[mode] = rec.pop("_step1_logits").cpu().double()
        first[mode] = rec.pop("_first_tokens").cpu()
        res["runs"].append(rec)
        del loop
        torch.cuda.empty_cache()
    i8, bf = res["runs"]
    a, b = step1["int8"], step1["bf16"]
    res["int8_vs_bf16"] = {
        "step1_logits_cos_min": round(float(torch.nn.functional.cosine_similarity(a, b, dim=1).min()), 6),
        "step1_logits_rel_l2": round(float((a - b).norm() / b.norm()), 6),
        "step1_top1_agreement": round(float((a.argmax(1) == b.argmax(1)).float().mean()), 4),
        "prefill_first_tokens_equal": bool(torch.equal(first["int8"], first["bf16"])),
        "tpot_speedup": round(bf["decode_tpot_ms"] / i8["decode_tpot_ms"], 4),
        "kv_bytes_ratio": round(i8["kv_cache_bytes"] / bf["kv_cache_bytes"], 4),
        "greedy_token_agreement": round(float((gens["int8"] == gens["bf16"]).float().mean()), 4),
        "first_divergence_step_median": int(torch.tensor(
            [int((r != s).nonzero()[0]) if (r != s).any() else new_tokens
             for r, s in zip(gens["int8"], gens["bf16"])]).median()),
    }
    log(f"cfg4: {json.dumps(res['int8_vs_bf16'])}")
    if out_path:
        Path(out_path).parent.mkdir(parents=True, exist_ok=True)
        Path(out_path).write_text(json.dumps(res, indent=1))
    return res


def calibrate_copy(dev) -> None:
    """Three plain 1 GiB device-to-device copies: each reads and writes exactly 1,048,576 KiB,
    which scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes."""
    import torch

    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20,
                    help="untimed calls before each timed loop (the first timed loop is also "
                         "preceded by the settle phase, whatever this is)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-budget", type=float, default=4.0,
                    help="seconds of one CPU-baseline pass (the sample is sized to it)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--no-writes", action="store_true", help="skip the cache-write legs")
    ap.add_argument("--writes-only", action="store_true",
                    help="run only the cache-write legs (config 1 eagerly, not as graph replays: "
                         "for rocprofv3 counter passes) and print their JSON")
    ap.add_argument("--midsize", metavar="JSON", default=None,
                    help="only the mid-size INT8 decode cases (B=32 x 8256 ...), results to JSON")
    ap.add_argument("--cold", metavar="JSON", default=None,
                    help="only config 4's per-layer decode call with warm and cold caches (28 "
                         "layer pools rotated, and between the decode step's GEMMs), results to JSON")
    ap.add_argument("--trace-table", nargs=2, metavar=("CSV", "JSON"), default=None,
                    help="summarise a rocprofv3 kernel trace of --cold (CPU only) into JSON")
    ap.add_argument("--step-table", nargs=2, metavar=("CSV", "JSON"), default=None,
                    help="summarise a rocprofv3 kernel trace of --tpot-only (CPU only) into JSON")
    ap.add_argument("--stamps", metavar="JSON", default=None,
                    help="only the per-wave timelines of the measurement build "
                         "(libint8kv_stamps.so), into JSON")
    ap.add_argument("--ceiling", metavar="JSON", default=None,
                    help="only the read-ceiling probes of the decode's K/V stream, into JSON")
    ap.add_argument("--counter-run", choices=("warm", "cold", "cfg3"), default=None,
                    help="only eager decode calls for a rocprofv3 counter pass (config 4's call on "
                         "a warm pool or between the step's GEMMs, or the headline workload)")
    ap.add_argument("--layouts", metavar="JSON", default=None,
                    help="only the layout comparison (automatic vs each forced layout over head_dim "
                         "64/128/256 short and few-sequence calls), results to JSON")
    ap.add_argument("--sweep", metavar="JSON", default=None,
                    help="also measure the config-2 decode sweep, written to JSON")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run 3 plain 1 GiB device copies (the reference kernel that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters to bytes)")
    ap.add_argument("--tpot", metavar="JSON", default=None,
                    help="also run config 4 (28-layer random-init Qwen2.5-7B decode loop, INT8 vs "
                         "BF16 KV: TPOT and KV bytes), written to JSON")
    ap.add_argument("--tpot-only", action="store_true",
                    help="run only config 4 (no headline line)")
    ap.add_argument("--tpot-shape", default="32,8192,128,28", metavar="B,CTX,NEW,LAYERS",
                    help="config-4 batch, prompt length, new tokens and layer count")
    ap.add_argument("--gemm-tuning", default="use", choices=("off", "use", "tune"),
                    help="config 4: torch GEMM solution choice (TunableOp results file, or tune it)")
    ap.add_argument("--gemm-tuning-file", default=None,
                    help="config 4: TunableOp results file (default: the one shipped with int8kv)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: every GPU box of this build has one GPU, and the "
              "decode op needs no exchange to shard (sequences and kv heads split across GPUs "
              "independently); run with --gpus 1.", file=sys.stderr)
        return 2
    if args.trace_table:
        trace_table(*args.trace_table)
        return 0
    if args.step_table:
        step_table(*args.step_table)
        return 0
    if args.stamps:
        os.environ["INT8KV_CTYPES"] = "1"  # the torch extension is linked to the product build

    import torch

    import int8kv
    from int8kv import _decode, _lib, roofline

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.stamps:
        from int8kv import _build

        _lib.LIB_PATH = _build.STAMPS_LIB_PATH
    _lib.load()
    dev = torch.device("cuda:0")
    tpot_args = [int(x) for x in args.tpot_shape.split(",")]
    if args.tpot_only:
        tpot_config4(dev, args.tpot, *tpot_args, gemm_tuning=args.gemm_tuning,
                     tuning_file=args.gemm_tuning_file)
        return 0
    if args.midsize:
        midsize_legs(dev, args.midsize)
        return 0
    if args.layouts:
        layout_legs(dev, args.layouts)
        return 0
    if args.cold:
        cold_legs(dev, args.cold)
        return 0
    if args.stamps:
        stamps_legs(dev, args.stamps)
        return 0
    if args.counter_run:
        counter_run(dev, args.counter_run)
        return 0
    if args.ceiling:
        ceiling_legs(dev, args.ceiling)
        return 0
    if args.writes_only:
        res = write_legs(dev, cfg1_graph=False)
        if args.calibrate_copy:
            calibrate_copy(dev)
        print(json.dumps({"writes": res}), flush=True)
        return 0
    log("building workload (B=64, ctx ~ U[1, 32768]) ...")
    w = build_workload(dev, seed=args.seed)
    lens = w["lens"]
    nbytes8 = roofline.decode_bytes(lens.numpy(), 4, 128, 1, 64, 28)
    nbytes16 = roofline.decode_bytes(lens.numpy(), 4, 128, 2, 64, 28)
    log(f"tokens={int(lens.sum())} blocks={w['num_blocks']} int8 bytes/call={nbytes8}")

    def int8_call():
        return int8kv.int8_paged_attention(w["q"], w["kc"], w["vc"], w["bt"], w["sl"], w["ks"], w["vs"])

    def bf16_call():
        return int8kv.bf16_paged_attention(w["q"], w["kc16"], w["vc16"], w["bt"], w["sl"])

    # Decode kernel alone (no merge), same arguments as int8_call, workspace preallocated.
    chunk = 0
    need = _lib.load().int8kv_decode_workspace_bytes(28, 4, 128, 16, chunk)
    ws = torch.zeros(max(need, 16), dtype=torch.uint8, device=dev)
    out_main = torch.empty_like(w["q"])

    def main_kernel():
        _decode.paged_decode(w["q"], w["kc"], w["vc"], w["bt"], w["sl"], w["ks"], w["vs"], out_main,
                             chunk, _lib.DECODE_MAIN, ws)

    def merge_kernel():
        _decode.paged_decode(w["q"], w["kc"], w["vc"], w["bt"], w["sl"], w["ks"], w["vs"], out_main,
                             chunk, _lib.DECODE_MERGE, ws)

    out = int8_call()
    torch.cuda.synchronize()
    st = settle(int8_call, min_ms=400.0)
    log(f"settle: {st}")
    ms = time_loop(int8_call, args.steps, args.warmup)
    ms_main = time_events(main_kernel, args.steps, args.warmup)
    plan = _lib.decode_plan(w["q"].dtype, w["kc"].dtype, 64, 28, 4, 128, w["num_blocks"], 16,
                            w["bt"].shape[1])
    # A separate merge kernel (when the layout has one) takes a few microseconds, less than the
    # host's cost of one call: HIP-graph replays give its device time.
    ms_merge = time_graph(merge_kernel) if plan["kernels"] == 2 else None
    # Each later op gets a short settle of its own: switching from one sustained load to another
    # (the BF16 op after the INT8 one) showed the same kind of dip for a few ms.
    settle(bf16_call, batch=10, min_ms=30.0)
    ms16 = time_loop(bf16_call, args.steps, args.warmup)

    def int8_q_call():
        return int8kv.int8_paged_attention(w["q"], w["kc"], w["vc"], w["bt"], w["sl"], w["ks"], w["vs"],
                                           quantize_q=True)

    settle(int8_q_call, batch=10, min_ms=30.0)
    ms_q = time_loop(int8_q_call, args.steps, args.warmup)
    # Host cost of one eager call, through the torch extension (the default path) and through the
    # ctypes binding of the same C ABI: the wall time of one call made when the device has caught
    # up (median of 50), and the wall time per call of enqueueing 50 calls without waiting (median
    # of five batches after one untimed), where each call's ~190 us of device work keeps the device
    # ever further behind the host: the HIP runtime's launches then cost ~3.5 us more per call
    # (MI355X, ROCm 7.2; 5.5 us per call with 20-us calls queued, 9 us with 190-us ones).
    from int8kv import _ext

    def call_us(calls=50):
        per_call = []
        for _ in range(calls + 1):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            int8_call()
            per_call.append((time.perf_counter() - t0) * 1e6)
        torch.cuda.synchronize()
        return statistics.median(per_call[1:])

    def enqueue_us(batches=5, calls=50):
        per_call = []
        for rep in range(batches + 1):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(calls):
                int8_call()
            if rep:
                per_call.append((time.perf_counter() - t0) * 1e6 / calls)
        torch.cuda.synchronize()
        return statistics.median(per_call)

    host_us, host_us_queued = call_us(), enqueue_us()
    with _ext.use_ctypes():
        host_us_ctypes, host_us_ctypes_queued = call_us(), enqueue_us()
    value = nbytes8 / (ms * 1e-3) / 1e9
    achieved = nbytes8 / (ms_main * 1e-3) / 1e9
    log(f"int8 op: {ms * 1e3:.1f} us/call ({value:.0f} GB/s); decode kernel {ms_main * 1e3:.1f} us "
        f"({achieved:.0f} GB/s); merge kernel {ms_merge and round(ms_merge * 1e3, 1)} us; "
        f"bf16 op {ms16 * 1e3:.1f} us "
        f"({nbytes16 / (ms16 * 1e-3) / 1e9:.0f} GB/s); int8 quantize_q op {ms_q * 1e3:.1f} us; "
        f"host enqueue {host_us:.1f} us/call, {host_us_queued:.1f} queued (ctypes path "
        f"{host_us_ctypes:.1f}, {host_us_ctypes_queued:.1f})")

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded Qwen2.5-7B-shaped K/V with outlier channels; no checkpoint)",
        "config": {
            "workload": "cfg3: one-layer INT8 paged decode, B=64, ctx ~ U[1,32768] ragged, "
                        "28q/4kv heads, head_dim 128, block 16, shuffled block pool",
            "batch": 64,
            "seed": args.seed,
            "tokens": int(lens.sum()),
            "max_ctx": int(lens.max()),
            "algorithmic_bytes_per_call": int(nbytes8),
            "us_per_call": round(ms * 1e3, 2),
            "bf16_us_per_call": round(ms16 * 1e3, 2),
            "bf16_algorithmic_bytes_per_call": int(nbytes16),
            "int8_speedup_vs_bf16": round(ms16 / ms, 3),
            "decode_kernel_us": round(ms_main * 1e3, 2),
            "merge_kernel_us_graph_replay": None if ms_merge is None else round(ms_merge * 1e3, 2),
            "plan": plan,
            "int8_quantize_q_us_per_call": round(ms_q * 1e3, 2),
            "frac_of_hbm_peak_whole_call": round(value / HBM_PEAK_GBS, 4),
            "host_enqueue_us_per_call": round(host_us, 2),
            "host_enqueue_us_per_call_ctypes": round(host_us_ctypes, 2),
            "host_enqueue_us_per_call_queued": round(host_us_queued, 2),
            "host_enqueue_us_per_call_ctypes_queued": round(host_us_ctypes_queued, 2),
            "host_path": "torch extension" if _ext.module() is not None else "ctypes",
            "settle": st,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": read_traffic(w, nbytes8),
            "traffic_source": "profiles/decode_int8_cfg3_traffic.json (rocprofv3 FETCH_SIZE + "
                              "WRITE_SIZE per launch, calibrated; used only when its seed, tokens "
                              "and algorithmic bytes match this workload)",
            "kernel": "decode_kernel<int8 cache, bf16 query>",
        },
        "cpu_baseline": None,
    }
    if not args.no_writes:
        result["config"]["writes"] = write_legs(dev)
    if not args.no_cpu:
        log(f"cpu baseline (torch, {cpu_threads()} threads) ...")
        cb, check = cpu_baseline(w, out, args.cpu_budget)
        cb["numpy_oracle_single_thread"] = cpu_oracle_single_thread(w)
        result["cpu_baseline"] = cb
        result["config"]["gpu_vs_cpu_on_sample"] = check
        log(f"cpu baseline {cb['value']} GB/s on {cb['cores']} threads; GPU vs CPU on sample: {check}")
    if args.sweep:
        sweep_configs(dev, args.sweep)
    if args.tpot:
        del w
        torch.cuda.empty_cache()
        tpot_config4(dev, args.tpot, *tpot_args, gemm_tuning=args.gemm_tuning,
                     tuning_file=args.gemm_tuning_file)
    if args.calibrate_copy:
        calibrate_copy(dev)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
