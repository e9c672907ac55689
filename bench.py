#!/usr/bin/env python3
"""Headline benchmark: INT8 PagedAttention decode on one MI355X (the large ragged batch).

Workload (the configuration the headline metric is quoted on): one decode step of one layer,
Qwen2.5-7B attention shape (28 query heads, 4 kv heads, head_dim 128, 16-token cache blocks),
B = 64 sequences with context lengths drawn uniformly from [1, 32768], block tables shuffled
over a shared pool of ~65.6k physical blocks (~1.07 GB of int8 K+V).  Inputs are synthetic
(seeded), written into the int8 cache by this library's own cache-write kernel, and resident
in HBM before the timed region starts.

A "step" is one int8_paged_attention call (decode kernel + split merge).  Reported:
  * value: whole-call algorithmic HBM GB/s (K+V bytes once, block-table entries, q, out,
    seq_lens, scales) over the measured step time;
  * roofline: the decode kernel alone, timed with one HIP event pair around back-to-back
    launches on the launch stream, against the 8 TB/s HBM peak; ``traffic`` comes from committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE counters when present;
  * the same-kernel BF16 path on the same data (bf16 cache), for the INT8-vs-BF16 comparison;
  * cpu_baseline: the CPU oracle (a numpy restatement of the reference's torch path) timed on a
    bounded sample (about 10 s of work) of the same sequences on this host, one thread.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import math
import os
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
                ks=ks_d, vs=vs_d, lens=lens, bt_cpu=bt, num_blocks=num_blocks)


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


def time_graph(fn, calls: int = 20, replays: int = 10) -> float:
    """Device time per call (ms) of ``fn`` captured ``calls`` times in one HIP graph and replayed:
    removes the host's per-call launch cost, which dominates calls of a few microseconds."""
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
    for _ in range(2):
        graph.replay()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(replays):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / (replays * calls)


def cpu_baseline(w, out_gpu, budget_s: float = 10.0):
    """Times the CPU oracle (one thread) over the workload's sequences, pass after pass, until
    ``budget_s`` seconds of oracle work are done; the first pass also measures the agreement of
    the GPU output with the oracle on every sequence."""
    import numpy as np

    from oracle import int8kv_oracle as O

    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    kc = w["kc"].cpu().numpy()
    vc = w["vc"].cpu().numpy()
    q = w["q"].float().cpu().numpy()
    bt = w["bt_cpu"].numpy()
    lens = w["lens"].numpy()
    ks, vs = w["ks"].cpu().numpy(), w["vs"].cpu().numpy()
    got = out_gpu.float().cpu().numpy()
    ctx = threadpool_limits(limits=1) if threadpool_limits else None
    calls, t_total, nbytes, tokens = 0, 0.0, 0, 0
    worst, dots, n1, n2 = 0.0, 0.0, 0.0, 0.0
    first_pass = True
    try:
        if ctx:
            ctx.__enter__()
        while t_total < budget_s:
            for b in range(len(lens)):
                t0 = time.perf_counter()
                ref = O.paged_attention_ref(q[b:b + 1], kc, vc, bt[b:b + 1], lens[b:b + 1], ks, vs)
                t_total += time.perf_counter() - t0
                nbytes += O.decode_bytes(lens[b:b + 1], 4, 128, 1, 1, 28)
                tokens += int(lens[b])
                calls += 1
                if first_pass:
                    d = got[b:b + 1].astype(np.float64)
                    r = ref.astype(np.float64)
                    worst = max(worst, float(np.abs(d - r).max()))
                    dots += float((d * r).sum())
                    n1 += float((d * d).sum())
                    n2 += float((r * r).sum())
                if t_total >= budget_s and not first_pass:
                    break
            first_pass = False
    finally:
        if ctx:
            ctx.__exit__(None, None, None)
    cos = dots / math.sqrt(n1 * n2) if n1 > 0 and n2 > 0 else 0.0
    return {
        "value": round(nbytes / t_total / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{calls} single-sequence oracle calls over the workload's {len(lens)} sequences "
                  f"({tokens} tokens; numpy gather, dequantise, fp32 softmax attention), "
                  f"{t_total:.1f} s on one thread",
        "us_per_call_extrapolated": round(t_total / max(tokens, 1) * int(lens.sum()) * 1e6, 1),
    }, {"sequences": len(lens), "max_abs": worst, "cos": cos}


def read_traffic():
    """HBM bytes per decode launch from the committed rocprofv3 counter summary (or None)."""
    if not TRAFFIC_FILE.exists():
        return None
    try:
        d = json.loads(TRAFFIC_FILE.read_text())
        return int(d["traffic_bytes_per_launch"])
    except (ValueError, KeyError):
        return None


def sweep_configs(dev, out_path: str | None) -> dict:
    """The two smaller benchmark configurations, reported beside the headline line:
    cfg1 -- the prefill cache write alone (8 x 2048 tokens + 512 padding slots into a
    2048-block cache through a random-permutation slot mapping); cfg2 -- INT8 and BF16 decode at
    B in {1, 2, 4, 8} x uniform ctx in {512, 1024, 2048, 4096}, automatic split vs one range per
    sequence.  Both working sets fit the 256 MB Infinity Cache, so their GB/s are cache-resident
    rates and µs/call is the meaningful figure.  Times are device times per call from HIP-graph
    replays (a few-microsecond call is otherwise dominated by the host's launch cost)."""
    import numpy as np
    import torch

    import int8kv
    from int8kv import synthetic as syn
    from oracle import int8kv_oracle as O

    res = {}
    g = torch.Generator().manual_seed(11)
    dist = syn.make_distribution(11)
    ks, vs = syn.calibrate_scales(dist, seed=12)
    n_tok, n_pad, nb = 16384, 512, 2048
    k, v = syn.sample_kv(n_tok + n_pad, dist, g)
    slots = torch.randperm(nb * 16, generator=g)[: n_tok + n_pad].to(torch.int64)
    slots[torch.randperm(n_tok + n_pad, generator=g)[:n_pad]] = -1
    kc = torch.zeros(nb, 16, 4, 128, dtype=torch.int8, device=dev)
    vc = torch.zeros_like(kc)
    k, v, slots_d, ks_d, vs_d = k.to(dev), v.to(dev), slots.to(dev), ks.to(dev), vs.to(dev)

    def write():
        int8kv.int8_kv_cache_write(k, v, kc, vc, slots_d, ks_d, vs_d)

    ms_w = time_graph(write)
    wbytes = n_tok * 4 * 128 * (2 + 2 + 1 + 1) + (n_tok + n_pad) * 8 + 2 * 4 * 4
    res["cfg1_write"] = {"tokens": n_tok, "padding_slots": n_pad, "us_per_call": round(ms_w * 1e3, 2),
                         "algorithmic_bytes": wbytes, "GBps": round(wbytes / ms_w / 1e6, 1)}
    log(f"cfg1 write: {ms_w * 1e3:.1f} us ({wbytes / ms_w / 1e6:.0f} GB/s)")

    # The dynamic per-(token, head) write (reshape_and_cache_int8) on the same inputs: the same
    # bytes plus one fp32 scale per (token, head) for K and V.
    from int8kv import cache_ops

    kcd, vcd = torch.zeros_like(kc), torch.zeros_like(vc)
    ksc = torch.zeros(nb, 16, 4, dtype=torch.float32, device=dev)
    vsc = torch.zeros_like(ksc)

    def dyn_write():
        cache_ops.reshape_and_cache_int8(k, v, kcd, vcd, ksc, vsc, slots_d)

    ms_d = time_graph(dyn_write)
    dbytes = wbytes - 2 * 4 * 4 + n_tok * 4 * 4 * 2
    res["cfg1_dynamic_write"] = {"us_per_call": round(ms_d * 1e3, 2), "algorithmic_bytes": dbytes,
                                 "GBps": round(dbytes / ms_d / 1e6, 1)}
    log(f"cfg1 dynamic write: {ms_d * 1e3:.1f} us ({dbytes / ms_d / 1e6:.0f} GB/s)")

    # The CPU oracle's static write on the same inputs (numpy, one thread), for comparison.
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    kn, vn, sn = k.float().cpu().numpy(), v.float().cpu().numpy(), slots.numpy()
    kcn = np.zeros((nb, 16, 4, 128), np.int8)
    vcn = np.zeros_like(kcn)
    ctx = threadpool_limits(limits=1) if threadpool_limits else None
    if ctx:
        ctx.__enter__()
    try:
        t0 = time.perf_counter()
        O.int8_kv_cache_write(kn, vn, kcn, vcn, sn, ks.numpy(), vs.numpy())
        t_cpu = time.perf_counter() - t0
    finally:
        if ctx:
            ctx.__exit__(None, None, None)
    same = bool(np.array_equal(kcn, kc.cpu().numpy()) and np.array_equal(vcn, vc.cpu().numpy()))
    res["cfg1_write_cpu_oracle"] = {"seconds": round(t_cpu, 4), "GBps": round(wbytes / t_cpu / 1e9, 3),
                                    "cores": 1, "kind": "port", "gpu_caches_bit_exact": same}
    log(f"cfg1 write on the CPU oracle: {t_cpu * 1e3:.1f} ms ({wbytes / t_cpu / 1e9:.2f} GB/s); "
        f"GPU caches bit-exact: {same}")

    # HBM-sized writes: 262,144 tokens into a 32,768-block pool (the sources alone exceed the
    # Infinity Cache).
    n_big, nb_big = 262144, 32768
    gb = torch.Generator(device=dev).manual_seed(13)
    kb_, vb_ = syn.sample_kv(n_big, dist, gb, device=dev)
    sb_ = torch.randperm(nb_big * 16, device=dev, generator=gb)[:n_big]
    kcb = torch.zeros(nb_big, 16, 4, 128, dtype=torch.int8, device=dev)
    vcb = torch.zeros_like(kcb)
    kscb = torch.zeros(nb_big, 16, 4, dtype=torch.float32, device=dev)
    vscb = torch.zeros_like(kscb)
    big_bytes = n_big * 4 * 128 * 6 + n_big * 8 + 32
    ms_sb = time_loop(lambda: int8kv.int8_kv_cache_write(kb_, vb_, kcb, vcb, sb_, ks_d, vs_d), 40, 10)
    ms_db = time_loop(lambda: cache_ops.reshape_and_cache_int8(kb_, vb_, kcb, vcb, kscb, vscb, sb_), 40, 10)
    res["hbm_write_262k"] = {
        "tokens": n_big, "static_us": round(ms_sb * 1e3, 2),
        "static_GBps": round(big_bytes / ms_sb / 1e6, 1), "dynamic_us": round(ms_db * 1e3, 2),
        "dynamic_GBps": round((big_bytes - 32 + n_big * 32) / ms_db / 1e6, 1)}
    log(f"262k-token writes: static {ms_sb * 1e3:.1f} us, dynamic {ms_db * 1e3:.1f} us")
    del kb_, vb_, sb_, kcb, vcb, kscb, vscb

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
            ):
                ms = time_graph(fn)
                e = 2 if name.startswith("bf16") else 1
                nbytes = O.decode_bytes([ctx] * B, 4, 128, e, B, 28)
                row[name + "_us"] = round(ms * 1e3, 2)
                row[name + "_GBps"] = round(nbytes / ms / 1e6, 1)
            rows.append(row)
            log(f"cfg2 B={B} ctx={ctx}: int8 {row['int8_auto_us']} us (single pass "
                f"{row['int8_single_pass_us']}), bf16 {row['bf16_auto_us']} us")
    res["cfg2_sweep"] = rows
    if out_path:
        Path(out_path).parent.mkdir(parents=True, exist_ok=True)
        Path(out_path).write_text(json.dumps(res, indent=1))
    return res


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


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=100,
                    help="untimed calls before each timed loop (the first ~50 calls after the "
                         "workload build run at lower clocks)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-budget", type=float, default=10.0,
                    help="seconds of CPU-oracle work for the cpu_baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--sweep", metavar="JSON", default=None,
                    help="also measure the cfg1 write and the cfg2 decode sweep, written to JSON")
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
        print("bench.py measures one GPU only: the decode op has no multi-GPU path in this build "
              "(sequences and kv heads shard across GPUs without any exchange); run with --gpus 1.",
              file=sys.stderr)
        return 2

    import torch

    import int8kv
    from int8kv import _decode, _lib
    from oracle import int8kv_oracle as O

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    _lib.load()
    dev = torch.device("cuda:0")
    tpot_args = [int(x) for x in args.tpot_shape.split(",")]
    if args.tpot_only:
        tpot_config4(dev, args.tpot, *tpot_args, gemm_tuning=args.gemm_tuning,
                     tuning_file=args.gemm_tuning_file)
        return 0
    log("building workload (B=64, ctx ~ U[1, 32768]) ...")
    w = build_workload(dev, seed=args.seed)
    lens = w["lens"]
    nbytes8 = O.decode_bytes(lens.numpy(), 4, 128, 1, 64, 28)
    nbytes16 = O.decode_bytes(lens.numpy(), 4, 128, 2, 64, 28)
    log(f"tokens={int(lens.sum())} blocks={w['num_blocks']} int8 bytes/call={nbytes8}")

    def int8_call():
        return int8kv.int8_paged_attention(w["q"], w["kc"], w["vc"], w["bt"], w["sl"], w["ks"], w["vs"])

    def bf16_call():
        return int8kv.bf16_paged_attention(w["q"], w["kc16"], w["vc16"], w["bt"], w["sl"])

    # Decode kernel alone (no merge), same arguments as int8_call, workspace preallocated.
    chunk = 0
    need = _lib.load().int8kv_decode_workspace_bytes(28, 4, 128, 16, chunk)
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
    out_main = torch.empty_like(w["q"])

    def main_kernel():
        _decode.paged_decode(w["q"], w["kc"], w["vc"], w["bt"], w["sl"], w["ks"], w["vs"], out_main,
                             chunk, _lib.DECODE_MAIN, ws)

    def merge_kernel():
        _decode.paged_decode(w["q"], w["kc"], w["vc"], w["bt"], w["sl"], w["ks"], w["vs"], out_main,
                             chunk, _lib.DECODE_MERGE, ws)

    out = int8_call()
    torch.cuda.synchronize()
    ms = time_loop(int8_call, args.steps, args.warmup)
    ms_main = time_events(main_kernel, args.steps, args.warmup)
    # The merge kernel takes a few microseconds, less than the host's cost of one call: HIP-graph
    # replays give its device time.
    ms_merge = time_graph(merge_kernel)
    ms16 = time_loop(bf16_call, args.steps, args.warmup)
    ms_q = time_loop(lambda: int8kv.int8_paged_attention(w["q"], w["kc"], w["vc"], w["bt"], w["sl"], w["ks"],
                                                         w["vs"], quantize_q=True), args.steps, args.warmup)
    value = nbytes8 / (ms * 1e-3) / 1e9
    achieved = nbytes8 / (ms_main * 1e-3) / 1e9
    log(f"int8 op: {ms * 1e3:.1f} us/call ({value:.0f} GB/s); decode kernel {ms_main * 1e3:.1f} us "
        f"({achieved:.0f} GB/s); merge kernel {ms_merge * 1e3:.1f} us; bf16 op {ms16 * 1e3:.1f} us "
        f"({nbytes16 / (ms16 * 1e-3) / 1e9:.0f} GB/s); int8 quantize_q op {ms_q * 1e3:.1f} us")

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
            "tokens": int(lens.sum()),
            "max_ctx": int(lens.max()),
            "algorithmic_bytes_per_call": int(nbytes8),
            "us_per_call": round(ms * 1e3, 2),
            "bf16_us_per_call": round(ms16 * 1e3, 2),
            "bf16_algorithmic_bytes_per_call": int(nbytes16),
            "int8_speedup_vs_bf16": round(ms16 / ms, 3),
            "decode_kernel_us": round(ms_main * 1e3, 2),
            "merge_kernel_us_graph_replay": round(ms_merge * 1e3, 2),
            "int8_quantize_q_us_per_call": round(ms_q * 1e3, 2),
            "frac_of_hbm_peak_whole_call": round(value / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": read_traffic(),
            "kernel": "decode_kernel<int8 cache, bf16 query>",
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        log("cpu baseline (numpy oracle, 1 thread) ...")
        cb, check = cpu_baseline(w, out, args.cpu_budget)
        result["cpu_baseline"] = cb
        result["config"]["gpu_vs_oracle_on_sample"] = {
            "sequences": check["sequences"], "max_abs": round(check["max_abs"], 6),
            "cos": round(check["cos"], 7)}
        log(f"cpu baseline {cb['value']} GB/s; GPU vs oracle on sample: {check}")
    if args.sweep:
        sweep_configs(dev, args.sweep)
    if args.tpot:
        del w
        torch.cuda.empty_cache()
        tpot_config4(dev, args.tpot, *tpot_args, gemm_tuning=args.gemm_tuning,
                     tuning_file=args.gemm_tuning_file)
    if args.calibrate_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
