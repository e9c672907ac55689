"""bench.py's output contract: the one JSON line the round-end harness parses.

CPU: ``--gpus N`` with N > 1 (or a multi-rank launch) is refused with a message and exit
status 2, before anything touches a GPU.  GPU: a short headline run (3 timed steps, no write
legs, a sub-second CPU sample) prints one JSON line whose every required key is present with
the right type, whose figures agree with one another (value × ms_per_step = the algorithmic
bytes of one call, frac = achieved / peak, the decode kernel no slower than the whole call),
and whose roofline and cpu_baseline objects have the documented fields.
"""

from __future__ import annotations

import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
BENCH = REPO / "bench.py"


def _run(args, env=None, timeout=60):
    e = dict(os.environ)
    e.update(env or {})
    return subprocess.run([sys.executable, str(BENCH), *args], cwd=REPO, env=e, text=True,
                          capture_output=True, timeout=timeout)


@pytest.mark.parametrize("args,env", [(["--gpus", "2"], None), (["--gpus", "8"], None),
                                      (["--gpus", "1"], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_is_refused(args, env):
    r = _run(args, env)
    assert r.returncode == 2, (r.returncode, r.stderr)
    assert "one GPU" in r.stderr and "--gpus 1" in r.stderr
    assert r.stdout.strip() == ""  # no JSON line: the harness must not read a number from it


@pytest.mark.gpu
def test_headline_line_keeps_the_contract():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    steps, warmup = 3, 1
    print(f"bench.py --no-writes --steps {steps} --warmup {warmup} --cpu-budget 0.3", flush=True)
    r = _run(["--no-writes", "--steps", str(steps), "--warmup", str(warmup), "--cpu-budget", "0.3"],
             timeout=240)
    assert r.returncode == 0, r.stderr[-3000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, r.stdout[-2000:]
    d = json.loads(lines[0])

    types = {"metric": str, "value": float, "unit": str, "n_gpus": int, "steps": int,
             "warmup": int, "ms_per_step": float, "higher_is_better": bool, "scaling": str,
             "dtype": str, "data": str, "config": dict, "roofline": dict, "cpu_baseline": dict}
    for key, t in types.items():
        assert isinstance(d.get(key), t), (key, d.get(key))
    assert "vs_baseline" in d and d["vs_baseline"] is None  # no published number for this metric
    assert (d["n_gpus"], d["steps"], d["warmup"]) == (1, steps, warmup)
    assert d["unit"] == "GB/s" and d["higher_is_better"] is True and d["scaling"] in ("weak", "strong")
    assert d["dtype"] == "int8" and "synthetic" in d["data"]
    cfg = d["config"]
    assert isinstance(cfg.get("workload"), str) and cfg["workload"]
    assert not ({"model", "global_batch", "seq_len", "parallelism"} & set(cfg))

    # value is the whole call's algorithmic bytes over the step time
    nbytes = cfg["algorithmic_bytes_per_call"]
    assert d["value"] > 0 and d["ms_per_step"] > 0
    assert abs(d["value"] * 1e9 * d["ms_per_step"] * 1e-3 / nbytes - 1) < 2e-3
    assert abs(cfg["us_per_call"] - d["ms_per_step"] * 1e3) < 0.02
    assert cfg["tokens"] > 0 and cfg["batch"] == 64

    rf = d["roofline"]
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in rf, key
    assert rf["bound"] in ("hbm", "mfma") and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert 0 < rf["frac"] <= 1 and abs(rf["frac"] - rf["achieved"] / rf["peak"]) < 1e-3
    # the decode kernel alone is part of the call: its rate over the same bytes is not lower
    assert rf["achieved"] >= d["value"] * 0.98
    assert abs(nbytes / (rf["achieved"] * 1e9) * 1e6 - cfg["decode_kernel_us"]) < 0.05
    assert rf["traffic"] is None or rf["traffic"] >= nbytes * 0.95

    cb = d["cpu_baseline"]
    for key in ("value", "unit", "cores", "kind", "sample"):
        assert key in cb, key
    assert cb["kind"] in ("reference", "port") and cb["cores"] >= 1 and cb["value"] > 0
    assert cb["unit"] == d["unit"] and isinstance(cb["sample"], str) and cb["sample"]
    # the GPU call agrees with the CPU restatement on the sampled sequences
    agree = cfg["gpu_vs_cpu_on_sample"]
    assert agree["sequences"] >= 1 and agree["max_abs"] <= 2e-2 and agree["cos"] >= 0.9999
