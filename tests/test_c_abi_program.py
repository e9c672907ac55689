"""The C-ABI smoke program (tests/c_abi/abi_smoke.cpp): a host-only C++ caller of libint8kv.so
that uses nothing but include/int8kv.h and the HIP runtime.  On the CPU it must compile and link
against the header and the built library; on the GPU (the in-tree binary that
``__graft_entry__.build()`` makes) it writes, decodes and checks its results itself (cache bytes
against the quantisation, attention against a double-precision restatement, the no-allocation
entry point against the workspace one) and exits 0."""

from __future__ import annotations

import importlib.util
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent / "c_abi"


def _builder():
    spec = importlib.util.spec_from_file_location("abi_smoke_build", HERE / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_program_compiles_against_the_header(tmp_path):
    b = _builder()
    if not (b.LIB_DIR / "libint8kv.so").exists():
        pytest.fail("libint8kv.so is not built (run __graft_entry__.build())")
    out = b.build(tmp_path / "abi_smoke")
    assert out.exists() and out.stat().st_size > 0


@pytest.mark.gpu
def test_program_runs_and_checks_itself():
    exe = HERE / "abi_smoke"
    assert exe.exists(), "tests/c_abi/abi_smoke is not built (run __graft_entry__.build())"
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ABI SMOKE OK" in r.stdout
