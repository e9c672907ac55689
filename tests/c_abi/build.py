"""Builds tests/c_abi/abi_smoke, a host-only C++ caller of libint8kv.so's C ABI (no torch): g++
against include/int8kv.h and the HIP runtime, linked to int8-kvcache_amd/int8kv/libint8kv.so
through an $ORIGIN-relative rpath, so the binary runs wherever the repository is copied."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
SRC = HERE / "abi_smoke.cpp"
BIN = HERE / "abi_smoke"
LIB_DIR = REPO / "int8-kvcache_amd" / "int8kv"
ROCM = Path("/opt/rocm")


def command(out: Path) -> list[str]:
    rel = Path("..") / ".." / LIB_DIR.relative_to(REPO)
    return ["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-Wall", "-D__HIP_PLATFORM_AMD__=1",
            f"-I{ROCM / 'include'}", f"-I{REPO / 'include'}", str(SRC), f"-L{LIB_DIR}", "-lint8kv",
            f"-Wl,-rpath,$ORIGIN/{rel}", f"-L{ROCM / 'lib'}", "-lamdhip64",
            f"-Wl,-rpath,{ROCM / 'lib'}", "-o", str(out)]


def build(out: Path = BIN) -> Path:
    subprocess.run(command(out), check=True)
    return out


if __name__ == "__main__":
    print(build(Path(sys.argv[1]) if len(sys.argv) > 1 else BIN))
