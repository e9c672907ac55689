"""Builds libint8kv.so (the HIP kernels plus the C ABI of include/int8kv*.h) for gfx950.

The library is compiled in-tree with hipcc, next to this file, so that it travels with the
source tree.  Usage: ``python -m int8kv._build`` (from the ``int8-kvcache_amd`` directory) or
``int8kv._build.build_library()``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC_DIR = PKG_DIR.parent / "csrc"
INCLUDE_DIR = PKG_DIR.parent.parent / "include"
LIB_PATH = PKG_DIR / "libint8kv.so"

SOURCES = ["cache_write.hip", "paged_decode.hip", "decode_loop_ops.hip"]

# -packed-fp32-ops keeps hipcc from emitting packed fp32 VALU instructions (v_pk_fma_f32 and
# friends) from ordinary float code; the host pass merely warns that it does not know it.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; ROCm is required to build libint8kv.so")


def _run(cmd, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in (proc.stdout + proc.stderr).splitlines() if noise not in ln]
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs), flush=True)


def build_library(verbose: bool = False) -> Path:
    """Compiles every HIP source into LIB_PATH (always rebuilds): one hipcc process per source,
    in parallel, then one link."""
    from concurrent.futures import ThreadPoolExecutor

    hipcc = hipcc_path()
    obj_dir = Path(tempfile.mkdtemp(prefix="int8kv_build_"))
    try:
        compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
        objs = [obj_dir / (Path(s).stem + ".o") for s in SOURCES]
        cmds = [[hipcc, *compile_flags, f"-I{INCLUDE_DIR}", "-c", str(CSRC_DIR / s), "-o", str(o)]
                for s, o in zip(SOURCES, objs)]
        with ThreadPoolExecutor(max_workers=len(cmds)) as pool:
            for fut in [pool.submit(_run, c, verbose) for c in cmds]:
                fut.result()
        tmp = LIB_PATH.with_suffix(".so.tmp")
        _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)],
             verbose)
        os.replace(tmp, LIB_PATH)
    finally:
        shutil.rmtree(obj_dir, ignore_errors=True)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv))
