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

# The paged decode's kernels compile per cache type in parallel (paged_decode_<type>.hip and, for
# head_dims below the kernels' 64 / 128 / 256, paged_decode_<type>_pad.hip, from
# paged_decode_kernels.h); paged_decode.hip is its host side.
SOURCES = ["cache_write.hip", "paged_decode.hip", "paged_decode_int8.hip", "paged_decode_bf16.hip",
           "paged_decode_fp16.hip", "paged_decode_int8_pad.hip", "paged_decode_bf16_pad.hip",
           "paged_decode_fp16_pad.hip", "decode_loop_ops.hip", "read_probe.hip"]
# The torch extension over the C ABI (host code only; torch headers, linked to libint8kv.so).
EXT_SOURCE = "torch_ops.cpp"
EXT_NAME = "_int8kv_torch"
EXT_PATH = PKG_DIR / f"{EXT_NAME}.so"

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


def _torch_ext_flags():
    """Compile and link flags of a host-only torch extension for this interpreter's torch."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    cflags = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-parameter",
              "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-DTORCH_EXTENSION_NAME={EXT_NAME}",
              "-DTORCH_API_INCLUDE_EXTENSION_H",
              f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
              *[f"-I{p}" for p in cpp_extension.include_paths()],
              f"-I{sysconfig.get_paths()['include']}", "-I/opt/rocm/include", f"-I{INCLUDE_DIR}"]
    lflags = [f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
              f"-L{PKG_DIR}", "-lint8kv", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"]
    return cflags, lflags


OBJ_CACHE = PKG_DIR.parent / "build"  # objects kept by incremental builds (git-ignored)

# The measurement build: the library with the units below compiled with -DINT8KV_STAMPS (per-wave
# s_memrealtime stamps in the INT8 and BF16 decode kernels and the load probe, read back through
# int8kv_stamps_read_<unit>; bench.py --stamps) and every other unit shared with the product
# build.  Never loaded by the operators.
STAMPS_LIB_PATH = PKG_DIR / "libint8kv_stamps.so"
STAMPS_SOURCES = ["paged_decode_int8.hip", "paged_decode_bf16.hip", "read_probe.hip"]


def build_library(verbose: bool = False, torch_ext: bool = True, incremental: bool = False,
                  stamps: bool = True) -> Path:
    """Compiles every HIP source into LIB_PATH and the torch extension into EXT_PATH: one
    compiler process per source, in parallel, then the links.  By default everything is rebuilt
    in a temporary directory; ``incremental`` keeps the objects in OBJ_CACHE and recompiles only
    the sources older than their object or than any header they may include (a developer's
    edit-build loop).  ``stamps``: also link the measurement build, STAMPS_LIB_PATH (its
    STAMPS_SOURCES compiled once more, in the same parallel batch)."""
    from concurrent.futures import ThreadPoolExecutor

    hipcc = hipcc_path()
    if incremental:
        obj_dir = OBJ_CACHE
        obj_dir.mkdir(parents=True, exist_ok=True)
    else:
        obj_dir = Path(tempfile.mkdtemp(prefix="int8kv_build_"))
    headers = [*CSRC_DIR.glob("*.h"), *INCLUDE_DIR.glob("*.h")]
    newest_header = max((h.stat().st_mtime for h in headers), default=0.0)

    def stale(src: Path, obj: Path) -> bool:
        if not incremental or not obj.exists():
            return True
        return obj.stat().st_mtime < max(src.stat().st_mtime, newest_header)

    try:
        compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
        objs = [obj_dir / (Path(s).stem + ".o") for s in SOURCES]
        cmds = [[hipcc, *compile_flags, f"-I{INCLUDE_DIR}", "-c", str(CSRC_DIR / s), "-o", str(o)]
                for s, o in zip(SOURCES, objs) if stale(CSRC_DIR / s, o)]
        stamp_objs = {s: obj_dir / (Path(s).stem + "_stamps.o") for s in STAMPS_SOURCES}
        if stamps:
            cmds += [[hipcc, *compile_flags, "-DINT8KV_STAMPS", f"-I{INCLUDE_DIR}", "-c",
                      str(CSRC_DIR / s), "-o", str(o)]
                     for s, o in stamp_objs.items() if stale(CSRC_DIR / s, o)]
        ext_obj = obj_dir / "torch_ops.o"
        if torch_ext:
            cflags, lflags = _torch_ext_flags()
            if stale(CSRC_DIR / EXT_SOURCE, ext_obj):
                cmds.append(["g++", *cflags, "-c", str(CSRC_DIR / EXT_SOURCE), "-o", str(ext_obj)])
        if cmds:
            with ThreadPoolExecutor(max_workers=len(cmds)) as pool:
                for fut in [pool.submit(_run, c, verbose) for c in cmds]:
                    fut.result()
        tmp = LIB_PATH.with_suffix(".so.tmp")
        _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)],
             verbose)
        os.replace(tmp, LIB_PATH)
        if stamps:
            mixed = [stamp_objs.get(s, o) for s, o in zip(SOURCES, objs)]
            tmp = STAMPS_LIB_PATH.with_suffix(".so.tmp")
            _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, mixed), "-o",
                  str(tmp)], verbose)
            os.replace(tmp, STAMPS_LIB_PATH)
        if torch_ext:
            tmp = EXT_PATH.with_suffix(".so.tmp")
            _run(["g++", "-shared", str(ext_obj), *lflags, "-o", str(tmp)], verbose)
            os.replace(tmp, EXT_PATH)
    finally:
        if not incremental:
            shutil.rmtree(obj_dir, ignore_errors=True)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv, incremental="--incremental" in sys.argv,
                        stamps="--no-stamps" not in sys.argv))
