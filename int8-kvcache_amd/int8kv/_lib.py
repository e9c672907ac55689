"""ctypes binding of libint8kv.so (the C ABI declared in include/int8kv.h and
include/int8kv_decode_loop.h).

The library is required: if it is missing every operator raises instead of computing anything
elsewhere.  Torch is used only to read tensor metadata (pointers, strides, the current stream).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libint8kv.so"

# enum int8kv_dtype
F32, F16, BF16, I8, I32, I64 = 0, 1, 2, 3, 4, 5
DTYPE_CODE = {
    torch.float32: F32,
    torch.float16: F16,
    torch.bfloat16: BF16,
    torch.int8: I8,
    torch.int32: I32,
    torch.int64: I64,
}

DECODE_MAIN, DECODE_MERGE, DECODE_ALL, DECODE_QUANTIZE_Q = 1, 2, 3, 4
DECODE_PER_SEQUENCE = 8
DECODE_SPLIT_SEQUENCES = 16

# int8kv_decode_plan_t.layout / .merge
LAYOUT_RANGES, LAYOUT_PER_SEQUENCE, LAYOUT_SPLIT = 0, 1, 2
LAYOUT_NAMES = {LAYOUT_RANGES: "ranges", LAYOUT_PER_SEQUENCE: "per_sequence", LAYOUT_SPLIT: "split"}
MERGE_NAMES = {0: "none", 1: "by_sequence", 2: "by_range", 3: "split"}


class DecodePlan(ctypes.Structure):
    """int8kv_decode_plan_t (include/int8kv.h)."""

    _fields_ = [(name, ctypes.c_int32) for name in (
        "layout", "kernels", "num_ranges", "min_tiles", "seq_cost", "ranges_per_workgroup", "depth",
        "kv_pair", "split", "non_temporal", "merge", "merge_waves", "merge_fold", "compute_units")
    ] + [("workspace_bytes", ctypes.c_uint64)]

    def as_dict(self) -> dict:
        d = {name: getattr(self, name) for name, _ in self._fields_}
        d["layout"] = LAYOUT_NAMES[self.layout]
        d["merge"] = MERGE_NAMES[self.merge]
        return d

ERRORS = {
    -1: "INT8KV_E_NULL (a required pointer is NULL)",
    -2: "INT8KV_E_DTYPE (unsupported element type)",
    -3: "INT8KV_E_SHAPE (unsupported or inconsistent size)",
    -4: "INT8KV_E_STRIDE (innermost stride != 1 or rows not 16-byte aligned)",
    -5: "INT8KV_E_WORKSPACE (workspace missing or too small)",
    -6: "INT8KV_E_SCRATCH (the call's split partials exceed the library's fixed scratch array)",
}

_c_i64p = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p
_lib = None


class Int8KVError(RuntimeError):
    """A non-zero status returned by libint8kv.so."""


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    _lib = bind(LIB_PATH)
    return _lib


def bind(path: Path) -> ctypes.CDLL:
    """Loads a build of the library (libint8kv.so, or the measurement build) and declares the
    C ABI's argument types on it."""
    if not path.exists():
        raise RuntimeError(
            f"{path} is not built; run `python -m int8kv._build` or "
            "__graft_entry__.build() first (there is no non-HIP implementation)"
        )
    lib = ctypes.CDLL(str(path))
    i32, i64, u32, f32, sz = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32, ctypes.c_float, ctypes.c_size_t
    lib.int8kv_cache_write.restype = ctypes.c_int
    lib.int8kv_cache_write.argtypes = [
        _vp, _vp, ctypes.c_int, i64, i32, i32, _c_i64p, _c_i64p, _vp, _vp, i64, i32,
        _c_i64p, _c_i64p, _vp, ctypes.c_int, _vp, _vp, _vp,
    ]
    lib.int8kv_dynamic_cache_write.restype = ctypes.c_int
    lib.int8kv_dynamic_cache_write.argtypes = [
        _vp, _vp, ctypes.c_int, i64, i32, i32, _c_i64p, _c_i64p, _vp, _vp, i64, i32,
        _c_i64p, _c_i64p, _vp, _vp, _c_i64p, _c_i64p, _vp, ctypes.c_int, _vp,
    ]
    lib.int8kv_decode_workspace_bytes.restype = sz
    lib.int8kv_decode_workspace_bytes.argtypes = [i32, i32, i32, i32, i32]
    lib.int8kv_decode_auto_ranges.restype = i32
    lib.int8kv_decode_auto_ranges.argtypes = [i32]
    lib.int8kv_decode_plan.restype = ctypes.c_int
    lib.int8kv_decode_plan.argtypes = [
        ctypes.c_int, ctypes.c_int, i64, i32, i32, i32, i64, i32, i64, i64, i64, i32, i32, u32, i32,
        i32, ctypes.POINTER(DecodePlan),
    ]
    lib.int8kv_paged_decode.restype = ctypes.c_int
    lib.int8kv_paged_decode.argtypes = [
        _vp, ctypes.c_int, i64, i32, i32, _c_i64p, _vp, _vp, ctypes.c_int, i64, i32, i32,
        _c_i64p, _c_i64p, _vp, ctypes.c_int, i64, _c_i64p, _vp, ctypes.c_int, _vp, _vp, f32,
        _vp, _c_i64p, _vp, sz, i32, i32, u32, _vp,
    ]
    lib.int8kv_paged_decode_noalloc.restype = ctypes.c_int
    lib.int8kv_paged_decode_noalloc.argtypes = [
        _vp, ctypes.c_int, i64, i32, i32, _c_i64p, _vp, _vp, ctypes.c_int, i64, i32, i32,
        _c_i64p, _c_i64p, _vp, ctypes.c_int, i64, _c_i64p, _vp, ctypes.c_int, _vp, _vp, f32,
        _vp, _c_i64p, i32, i32, u32, _vp,
    ]
    lib.int8kv_add_rms_norm.restype = ctypes.c_int
    lib.int8kv_add_rms_norm.argtypes = [_vp, _vp, _vp, _vp, i64, i32, i64, i64, i64, f32, _vp]
    lib.int8kv_rotary_inplace.restype = ctypes.c_int
    lib.int8kv_rotary_inplace.argtypes = [_vp, i64, i64, i32, i32, _vp, _vp, _vp, i64, _vp]
    lib.int8kv_silu_mul.restype = ctypes.c_int
    lib.int8kv_silu_mul.argtypes = [_vp, _vp, i64, i32, i64, i64, _vp]
    lib.int8kv_rotary_cache_write.restype = ctypes.c_int
    lib.int8kv_rotary_cache_write.argtypes = [
        _vp, i64, i64, i32, i32, i32, _vp, _vp, _vp, i64, _vp, i64, i64, i64, i32, ctypes.c_int,
        _vp, _vp, _c_i64p, _c_i64p, _vp, _vp, _vp,
    ]
    lib.int8kv_argmax_rows.restype = ctypes.c_int
    lib.int8kv_argmax_rows.argtypes = [_vp, i64, i64, i64, _vp, _vp]
    lib.int8kv_version.restype = ctypes.c_char_p
    lib.int8kv_version.argtypes = []
    # include/int8kv_probe.h (measurement only: bench.py --ceiling and --cold)
    lib.int8kv_probe_stream_read.restype = ctypes.c_int
    lib.int8kv_probe_stream_read.argtypes = [_vp, sz, i32, _vp, i32, _vp]
    lib.int8kv_probe_clock.restype = ctypes.c_int
    lib.int8kv_probe_clock.argtypes = [_vp, i32, ctypes.c_uint32, _vp]
    lib.int8kv_probe_decode_loads.restype = ctypes.c_int
    lib.int8kv_probe_decode_loads.argtypes = [_vp, _vp, i64, i32, _vp, i64, i32, i32, i32, _vp, i64,
                                              _vp]
    if hasattr(lib, "int8kv_stamps_read_i8"):  # the measurement build
        for unit in ("i8", "bf16", "probe"):
            getattr(lib, f"int8kv_stamps_read_{unit}").restype = ctypes.c_int
            getattr(lib, f"int8kv_stamps_read_{unit}").argtypes = [_vp, sz]
            getattr(lib, f"int8kv_stamps_clear_{unit}").restype = ctypes.c_int
            getattr(lib, f"int8kv_stamps_clear_{unit}").argtypes = []
    return lib


def decode_plan(query_dtype, cache_dtype, batch: int, num_q_heads: int, num_kv_heads: int,
                head_dim: int, num_blocks: int, block_size: int, table_width: int,
                key_head_stride: int | None = None, value_head_stride: int | None = None,
                num_ranges: int = 0, min_tiles: int = 0, flags: int = DECODE_ALL,
                compute_units: int = 0, no_alloc: bool = False) -> dict:
    """What int8kv_paged_decode (or, with ``no_alloc``, int8kv_paged_decode_noalloc) does for
    these sizes: layout, range count, tiles in flight, merge kernel... (int8kv_decode_plan).
    Dtypes are torch dtypes or dtype codes; the head strides default to head_dim (contiguous
    caches); ``compute_units`` 0 means the current device.  Pure host computation: no kernel is
    launched and no device memory is read."""
    lib = load()
    qd = DTYPE_CODE.get(query_dtype, query_dtype)
    cd = DTYPE_CODE.get(cache_dtype, cache_dtype)
    ks = head_dim if key_head_stride is None else key_head_stride
    vs = head_dim if value_head_stride is None else value_head_stride
    plan = DecodePlan()
    st = lib.int8kv_decode_plan(qd, cd, batch, num_q_heads, num_kv_heads, head_dim, num_blocks,
                                block_size, table_width, ks, vs, num_ranges, min_tiles, flags,
                                compute_units, int(bool(no_alloc)), ctypes.byref(plan))
    check(st, "int8kv_decode_plan")
    return plan.as_dict()


_STRIDE_ARRAYS: dict = {}


def strides(t: torch.Tensor):
    """The tensor's strides as a ctypes int64 array (cached per stride tuple; the library only
    reads them during the call)."""
    st = t.stride()
    arr = _STRIDE_ARRAYS.get(st)
    if arr is None:
        if len(_STRIDE_ARRAYS) > 4096:
            _STRIDE_ARRAYS.clear()
        arr = _STRIDE_ARRAYS[st] = (ctypes.c_int64 * len(st))(*st)
    return arr


def aligned_rows(t: torch.Tensor) -> torch.Tensor:
    """A contiguous copy of ``t`` at a fresh (16-byte aligned) address: for inputs whose rows
    the kernels could not read with 16-byte loads.  ``contiguous()`` alone keeps a misaligned
    storage offset of an already contiguous view."""
    return t.clone(memory_format=torch.contiguous_format)


def check(status: int, what: str) -> None:
    if status != 0:
        msg = ERRORS.get(status, f"hipError_t {status}")
        raise Int8KVError(f"{what} failed: {msg}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on ``device`` (the raw handle, read without building
    a torch Stream object)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return _raw_stream(idx)
    return torch.cuda.current_stream(idx).cuda_stream
