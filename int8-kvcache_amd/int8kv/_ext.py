"""The torch extension over libint8kv.so's C ABI (``_int8kv_torch``, built from
csrc/torch_ops.cpp): one pybind11 call per operator, with the reference's argument checks, the
output/workspace allocation and the current stream handled in C++.

``module()`` returns it once built (None when it is absent: the operators then reach the same C
ABI through ctypes).  A present but unloadable extension raises.  ``INT8KV_CTYPES=1`` in the
environment, or ``use_ctypes()`` in a ``with`` block, selects the ctypes path instead (both call
the same kernels; the tests compare them).
"""

from __future__ import annotations

import os
from contextlib import contextmanager
from pathlib import Path

from . import _lib

EXT_PATH = Path(__file__).resolve().parent / "_int8kv_torch.so"

_module = None
_loaded = False
_forced_off = os.environ.get("INT8KV_CTYPES", "0") not in ("", "0")


def _load():
    global _module, _loaded
    _loaded = True
    if EXT_PATH.exists():
        from . import _int8kv_torch as m

        m.set_library_error(_lib.Int8KVError)
        _module = m
    return _module


def module():
    """The extension module, or None (not built, or the ctypes path selected)."""
    if _forced_off:
        return None
    return _module if _loaded else _load()


@contextmanager
def use_ctypes():
    """Routes the operators through the ctypes binding inside the block."""
    global _forced_off
    before = _forced_off
    _forced_off = True
    try:
        yield
    finally:
        _forced_off = before
