"""Reference module paths for unmodified callers.

The reference's callers import the operators from ``src.triton_ops.*``
(vllm_int8/vllm_shadow_cache_patch.py:5, vllm_int8/vllm_int8_cache_ops.py:281,
vllm_int8/vllm_int8_attention_patch.py:8-10, vllm_int8/vllm_int8_attention_backend.py:10-12).
``install_reference_aliases()`` registers this package's modules under those names in
``sys.modules`` so those imports bind to the HIP operators without editing the callers.  Only the
operator modules are aliased; the reference's pure-torch checking helpers are not provided.
"""

from __future__ import annotations

import importlib
import importlib.util
import sys
import types

ALIASES = {
    "src.triton_ops.int8_cache_write": "int8kv.int8_cache_write",
    "src.triton_ops.int8_paged_attention": "int8kv.int8_paged_attention",
    "src.triton_ops.bf16_paged_attention": "int8kv.bf16_paged_attention",
}


def _ensure_package(name: str) -> None:
    if name in sys.modules:
        return
    try:
        spec = importlib.util.find_spec(name)
    except (ImportError, ValueError):
        spec = None
    if spec is not None:
        importlib.import_module(name)  # a real (namespace) package of that name exists
        return
    mod = types.ModuleType(name)
    mod.__path__ = []  # a package with no files: only the aliased submodules resolve
    sys.modules[name] = mod


def install_reference_aliases() -> list:
    """Makes ``import src.triton_ops.<op>`` resolve to this package; returns the aliased names."""
    done = []
    for alias, target in ALIASES.items():
        parent = alias.rsplit(".", 1)[0]
        _ensure_package(parent.split(".")[0])
        _ensure_package(parent)
        mod = importlib.import_module(target)
        sys.modules[alias] = mod
        setattr(sys.modules[parent], alias.rsplit(".", 1)[1], mod)
        done.append(alias)
    return done
