"""Reference module paths for unmodified callers.

The reference's callers import the operators from ``src.triton_ops.*``
(vllm_int8/vllm_shadow_cache_patch.py:5, vllm_int8/vllm_int8_cache_ops.py:281,
vllm_int8/vllm_int8_attention_patch.py:8-10, vllm_int8/vllm_int8_attention_backend.py:10-12).
``install_reference_aliases()`` registers this package's modules under those names in
``sys.modules`` so those imports bind to the HIP operators without editing the callers.  The
aliased operator modules also export the reference's two pure-torch checkers under their names
(``torch_int8_kv_cache_write_reference`` and ``torch_int8_paged_attention_reference``, from
``int8kv.torch_reference``), for callers' own tests; no operator calls them.
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

# The integration layer itself, for callers that import the reference's vllm_int8 modules.
VLLM_INT8_ALIASES = {
    f"vllm_int8.{m}": f"int8kv.vllm_int8.{m}"
    for m in ("cache_manager", "static_scales", "vllm_int8_kvcache_adapter",
              "vllm_int8_cache_ops", "vllm_shadow_cache_patch", "vllm_int8_attention_patch")
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


def install_reference_aliases(include_vllm_int8: bool = False) -> list:
    """Makes ``import src.triton_ops.<op>`` (and, with ``include_vllm_int8``, the reference's
    ``vllm_int8.<module>`` imports) resolve to this package; returns the aliased names."""
    done = []
    table = dict(ALIASES)
    if include_vllm_int8:
        table.update(VLLM_INT8_ALIASES)
    for alias, target in table.items():
        parent = alias.rsplit(".", 1)[0]
        _ensure_package(parent.split(".")[0])
        _ensure_package(parent)
        mod = importlib.import_module(target)
        sys.modules[alias] = mod
        setattr(sys.modules[parent], alias.rsplit(".", 1)[1], mod)
        done.append(alias)
    return done
