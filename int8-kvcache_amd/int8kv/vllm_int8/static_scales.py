"""Static per-(layer, kv-head) scales (vllm_int8/static_scales.py of the reference).

The scale file is the calibration output of scripts/04_calibrate_static_scale.py:55-65:
``{"k_scale": [L, Hkv], "v_scale": [L, Hkv], ...}`` float32.  It is loaded as data only
(``torch.load(..., weights_only=True)``).
"""

from __future__ import annotations

import re

import torch

_SCALE_DATA = None
_LAYER_INDEX = re.compile(r"layers\.(\d+)")


def load_static_scales(path: str):
    """Loads the scale file as data and makes it the process's scale source
    (vllm_int8/static_scales.py:9-28).  KeyError when a scale is absent, ValueError when one is
    not a [layers, kv heads] table."""
    global _SCALE_DATA
    data = torch.load(path, map_location="cpu", weights_only=True)
    for key in ("k_scale", "v_scale"):
        if key not in data:
            raise KeyError(f"scale file {path} holds no {key!r} table")
        if data[key].ndim != 2:
            raise ValueError(f"scale file {path}: {key!r} has shape {tuple(data[key].shape)}, "
                             f"expected [layers, kv heads]")
    _SCALE_DATA = data
    print(f"[int8kv] static scales from {path}: k {tuple(data['k_scale'].shape)}, "
          f"v {tuple(data['v_scale'].shape)}")
    return data


def set_static_scales(k_scale: torch.Tensor, v_scale: torch.Tensor):
    """Installs [L, Hkv] scales directly (without a file)."""
    global _SCALE_DATA
    _SCALE_DATA = {"k_scale": k_scale.detach().float().cpu(), "v_scale": v_scale.detach().float().cpu()}
    return _SCALE_DATA


def extract_layer_idx(layer_name: str) -> int:
    """'model.layers.0.self_attn.attn' -> 0 (vllm_int8/static_scales.py:31-47)."""
    match = _LAYER_INDEX.search(layer_name)
    if match is None:
        raise RuntimeError(f"layer name {layer_name!r} has no 'layers.<index>' part to pick its "
                           f"scales by")
    return int(match.group(1))


def get_layer_scales(layer_name: str, device):
    """(k_scale, v_scale) of the layer as contiguous float32 [Hkv] on ``device`` (:50-75)."""
    if _SCALE_DATA is None:
        raise RuntimeError("no static scales installed: load_static_scales(path) or "
                           "set_static_scales(k, v) must run before the first INT8 cache write")
    idx = extract_layer_idx(layer_name)
    k_scale = _SCALE_DATA["k_scale"][idx].to(device=device, dtype=torch.float32).contiguous()
    v_scale = _SCALE_DATA["v_scale"][idx].to(device=device, dtype=torch.float32).contiguous()
    return k_scale, v_scale
