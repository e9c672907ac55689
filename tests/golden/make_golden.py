"""Writes the golden fixtures of tests/golden/ (run once, in a container holding the reference).

Inputs come from the reference's own data files, loaded as data only
(``torch.load(..., weights_only=True)``; nothing from the reference is imported or executed):

  * outputs/static_per_head_scales.pt  -- calibrated static scales, k_scale / v_scale [28, 4] fp32
    (written by scripts/04_calibrate_static_scale.py:55-65 of the reference);
  * outputs/kv_sample.pt               -- real Qwen2.5-7B K/V, {layer: {k, v}} [4, 4, 10, 128] fp16
    for layers 0, 7, 14, 21, 27 (scripts/01_collect_kv.py:53-59).

Expected outputs are computed here from the definitions, independently of the oracle's numpy
code paths:

  * int8 codes: q = clamp(rne(fl32(x / s)), -127, 127), with the fp32 quotient fl32(x / s)
    rounded exactly from the rational x / s (fractions.Fraction), i.e. IEEE division, and both
    roundings half-to-even (src/quant.py:37-40: torch.round of an fp32 quotient);
  * attention: out[b, h] = sum_t softmax_t(<q, k_t> / sqrt(128)) v_t over the dequantised codes
    (k_t = code * k_scale, fp32 products as the reference's dequantisation, then exact
    float64 sums with math.fsum), for a seeded bf16 query (stored as its bf16 bit patterns) on
    the first two sequences of each layer sample; GQA head h reads kv head h // 7; stored as
    float32.

Usage: python tests/golden/make_golden.py [/root/reference]
"""

from __future__ import annotations

import json
import math
import sys
from fractions import Fraction
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LAYERS = (0, 27)
ATTN_ROWS = 2  # attention golden on the first two sequences of each layer sample


def fp32_round(q: Fraction) -> Fraction:
    """The fp32 value nearest to the rational q (ties to even), as an exact Fraction."""
    if q == 0:
        return Fraction(0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    # fix e so that 2^e <= a < 2^(e+1)
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)  # subnormals share the exponent of the smallest normal
    ulp = Fraction(2) ** (e - 23)
    m = a / ulp
    lo = math.floor(m)
    r = m - lo
    n = lo + 1 if (r > Fraction(1, 2) or (r == Fraction(1, 2) and lo % 2 == 1)) else lo
    return sign * n * ulp


def rne_int(x: Fraction) -> int:
    lo = math.floor(x)
    r = x - lo
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and lo % 2 == 1):
        return lo + 1
    return lo


def quantize_exact(x: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """x [..., H, T, D] (exact fp16/fp32 values), scale [H] fp32 -> int8 codes."""
    out = np.empty(x.shape, np.int8)
    it = np.nditer(x, flags=["multi_index"])
    cache = {}
    for v in it:
        h = it.multi_index[-3]
        key = (float(v), h)
        if key not in cache:
            s = Fraction(float(np.float32(max(float(scale[h]), float(np.float32(1e-6))))))
            qf = fp32_round(Fraction(float(v)) / s)
            cache[key] = max(-127, min(127, rne_int(qf)))
        out[it.multi_index] = cache[key]
    return out


def attention_exact(q: np.ndarray, kq: np.ndarray, vq: np.ndarray, ks: np.ndarray, vs: np.ndarray):
    """q [B, 28, D] fp32 values; kq/vq int8 [B, 4, T, D]; -> float64 [B, 28, D]."""
    B, hq, d = q.shape
    hkv, T = kq.shape[1], kq.shape[2]
    g = hq // hkv
    out = np.zeros((B, hq, d))
    for b in range(B):
        for h in range(hq):
            kvh = h // g
            k = (kq[b, kvh].astype(np.float32) * np.float32(ks[kvh])).astype(np.float64)
            v = (vq[b, kvh].astype(np.float32) * np.float32(vs[kvh])).astype(np.float64)
            s = [math.fsum(float(q[b, h, i]) * k[t, i] for i in range(d)) / math.sqrt(d) for t in range(T)]
            m = max(s)
            w = [math.exp(x - m) for x in s]
            z = math.fsum(w)
            for i in range(d):
                out[b, h, i] = math.fsum(w[t] * v[t, i] for t in range(T)) / z
    return out


def main() -> None:
    import torch

    ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    scales = torch.load(ref / "outputs" / "static_per_head_scales.pt", weights_only=True)
    kv = torch.load(ref / "outputs" / "kv_sample.pt", weights_only=True)
    ks_all = scales["k_scale"].float().numpy()
    vs_all = scales["v_scale"].float().numpy()
    json.dump({"k_scale": ks_all.tolist(), "v_scale": vs_all.tolist(),
               "source": "outputs/static_per_head_scales.pt of cjsmt/Int8-kvcache"},
              open(HERE / "static_per_head_scales.json", "w"))

    g = torch.Generator().manual_seed(2024)
    arrays = {}
    for layer in LAYERS:
        k = kv[layer]["k"].numpy()  # [4, 4, 10, 128] fp16
        v = kv[layer]["v"].numpy()
        ks, vs = ks_all[layer], vs_all[layer]
        kq = quantize_exact(k.astype(np.float32), ks)
        vq = quantize_exact(v.astype(np.float32), vs)
        qb = torch.randn(ATTN_ROWS, 28, 128, generator=g).to(torch.bfloat16)
        q = qb.float().numpy()
        out = attention_exact(q, kq[:ATTN_ROWS], vq[:ATTN_ROWS], ks, vs)
        arrays[f"l{layer}_k"] = k
        arrays[f"l{layer}_v"] = v
        arrays[f"l{layer}_kq"] = kq
        arrays[f"l{layer}_vq"] = vq
        arrays[f"l{layer}_q_bf16_bits"] = qb.view(torch.int16).numpy()
        arrays[f"l{layer}_out"] = out.astype(np.float32)
        print(f"layer {layer}: K codes clamp {int((np.abs(kq) == 127).sum())}, "
              f"V codes clamp {int((np.abs(vq) == 127).sum())}", flush=True)
    np.savez_compressed(HERE / "qwen_kv_sample_golden.npz", **arrays)


if __name__ == "__main__":
    main()
