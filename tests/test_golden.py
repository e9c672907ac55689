"""The CPU oracle against the golden fixtures of tests/golden/ (made by make_golden.py).

The fixtures hold the reference's own data (real Qwen2.5-7B K/V samples and the calibrated
static per-head scales from its outputs/ directory) with expected results computed from the
definitions by exact rational / float64 arithmetic, independently of the oracle's code paths.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import int8kv_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"
LAYERS = (0, 27)


@pytest.fixture(scope="module")
def golden():
    data = dict(np.load(GOLDEN / "qwen_kv_sample_golden.npz"))
    sc = json.loads((GOLDEN / "static_per_head_scales.json").read_text())
    data["k_scale"] = np.asarray(sc["k_scale"], np.float32)
    data["v_scale"] = np.asarray(sc["v_scale"], np.float32)
    return data


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint16).astype(np.uint32) << 16).view(np.float32)


def paged_from_dense(kq: np.ndarray, vq: np.ndarray, seed: int = 0, block_size: int = 16):
    """int8 [B, Hkv, T, D] -> shuffled paged caches + tables (one block per 16 tokens)."""
    B, hkv, T, d = kq.shape
    n = (T + block_size - 1) // block_size
    rng = np.random.default_rng(seed)
    nb = B * n + 3
    perm = rng.permutation(nb)
    kc = rng.integers(-128, 128, (nb, block_size, hkv, d)).astype(np.int8)
    vc = rng.integers(-128, 128, (nb, block_size, hkv, d)).astype(np.int8)
    bt = np.zeros((B, n), np.int32)
    for b in range(B):
        for lb in range(n):
            p = perm[b * n + lb]
            bt[b, lb] = p
            s, e = lb * block_size, min(T, (lb + 1) * block_size)
            kc[p, : e - s] = kq[b, :, s:e].transpose(1, 0, 2)
            vc[p, : e - s] = vq[b, :, s:e].transpose(1, 0, 2)
    return kc, vc, bt, np.full(B, T, np.int32)


def test_scales_fixture(golden):
    assert golden["k_scale"].shape == (28, 4) and golden["v_scale"].shape == (28, 4)
    assert (golden["k_scale"] > 0).all() and (golden["v_scale"] > 0).all()


@pytest.mark.parametrize("layer", LAYERS)
def test_oracle_quant_matches_golden_codes(golden, layer):
    k = golden[f"l{layer}_k"].astype(np.float32)  # [4, 4, 10, 128]
    v = golden[f"l{layer}_v"].astype(np.float32)
    ks, vs = golden["k_scale"][layer], golden["v_scale"][layer]
    kq = O.quant_kv_static_per_head(k, ks[None, :, None, None])
    vq = O.quant_kv_static_per_head(v, vs[None, :, None, None])
    assert np.array_equal(kq, golden[f"l{layer}_kq"])
    assert np.array_equal(vq, golden[f"l{layer}_vq"])
    # the fixture exercises clamping (values beyond the calibrated absmax)
    assert (np.abs(golden[f"l{layer}_kq"]) == 127).any()


@pytest.mark.parametrize("layer", LAYERS)
def test_oracle_write_matches_golden_codes(golden, layer):
    k = golden[f"l{layer}_k"].astype(np.float32)  # [B, Hkv, T, D]
    v = golden[f"l{layer}_v"].astype(np.float32)
    B, hkv, T, d = k.shape
    kq, vq = golden[f"l{layer}_kq"], golden[f"l{layer}_vq"]
    kc_ref, vc_ref, bt, sl = paged_from_dense(kq, vq, seed=layer)
    kc = np.full_like(kc_ref, 0x5A)
    vc = np.full_like(vc_ref, 0x5A)
    slots = np.concatenate([bt[b, np.arange(T) // 16].astype(np.int64) * 16 + np.arange(T) % 16
                            for b in range(B)])
    key = k.transpose(0, 2, 1, 3).reshape(B * T, hkv, d)
    val = v.transpose(0, 2, 1, 3).reshape(B * T, hkv, d)
    O.int8_kv_cache_write(key, val, kc, vc, slots, golden["k_scale"][layer], golden["v_scale"][layer])
    written = np.zeros(kc.shape[:2], bool)
    written.reshape(-1)[slots] = True
    assert np.array_equal(kc[written], kc_ref[written]) and np.array_equal(vc[written], vc_ref[written])
    assert (kc[~written] == 0x5A).all()


@pytest.mark.parametrize("layer", LAYERS)
def test_oracle_attention_matches_golden(golden, layer):
    out = golden[f"l{layer}_out"]  # [2, 28, 128]
    rows = out.shape[0]
    q = bf16_bits_to_f32(golden[f"l{layer}_q_bf16_bits"])
    kc, vc, bt, sl = paged_from_dense(golden[f"l{layer}_kq"][:rows], golden[f"l{layer}_vq"][:rows],
                                      seed=10 + layer)
    got = O.paged_attention_ref(q, kc, vc, bt, sl, golden["k_scale"][layer], golden["v_scale"][layer])
    # fp32 oracle vs float64 definition: scores reach ~100 on layer 27 (k_scale up to 3.3)
    np.testing.assert_allclose(got, out, rtol=1e-4, atol=1e-4)


def test_dequantize_paged_cache_known_answer():
    c = np.array([[[[1, -2], [127, -127]]]], np.int8)  # [1, 1, 2, 2]
    out = O.dequantize_paged_cache(c, np.array([0.5, 0.25], np.float32))
    assert out.dtype == np.float32
    assert out.tolist() == [[[[0.5, -1.0], [31.75, -31.75]]]]
