"""CPU tests of the decode loop's host-side pieces (no HIP calls): sizes, rotary tables, norms,
prefill attention, calibration.

Each check is against mathematics that fixes the answer (closed forms, invariants, a brute-force
softmax), not against the code's own formula.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from int8kv import decode_loop as DL


def test_config4_kv_bytes():
    """Config 4: B=32, 8192 + 128 tokens -> 520 blocks per sequence; int8 7.63 GB vs bf16 15.27 GB."""
    nb = 32 * DL.blocks_per_sequence(8192 + 128)
    assert nb == 32 * 520
    i8 = DL.kv_cache_bytes(DL.QWEN25_7B, nb, "int8")
    bf = DL.kv_cache_bytes(DL.QWEN25_7B, nb, "bf16")
    assert i8["kv_bytes"] == 7_633_633_280 and bf["kv_bytes"] == 15_267_266_560
    assert i8["scale_bytes"] == 2 * 28 * 4 * 4 and bf["scale_bytes"] == 0
    with pytest.raises(ValueError):
        DL.kv_cache_bytes(DL.QWEN25_7B, nb, "fp8")


def test_qwen_shape():
    s = DL.QWEN25_7B
    assert (s.hidden, s.layers, s.q_heads, s.kv_heads, s.head_dim, s.ffn, s.vocab) == \
        (3584, 28, 28, 4, 128, 18944, 152064)
    assert s.qkv_width == 4608 and s.rope_theta == 1e6


def test_rope_tables_closed_form():
    s = DL.QWEN25_7B
    cos, sin = DL.rope_tables(s, 9000, "cpu")
    for pos, i in [(0, 0), (1, 0), (8191, 5), (8319, 63), (123, 31)]:
        ang = pos / (1e6 ** (2 * i / 128))
        assert cos[pos, i].item() == pytest.approx(math.cos(ang), abs=2e-7)
        assert sin[pos, i + 64].item() == pytest.approx(math.sin(ang), abs=2e-7)


def test_rope_invariants():
    """Identity at position 0, norm preserved, and q.k depends only on the position difference."""
    s = DL.QWEN25_7B
    cos, sin = DL.rope_tables(s, 4096, "cpu")
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, 1, 2, 128, generator=g)
    k = torch.randn(1, 1, 2, 128, generator=g)
    assert torch.allclose(DL.apply_rope(q, cos[:1], sin[:1]), q)

    def at(x, p):
        return DL.apply_rope(x, cos[p:p + 1], sin[p:p + 1])

    assert torch.allclose(at(q, 777).norm(dim=-1), q.norm(dim=-1), rtol=1e-5)
    d1 = (at(q, 100) * at(k, 40)).sum(-1)
    d2 = (at(q, 3100) * at(k, 3040)).sum(-1)
    assert torch.allclose(d1, d2, atol=2e-4)
    # Pairing: element i rotates with element i + 64 (rotate-half form), by angle pos * theta^(-2i/D).
    e = torch.zeros(1, 1, 1, 128)
    e[..., 3] = 1.0
    r = at(e, 10).reshape(-1)
    ang = 10 / (1e6 ** (6 / 128))
    assert r[3].item() == pytest.approx(math.cos(ang), abs=1e-6)
    assert r[67].item() == pytest.approx(math.sin(ang), abs=1e-6)
    assert float(r.abs().sum() - abs(r[3]) - abs(r[67])) == 0.0


def test_rms_norm_closed_form():
    x = torch.tensor([[3.0, 4.0, 0.0, 0.0]])
    w = torch.tensor([1.0, 2.0, 1.0, 1.0])
    got = DL.rms_norm(x, w, 0.0)
    rms = math.sqrt((9 + 16) / 4)
    assert torch.allclose(got, torch.tensor([[3 / rms, 8 / rms, 0.0, 0.0]]))


def test_prefill_attention_causal_gqa():
    """Causal attention with query head h reading kv head h // G, against a float64 brute force."""
    g = torch.Generator().manual_seed(1)
    c, hq, hkv, S, D = 2, 6, 2, 9, 16
    q = torch.randn(c, hq, S, D, generator=g)
    k = torch.randn(c, hkv, S, D, generator=g)
    v = torch.randn(c, hkv, S, D, generator=g)
    got = DL.prefill_attention(q, k, v).double().numpy()
    qn, kn, vn = q.double().numpy(), k.double().numpy(), v.double().numpy()
    G = hq // hkv
    for b in range(c):
        for h in range(hq):
            for t in range(S):
                s = kn[b, h // G, : t + 1] @ qn[b, h, t] / math.sqrt(D)
                p = np.exp(s - s.max())
                ref = (p / p.sum()) @ vn[b, h // G, : t + 1]
                assert np.abs(got[b, h, t] - ref).max() < 1e-5


def test_calibration_cpu_tiny_model():
    """Scales are amax/127 per (layer, kv head): quantising the calibration K hits exactly +-127."""
    shape = DL.QwenShape(hidden=64, layers=2, q_heads=4, kv_heads=2, head_dim=16, ffn=96, vocab=50)
    w = DL.random_weights(shape, "cpu", seed=3, dtype=torch.float32)
    ids = torch.randint(0, shape.vocab, (2, 12), generator=torch.Generator().manual_seed(4))
    ks, vs = DL.calibrate_static_scales(w, ids)
    assert ks.shape == (2, 2) and vs.shape == (2, 2)
    assert (ks >= 1e-6).all() and (vs >= 1e-6).all()
    # Recompute the layer-0 K and V of the calibration batch from the definitions.
    x = w.embed[ids.reshape(-1)]
    lw = w.layers[0]
    h = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + shape.rms_eps)
    qkv = h @ lw.wqkv.t() + lw.bqkv
    k = qkv[:, 4 * 16:6 * 16].reshape(2, 12, 2, 16)
    v = qkv[:, 6 * 16:].reshape(2, 12, 2, 16)
    pos = torch.arange(12, dtype=torch.float64)
    inv = 1.0 / (1e6 ** (torch.arange(8, dtype=torch.float64) * 2 / 16))
    ang = pos[:, None] * inv[None, :]
    cos = torch.cat([ang.cos(), ang.cos()], 1).float()[:, None, :]
    sin = torch.cat([ang.sin(), ang.sin()], 1).float()[:, None, :]
    k = k * cos + torch.cat([-k[..., 8:], k[..., :8]], -1) * sin
    kmax = k.abs().amax(dim=(0, 1, 3))
    vmax = v.abs().amax(dim=(0, 1, 3))
    assert torch.allclose(ks[0] * 127, kmax, rtol=1e-5)
    assert torch.allclose(vs[0] * 127, vmax, rtol=1e-5)


def test_gemm_tuning_modes_and_shipped_file():
    """The shipped TunableOp file covers exactly the decode step's five GEMM shapes at M = 32."""
    with pytest.raises(ValueError):  # rejected before torch's TunableOp (which needs a GPU)
        DL.configure_gemm_tuning("fast")
    rows = [ln.split(",") for ln in DL.GEMM_TUNING_FILE.read_text().splitlines()]
    validators = {r[1] for r in rows if r[0] == "Validator"}
    assert {"PT_VERSION", "HIPBLASLT_VERSION", "GCN_ARCH_NAME"} <= validators
    shapes = sorted(r[1] for r in rows if r[0] != "Validator")
    s = DL.QWEN25_7B
    want = sorted(f"tn_{n}_32_{k}_ld_{k}_{k}_{n}" for n, k in (
        (s.qkv_width, s.hidden), (s.hidden, s.q_heads * s.head_dim), (2 * s.ffn, s.hidden),
        (s.hidden, s.ffn), (s.vocab, s.hidden)))
    assert shapes == want
