"""GPU kernels against the golden fixtures (real Qwen2.5-7B K/V samples and calibrated scales
from the reference's outputs/, expected results from exact arithmetic; see golden/make_golden.py).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import int8kv
from conftest import MAX_ABS, MIN_COS, metrics
from test_golden import LAYERS, bf16_bits_to_f32, golden, paged_from_dense  # noqa: F401

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("layer", LAYERS)
def test_write_kernel_matches_golden_codes(cuda, golden, layer):  # noqa: F811
    k = torch.from_numpy(golden[f"l{layer}_k"])  # fp16 [B, Hkv, T, D]
    v = torch.from_numpy(golden[f"l{layer}_v"])
    B, hkv, T, d = k.shape
    kc_ref, vc_ref, bt, _ = paged_from_dense(golden[f"l{layer}_kq"], golden[f"l{layer}_vq"], seed=layer)
    slots = np.concatenate([bt[b, np.arange(T) // 16].astype(np.int64) * 16 + np.arange(T) % 16
                            for b in range(B)])
    key = k.permute(0, 2, 1, 3).reshape(B * T, hkv, d).contiguous()
    val = v.permute(0, 2, 1, 3).reshape(B * T, hkv, d).contiguous()
    kc = torch.full(kc_ref.shape, 0x5A, dtype=torch.int8, device=cuda)
    vc = torch.full_like(kc, 0x5A)
    ks = torch.from_numpy(golden["k_scale"][layer].copy()).to(cuda)
    vs = torch.from_numpy(golden["v_scale"][layer].copy()).to(cuda)
    int8kv.int8_kv_cache_write(key.to(cuda), val.to(cuda), kc, vc, torch.from_numpy(slots).to(cuda), ks, vs)
    torch.cuda.synchronize()
    kg, vg = kc.cpu().numpy(), vc.cpu().numpy()
    written = np.zeros(kg.shape[:2], bool)
    written.reshape(-1)[slots] = True
    assert np.array_equal(kg[written], kc_ref[written]), "K codes differ from the golden codes"
    assert np.array_equal(vg[written], vc_ref[written]), "V codes differ from the golden codes"
    assert (kg[~written] == 0x5A).all() and (vg[~written] == 0x5A).all()


@pytest.mark.parametrize("layer", LAYERS)
@pytest.mark.parametrize("num_splits", [None, 1, 3])
@pytest.mark.parametrize("qdtype", [torch.float32, torch.bfloat16])
def test_decode_kernel_matches_golden(cuda, golden, layer, num_splits, qdtype):  # noqa: F811
    """The output has the query's dtype.  With an fp32 query (the bf16 values widened exactly) the
    bar is the north-star one; a bf16 output adds its own rounding (up to 2^-8 of |out|; layer 27's
    outputs reach 49, where a bf16 ulp is 0.25)."""
    out_ref = golden[f"l{layer}_out"]
    rows = out_ref.shape[0]
    q = torch.from_numpy(golden[f"l{layer}_q_bf16_bits"]).view(torch.bfloat16).to(qdtype)
    kc, vc, bt, sl = paged_from_dense(golden[f"l{layer}_kq"][:rows], golden[f"l{layer}_vq"][:rows],
                                      seed=10 + layer)
    ks = torch.from_numpy(golden["k_scale"][layer].copy()).to(cuda)
    vs = torch.from_numpy(golden["v_scale"][layer].copy()).to(cuda)
    out = int8kv.int8_paged_attention(q.to(cuda), torch.from_numpy(kc).to(cuda), torch.from_numpy(vc).to(cuda),
                                      torch.from_numpy(bt).to(cuda), torch.from_numpy(sl).to(cuda), ks, vs,
                                      num_splits=num_splits)
    torch.cuda.synchronize()
    assert out.dtype == qdtype
    got = out.float().cpu().numpy()
    err, cos, _ = metrics(got, out_ref)
    print(f"layer {layer} splits={num_splits} {qdtype}: max|diff|={err:.3e} cos={cos:.7f}", flush=True)
    assert cos >= MIN_COS
    if qdtype == torch.float32:
        assert err <= MAX_ABS
    else:
        excess = np.abs(got - out_ref) - (MAX_ABS + np.abs(out_ref) * 2.0 ** -8)
        assert excess.max() <= 0, f"beyond 2e-2 + bf16 rounding by {excess.max():.3e}"
