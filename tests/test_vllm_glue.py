"""CPU checks of the vLLM integration layer (int8kv.vllm_int8, counterpart of the reference's
vllm_int8/): scale file format, page-geometry inference, the decode gate, the adapter's
quantisation, the cache pool and the patch plumbing with a fake vLLM."""

from __future__ import annotations

import json
import types
from pathlib import Path

import numpy as np
import pytest
import torch

import fake_vllm
from int8kv.vllm_int8 import cache_manager, static_scales
from int8kv.vllm_int8 import vllm_int8_attention_patch as attn_patch
from int8kv.vllm_int8 import vllm_int8_kvcache_adapter as adapter
from int8kv.vllm_int8 import vllm_shadow_cache_patch as shadow_patch

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_static_scales_file_round_trip(tmp_path):
    """The calibration file format (scripts/04_calibrate_static_scale.py:55-65) with the
    reference's own calibrated values."""
    sc = json.loads((GOLDEN / "static_per_head_scales.json").read_text())
    ks, vs = torch.tensor(sc["k_scale"]), torch.tensor(sc["v_scale"])
    path = tmp_path / "scales.pt"
    torch.save({"k_scale": ks, "v_scale": vs, "k_amax": ks * 127, "v_amax": vs * 127}, path)
    static_scales.load_static_scales(str(path))
    k, v = static_scales.get_layer_scales("model.layers.27.self_attn.attn", "cpu")
    assert k.dtype == torch.float32 and k.is_contiguous() and torch.equal(k, ks[27])
    assert torch.equal(v, vs[27])
    assert static_scales.extract_layer_idx("model.layers.13.self_attn.attn") == 13
    with pytest.raises(RuntimeError):
        static_scales.extract_layer_idx("lm_head")
    bad = tmp_path / "bad.pt"
    torch.save({"k_scale": ks}, bad)
    with pytest.raises(KeyError):
        static_scales.load_static_scales(str(bad))


def test_native_page_geometry():
    f = shadow_patch.native_page_geometry
    assert f(torch.empty(10, 4, 16, 256), 4) == (10, 16)  # v0.26 fused
    assert f(torch.empty(10, 2, 16, 4, 128), 4) == (10, 16)  # v0.16 split
    assert f(torch.empty(2, 10, 16, 4, 128), 4) == (10, 16)  # older split
    with pytest.raises(ValueError):
        f(torch.empty(10, 16, 4, 128), 4)


def _meta(B, num_tokens=None, max_query_len=1, name="block_table"):
    m = types.SimpleNamespace(seq_lens=torch.full((B,), 40, dtype=torch.int32),
                              num_actual_tokens=B if num_tokens is None else num_tokens,
                              max_query_len=max_query_len)
    setattr(m, name, torch.zeros(B, 3, dtype=torch.int32))
    return m


def test_decode_gate():
    q = torch.zeros(4, 28, 128)

    def gate(query, meta):
        return attn_patch.decode_step_of(query, meta) is not None

    assert gate(q, _meta(4))
    assert gate(q, _meta(4, name="block_tables"))  # wrapper naming
    assert not gate(q, _meta(4, num_tokens=9))  # prefill tokens
    assert not gate(q, _meta(4, max_query_len=2))  # chunked prefill
    assert not gate(q[0], _meta(4))  # not [tokens, heads, dim]
    assert not gate(q, None)
    padded = torch.zeros(8, 28, 128)  # vLLM 0.16 pads the query; num_actual_tokens decides
    assert gate(padded, _meta(4))
    step = attn_patch.decode_step_of(padded, _meta(4))
    assert step.query.shape == (4, 28, 128) and step.block_table.shape == (4, 3)
    assert step.seq_lens.is_contiguous() and step.block_table.is_contiguous()
    assert not gate(q, _meta(0))  # empty batch


def test_agreement_metrics():
    a = torch.tensor([[1.0, 2.0], [3.0, 4.0]])
    m = attn_patch.agreement(a, a)
    assert m == {"cosine": 1.0, "rel_l2": 0.0, "mae": 0.0}
    m = attn_patch.agreement(-a, a)
    assert m["cosine"] == -1.0 and m["rel_l2"] == 2.0 and m["mae"] == 5.0


def test_backend_registration_class():
    """INT8PagedAttentionBackend (vllm_int8/vllm_int8_attention_backend.py:81-87): the name and
    the implementation class a caller registers with vLLM."""
    import importlib

    with fake_vllm.installed() as mods:
        import int8kv.vllm_int8.vllm_int8_attention_backend as backend

        backend = importlib.reload(backend)
        assert issubclass(backend.INT8PagedAttentionBackend,
                          mods["vllm.v1.attention.backend"].AttentionBackend)
        assert backend.INT8PagedAttentionBackend.get_name() == "INT8_PAGED_ATTENTION"
        impl_cls = backend.INT8PagedAttentionBackend.get_impl_cls()
        assert impl_cls is backend.INT8PagedAttentionImpl
        impl = impl_cls("model.layers.3.self_attn.attn", 28, 128, 4, 128 ** -0.5)
        assert (impl.num_heads, impl.head_size, impl.num_kv_heads) == (28, 128, 4)


def test_adapter_quantize_per_head():
    x = torch.zeros(1, 2, 1, 4)
    x[0, 0, 0] = torch.tensor([127.0, 2.5, -2.5, 3.5])
    x[0, 1, 0] = torch.tensor([0.0, 0.0, 0.0, 0.0])
    q, s = adapter.quantize_per_head(x)
    assert s.tolist() == [1.0, pytest.approx(1e-6)]
    assert q[0, 0, 0].tolist() == [127, 2, -2, 4]  # torch.round: half to even
    assert (q[0, 1] == 0).all()
    g = torch.Generator().manual_seed(0)
    kv = torch.randn(6, 4, 16, 256, generator=g).to(torch.bfloat16)
    k8, v8, ks, vs = adapter.convert_vllm_fused_kv_cache_to_int8(kv)
    assert k8.shape == (6, 4, 16, 128) and ks.shape == (4,)
    err = (adapter.dequant_kv_cache(k8, ks) - kv[..., :128].float()).abs().mean()
    assert float(err) < 0.02  # tests/test_vllm_cache_quant.py:8-61 bound


def test_cache_pool():
    cache_manager.clear_cache_pool()
    c = cache_manager.allocate_layer_cache(layer_name="model.layers.0.attn", num_blocks=3,
                                           block_size=16, num_kv_heads=4, head_dim=128,
                                           k_scale=torch.ones(4), v_scale=torch.ones(4),
                                           device=torch.device("cpu"))
    assert cache_manager.has_layer_cache("model.layers.0.attn")
    assert c.key_cache.shape == (3, 16, 4, 128) and (c.key_cache == 0).all()
    assert cache_manager.int8_cache_bytes() == 2 * 3 * 16 * 4 * 128
    cache_manager.clear_cache_pool()
    assert not cache_manager.has_layer_cache("model.layers.0.attn")


def test_attention_patch_modes_and_prefill_fallback():
    with pytest.raises(ValueError):
        attn_patch.apply_int8_attention_patch(mode="fp8")
    with fake_vllm.installed():
        impl = fake_vllm.TritonAttentionImpl(28, 128, 4)
        calls = []

        def original(self, layer, query, key, value, kv_cache, attn_metadata, output, **kw):
            calls.append("vllm")
            return output

        patched = attn_patch.make_patched_forward(original, mode="int8_only")
        layer = types.SimpleNamespace(layer_name="model.layers.0.self_attn.attn")
        q = torch.zeros(9, 28, 128)
        out = torch.zeros(9, 28 * 128)
        # no shadow cache for the layer -> vLLM path
        patched(impl, layer, q, None, None, None, _meta(4, num_tokens=9), out)
        # prefill metadata -> vLLM path even with a shadow cache
        cache_manager.allocate_layer_cache(layer_name=layer.layer_name, num_blocks=2, block_size=16,
                                           num_kv_heads=4, head_dim=128, k_scale=torch.ones(4),
                                           v_scale=torch.ones(4), device=torch.device("cpu"))
        patched(impl, layer, q, None, None, None, _meta(4, num_tokens=9), out)
        assert calls == ["vllm", "vllm"]
        cache_manager.clear_cache_pool()


def test_apply_patches_with_fake_vllm():
    with fake_vllm.installed() as mods:
        cls = mods["vllm.v1.attention.backends.triton_attn"].TritonAttentionImpl
        before = (cls.do_kv_cache_update, cls.forward)
        shadow_patch._PATCHED = False
        attn_patch._PATCHED = False
        try:
            shadow_patch.apply_shadow_cache_patch()
            attn_patch.apply_int8_attention_patch(mode="int8_only")
            assert cls.do_kv_cache_update is not before[0] and cls.forward is not before[1]
            with pytest.raises(RuntimeError):
                attn_patch.apply_int8_attention_patch(mode="int8_only")
        finally:
            shadow_patch._PATCHED = False
            attn_patch._PATCHED = False
