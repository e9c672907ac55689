"""The vLLM integration layer end to end on the GPU, against a fake vLLM (tests/fake_vllm.py):
the shadow write mirrors vLLM's BF16 write into the INT8 cache (bit-exact to the oracle), and
the patched forward runs the INT8 decode in shadow / takeover / int8_only modes
(vllm_int8/vllm_shadow_cache_patch.py:58-188, vllm_int8/vllm_int8_attention_patch.py:160-321)."""

from __future__ import annotations

import types

import numpy as np
import pytest
import torch

import fake_vllm
from conftest import MAX_ABS, MIN_COS, metrics
from int8kv import synthetic as syn
from int8kv.vllm_int8 import cache_manager, static_scales
from int8kv.vllm_int8 import vllm_int8_attention_patch as attn_patch
from int8kv.vllm_int8 import vllm_shadow_cache_patch as shadow_patch
from oracle import int8kv_oracle as O

pytestmark = pytest.mark.gpu

LAYER = "model.layers.1.self_attn.attn"


@pytest.fixture()
def engine(cuda):
    """A fake vLLM layer with a 3-sequence prefill already written (native BF16 + INT8 shadow)."""
    cache_manager.clear_cache_pool()
    dist = syn.make_distribution(5)
    ks, vs = syn.calibrate_scales(dist, seed=6)
    static_scales.set_static_scales(torch.stack([ks * 2, ks]), torch.stack([vs * 2, vs]))
    g = torch.Generator().manual_seed(7)
    lens = [37, 300, 129]
    nb = 64
    bt = syn.random_block_tables([n + 1 for n in lens], nb, g, width=24)
    slots = syn.slot_mapping_for(bt, lens)
    k, v = syn.sample_kv(sum(lens), dist, g)
    native = torch.zeros(nb, 2, 16, 4, 128, dtype=torch.bfloat16, device=cuda)
    impl = fake_vllm.TritonAttentionImpl(28, 128, 4)
    layer = types.SimpleNamespace(layer_name=LAYER)
    write = shadow_patch.make_patched_do_kv_cache_update(fake_vllm.TritonAttentionImpl.do_kv_cache_update)
    write(impl, layer, k.to(cuda), v.to(cuda), native, slots.to(cuda))
    yield types.SimpleNamespace(impl=impl, layer=layer, write=write, native=native, bt=bt,
                                lens=lens, slots=slots, k=k, v=v, ks=ks, vs=vs, dist=dist, g=g,
                                nb=nb, dev=cuda)
    cache_manager.clear_cache_pool()


def test_shadow_write_is_bit_exact(engine):
    e = engine
    shadow = cache_manager.get_layer_cache(LAYER)
    assert shadow.key_cache.shape == (e.nb, 16, 4, 128)  # geometry of the native cache
    assert torch.equal(shadow.k_scale.cpu(), e.ks)  # layer 1 of the scale table
    kr = np.zeros((e.nb, 16, 4, 128), np.int8)
    vr = np.zeros_like(kr)
    O.int8_kv_cache_write(e.k.float().numpy(), e.v.float().numpy(), kr, vr, e.slots.numpy(),
                          e.ks.numpy(), e.vs.numpy())
    assert np.array_equal(shadow.key_cache.cpu().numpy(), kr)
    assert np.array_equal(shadow.value_cache.cpu().numpy(), vr)
    assert shadow_patch.WRITE_CALL_COUNT[LAYER] >= 1


def _decode_step(e, mode, query=None):
    """One decode token per sequence: write it, then run the patched forward."""
    B = len(e.lens)
    k1, v1 = syn.sample_kv(B, e.dist, e.g)
    new_slots = torch.tensor([int(e.bt[b, n // 16]) * 16 + n % 16 for b, n in enumerate(e.lens)])
    e.write(e.impl, e.layer, k1.to(e.dev), v1.to(e.dev), e.native, new_slots.to(e.dev))
    lens = [n + 1 for n in e.lens]
    meta = types.SimpleNamespace(seq_lens=torch.tensor(lens, dtype=torch.int32, device=e.dev),
                                 block_table=e.bt.to(e.dev), num_actual_tokens=B, max_query_len=1)
    q = syn.sample_query(B, e.g).to(e.dev) if query is None else query
    out = torch.zeros(B, 28, 128, dtype=torch.bfloat16, device=e.dev)
    fwd = attn_patch.make_patched_forward(fake_vllm.TritonAttentionImpl.forward, mode=mode)
    res = fwd(e.impl, e.layer, q, None, None, e.native, meta, out)
    torch.cuda.synchronize()
    shadow = cache_manager.get_layer_cache(LAYER)
    ref = O.paged_attention_ref(q.float().cpu().numpy(), shadow.key_cache.cpu().numpy(),
                                shadow.value_cache.cpu().numpy(), e.bt.numpy(), np.array(lens),
                                e.ks.numpy(), e.vs.numpy())
    return res, ref, out


def test_int8_only_decode_matches_oracle(engine):
    calls = engine.impl.forward_calls
    res, ref, out = _decode_step(engine, "int8_only")
    err, cos, _ = metrics(out.float().cpu().numpy(), ref)
    assert err <= MAX_ABS and cos >= MIN_COS
    assert engine.impl.forward_calls == calls  # vLLM's attention did not run
    assert attn_patch.ATTN_INT8_HITS[LAYER] >= 1


def test_shadow_mode_keeps_vllm_output_and_compares(engine):
    res, ref, out = _decode_step(engine, "shadow")
    m = attn_patch.ATTN_METRICS[LAYER][-1]
    assert m["cosine"] > 0.99 and m["batch"] == 3
    # the returned output is vLLM's (fake BF16), not the INT8 one
    err_int8, _, _ = metrics(out.float().cpu().numpy(), ref)
    assert err_int8 > 0  # BF16 attention differs from INT8 attention by the quantisation error


def test_takeover_mode_returns_int8(engine):
    res, ref, out = _decode_step(engine, "takeover")
    err, cos, _ = metrics(out.float().cpu().numpy(), ref)
    assert err <= MAX_ABS and cos >= MIN_COS


def test_int8_only_nan_raises(engine):
    q = torch.full((3, 28, 128), float("nan"), dtype=torch.bfloat16, device=engine.dev)
    with pytest.raises(RuntimeError, match="NaN"):
        _decode_step(engine, "int8_only", query=q)


def test_attention_backend_class(engine):
    with fake_vllm.installed():
        import importlib

        import int8kv.vllm_int8.vllm_int8_attention_backend as backend

        backend = importlib.reload(backend)
        impl = backend.INT8PagedAttentionImpl(LAYER, 28, 128, 4, 128 ** -0.5)
        e = engine
        lens = torch.tensor(e.lens, dtype=torch.int32, device=e.dev)
        meta = backend.INT8AttentionMetadata(e.bt.to(e.dev), lens)
        q = syn.sample_query(3, e.g).to(e.dev)
        out = torch.zeros(3, 28 * 128, dtype=torch.bfloat16, device=e.dev)
        impl.forward(None, q, None, None, None, meta, out)
        torch.cuda.synchronize()
        shadow = cache_manager.get_layer_cache(LAYER)
        ref = O.paged_attention_ref(q.float().cpu().numpy(), shadow.key_cache.cpu().numpy(),
                                    shadow.value_cache.cpu().numpy(), e.bt.numpy(),
                                    np.array(e.lens), e.ks.numpy(), e.vs.numpy())
        err, cos, _ = metrics(out.view(3, 28, 128).float().cpu().numpy(), ref)
        assert err <= MAX_ABS and cos >= MIN_COS
