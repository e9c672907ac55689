"""CPU tests of the reference's torch checking helpers (int8kv.torch_reference) against the oracle.

The helpers are restatements the reference's own tests import from the operator modules
(src/triton_ops/int8_cache_write.py:150-181, src/triton_ops/int8_paged_attention.py:776-814);
here they are held to the numpy oracle on the same inputs, and to the names the drop-in modules
must export.
"""

from __future__ import annotations

import numpy as np
import torch

from cases import decode_case
from conftest import metrics
from oracle import int8kv_oracle as O


def test_checkers_exported_from_operator_modules():
    """Importable under the reference's module paths once the aliases are installed."""
    import importlib

    from int8kv import torch_reference
    from int8kv.compat import install_reference_aliases

    install_reference_aliases()
    w = importlib.import_module("src.triton_ops.int8_cache_write")
    a = importlib.import_module("src.triton_ops.int8_paged_attention")
    assert w.torch_int8_kv_cache_write_reference is torch_reference.torch_int8_kv_cache_write_reference
    assert a.torch_int8_paged_attention_reference is torch_reference.torch_int8_paged_attention_reference


def test_write_checker_matches_oracle():
    from int8kv.torch_reference import torch_int8_kv_cache_write_reference as ref_write

    g = torch.Generator().manual_seed(0)
    T, Hkv, D, NB = 45, 4, 128, 8
    key = (torch.randn(T, Hkv, D, generator=g) * 3).to(torch.bfloat16)
    value = torch.randn(T, Hkv, D, generator=g).to(torch.bfloat16)
    ks = torch.rand(Hkv, generator=g) * 0.05 + 0.01
    vs = torch.rand(Hkv, generator=g) * 0.02 + 0.005
    slots = torch.randperm(NB * 16, generator=g)[:T]
    slots[::7] = -1
    kc = torch.full((NB, 16, Hkv, D), 0x5A, dtype=torch.int8)
    vc = kc.clone()
    ref_write(key, value, kc, vc, slots, ks, vs)
    kc_o = np.full((NB, 16, Hkv, D), 0x5A, np.int8)
    vc_o = kc_o.copy()
    O.int8_kv_cache_write(key.float().numpy(), value.float().numpy(), kc_o, vc_o, slots.numpy(),
                          ks.numpy(), vs.numpy())
    assert np.array_equal(kc.numpy(), kc_o) and np.array_equal(vc.numpy(), vc_o)


def test_attention_checker_matches_oracle():
    from int8kv.torch_reference import torch_int8_paged_attention_reference as ref_attn

    c = decode_case([1, 17, 64, 200], seed=3, extra_blocks=6)
    kc, vc = torch.from_numpy(c.kc), torch.from_numpy(c.vc)
    for quantize_q in (False, True):
        got = ref_attn(c.query.float(), kc, vc, c.block_tables, c.seq_lens, c.k_scale, c.v_scale,
                       quantize_q=quantize_q)
        assert got.dtype == torch.float32
        ref = O.paged_attention_ref(c.query.float().numpy(), c.kc, c.vc, c.block_tables.numpy(),
                                    c.seq_lens.numpy(), c.k_scale.numpy(), c.v_scale.numpy(),
                                    quantize_q=quantize_q)
        err, cos, _ = metrics(got.numpy(), ref)
        assert err <= 1e-4 and cos >= 0.999999, (quantize_q, err, cos)
    out16 = ref_attn(c.query, kc, vc, c.block_tables, c.seq_lens, c.k_scale, c.v_scale)
    assert out16.dtype == torch.bfloat16
