"""Pins the torch CPU restatement (oracle/torch_cpu_path.py), the timed CPU baseline.

Checks: known answers of the static quantisation (ties to even, clamp, sign), the paged write
bit-exact against the numpy oracle's slot-mapping write, gather(write(x)) == codes of x, the
decode step against the numpy oracle on a ragged batch with shuffled tables (and an empty
sequence), and the reference attention against torch's scaled_dot_product_attention in float64.
"""

from __future__ import annotations

import numpy as np
import torch

from int8kv import synthetic as syn
from oracle import int8kv_oracle as O
from oracle import torch_cpu_path as TP


def test_quant_known_answers():
    x = torch.tensor([2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 127.5, 300.0, -300.0, 126.49])
    q = TP.quant_kv_static_per_head(x, torch.tensor(1.0))
    assert q.dtype == torch.int8
    assert q.tolist() == [2, 4, -2, -4, 0, 0, 127, 127, -127, 126]


def _ragged(seed=0, lens=(37, 1, 0, 200, 64), pool_extra=9):
    g = torch.Generator().manual_seed(seed)
    dist = syn.make_distribution(seed)
    ks, vs = syn.calibrate_scales(dist, seed=seed + 1)
    nb = sum((n + 15) // 16 for n in lens) + pool_extra
    bt = syn.random_block_tables(lens, nb, g)
    k, v = syn.sample_kv(sum(lens), dist, g)
    q = syn.sample_query(len(lens), g)
    return lens, nb, bt, k, v, q, ks, vs


def test_write_matches_numpy_oracle_and_gathers_back():
    lens, nb, bt, k, v, q, ks, vs = _ragged()
    kc = torch.zeros(nb, 16, 4, 128, dtype=torch.int8)
    vc = torch.zeros_like(kc)
    off = 0
    for b, n in enumerate(lens):
        TP.write_paged(k[off:off + n], v[off:off + n], kc, vc, bt[b], ks, vs)
        off += n
    kc_ref = np.zeros((nb, 16, 4, 128), np.int8)
    vc_ref = np.zeros_like(kc_ref)
    slots = syn.slot_mapping_for(bt, lens)
    O.int8_kv_cache_write(k.float().numpy(), v.float().numpy(), kc_ref, vc_ref, slots.numpy(),
                          ks.numpy(), vs.numpy())
    assert np.array_equal(kc.numpy(), kc_ref) and np.array_equal(vc.numpy(), vc_ref)
    off = 0
    for b, n in enumerate(lens):
        got = TP.gather_sequence(kc, bt[b], n).permute(1, 0, 2)
        want = TP.quant_kv_static_per_head(k[off:off + n].float(), ks.reshape(1, 4, 1))
        assert torch.equal(got, want)
        off += n


def test_decode_step_matches_numpy_oracle():
    lens, nb, bt, k, v, q, ks, vs = _ragged(seed=3)
    kc = np.zeros((nb, 16, 4, 128), np.int8)
    vc = np.zeros_like(kc)
    slots = syn.slot_mapping_for(bt, lens)
    O.int8_kv_cache_write(k.float().numpy(), v.float().numpy(), kc, vc, slots.numpy(), ks.numpy(),
                          vs.numpy())
    lens_t = torch.tensor(lens, dtype=torch.int32)
    got = TP.decode_step(q, torch.from_numpy(kc), torch.from_numpy(vc), bt, lens_t, ks, vs)
    ref = O.paged_attention_ref(q.float().numpy(), kc, vc, bt.numpy(), lens_t.numpy(), ks.numpy(),
                                vs.numpy())
    assert float(np.abs(got.numpy() - ref).max()) < 1e-5
    assert float(got[2].abs().max()) == 0.0  # the empty sequence
    part = TP.decode_step(q, torch.from_numpy(kc), torch.from_numpy(vc), bt, lens_t, ks, vs,
                          sequences=[3])
    assert torch.equal(part[3], got[3]) and float(part[0].abs().max()) == 0.0


def test_attention_matches_sdpa_float64():
    g = torch.Generator().manual_seed(5)
    q = torch.randn(2, 28, 128, generator=g)
    k = torch.randn(2, 4, 77, 128, generator=g)
    v = torch.randn(2, 4, 77, 128, generator=g)
    got = TP.decode_attention_ref(q, k, v).double()
    kk = k.double().repeat_interleave(7, dim=1)
    vv = v.double().repeat_interleave(7, dim=1)
    ref = torch.nn.functional.scaled_dot_product_attention(q.double()[:, :, None], kk, vv)[:, :, 0]
    assert float((got - ref).abs().max()) < 1e-5
    # kv head g serves query heads 7g .. 7g + 6: moving kv head 1's data moves only those rows
    k2 = k.clone()
    k2[:, 1] = torch.randn(2, 77, 128, generator=g)
    got2 = TP.decode_attention_ref(q, k2, v)
    changed = (got2 - got.float()).abs().amax(dim=(0, 2)) > 0
    assert changed.tolist() == [7 <= h < 14 for h in range(28)]
