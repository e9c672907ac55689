"""GPU parity of the static INT8 cache write: bit-exact against the oracle.

Mirrors the reference's write tests (tests/test_int8_paged_attention.py:183-210,
tests/test_cache_write.py, tests/test_runtime_cache_write.py) with the stricter bar the build
targets: every int8 byte equal to the round-half-even oracle (the reference tolerated |diff| <= 1
because its Triton kernel rounds half away from zero).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import int8kv
from int8kv import synthetic as syn
from oracle import int8kv_oracle as O

pytestmark = pytest.mark.gpu

SENTINEL = 0x5A


def _run(key, value, slots, ks, vs, nb, dev, sentinel=SENTINEL, kc=None, vc=None):
    hkv, d = key.shape[1], key.shape[2]
    if kc is None:
        kc = torch.full((nb, 16, hkv, d), sentinel, dtype=torch.int8, device=dev)
        vc = torch.full_like(kc, sentinel)
    int8kv.int8_kv_cache_write(key.to(dev), value.to(dev), kc, vc, slots.to(dev), ks.to(dev), vs.to(dev))
    torch.cuda.synchronize()
    kr = np.full((nb, 16, hkv, d), sentinel, np.int8)
    vr = np.full_like(kr, sentinel)
    O.int8_kv_cache_write(key.float().cpu().numpy(), value.float().cpu().numpy(), kr, vr,
                          slots.cpu().numpy(), ks.cpu().numpy(), vs.cpu().numpy())
    return kc, vc, kr, vr


def _assert_equal(kc, vc, kr, vr):
    kg, vg = kc.cpu().numpy(), vc.cpu().numpy()
    nk = int((kg != kr).sum())
    nv = int((vg != vr).sum())
    assert nk == 0 and nv == 0, f"{nk} K bytes and {nv} V bytes differ from the oracle"


def test_write_config0_shape(cuda):
    g = torch.Generator().manual_seed(0)
    dist = syn.make_distribution(0)
    ks, vs = syn.calibrate_scales(dist, seed=1)
    k, v = syn.sample_kv(512, dist, g)
    bt = syn.random_block_tables([512], 64, g)
    slots = syn.slot_mapping_for(bt, [512])
    _assert_equal(*_run(k, v, slots, ks, vs, 64, cuda))


def test_write_config1_prefill_with_padding(cuda):
    """8 x 2048 tokens into 2048 blocks x 16 via a random-permutation slot mapping, -1 pads."""
    g = torch.Generator().manual_seed(11)
    dist = syn.make_distribution(11)
    ks, vs = syn.calibrate_scales(dist, seed=12)
    n_tok, n_pad, nb = 16384, 512, 2048
    k, v = syn.sample_kv(n_tok + n_pad, dist, g)
    slots = torch.randperm(nb * 16, generator=g)[: n_tok + n_pad].to(torch.int64)
    pad_rows = torch.randperm(n_tok + n_pad, generator=g)[:n_pad]
    slots[pad_rows] = -1
    kc, vc, kr, vr = _run(k, v, slots, ks, vs, nb, cuda)
    _assert_equal(kc, vc, kr, vr)
    untouched = np.ones(nb * 16, bool)
    untouched[slots[slots >= 0].numpy()] = False
    assert (kc.cpu().numpy().reshape(nb * 16, -1)[untouched] == SENTINEL).all()


@pytest.mark.parametrize("src_dtype", [torch.float16, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("slot_dtype", [torch.int32, torch.int64])
def test_write_dtypes(cuda, src_dtype, slot_dtype):
    g = torch.Generator().manual_seed(3)
    k = (torch.randn(300, 4, 128, generator=g) * 2).to(src_dtype)
    v = torch.randn(300, 4, 128, generator=g).to(src_dtype)
    ks = (k.float().abs().amax(dim=(0, 2)) / 127.0).clamp_min(1e-6)
    vs = (v.float().abs().amax(dim=(0, 2)) / 127.0).clamp_min(1e-6)
    slots = torch.randperm(40 * 16, generator=g)[:300].to(slot_dtype)
    _assert_equal(*_run(k, v, slots, ks, vs, 40, cuda))


def test_write_divide_and_tie_known_answers(cuda):
    """IEEE fp32 quotients on exact .5 ties: -23, -21, -18 (a reciprocal multiply gives -22, -20,
    -17; an fp64 divide gives -17 for the last one)."""
    kats = [(-0.08251953125, 0.0036675346, -23), (-0.232421875, 0.011337652, -21),
            (-0.9296875, 0.053125, -18)]
    key = torch.zeros(2, 4, 128, dtype=torch.bfloat16)
    ks = torch.ones(4)
    for h, (x, s, _) in enumerate(kats):
        key[0, h, :] = x
        ks[h] = s
    key[0, 3, :8] = torch.tensor([2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 300.0, -300.0])
    key[1] = key[0]
    value = key.clone()
    slots = torch.tensor([5, 17], dtype=torch.int64)
    kc, vc, kr, vr = _run(key, value, slots, ks, ks, 2, cuda)
    _assert_equal(kc, vc, kr, vr)
    got = kc.cpu()
    for h, (_, _, want) in enumerate(kats):
        assert (got[0, 5, h] == want).all() and (got[1, 1, h] == want).all()
    assert got[0, 5, 3, :8].tolist() == [2, 4, -2, -4, 0, 0, 127, -127]


def test_write_reference_fixed_scales_and_slots(cuda):
    """tests/test_cache_write.py:21-38 (scales that clamp; slots 16..31, 64..79, 96..100) and
    tests/test_runtime_cache_write.py:28-29 (slots 7..29 across a block boundary)."""
    g = torch.Generator().manual_seed(41)
    key = torch.randn(37, 4, 128, generator=g).to(torch.bfloat16)
    value = torch.randn(37, 4, 128, generator=g).to(torch.bfloat16)
    ks = torch.tensor([0.03, 0.025, 0.04, 0.035])
    vs = torch.tensor([0.035, 0.03, 0.025, 0.04])
    slots = torch.tensor(list(range(16, 32)) + list(range(64, 80)) + list(range(96, 101)))
    _assert_equal(*_run(key, value, slots, ks, vs, 8, cuda, sentinel=0))
    k23, v23 = key[:23], value[:23]
    ks2 = (k23.float().abs().amax(dim=(0, 2)) / 127).clamp_min(1e-6)
    vs2 = (v23.float().abs().amax(dim=(0, 2)) / 127).clamp_min(1e-6)
    _assert_equal(*_run(k23, v23, torch.arange(7, 30), ks2, vs2, 16, cuda, sentinel=0))


def test_write_strided_views(cuda):
    """key/value as head-slices of a fused qkv projection and caches as views of the
    [num_blocks, 2, BS, Hkv, D] split layout (vllm_shadow_cache_patch.py:26-43)."""
    g = torch.Generator().manual_seed(5)
    T, hq, hkv, d, nb = 77, 28, 4, 128, 12
    qkv = torch.randn(T, (hq + 2 * hkv) * d, generator=g).to(torch.bfloat16).to(cuda)
    key = qkv[:, hq * d:(hq + hkv) * d].view(T, hkv, d)
    value = qkv[:, (hq + hkv) * d:].view(T, hkv, d)
    assert not key.is_contiguous()
    ks = (key.float().abs().amax(dim=(0, 2)) / 127).clamp_min(1e-6)
    vs = (value.float().abs().amax(dim=(0, 2)) / 127).clamp_min(1e-6)
    kv = torch.full((nb, 2, 16, hkv, d), SENTINEL, dtype=torch.int8, device=cuda)
    slots = torch.randperm(nb * 16, generator=g)[:T]
    kc, vc, kr, vr = _run(key, value, slots, ks, vs, nb, cuda, kc=kv[:, 0], vc=kv[:, 1])
    _assert_equal(kc, vc, kr, vr)


@pytest.mark.parametrize("head_dim,pad", [(72, 0), (128, 8), (136, 0)])
def test_write_narrow_layouts(cuda, head_dim, pad):
    """Layouts the 16-element kernel does not take -- head_dim % 16 == 8, or cache rows only
    8-byte aligned (a view 8 bytes into a wider row) -- run the 8-element kernel, bit-exact."""
    g = torch.Generator().manual_seed(head_dim + pad)
    T, hkv, nb = 61, 4, 6
    k = (torch.randn(T, hkv, head_dim, generator=g) * 2).to(torch.bfloat16)
    v = torch.randn(T, hkv, head_dim, generator=g).to(torch.bfloat16)
    ks = (k.float().abs().amax(dim=(0, 2)) / 127).clamp_min(1e-6)
    vs = (v.float().abs().amax(dim=(0, 2)) / 127).clamp_min(1e-6)
    slots = torch.randperm(nb * 16, generator=g)[:T]
    slots[::9] = -1
    big = torch.full((2, nb, 16, hkv, head_dim + 2 * pad), SENTINEL, dtype=torch.int8, device=cuda)
    kc, vc = big[0, ..., pad:pad + head_dim], big[1, ..., pad:pad + head_dim]
    kc, vc, kr, vr = _run(k, v, slots, ks, vs, nb, cuda, kc=kc, vc=vc)
    _assert_equal(kc, vc, kr, vr)
    if pad:
        assert (big[..., :pad] == SENTINEL).all() and (big[..., pad + head_dim:] == SENTINEL).all()


def test_write_empty_and_out_of_range(cuda):
    k = torch.zeros(0, 4, 128, dtype=torch.bfloat16, device=cuda)
    kc = torch.full((2, 16, 4, 128), SENTINEL, dtype=torch.int8, device=cuda)
    vc = kc.clone()
    s = torch.ones(4, device=cuda)
    int8kv.int8_kv_cache_write(k, k, kc, vc, torch.zeros(0, dtype=torch.int64, device=cuda), s, s)
    torch.cuda.synchronize()
    assert (kc == SENTINEL).all()
    # Slots beyond the cache are skipped (no write outside the allocation).
    k = torch.ones(3, 4, 128, dtype=torch.bfloat16)
    slots = torch.tensor([32, 1000, 3], dtype=torch.int64)
    kc, vc, kr, vr = _run(k, k, slots, torch.ones(4), torch.ones(4), 2, cuda)
    _assert_equal(kc, vc, kr, vr)
    assert (kc.cpu()[0, 3] == 1).all()


# ----------------------------------------------------------------------------- dynamic write
def _run_dynamic(key, value, slots, nb, dev, kc=None, vc=None, ksc=None, vsc=None):
    from int8kv import cache_ops

    hkv, d = key.shape[1], key.shape[2]
    if kc is None:
        kc = torch.full((nb, 16, hkv, d), SENTINEL, dtype=torch.int8, device=dev)
        vc = torch.full_like(kc, SENTINEL)
        ksc = torch.full((nb, 16, hkv), -1.0, device=dev)
        vsc = torch.full_like(ksc, -1.0)
    cache_ops.reshape_and_cache_int8(key.to(dev), value.to(dev), kc, vc, ksc, vsc, slots.to(dev))
    torch.cuda.synchronize()
    ref = [np.full(tuple(kc.shape), SENTINEL, np.int8), np.full(tuple(vc.shape), SENTINEL, np.int8),
           np.full(tuple(ksc.shape), -1.0, np.float32), np.full(tuple(vsc.shape), -1.0, np.float32)]
    O.reshape_and_cache_int8(key.float().cpu().numpy(), value.float().cpu().numpy(), *ref,
                             slots.cpu().numpy())
    got = [kc.cpu().numpy(), vc.cpu().numpy(), ksc.cpu().numpy(), vsc.cpu().numpy()]
    return got, ref


@pytest.mark.parametrize("src_dtype", [torch.float16, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("slot_dtype", [torch.int32, torch.int64])
def test_dynamic_write_bit_exact(cuda, src_dtype, slot_dtype):
    g = torch.Generator().manual_seed(17)
    T, nb = 300, 40
    k = (torch.randn(T, 4, 128, generator=g) * 3).to(src_dtype)
    v = torch.randn(T, 4, 128, generator=g).to(src_dtype)
    k[5, 2] = 0  # all-zero row: scale floor, zero codes
    slots = torch.randperm(nb * 16, generator=g)[:T].to(slot_dtype)
    slots[::17] = -1
    got, ref = _run_dynamic(k, v, slots, nb, cuda)
    for name, a, b in zip(("K codes", "V codes", "K scales", "V scales"), got, ref):
        assert np.array_equal(a, b), f"{name} differ from the oracle"


@pytest.mark.parametrize("head_dim", [64, 256])
def test_dynamic_write_head_dims(cuda, head_dim):
    g = torch.Generator().manual_seed(head_dim)
    k = torch.randn(50, 2, head_dim, generator=g).to(torch.bfloat16)
    v = torch.randn(50, 2, head_dim, generator=g).to(torch.bfloat16)
    slots = torch.randperm(8 * 16, generator=g)[:50]
    got, ref = _run_dynamic(k, v, slots, 8, cuda)
    assert all(np.array_equal(a, b) for a, b in zip(got, ref))


def test_dynamic_write_reference_scenario(cuda):
    """tests/test_vllm_int8_cache_ops.py:10-118: 23 bf16 tokens into slots 7..29 (across a block
    boundary); per-token dequantisation error below 0.02 on average; plus bit-exactness."""
    from int8kv import cache_ops

    g = torch.Generator().manual_seed(0)
    key = torch.randn(23, 4, 128, generator=g).to(torch.bfloat16)
    value = torch.randn(23, 4, 128, generator=g).to(torch.bfloat16)
    kc, vc, ksc, vsc = cache_ops.allocate_int8_kv_cache(32, 16, 4, 128, device=cuda)
    slots = torch.arange(7, 30, dtype=torch.int64)
    got, ref = _run_dynamic(key, value, slots, 32, cuda, kc, vc, ksc, vsc)
    written = np.zeros((32, 16), bool)
    written.reshape(-1)[slots.numpy()] = True
    for a, b in zip(got, ref):
        assert np.array_equal(a[written], b[written])
    kd = cache_ops.dequantize_int8_cache(kc, ksc).cpu().reshape(-1, 4, 128)[slots]
    vd = cache_ops.dequantize_int8_cache(vc, vsc).cpu().reshape(-1, 4, 128)[slots]
    assert float((kd - key.float()).abs().mean()) < 0.02
    assert float((vd - value.float()).abs().mean()) < 0.02


def test_dynamic_write_narrow_layout(cuda):
    """Cache rows only 8-byte aligned: the 8-element dynamic kernel, bit-exact."""
    g = torch.Generator().manual_seed(31)
    T, hkv, d, nb = 37, 4, 128, 5
    k = (torch.randn(T, hkv, d, generator=g) * 3).to(torch.bfloat16)
    v = torch.randn(T, hkv, d, generator=g).to(torch.bfloat16)
    big = torch.full((2, nb, 16, hkv, d + 16), SENTINEL, dtype=torch.int8, device=cuda)
    sc = torch.full((2, nb, 16, hkv), -1.0, device=cuda)
    slots = torch.randperm(nb * 16, generator=g)[:T]
    got, ref = _run_dynamic(k, v, slots, nb, cuda, big[0, ..., 8:8 + d], big[1, ..., 8:8 + d], sc[0], sc[1])
    assert all(np.array_equal(a, b) for a, b in zip(got, ref))


def test_dynamic_write_strided_views(cuda):
    """key/value as head slices of a fused qkv projection; caches and scale caches as views of
    joint K/V allocations."""
    g = torch.Generator().manual_seed(9)
    T, hq, hkv, d, nb = 41, 28, 4, 128, 6
    qkv = torch.randn(T, (hq + 2 * hkv) * d, generator=g).to(torch.bfloat16).to(cuda)
    key = qkv[:, hq * d:(hq + hkv) * d].view(T, hkv, d)
    value = qkv[:, (hq + hkv) * d:].view(T, hkv, d)
    kv = torch.full((nb, 2, 16, hkv, d), SENTINEL, dtype=torch.int8, device=cuda)
    sc = torch.full((2, nb, 16, hkv), -1.0, device=cuda)
    slots = torch.randperm(nb * 16, generator=g)[:T]
    got, ref = _run_dynamic(key, value, slots, nb, cuda, kv[:, 0], kv[:, 1], sc[0], sc[1])
    assert all(np.array_equal(a, b) for a, b in zip(got, ref))


def test_debug_checks_reject_duplicate_slots(cuda, monkeypatch):
    """With INT8KV_DEBUG on, a duplicated slot raises before the write is launched (the caches
    keep their sentinel)."""
    from int8kv import _decode, cache_ops

    monkeypatch.setattr(_decode, "DEBUG_CHECKS", True)
    k = torch.ones(3, 4, 128, dtype=torch.bfloat16, device=cuda)
    kc = torch.full((2, 16, 4, 128), SENTINEL, dtype=torch.int8, device=cuda)
    vc = kc.clone()
    s = torch.ones(4, device=cuda)
    slots = torch.tensor([4, 9, 4], dtype=torch.int64, device=cuda)
    with pytest.raises(AssertionError, match="repeats"):
        int8kv.int8_kv_cache_write(k, k, kc, vc, slots, s, s)
    ksc = torch.zeros(2, 16, 4, device=cuda)
    with pytest.raises(AssertionError, match="repeats"):
        cache_ops.reshape_and_cache_int8(k, k, kc, vc, ksc, ksc.clone(), slots)
    torch.cuda.synchronize()
    assert (kc == SENTINEL).all() and (vc == SENTINEL).all()


def test_write_misaligned_sources_are_copied(cuda):
    """Contiguous key/value at an odd storage offset (rows not 16-byte aligned) are read through
    aligned copies; the caches are bit-exact to the oracle."""
    g = torch.Generator().manual_seed(17)
    T, hkv, d, nb = 45, 4, 128, 8
    k = torch.randn(T, hkv, d, generator=g).to(torch.bfloat16).to(cuda)
    v = torch.randn(T, hkv, d, generator=g).to(torch.bfloat16).to(cuda)
    bufk = torch.empty(k.numel() + 1, dtype=k.dtype, device=cuda)
    bufv = torch.empty(v.numel() + 3, dtype=v.dtype, device=cuda)
    k_odd, v_odd = bufk[1:].view(k.shape), bufv[3:].view(v.shape)
    k_odd.copy_(k)
    v_odd.copy_(v)
    assert k_odd.data_ptr() % 16 and v_odd.data_ptr() % 16
    ks = (k.float().abs().amax(dim=(0, 2)) / 127).clamp_min(1e-6)
    vs = (v.float().abs().amax(dim=(0, 2)) / 127).clamp_min(1e-6)
    slots = torch.randperm(nb * 16, generator=g)[:T]
    _assert_equal(*_run(k_odd, v_odd, slots, ks, vs, nb, cuda))
    from int8kv import cache_ops
    kc = torch.zeros(nb, 16, hkv, d, dtype=torch.int8, device=cuda)
    vc = torch.zeros_like(kc)
    ksc = torch.zeros(nb, 16, hkv, device=cuda)
    vsc = torch.zeros_like(ksc)
    cache_ops.reshape_and_cache_int8(k_odd, v_odd, kc, vc, ksc, vsc, slots.to(cuda))
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    ksc2, vsc2 = torch.zeros_like(ksc), torch.zeros_like(vsc)
    cache_ops.reshape_and_cache_int8(k, v, kc2, vc2, ksc2, vsc2, slots.to(cuda))
    torch.cuda.synchronize()
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
    assert torch.equal(ksc, ksc2) and torch.equal(vsc, vsc2)


@pytest.mark.parametrize("hkv,d", [(1, 128), (3, 128), (8, 128), (4, 256), (8, 256), (2, 64)])
def test_writes_across_kv_head_counts(cuda, hkv, d):
    """Static and dynamic writes for kv-head counts and head sizes on both sides of the
    token-major lane map (a token's heads in one wave when Hkv is a power of two and
    Hkv * head_dim / 16 <= 64; the head-major kernels otherwise): bit-exact to the oracle."""
    g = torch.Generator().manual_seed(100 * hkv + d)
    T, nb = 77, 9
    k = (torch.randn(T, hkv, d, generator=g) * 2).to(torch.bfloat16)
    v = torch.randn(T, hkv, d, generator=g).to(torch.bfloat16)
    slots = torch.randperm(nb * 16, generator=g)[:T]
    slots[3::11] = -1
    ks = (k.float().abs().amax(dim=(0, 2)) / 127).clamp_min(1e-6)
    vs = (v.float().abs().amax(dim=(0, 2)) / 127).clamp_min(1e-6)
    _assert_equal(*_run(k, v, slots, ks, vs, nb, cuda))
    got, ref = _run_dynamic(k, v, slots, nb, cuda)
    for name, a, b in zip(("K codes", "V codes", "K scales", "V scales"), got, ref):
        assert np.array_equal(a, b), f"{name} differ from the oracle (Hkv={hkv}, D={d})"


def test_dynamic_write_head_strided_scale_cache(cuda):
    """Scale caches whose kv-head stride is not 1 (a transposed view): per-head scale stores."""
    g = torch.Generator().manual_seed(55)
    T, hkv, d, nb = 60, 4, 128, 7
    k = (torch.randn(T, hkv, d, generator=g) * 3).to(torch.bfloat16)
    v = torch.randn(T, hkv, d, generator=g).to(torch.bfloat16)
    slots = torch.randperm(nb * 16, generator=g)[:T]
    kc = torch.full((nb, 16, hkv, d), SENTINEL, dtype=torch.int8, device=cuda)
    vc = torch.full_like(kc, SENTINEL)
    ksc = torch.full((hkv, nb, 16), -1.0, device=cuda).permute(1, 2, 0)  # [nb, 16, hkv], stride(2) != 1
    vsc = torch.full((hkv, nb, 16), -1.0, device=cuda).permute(1, 2, 0)
    assert ksc.stride(2) != 1
    got, ref = _run_dynamic(k, v, slots, nb, cuda, kc, vc, ksc, vsc)
    for name, a, b in zip(("K codes", "V codes", "K scales", "V scales"), got, ref):
        assert np.array_equal(a, b), f"{name} differ from the oracle"


@pytest.mark.parametrize("src_dtype,T", [(torch.bfloat16, 262_144), (torch.float32, 65_536)])
def test_hbm_sized_writes_sampled(cuda, src_dtype, T):
    """Writes larger than the 256 MB Infinity Cache (the static write's token-major kernel runs
    only there): every sampled token's K/V codes (and dynamic scales) equal the oracle's for that
    token, and every slot the mapping does not name keeps the sentinel."""
    g = torch.Generator().manual_seed(T)
    hkv, d, nb = 4, 128, 2 * T // 16
    k = (torch.randn(T, hkv, d, generator=g) * 2).to(src_dtype).to(cuda)
    v = torch.randn(T, hkv, d, generator=g).to(src_dtype).to(cuda)
    slots = torch.randperm(nb * 16, generator=g)[:T]
    slots[7::1001] = -1
    ks = (k.float().abs().amax(dim=(0, 2)) / 127).clamp_min(1e-6).cpu()
    vs = (v.float().abs().amax(dim=(0, 2)) / 127).clamp_min(1e-6).cpu()
    idx = torch.cat([torch.tensor([0, T - 1]), torch.randperm(T, generator=g)[:4094]])
    idx = idx[slots[idx] >= 0]
    n = idx.numel()
    small = (n + 15) // 16
    kx, vx = k[idx.to(cuda)].float().cpu().numpy(), v[idx.to(cuda)].float().cpu().numpy()
    written = torch.zeros(nb * 16, dtype=torch.bool, device=cuda)
    written[slots[slots >= 0].to(cuda)] = True
    rows = slots[idx].to(cuda)

    kc = torch.full((nb, 16, hkv, d), SENTINEL, dtype=torch.int8, device=cuda)
    vc = torch.full_like(kc, SENTINEL)
    int8kv.int8_kv_cache_write(k, v, kc, vc, slots.to(cuda), ks.to(cuda), vs.to(cuda))
    torch.cuda.synchronize()
    kr = np.full((small, 16, hkv, d), SENTINEL, np.int8)
    vr = np.full_like(kr, SENTINEL)
    O.int8_kv_cache_write(kx, vx, kr, vr, np.arange(n), ks.numpy(), vs.numpy())
    for name, c, r in (("K", kc, kr), ("V", vc, vr)):
        flat = c.view(nb * 16, hkv * d)
        assert np.array_equal(flat[rows].cpu().numpy(), r.reshape(-1, hkv * d)[:n]), f"static {name}"
        assert bool((flat[~written] == SENTINEL).all()), f"static {name}: unnamed slot written"

    from int8kv import cache_ops
    kc.fill_(SENTINEL)
    vc.fill_(SENTINEL)
    ksc = torch.full((nb, 16, hkv), -1.0, device=cuda)
    vsc = torch.full_like(ksc, -1.0)
    cache_ops.reshape_and_cache_int8(k, v, kc, vc, ksc, vsc, slots.to(cuda))
    torch.cuda.synchronize()
    ref = [np.full((small, 16, hkv, d), SENTINEL, np.int8), np.full((small, 16, hkv, d), SENTINEL, np.int8),
           np.full((small, 16, hkv), -1.0, np.float32), np.full((small, 16, hkv), -1.0, np.float32)]
    O.reshape_and_cache_int8(kx, vx, *ref, np.arange(n))
    for name, c, r, fill in (("K", kc, ref[0], SENTINEL), ("V", vc, ref[1], SENTINEL),
                             ("K scale", ksc, ref[2], -1.0), ("V scale", vsc, ref[3], -1.0)):
        flat = c.view(nb * 16, -1)
        assert np.array_equal(flat[rows].cpu().numpy(), r.reshape(small * 16, -1)[:n]), f"dynamic {name}"
        assert bool((flat[~written] == fill).all()), f"dynamic {name}: unnamed slot written"
