"""Pins the CPU oracle (oracle/int8kv_oracle.py) before it is trusted as the checker.

The reference ships no golden vectors for this path, so each oracle function is pinned by
checks chosen so that a plausible slip fails one of them:
  * quantisation / write: hand known-answer tests (ties round to even, clamping, sign, the
    1e-6 scale floor, K vs V scale, slot -> (block, offset) split, skipped slots), the
    reference test's fixed scales and slot patterns (tests/test_cache_write.py:21-38,
    tests/test_runtime_cache_write.py:28-29), and a brute-force pure-Python loop;
  * paged layout: gather(scatter(x)) == x (tests/test_paged_cache.py:3-10) and permutation
    invariance;
  * attention: closed forms (one token -> v0 * v_scale, constant keys -> mean of v), the GQA
    head mapping h -> h // group, permutation of physical blocks, a float64 brute-force loop,
    and torch's scaled_dot_product_attention (float64) as an independent library routine.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import int8kv_oracle as O


# ----------------------------------------------------------------------------- quantisation
def test_quant_known_answers():
    x = np.array([2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5, 127.5, 300.0, -300.0, 126.49, -0.0],
                 np.float32)
    q = O.quant_kv_static_per_head(x, np.float32(1.0))
    assert q.tolist() == [2, 4, -2, -4, 0, 0, 2, 127, 127, -127, 126, 0]
    assert q.dtype == np.int8


def _fp32_quotient_exact(x: np.float32, s: np.float32) -> float:
    """Correctly rounded fp32 quotient from exact rational arithmetic (round to nearest even)."""
    from fractions import Fraction

    q = Fraction(float(x)) / Fraction(float(s))
    lo = np.float32(float(q))  # a neighbour; search the fp32 grid around it
    cands = [np.nextafter(lo, np.float32(-np.inf)), lo, np.nextafter(lo, np.float32(np.inf))]
    best = min(cands, key=lambda c: (abs(Fraction(float(c)) - q), int(np.float32(c).view(np.int32)) & 1))
    return float(best)


# (bf16 value, fp32 scale, int8 under an IEEE fp32 divide + half-even rounding).  The last two
# columns show what a reciprocal multiply and a float64 divide would give instead.
DIVIDE_KATS = [
    (-0.08251953125, 0.0036675346, -23, -22, -23),
    (-0.232421875, 0.011337652, -21, -20, -21),
    (-0.9296875, 0.053125, -18, -17, -17),
]


@pytest.mark.parametrize("x,s,want,rcp,f64", DIVIDE_KATS)
def test_quant_divides_in_fp32(x, s, want, rcp, f64):
    x, s = np.float32(x), np.float32(s)
    q = _fp32_quotient_exact(x, s)
    assert np.float32(x / s) == np.float32(q)
    assert int(np.rint(q)) == want
    assert int(np.rint(np.float32(x * np.float32(np.float32(1) / s)))) == rcp != want
    assert int(np.rint(np.float64(x) / np.float64(s))) == f64
    assert O.quant_kv_static_per_head(np.array([x], np.float32), s)[0] == want


def _brute_write(key, value, kc, vc, slots, ks, vs):
    nb, bs = kc.shape[:2]
    for t in range(key.shape[0]):
        s = int(slots[t])
        if s < 0 or s >= nb * bs:
            continue
        for h in range(key.shape[1]):
            for d in range(key.shape[2]):
                for src, dst, sc in ((key, kc, ks), (value, vc, vs)):
                    scale = max(float(sc[h]), float(np.float32(1e-6)))
                    qv = float(np.float32(src[t, h, d]) / np.float32(scale))
                    r = round(qv)  # Python round(): half to even
                    dst[s // bs, s % bs, h, d] = max(-127, min(127, r))


def test_write_known_answers():
    nb, bs, hkv, d = 3, 4, 2, 8
    key = np.zeros((4, hkv, d), np.float32)
    value = np.zeros((4, hkv, d), np.float32)
    key[0, 0, 0], key[0, 1, 0] = 2.5, 2.5  # head scales differ
    value[0, 0, 0] = 2.5
    key[1, 0, :2] = [300.0, -300.0]
    key[2, 1, 3] = 1e-4  # scale floor: 1e-4 / 1e-6 = 100
    key[3, 0, 0] = 9.0
    slots = np.array([5, 0, 11, -1], np.int64)  # token 3 skipped
    ks = np.array([1.0, 0.5], np.float32)
    vs = np.array([2.0, 1.0], np.float32)
    ks2 = ks.copy()
    kc = np.full((nb, bs, hkv, d), 0x5A, np.int8)
    vc = np.full((nb, bs, hkv, d), 0x5A, np.int8)
    # head-1 scale of token 2 is the floored one
    ks2[1] = 0.0
    O.int8_kv_cache_write(key[:2], value[:2], kc, vc, slots[:2], ks, vs)
    O.int8_kv_cache_write(key[2:], value[2:], kc, vc, slots[2:], ks2, vs)
    assert kc[1, 1, 0, 0] == 2 and kc[1, 1, 1, 0] == 5  # slot 5 -> block 1, offset 1
    assert vc[1, 1, 0, 0] == 1  # 2.5 / 2.0 = 1.25 -> 1 (V uses v_scale)
    assert kc[0, 0, 0, 0] == 127 and kc[0, 0, 0, 1] == -127
    assert kc[2, 3, 1, 3] == 100  # slot 11 -> block 2, offset 3, floored scale
    written = np.zeros((nb, bs), bool)
    written[1, 1] = written[0, 0] = written[2, 3] = True
    assert (kc[~written] == 0x5A).all() and (vc[~written] == 0x5A).all()


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_write_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    T, hkv, d, nb, bs = 9, 4, 16, 4, 4
    key = (rng.standard_normal((T, hkv, d)) * 3).astype(np.float32)
    value = rng.standard_normal((T, hkv, d)).astype(np.float32)
    # exact ties: multiples of scale/2
    key[0, 0, :] = (np.arange(d) - 8) * np.float32(0.5) * np.float32(0.25)
    slots = rng.permutation(nb * bs)[:T].astype(np.int64)
    slots[3] = -1
    ks = np.array([0.25, 0.03, 0.04, 0.035], np.float32)
    vs = np.array([0.035, 0.03, 0.025, 0.04], np.float32)
    kc = np.zeros((nb, bs, hkv, d), np.int8)
    vc = np.zeros_like(kc)
    kb, vb = kc.copy(), vc.copy()
    O.int8_kv_cache_write(key, value, kc, vc, slots, ks, vs)
    _brute_write(key, value, kb, vb, slots, ks, vs)
    assert np.array_equal(kc, kb) and np.array_equal(vc, vb)


def test_write_reference_test_patterns():
    # tests/test_cache_write.py:21-38: fixed scales (clamping is exercised) and the slot
    # pattern 16..31, 64..79, 96..100 over 8 blocks of 16.
    rng = np.random.default_rng(41)
    key = rng.standard_normal((37, 4, 128)).astype(np.float32) * 4
    value = rng.standard_normal((37, 4, 128)).astype(np.float32) * 4
    ks = np.array([0.03, 0.025, 0.04, 0.035], np.float32)
    vs = np.array([0.035, 0.03, 0.025, 0.04], np.float32)
    slots = np.array(list(range(16, 32)) + list(range(64, 80)) + list(range(96, 101)), np.int64)
    kc = np.zeros((8, 16, 4, 128), np.int8)
    vc = np.zeros_like(kc)
    O.int8_kv_cache_write(key, value, kc, vc, slots, ks, vs)
    assert (np.abs(kc[1]) == 127).any()  # clamping happens with these scales
    ref = O.quant_kv_static_per_head(key, ks[None, :, None])
    assert np.array_equal(kc[1], ref[:16]) and np.array_equal(kc[4], ref[16:32])
    assert np.array_equal(kc[6, :5], ref[32:37]) and (kc[6, 5:] == 0).all()
    # tests/test_runtime_cache_write.py:28-29: slots arange(7, 30) cross a block boundary.
    kc2 = np.zeros((16, 16, 4, 128), np.int8)
    vc2 = np.zeros_like(kc2)
    O.int8_kv_cache_write(key[:23], value[:23], kc2, vc2, np.arange(7, 30), ks, vs)
    assert np.array_equal(kc2[0, 7:], ref[:9]) and np.array_equal(kc2[1, :14], ref[9:23])


# ----------------------------------------------------------------------------- paged layout
def test_paged_round_trip_and_permutation():
    rng = np.random.default_rng(3)
    k = rng.standard_normal((2, 4, 127, 16)).astype(np.float32)
    v = rng.standard_normal((2, 4, 127, 16)).astype(np.float32)
    kc, vc, bt, sl = O.make_paged_cache(k, v, 16)
    k2, v2 = O.gather_from_paged_cache(kc, vc, bt, sl)
    assert np.array_equal(k, k2) and np.array_equal(v, v2)
    perm = rng.permutation(kc.shape[0])
    inv = np.argsort(perm)
    k3, v3 = O.gather_from_paged_cache(kc[perm], vc[perm], inv[bt], sl)
    assert np.array_equal(k, k3) and np.array_equal(v, v3)


# ----------------------------------------------------------------------------- attention
def _brute_attention(q, k, v):
    """float64 loops: q [Hq, D], k/v [T, Hkv, D]."""
    hq, d = q.shape
    T, hkv, _ = k.shape
    g = hq // hkv
    out = np.zeros((hq, d))
    for h in range(hq):
        kvh = h // g
        s = [sum(float(q[h, i]) * float(k[t, kvh, i]) for i in range(d)) / math.sqrt(d) for t in range(T)]
        m = max(s)
        w = [math.exp(x - m) for x in s]
        z = sum(w)
        for i in range(d):
            out[h, i] = sum(w[t] * float(v[t, kvh, i]) for t in range(T)) / z
    return out


def _random_paged(rng, lens, hq=8, hkv=2, d=16, bs=4, extra=5):
    nblk = [(n + bs - 1) // bs for n in lens]
    nb = sum(nblk) + extra
    pool = rng.permutation(nb)
    width = max(nblk)
    bt = np.full((len(lens), width), nb - 1, np.int64)
    p = 0
    for b, n in enumerate(nblk):
        bt[b, :n] = pool[p:p + n]
        p += n
    kc = rng.integers(-127, 128, (nb, bs, hkv, d)).astype(np.int8)
    vc = rng.integers(-127, 128, (nb, bs, hkv, d)).astype(np.int8)
    q = rng.standard_normal((len(lens), hq, d)).astype(np.float32)
    return q, kc, vc, bt, np.array(lens, np.int64)


def test_paged_attention_matches_brute_force():
    rng = np.random.default_rng(5)
    q, kc, vc, bt, sl = _random_paged(rng, [1, 7, 13])
    ks = np.array([0.02, 0.05], np.float32)
    vs = np.array([0.03, 0.01], np.float32)
    out = O.paged_attention_ref(q, kc, vc, bt, sl, ks, vs)
    for b in range(3):
        k = O.gather_sequence(kc, bt[b], sl[b]).astype(np.float64) * ks[None, :, None]
        v = O.gather_sequence(vc, bt[b], sl[b]).astype(np.float64) * vs[None, :, None]
        ref = _brute_attention(q[b].astype(np.float64), k, v)
        np.testing.assert_allclose(out[b], ref, rtol=2e-5, atol=2e-6)


def test_paged_attention_matches_torch_sdpa():
    rng = np.random.default_rng(6)
    lens = [33, 64, 5]
    q, kc, vc, bt, sl = _random_paged(rng, lens, hq=28, hkv=4, d=32, bs=16)
    ks = np.array([0.02, 0.05, 0.01, 0.04], np.float32)
    vs = np.array([0.03, 0.01, 0.02, 0.05], np.float32)
    out = O.paged_attention_ref(q, kc, vc, bt, sl, ks, vs, dtype=np.float64)
    for b, T in enumerate(lens):
        # dequantise in fp32 as the reference does (int8_paged_attention.py:808-809)
        k = torch.from_numpy((O.gather_sequence(kc, bt[b], T).astype(np.float32) * ks[None, :, None]).astype(np.float64))
        v = torch.from_numpy((O.gather_sequence(vc, bt[b], T).astype(np.float32) * vs[None, :, None]).astype(np.float64))
        qq = torch.from_numpy(q[b].astype(np.float64))[:, None, :]  # [Hq, 1, D]
        kk = k.permute(1, 0, 2).repeat_interleave(7, dim=0)  # [Hq, T, D]
        vv = v.permute(1, 0, 2).repeat_interleave(7, dim=0)
        ref = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv)[:, 0, :].numpy()
        np.testing.assert_allclose(out[b], ref, rtol=1e-10, atol=1e-12)


def test_attention_closed_forms():
    rng = np.random.default_rng(7)
    q, kc, vc, bt, _ = _random_paged(rng, [16, 16], hq=8, hkv=2, d=16, bs=4)
    ks = np.array([0.5, 0.25], np.float32)
    vs = np.array([0.125, 2.0], np.float32)
    # one token: every head of a group returns v0 * v_scale exactly
    out = O.paged_attention_ref(q, kc, vc, bt, np.array([1, 1]), ks, vs)
    for b in range(2):
        v0 = vc[bt[b, 0], 0].astype(np.float32) * vs[:, None]
        assert np.allclose(out[b, :4], v0[0], rtol=0, atol=1e-6)
        assert np.allclose(out[b, 4:], v0[1], rtol=0, atol=1e-6)
    # constant keys: uniform softmax -> mean of the values
    kc_const = np.ones_like(kc) * 3
    out = O.paged_attention_ref(q, kc_const, vc, bt, np.array([16, 11]), ks, vs)
    for b, T in enumerate([16, 11]):
        v = O.gather_sequence(vc, bt[b], T).astype(np.float64) * vs[None, :, None]
        np.testing.assert_allclose(out[b, :4], np.broadcast_to(v[:, 0].mean(0), (4, 16)), atol=1e-5)
        np.testing.assert_allclose(out[b, 4:], np.broadcast_to(v[:, 1].mean(0), (4, 16)), atol=1e-4)
    # empty sequence -> zeros
    assert (O.paged_attention_ref(q, kc, vc, bt, np.array([0, 0]), ks, vs) == 0).all()


def test_attention_gqa_mapping_and_block_permutation():
    rng = np.random.default_rng(8)
    q, kc, vc, bt, sl = _random_paged(rng, [12, 9], hq=6, hkv=3, d=8, bs=4)
    ks = np.full(3, 0.1, np.float32)
    vs = np.full(3, 0.1, np.float32)
    out = O.paged_attention_ref(q, kc, vc, bt, sl, ks, vs)
    # Query head h must attend kv head h // 2: zeroing kv head 2's values only affects heads 4, 5.
    vc2 = vc.copy()
    vc2[:, :, 2, :] = 0
    out2 = O.paged_attention_ref(q, kc, vc2, bt, sl, ks, vs)
    assert np.array_equal(out[:, :4], out2[:, :4]) and (out2[:, 4:] == 0).all()
    # Physical block permutation leaves the result unchanged.
    perm = rng.permutation(kc.shape[0])
    inv = np.argsort(perm)
    out3 = O.paged_attention_ref(q, kc[perm], vc[perm], inv[bt], sl, ks, vs)
    np.testing.assert_allclose(out, out3, rtol=0, atol=0)


def test_decode_attention_ref_equals_paged_form():
    rng = np.random.default_rng(9)
    q = rng.standard_normal((2, 8, 16)).astype(np.float32)
    k = rng.standard_normal((2, 2, 21, 16)).astype(np.float32)
    v = rng.standard_normal((2, 2, 21, 16)).astype(np.float32)
    dense = O.decode_attention_ref(q, k, v, dtype=np.float64)
    kc, vc, bt, sl = O.make_paged_cache(k, v, 4)
    paged = O.paged_attention_ref(q, kc, vc, bt, sl, dtype=np.float64)
    np.testing.assert_allclose(dense, paged, rtol=1e-12, atol=1e-12)
    e = O.expand_kv_for_gqa(k, 8)
    assert e.shape == (2, 8, 21, 16) and np.array_equal(e[:, 3], k[:, 0]) and np.array_equal(e[:, 4], k[:, 1])


def test_decode_bytes_formula():
    # B=1, one 512-token sequence: 512*4*128*2 (K+V int8) + 32 table entries*4 + q/out + lens + scales
    n = O.decode_bytes([512], 4, 128, 1, 1, 28)
    assert n == 512 * 4 * 128 * 2 + 32 * 4 + 2 * 28 * 128 * 2 + 4 + 2 * 4 * 4


def test_query_quantisation_known_answers():
    """quantize_q rounds half away from zero (src/triton_ops/int8_paged_attention.py:772-773):
    with absmax 127 the scale is exactly 1, so q/scale = q."""
    q = np.array([[127.0, 2.5, -2.5, 0.5, -0.5, 1.49, -126.5, 3.0]], np.float32)
    got = O.quantize_query_rows(q)
    assert got.tolist() == [[127.0, 3.0, -3.0, 1.0, -1.0, 1.0, -127.0, 3.0]]
    assert O.round_half_away(np.array([2.5, -2.5, 3.5, -0.4], np.float32)).tolist() == [3, -3, 4, -0]
    # all-zero row: scale floor 1e-6, codes 0
    assert (O.quantize_query_rows(np.zeros((1, 8), np.float32)) == 0).all()
    # brute force on random rows
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 16)).astype(np.float32)
    ref = np.empty_like(x)
    for i in range(4):
        s = max(float(np.float32(np.abs(x[i]).max() / np.float32(127))), float(np.float32(1e-6)))
        s = np.float32(s)
        for j in range(16):
            v = float(np.float32(x[i, j] / s))
            r = math.floor(v + 0.5) if v >= 0 else -math.floor(-v + 0.5)
            ref[i, j] = np.float32(max(-127, min(127, r)) * s)
    assert np.array_equal(O.quantize_query_rows(x), ref)


def test_paged_attention_quantize_q_changes_only_q():
    rng = np.random.default_rng(11)
    q, kc, vc, bt, sl = _random_paged(rng, [9, 20], hq=8, hkv=2, d=16, bs=4)
    ks = np.array([0.02, 0.05], np.float32)
    vs = np.array([0.03, 0.01], np.float32)
    qq = np.stack([O.quantize_query_rows(q[b]) for b in range(2)])
    a = O.paged_attention_ref(q, kc, vc, bt, sl, ks, vs, quantize_q=True)
    b = O.paged_attention_ref(qq, kc, vc, bt, sl, ks, vs)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, O.paged_attention_ref(q, kc, vc, bt, sl, ks, vs))


# ----------------------------------------------------------------------------- dynamic write
def test_dynamic_write_known_answers():
    """vllm_int8/vllm_int8_cache_ops.py:70-92: a row whose absmax is 127 has scale 1, so codes are
    x rounded half away from zero; an all-zero row has the 1e-6 floor and zero codes."""
    nb, bs, hkv, d = 2, 4, 2, 8
    key = np.zeros((3, hkv, d), np.float32)
    key[0, 0] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.49, -126.5, 3.0]
    key[0, 1] = [254.0, 5.0, -5.0, 1.0, -1.0, 0, 0, 0]  # scale 2 -> same codes as halves
    value = key * 0.5
    kc = np.full((nb, bs, hkv, d), 0x5A, np.int8)
    vc = kc.copy()
    ksc = np.full((nb, bs, hkv), -1.0, np.float32)
    vsc = ksc.copy()
    O.reshape_and_cache_int8(key, value, kc, vc, ksc, vsc, np.array([5, 2, -1]))
    assert kc[1, 1, 0].tolist() == [127, 3, -3, 1, -1, 1, -127, 3]
    assert kc[1, 1, 1].tolist()[:5] == [127, 3, -3, 1, -1]
    assert ksc[1, 1].tolist() == [1.0, 2.0] and vsc[1, 1].tolist() == [0.5, 1.0]
    assert (kc[0, 2] == 0).all() and ksc[0, 2].tolist() == [np.float32(1e-6)] * 2
    written = np.zeros((nb, bs), bool)
    written[1, 1] = written[0, 2] = True
    assert (kc[~written] == 0x5A).all() and (ksc[~written] == -1.0).all()


def test_dynamic_write_matches_brute_force():
    rng = np.random.default_rng(4)
    T, hkv, d, nb, bs = 7, 3, 16, 3, 4
    key = (rng.standard_normal((T, hkv, d)) * 2).astype(np.float32)
    value = rng.standard_normal((T, hkv, d)).astype(np.float32)
    slots = rng.permutation(nb * bs)[:T].astype(np.int64)
    slots[2] = -1
    got = [np.zeros((nb, bs, hkv, d), np.int8) for _ in range(2)] + \
        [np.zeros((nb, bs, hkv), np.float32) for _ in range(2)]
    O.reshape_and_cache_int8(key, value, got[0], got[1], got[2], got[3], slots)
    exp = [np.zeros((nb, bs, hkv, d), np.int8) for _ in range(2)] + \
        [np.zeros((nb, bs, hkv), np.float32) for _ in range(2)]
    for t in range(T):
        s = int(slots[t])
        if s < 0:
            continue
        for h in range(hkv):
            for src, dst, sdst in ((key, exp[0], exp[2]), (value, exp[1], exp[3])):
                amax = max(abs(float(v)) for v in src[t, h])
                scale = np.float32(max(float(np.float32(np.float32(amax) / np.float32(127))),
                                       float(np.float32(1e-6))))
                sdst[s // bs, s % bs, h] = scale
                for i in range(d):
                    q = float(np.float32(src[t, h, i] / scale))
                    q = max(-127.0, min(127.0, q))
                    dst[s // bs, s % bs, h, i] = math.floor(q + 0.5) if q >= 0 else math.ceil(q - 0.5)
    for g, e in zip(got, exp):
        assert np.array_equal(g, e)
