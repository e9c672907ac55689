"""Seeded random cache-write configurations, bit-exact against the oracle.

Each case draws the token count (0-3000, some slots -1 or past the cache, which the writes skip),
kv heads (1, 2, 3, 4 or 8), head_dim (64, 128, 256, and 72 / 136 for the static write's narrow
kernels; a second set at the other multiples of 16 from 16 to 240), the cache block size (16-64), the source dtype (bf16, fp16, fp32; K and V of one
dtype), the slot dtype (int32 / int64), source views with padded token or head strides, and the
value scale (data spanning small and large magnitudes, so some quotients clamp), then runs the
static write (``int8_kv_cache_write``) and the dynamic per-(token, head) write
(``reshape_and_cache_int8``) into sentinel-filled caches and compares every byte (and every
dynamic scale) with the oracle, including the slots that must stay untouched.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import int8kv
from int8kv import cache_ops
from oracle import int8kv_oracle as O

pytestmark = pytest.mark.gpu

SENTINEL = 0x5A
SRC = [torch.bfloat16, torch.float16, torch.float32]


def _draw(seed: int) -> dict:
    rng = np.random.default_rng(5000 + seed)
    return dict(T=int(rng.choice([0, 1, 17, 300, 1000, 3000])), hkv=int(rng.choice([1, 2, 3, 4, 8])),
                d=int(rng.choice([64, 128, 256, 72, 136])), bs=int(rng.choice([16, 32, 64])),
                src=SRC[rng.integers(3)], slot64=bool(rng.random() < 0.5),
                view=int(rng.integers(3)), amp=float(rng.choice([0.01, 1.0, 30.0])))


def _source(T, hkv, d, dtype, view, g):
    """[T, hkv, d] of dtype, contiguous (view 0) or a strided view: padded token rows (1) or a
    slice of twice as many heads (2)."""
    if view == 1:
        base = torch.randn(T, hkv * d + 24, generator=g)
        x = base[:, : hkv * d].reshape(T, hkv, d) if T else base[:, : hkv * d].reshape(0, hkv, d)
    elif view == 2:
        x = torch.randn(T, 2 * hkv, d, generator=g)[:, ::2]
    else:
        x = torch.randn(T, hkv, d, generator=g)
    return x


@pytest.mark.parametrize("seed", range(20))
def test_random_writes(cuda, seed):
    _run(cuda, _draw(seed), seed)


@pytest.mark.parametrize("seed", range(50, 62))
def test_random_writes_other_head_dims(cuda, seed):
    """The random draws at the other multiples of 16 the decode takes (16-240): wide kernels with
    1-15 lanes per row (not a power of two: the head-major map at every size), and the dynamic
    write where head_dim / 8 is a power of two (16, 32)."""
    p = _draw(seed)
    p["d"] = [16, 32, 48, 80, 96, 112, 144, 160, 176, 192, 208, 240][seed % 12]
    _run(cuda, p, seed)


def _run(cuda, p, seed):
    what = f"seed {seed}: {p}"
    T, hkv, d, bs = p["T"], p["hkv"], p["d"], p["bs"]
    g = torch.Generator().manual_seed(seed)
    k32 = _source(T, hkv, d, p["src"], p["view"], g) * p["amp"]
    v32 = _source(T, hkv, d, p["src"], p["view"], g) * p["amp"] * 0.5
    k32[T // 3:T // 3 + 1] *= 300.0  # a token far outside the calibrated range: clamped codes
    k = k32.to(p["src"])
    v = v32.to(p["src"])
    nb = max(1, (T + 40) // bs + 2)
    cap = nb * bs
    slots = torch.randperm(cap, generator=g)[:T] if T <= cap else torch.arange(T) % cap
    if T:
        slots[torch.randperm(T, generator=g)[: T // 10]] = -1
        slots[torch.randperm(T, generator=g)[: T // 20]] = cap + 7  # past the cache: skipped
    slots = slots.to(torch.int64 if p["slot64"] else torch.int32)
    kf, vf = k.float().numpy(), v.float().numpy()
    ks = (torch.tensor(np.abs(kf).reshape(-1, hkv, d).max(axis=(0, 2)) if T else np.ones(hkv)) /
          127 * 0.7).float().clamp_min(1e-6)
    vs = (torch.tensor(np.abs(vf).reshape(-1, hkv, d).max(axis=(0, 2)) if T else np.ones(hkv)) /
          127).float().clamp_min(1e-6)

    # static write
    kc = torch.full((nb, bs, hkv, d), SENTINEL, dtype=torch.int8, device=cuda)
    vc = torch.full_like(kc, SENTINEL)
    kd = k.to(cuda) if p["view"] == 0 else _as_view(k, cuda, p["view"])
    vd = v.to(cuda) if p["view"] == 0 else _as_view(v, cuda, p["view"])
    int8kv.int8_kv_cache_write(kd, vd, kc, vc, slots.to(cuda), ks.to(cuda), vs.to(cuda))
    torch.cuda.synchronize()
    kr = np.full((nb, bs, hkv, d), SENTINEL, np.int8)
    vr = np.full_like(kr, SENTINEL)
    O.int8_kv_cache_write(kf, vf, kr, vr, slots.numpy(), ks.numpy(), vs.numpy())
    assert np.array_equal(kc.cpu().numpy(), kr), "static K " + what
    assert np.array_equal(vc.cpu().numpy(), vr), "static V " + what

    # dynamic write (head_dim / 8 must be a power of two)
    if (d // 8) & (d // 8 - 1):
        return
    kc.fill_(SENTINEL)
    vc.fill_(SENTINEL)
    ksc = torch.full((nb, bs, hkv), -1.0, device=cuda)
    vsc = torch.full_like(ksc, -1.0)
    cache_ops.reshape_and_cache_int8(kd, vd, kc, vc, ksc, vsc, slots.to(cuda))
    torch.cuda.synchronize()
    ref = [np.full((nb, bs, hkv, d), SENTINEL, np.int8), np.full((nb, bs, hkv, d), SENTINEL, np.int8),
           np.full((nb, bs, hkv), -1.0, np.float32), np.full((nb, bs, hkv), -1.0, np.float32)]
    O.reshape_and_cache_int8(kf, vf, *ref, slots.numpy())
    for name, got, want in zip(("K", "V", "K scale", "V scale"), (kc, vc, ksc, vsc), ref):
        assert np.array_equal(got.cpu().numpy(), want), f"dynamic {name} " + what


def _as_view(x: torch.Tensor, dev, view: int) -> torch.Tensor:
    """The same values on the device as the kind of strided view the case drew."""
    T, hkv, d = x.shape
    if view == 1:
        base = torch.zeros(T, hkv * d + 24, dtype=x.dtype, device=dev)
        base[:, : hkv * d] = x.reshape(T, hkv * d).to(dev)
        return base[:, : hkv * d].view(T, hkv, d)
    base = torch.zeros(T, 2 * hkv, d, dtype=x.dtype, device=dev)
    base[:, ::2] = x.to(dev)
    return base[:, ::2]
