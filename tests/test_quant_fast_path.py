"""The cache-write kernels' quantisation shortcut, checked exhaustively on the CPU.

The kernels need clamp(rint(RN(x / s)), -127, 127), with RN the correctly rounded fp32 divide.
They compute q0 = RN(x * r) with r = RN(1 / s), clamp it to qc in [-127, 127], and keep
n = rint(qc) unless |qc - n| >= 0.5 - 127 * 2^-20 (qc within 127 * 2^-20 of a half-integer), in
which case they divide (and for every element when s >= 2^100, where r could be subnormal).

Why that is exact: |r - 1/s| <= 2^-24 / s, so |x r - x/s| <= 2^-24 |x/s|; the product and the
divide each round by at most 2^-24 relative; hence |q0 - RN(x/s)| <= 3.0000002 * 2^-24 |x/s|,
at most 2.28e-5 while |q0| <= 127, well inside 127 * 2^-20 = 1.21e-4.  When no half-integer lies
that close to qc, RN(x/s) is in the same open interval between consecutive half-integers and
rounds to the same integer.  When |q0| > 127 (infinities included) qc = n = +-127 and RN(x/s) lies
beyond +-126.5, so the code is +-127 either way; a NaN becomes -127 on both paths: fmaxf/fminf
return the non-NaN operand, and the lower bound is applied first.  |qc - n| is exact (Sterbenz).
The same boundary argument holds for the dynamic write's half-away-from-zero rounding (rint and
half-away differ only at half-integers).

This file restates the kernels' steps in numpy float32 (each numpy float32 operation is one
correctly rounded IEEE operation, like the GPU's) and compares them with the divide for every
finite bf16 and fp16 value against a few hundred scales, including the reference's calibrated
Qwen scales and scales chosen to put quotients on and next to half-integers.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"
F32 = np.float32


def _all_finite(dtype) -> np.ndarray:
    bits = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16)
    vals = bits.view(dtype).float().numpy()
    return vals[np.isfinite(vals)]


def _clamp(v, lo, hi):
    """fminf(fmaxf(v, lo), hi): C semantics, a NaN operand yields the other operand."""
    return np.fmin(np.fmax(v, F32(lo)), F32(hi))


def _exact_codes(x, s, half_away=False):
    with np.errstate(over="ignore", invalid="ignore"):
        q = (x / s).astype(F32)  # IEEE fp32 divide
    if half_away:
        q = _clamp(q, -127, 127)
        return np.where(q >= 0, np.floor(q + F32(0.5)), -np.floor(-q + F32(0.5)))
    return _clamp(np.rint(q), -127, 127)


def _fast_codes(x, s):
    """The kernels' shortcut; returns (codes where the shortcut is kept, mask of lanes that
    divide instead)."""
    r = (F32(1) / s).astype(F32)
    with np.errstate(over="ignore", invalid="ignore"):
        q0 = (x * r).astype(F32)
    qc = _clamp(q0, -127, 127)
    n = np.rint(qc)
    d = np.abs(qc - n).astype(F32)
    keep_below = F32(0.5) - F32(127 * 2.0 ** -20)  # exact in float32, as in the kernels
    slow = ~(d < keep_below) | (s >= F32(2.0 ** 100))
    return n, slow


def _scales(seed=0):
    g = np.random.default_rng(seed)
    sc = json.loads((GOLDEN / "static_per_head_scales.json").read_text())
    out = [F32(v) for v in np.ravel(sc["k_scale"]) + np.ravel(sc["v_scale"])]  # reference's
    out += list(g.uniform(1e-6, 1.0, 64).astype(F32))
    out += list((10.0 ** g.uniform(-6, 3, 64)).astype(F32))
    out += [F32(2.0) ** k for k in range(-19, 8)]  # reciprocals exact
    # scales making x / s land on or right next to half-integers for many bf16 x
    for h in (0.5, 1.5, 2.5, 63.5, 126.5, 127.5):
        base = F32(1.0) / F32(h)
        out += [base, np.nextafter(base, F32(0)), np.nextafter(base, F32(1e9))]
    out += [F32(1e-6), np.nextafter(F32(1e-6), F32(1)), F32(1) / F32(3), F32(1) / F32(7)]
    return np.array(out, F32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("half_away", [False, True])
def test_shortcut_matches_the_divide_everywhere(dtype, half_away):
    x = _all_finite(dtype)
    slow_total, n_total = 0, 0
    for s in _scales():
        want = _exact_codes(x, s, half_away)
        fast, slow = _fast_codes(x, s)
        got = np.where(slow, want, fast)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, (f"scale {s!r}: x={x[bad[:5]]} fast={fast[bad[:5]]} "
                               f"divide={want[bad[:5]]}")
        inside = np.abs(x.astype(np.float64) / float(s)) < 256  # quotients that are not clamped
        slow_total += int(slow[inside].sum())
        n_total += int(inside.sum())
    # the divide is the exception among unclamped quotients (every one of which is probed here,
    # so half-integer quotients are far more frequent than in real data)
    assert slow_total < 2e-3 * n_total, slow_total / n_total


def test_shortcut_on_random_fp32_sources():
    g = np.random.default_rng(1)
    for s in _scales(2)[::3]:
        x = (g.standard_normal(200_000) * g.uniform(0.5, 300) * s).astype(F32)
        x[:50] = (np.arange(50) - 25 + 0.5).astype(F32) * s  # quotients at half-integers
        want = _exact_codes(x, s)
        fast, slow = _fast_codes(x, s)
        assert np.array_equal(np.where(slow, want, fast), want), s


def test_special_values():
    s = F32(0.01)
    x = np.array([np.inf, -np.inf, np.nan, 3e38, -3e38, 1e-40, 0.0, -0.0], F32)
    fast, slow = _fast_codes(x, s)
    assert not slow.any()
    assert fast.tolist() == [127, -127, -127, 127, -127, 0, 0, 0]
    assert np.array_equal(fast, _exact_codes(x, s))
    assert np.array_equal(fast, _exact_codes(x, s, half_away=True))
    _, slow = _fast_codes(np.array([1.0, 2.0], F32), F32(2.0 ** 101))
    assert slow.all()  # reciprocal could be subnormal: always divide


def test_the_window_is_needed():
    """Without the window (keeping rint(qc) whenever |qc - n| < 0.5) some bf16 values and scales
    round differently from the divide: the window is what makes the shortcut exact."""
    x = _all_finite(torch.bfloat16)
    wrong = 0
    for s in _scales():
        r = (F32(1) / s).astype(F32)
        with np.errstate(over="ignore", invalid="ignore"):
            q0 = (x * r).astype(F32)
        n = np.rint(_clamp(q0, -127, 127))
        want = _exact_codes(x, s)
        wrong += int((n != want).sum())
    assert wrong > 0
