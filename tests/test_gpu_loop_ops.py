"""GPU tests of the decode loop's fused elementwise kernels against their unfused definitions.

* residual add: bit-exact (one bf16 rounding of the fp32 sum);
* rotary embedding: bit-exact to the fp32 rotate-half definition with separately rounded
  products and sum, evaluated in float64 on the CPU and rounded the same way; rows outside the
  position table and heads past ``num_heads`` are untouched;
* RMSNorm and SwiGLU: within one bf16 rounding step of a float64 evaluation (the fp32 sum order
  and the last bit of exp are implementation details).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from int8kv import decode_loop as DL

pytestmark = pytest.mark.gpu


def _bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |x| (2^(e-7)), for a tolerance of about one rounding step."""
    ax = x.abs().clamp_min(1e-30)
    return torch.exp2(torch.floor(torch.log2(ax)) - 7)


@pytest.mark.parametrize("rows,hidden", [(32, 3584), (3, 512), (5, 8192), (1, 8)])
@pytest.mark.parametrize("with_delta", [True, False])
def test_add_rms_norm(cuda, rows, hidden, with_delta):
    g = torch.Generator().manual_seed(rows * 7 + hidden)
    x = (torch.randn(rows, hidden, generator=g) * 3).to(torch.bfloat16)
    d = (torch.randn(rows, hidden, generator=g) * 2).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16)
    res = x.to(cuda)
    out = torch.empty_like(res)
    DL.hip_add_rms_norm(res, d.to(cuda) if with_delta else None, w.to(cuda), out, 1e-6)
    exp_res = (x.float() + d.float()).to(torch.bfloat16) if with_delta else x
    assert torch.equal(res.cpu(), exp_res)
    r64 = exp_res.double()
    xn = r64 / torch.sqrt((r64 * r64).mean(-1, keepdim=True) + 1e-6)
    ref = w.double() * xn
    err = (out.cpu().double() - ref).abs()
    # Two bf16 roundings (the normalised value, then the weighted output): one step of each.
    tol = 1.01 * (_bf16_ulp(xn) * w.double().abs() + _bf16_ulp(ref))
    assert (err <= tol).all(), float((err - tol).max())


def _rope_ref(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, pos: torch.Tensor, heads: int,
              D: int) -> torch.Tensor:
    """Rotate-half rotary with each fp32 product and the sum rounded separately (fp32 numpy)."""
    out = x.clone()
    half = D // 2
    xf = x.float().numpy()
    c = cos.numpy()
    s = sin.numpy()
    res = out.float().numpy()
    for r in range(x.shape[0]):
        p = int(pos[r])
        if p < 0 or p >= c.shape[0]:
            continue
        for h in range(heads):
            v = xf[r, h * D:(h + 1) * D]
            x1, x2 = v[:half], v[half:]
            o1 = np.float32(x1 * c[p, :half]) + np.float32(-x2 * s[p, :half])
            o2 = np.float32(x2 * c[p, half:]) + np.float32(x1 * s[p, half:])
            res[r, h * D:h * D + half] = o1
            res[r, h * D + half:(h + 1) * D] = o2
    ref = torch.from_numpy(res).to(torch.bfloat16)
    keep = torch.zeros_like(out, dtype=torch.bool)
    for r in range(x.shape[0]):
        p = int(pos[r])
        if p < 0 or p >= c.shape[0]:
            keep[r] = True
    keep[:, heads * D:] = True
    return torch.where(keep, out, ref)


def test_rotary_inplace_bit_exact(cuda):
    shape = DL.QWEN25_7B
    D = shape.head_dim
    cos, sin = DL.rope_tables(shape, 9000, "cpu")
    g = torch.Generator().manual_seed(3)
    rows = 37
    qkv = (torch.randn(rows, shape.qkv_width, generator=g) * 4).to(torch.bfloat16)
    pos = torch.randint(0, 9000, (rows,), generator=g)
    pos[0], pos[1], pos[2], pos[3] = 0, 8999, -1, 9000  # the last two are outside the table
    got = qkv.to(cuda)
    DL.hip_rotary_(got, shape.q_heads + shape.kv_heads, D, pos.to(cuda), cos.to(cuda), sin.to(cuda))
    ref = _rope_ref(qkv, cos, sin, pos, shape.q_heads + shape.kv_heads, D)
    assert torch.equal(got.cpu(), ref)
    assert torch.equal(got.cpu()[2], qkv[2]) and torch.equal(got.cpu()[3], qkv[3])
    # The same rotation through the unfused torch definition.
    heads = shape.q_heads + shape.kv_heads
    x = qkv[4:, : heads * D].view(rows - 4, 1, heads, D)
    unfused = DL.apply_rope(x, cos[pos[4:]].view(rows - 4, 1, D), sin[pos[4:]].view(rows - 4, 1, D))
    assert torch.equal(got.cpu()[4:, : heads * D], unfused.reshape(rows - 4, heads * D))


@pytest.mark.parametrize("rows,ffn", [(32, 18944), (3, 1024), (1, 8)])
def test_silu_mul(cuda, rows, ffn):
    g = torch.Generator().manual_seed(ffn + rows)
    gu = (torch.randn(rows, 2 * ffn, generator=g) * 4).to(torch.bfloat16)
    gu[0, :4] = torch.tensor([-100.0, 100.0, 0.0, -0.0]).to(torch.bfloat16)  # saturating and zero gates
    out = torch.empty(rows, ffn, dtype=torch.bfloat16, device=cuda)
    DL.hip_silu_mul(gu.to(cuda), out)
    gate, up = gu[:, :ffn].double(), gu[:, ffn:].double()
    silu = (gate / (1 + torch.exp(-gate))).to(torch.bfloat16).double()
    ref = silu * up
    err = (out.cpu().double() - ref).abs()
    tol = 1.01 * (_bf16_ulp(ref) + _bf16_ulp(silu) * up.abs())
    assert (err <= tol).all(), float(err.max())
    unfused = torch.nn.functional.silu(gu[:, :ffn].to(cuda)) * gu[:, ffn:].to(cuda)
    assert (out.float() - unfused.float()).abs().max().item() <= float(tol.max())


def test_strided_rows(cuda):
    """Row strides larger than the row (views into wider buffers) are honoured."""
    g = torch.Generator().manual_seed(9)
    big = (torch.randn(6, 640, generator=g)).to(torch.bfloat16).to(cuda)
    res = big[:, :512]
    d = big[:, 64:576].clone()
    w = torch.ones(512, dtype=torch.bfloat16, device=cuda)
    out_big = torch.zeros(6, 520, dtype=torch.bfloat16, device=cuda)
    before = big.clone()
    DL.hip_add_rms_norm(res, d, w, out_big[:, :512], 1e-6)
    assert torch.equal(big[:, 512:], before[:, 512:])
    assert torch.equal(out_big[:, 512:], torch.zeros(6, 8, dtype=torch.bfloat16, device=cuda))
    assert torch.equal(res, (before[:, :512].float() + d.float()).to(torch.bfloat16))
