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


@pytest.mark.parametrize("mode", ["int8", "bf16"])
def test_rotary_cache_write_matches_unfused(cuda, mode):
    """The fused rotary + cache write equals the rotary kernel followed by the cache write
    (int8_kv_cache_write, or a bf16 scatter) bit for bit: the qkv rows and both caches.  Rows
    with a position outside the rotary table, or a negative block id, write nothing."""
    from int8kv import int8_kv_cache_write

    shape = DL.QwenShape(hidden=64, layers=1, q_heads=8, kv_heads=2, head_dim=128, ffn=64, vocab=16)
    B, width, nb = 9, 6, 60
    g = torch.Generator().manual_seed(5 if mode == "int8" else 6)
    qkv = (torch.randn(B, shape.qkv_width, generator=g) * 2).to(torch.bfloat16).to(cuda)
    pos = torch.randint(0, width * 16, (B,), generator=g)
    pos[3] = 10_000  # beyond the rotary table: untouched, nothing written
    bt = torch.randperm(nb, generator=g)[: B * width].view(B, width).to(torch.int32)
    bt[5, pos[5] // 16] = -1  # a negative block id: the row is rotated, its cache write skipped
    cos, sin = DL.rope_tables(shape, width * 16, cuda)
    dtype = torch.int8 if mode == "int8" else torch.bfloat16
    kc = torch.randint(-100, 100, (nb, 16, 2, 128), generator=g).to(dtype).to(cuda)
    vc = torch.randint(-100, 100, (nb, 16, 2, 128), generator=g).to(dtype).to(cuda)
    ks = torch.tensor([0.02, 0.05], device=cuda)
    vs = torch.tensor([0.03, 0.01], device=cuda)
    pos_d, bt_d = pos.to(cuda), bt.to(cuda)

    ref_qkv, ref_k, ref_v = qkv.clone(), kc.clone(), vc.clone()
    DL.hip_rotary_(ref_qkv, shape.q_heads + shape.kv_heads, 128, pos_d, cos, sin)
    q, k, v = DL._split_qkv(ref_qkv, shape)
    ok = (pos < width * 16) & (bt[torch.arange(B), (pos // 16).clamp(max=width - 1)] >= 0)
    rows = torch.nonzero(ok).view(-1)
    slots = (bt[rows, pos[rows] // 16].long() * 16 + pos[rows] % 16).to(cuda)
    if mode == "int8":
        int8_kv_cache_write(k[rows.to(cuda)], v[rows.to(cuda)], ref_k, ref_v, slots, ks, vs)
    else:
        ref_k.view(-1, 2, 128).index_copy_(0, slots, k[rows.to(cuda)].contiguous())
        ref_v.view(-1, 2, 128).index_copy_(0, slots, v[rows.to(cuda)].contiguous())

    DL.hip_rotary_cache_write_(qkv, shape, pos_d, cos, sin, bt_d, kc, vc,
                               ks if mode == "int8" else None, vs if mode == "int8" else None)
    torch.cuda.synchronize()
    assert torch.equal(qkv, ref_qkv)
    assert torch.equal(kc, ref_k) and torch.equal(vc, ref_v)


def test_argmax_rows_matches_torch(cuda):
    """First maximum per row, as torch.argmax on the same device: ties, -inf rows, a NaN."""
    g = torch.Generator().manual_seed(9)
    x = torch.randn(12, 152064, generator=g).to(torch.bfloat16)
    x[1, 1000] = x[1, 99_000] = 50.0  # tie: the lower index wins
    x[2, :] = -float("inf")
    x[3, 77] = float("inf")
    x[4, 5] = x[4, 6] = float("inf")
    x[5, 123_456] = float("nan")
    x[6, :] = 1.0  # all equal
    x[7, 152_058] = 70.0  # the maximum in the last, partial 8-element piece of a shortened row
    x[8, 3] = x[8, 152_059] = 80.0  # a tie between a 16-byte piece and that partial piece
    x[9, 500] = x[9, 20] = float("nan")  # two NaNs: the first one
    xd = x.to(cuda)
    out = torch.empty(12, dtype=torch.int64, device=cuda)
    DL.hip_argmax_rows(xd, out)
    view = xd[:, 1:-3]  # misaligned rows, row stride above the row length: 2-byte loads
    out2 = torch.empty(12, dtype=torch.int64, device=cuda)
    DL.hip_argmax_rows(view, out2)
    short = xd[:, :152_061]  # aligned rows with a 5-element remainder after the 16-byte loads
    out3 = torch.empty(12, dtype=torch.int64, device=cuda)
    DL.hip_argmax_rows(short, out3)
    torch.cuda.synchronize()
    assert torch.equal(out, xd.argmax(-1))
    assert torch.equal(out2, view.argmax(-1))
    assert torch.equal(out3, short.argmax(-1))
    assert out[1].item() == 1000 and out[6].item() == 0 and out[4].item() == 5
    assert out3[7].item() == 152_058 and out3[8].item() == 3 and out[9].item() == 20
