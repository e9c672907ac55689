"""GPU tests of the config-4 decode loop (int8kv.decode_loop) on a small model of the same head layout.

What is checked, each against something independent of the loop's own code:
* every K/V row the loop writes (prefill and decode steps) lands in the slot the block table
  names for its position, bit-exact to the oracle's static quantisation, and nothing else in the
  cache changes;
* each decode step's attention equals the fp32 oracle over the cache at length position + 1;
* a decode step's logits agree with an fp32 torch restatement of the model (dense attention over
  the dequantised cache);
* HIP-graph replays reproduce eager steps exactly (logits and tokens, every replay checked,
  with eager work and synchronisations between replays);
* the INT8 and BF16 cache modes agree to quantisation noise.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import MAX_ABS, MIN_COS, metrics
from int8kv import decode_loop as DL
from oracle import int8kv_oracle as O

pytestmark = pytest.mark.gpu

SHAPE = DL.QwenShape(hidden=512, layers=2, q_heads=28, kv_heads=4, head_dim=128, ffn=1024, vocab=2048)
B, S, NEW = 3, 21, 6


@pytest.fixture(scope="module")
def model(cuda):
    w = DL.random_weights(SHAPE, cuda, seed=0)
    g = torch.Generator().manual_seed(5)
    calib = torch.randint(0, SHAPE.vocab, (2, 48), generator=g)
    scales = DL.calibrate_static_scales(w, calib)
    prompt = torch.randint(0, SHAPE.vocab, (B, S), generator=g)
    return w, scales, prompt


class _Recorder:
    """Wraps PagedKVCache.write / attend of one loop to keep what they were given (eager only)."""

    def __init__(self, loop):
        self.loop, self.writes, self.attends = loop, [], []
        cache = loop.cache
        self._write, self._attend, self._rw = cache.write, cache.attend, cache.rotary_write

        def write(layer, k, v, slots):
            self.writes.append((layer, k.detach().clone(), v.detach().clone(), slots.detach().clone()))
            self._write(layer, k, v, slots)

        def rotary_write(layer, qkv, positions, cos, sin, bt):
            # The decode step's fused rotary + write: record the rotated k (left in qkv) and v
            # with the slots of the rows' positions, as an unfused write would have received.
            self._rw(layer, qkv, positions, cos, sin, bt)
            _, k, v = DL._split_qkv(qkv, SHAPE)
            pos = positions.long()
            slots = bt.long().gather(1, (pos // 16).view(-1, 1)).view(-1) * 16 + pos % 16
            self.writes.append((layer, k.detach().clone(), v.detach().clone(), slots.detach().clone()))

        def attend(layer, q, bt, sl, out, ws):
            r = self._attend(layer, q, bt, sl, out, ws)
            self.attends.append((layer, q.detach().clone(), sl.detach().clone(), r.detach().clone()))
            return r

        cache.write, cache.attend, cache.rotary_write = write, attend, rotary_write

    def detach(self):
        c = self.loop.cache
        c.write, c.attend, c.rotary_write = self._write, self._attend, self._rw


def _make(model, mode):
    w, scales, _ = model
    return DL.DecodeLoop(w, B, S, NEW, mode, scales=scales if mode == "int8" else None)


def _expected_slots(loop, positions):
    bt = loop.block_tables.cpu().to(torch.int64)
    return torch.stack([bt[b, p // 16] * 16 + p % 16 for b, p in enumerate(positions)])


def _check_writes(loop, writes):
    """Each recorded write is in the cache, bit-exact; every other row is still zero."""
    Hkv, D = SHAPE.kv_heads, SHAPE.head_dim
    ks = loop.cache.k_scale.cpu().numpy()
    vs = loop.cache.v_scale.cpu().numpy()
    written = [set() for _ in range(SHAPE.layers)]
    for layer, k, v, slots in writes:
        kc = loop.cache.key[layer].view(-1, Hkv, D)[slots].cpu().numpy()
        vc = loop.cache.value[layer].view(-1, Hkv, D)[slots].cpu().numpy()
        kq = O.quant_kv_static_per_head(k.float().cpu().numpy(), ks[layer][None, :, None])
        vq = O.quant_kv_static_per_head(v.float().cpu().numpy(), vs[layer][None, :, None])
        assert np.array_equal(kc, kq) and np.array_equal(vc, vq), f"layer {layer}: cache != oracle quant"
        written[layer].update(slots.cpu().tolist())
    for layer in range(SHAPE.layers):
        rows = loop.cache.key[layer].view(-1, Hkv * D).cpu()
        mask = torch.ones(rows.shape[0], dtype=torch.bool)
        mask[list(written[layer])] = False
        assert not rows[mask].any(), f"layer {layer}: rows outside the written slots changed"


def test_caches_written_at_table_slots_bit_exact(model):
    loop = _make(model, "int8")
    rec = _Recorder(loop)
    loop.prefill(model[2])
    torch.cuda.synchronize()
    prompt_slots = loop.prefill_slots(slice(0, B)).cpu()
    for layer, _, _, slots in rec.writes:
        assert torch.equal(slots.cpu(), prompt_slots)
    n_prefill = len(rec.writes)
    assert n_prefill == SHAPE.layers
    for step in range(3):
        loop.step_eager()
        torch.cuda.synchronize()
        exp = _expected_slots(loop, [S + step] * B)
        for _, _, _, slots in rec.writes[n_prefill + step * SHAPE.layers:]:
            assert torch.equal(slots.cpu(), exp), f"step {step}: slots {slots.tolist()} != {exp.tolist()}"
    rec.detach()
    _check_writes(loop, rec.writes)
    assert loop.positions.cpu().tolist() == [S + 3] * B
    assert loop.seq_lens.cpu().tolist() == [S + 4] * B


def test_step_attention_matches_oracle(model):
    loop = _make(model, "int8")
    loop.prefill(model[2])
    rec = _Recorder(loop)
    for step in range(2):
        loop.step_eager()
    torch.cuda.synchronize()
    rec.detach()
    kc = loop.cache.key.cpu().numpy()
    vc = loop.cache.value.cpu().numpy()
    ks = loop.cache.k_scale.cpu().numpy()
    vs = loop.cache.v_scale.cpu().numpy()
    bt = loop.block_tables.cpu().numpy()
    for i, (layer, q, sl, out) in enumerate(rec.attends):
        step = i // SHAPE.layers
        assert sl.cpu().tolist() == [S + 1 + step] * B
        ref = O.paged_attention_ref(q.float().cpu().numpy(), kc[layer], vc[layer], bt,
                                    np.full(B, S + 1 + step), ks[layer], vs[layer])
        err, cos, _ = metrics(out.float().cpu().numpy(), ref)
        assert err <= MAX_ABS and cos >= MIN_COS, f"step {step} layer {layer}: {err} {cos}"


def _fp32_step_logits(loop, tokens, pos):
    """fp32 restatement of one decode step over the (already written) int8 cache."""
    w, sh = loop.w, SHAPE
    Hq, Hkv, D = sh.q_heads, sh.kv_heads, sh.head_dim
    G = Hq // Hkv
    dev = loop.dev

    def rms(x, wt):
        return wt.float() * (x * torch.rsqrt((x * x).mean(-1, keepdim=True) + sh.rms_eps))

    half = D // 2
    inv = 1.0 / (sh.rope_theta ** (torch.arange(half, dtype=torch.float64) * 2.0 / D))
    ang = torch.tensor(pos, dtype=torch.float64)[:, None] * inv[None, :]
    cos = torch.cat([ang.cos(), ang.cos()], 1).float().to(dev)[:, None, :]
    sin = torch.cat([ang.sin(), ang.sin()], 1).float().to(dev)[:, None, :]

    def rope(x):
        return x * cos + torch.cat([-x[..., half:], x[..., :half]], -1) * sin

    bt = loop.block_tables.to(torch.int64)
    x = w.embed.float()[tokens]
    k0 = None
    for l, lw in enumerate(w.layers):
        h = rms(x, lw.ln1)
        qkv = h @ lw.wqkv.float().t() + lw.bqkv.float()
        q = rope(qkv[:, : Hq * D].reshape(-1, Hq, D))
        if l == 0:
            k0 = rope(qkv[:, Hq * D:(Hq + Hkv) * D].reshape(-1, Hkv, D))
        outs = []
        for b in range(len(tokens)):
            n = pos[b] + 1
            t = torch.arange(n, device=dev)
            rows = bt[b, t // 16] * 16 + t % 16
            kk = loop.cache.key[l].view(-1, Hkv, D)[rows].float() * loop.cache.k_scale[l][None, :, None]
            vv = loop.cache.value[l].view(-1, Hkv, D)[rows].float() * loop.cache.v_scale[l][None, :, None]
            o = []
            for hq in range(Hq):
                s = (kk[:, hq // G, :] @ q[b, hq]) / np.sqrt(D)
                o.append(torch.softmax(s, 0) @ vv[:, hq // G, :])
            outs.append(torch.stack(o))
        attn = torch.stack(outs).reshape(len(tokens), Hq * D)
        x = x + attn @ lw.wo.float().t()
        h = rms(x, lw.ln2)
        gu = h @ lw.w_gate_up.float().t()
        x = x + (torch.nn.functional.silu(gu[:, : sh.ffn]) * gu[:, sh.ffn:]) @ lw.w_down.float().t()
    return rms(x, w.ln_f) @ w.lm_head.float().t(), k0


def test_step_logits_match_fp32_model(model):
    loop = _make(model, "int8")
    loop.prefill(model[2])
    tokens = loop.tokens.clone()
    rec = _Recorder(loop)
    loop.step_eager()
    torch.cuda.synchronize()
    rec.detach()
    ref, k0 = _fp32_step_logits(loop, tokens, [S] * B)
    err, cos, _ = metrics(rec.writes[0][1].float().cpu().numpy(), k0.cpu().numpy())
    assert cos >= 0.9999, f"layer-0 post-rotary k: cos {cos} (position or rotary mismatch)"
    err, cos, rel = metrics(loop.logits.float().cpu().numpy(), ref.cpu().numpy())
    print(f"logits vs fp32 model: max|diff|={err:.3e} cos={cos:.6f} rel={rel:.3e}", flush=True)
    assert cos >= 0.999 and rel <= 0.05


@pytest.mark.parametrize("mode", DL.MODES)
def test_graph_replays_match_eager(model, mode):
    loop = _make(model, mode)
    loop.prefill(model[2])
    saved = loop.state()
    eager = []
    for _ in range(4):
        loop.step_eager()
        eager.append((loop.logits.clone(), loop.tokens.clone()))
    gen_eager = loop.generated.clone()
    torch.cuda.synchronize()
    loop.restore(saved)
    loop.capture()
    for i in range(4):
        loop.replay()
        torch.cuda.synchronize()
        _ = (loop.logits.float() * 2).sum().item()  # eager work between replays
        assert torch.equal(loop.logits, eager[i][0]), f"replay {i}: logits differ from the eager step"
        assert torch.equal(loop.tokens, eager[i][1]), f"replay {i}: tokens differ"
    assert torch.equal(loop.generated, gen_eager)
    assert loop.positions.cpu().tolist() == [S + 4] * B


def test_int8_and_bf16_modes_agree(model):
    a = _make(model, "int8")
    b = _make(model, "bf16")
    fa = a.prefill(model[2])
    fb = b.prefill(model[2])
    _, cos, _ = metrics(a.prefill_logits.float().cpu().numpy(), b.prefill_logits.float().cpu().numpy())
    assert cos >= 0.99999
    assert torch.equal(fa, fb)
    a.step_eager()
    b.step_eager()
    torch.cuda.synchronize()
    _, cos, rel = metrics(a.logits.float().cpu().numpy(), b.logits.float().cpu().numpy())
    print(f"int8 vs bf16 step logits: cos={cos:.6f} rel={rel:.3e}", flush=True)
    assert cos >= 0.999
    # The bf16 cache holds the prompt's K exactly as computed; the int8 cache is its quantisation.
    Hkv, D = SHAPE.kv_heads, SHAPE.head_dim
    slots = a.prefill_slots(slice(0, B))
    for l in range(SHAPE.layers):
        kb = b.cache.key[l].view(-1, Hkv, D)[slots].float().cpu().numpy()
        ki = a.cache.key[l].view(-1, Hkv, D)[slots].cpu().numpy()
        deq = ki.astype(np.float32) * a.cache.k_scale[l].cpu().numpy()[None, :, None]
        step = a.cache.k_scale[l].cpu().numpy()[None, :, None]
        assert (np.abs(deq - np.clip(kb, -127 * step, 127 * step)) <= 0.5 * step * 1.0001).all()


@pytest.mark.parametrize("mode", DL.MODES)
def test_fused_step_matches_unfused(model, mode, monkeypatch):
    """The decode step with the fused kernels (rotary + cache write in one launch, the library
    argmax) equals the unfused sequence (rotary kernel, slot arithmetic, cache write, torch
    argmax) bit for bit: logits, greedy tokens and every layer's K/V cache over three steps."""
    loops = {}
    for fused in (True, False):
        monkeypatch.setattr(DL, "FUSED_STEP", fused)
        loop = _make(model, mode)
        loop.prefill(model[2])
        steps = []
        for _ in range(3):
            loop.step_eager()
            steps.append((loop.logits.clone(), loop.tokens.clone()))
        torch.cuda.synchronize()
        loops[fused] = (loop, steps)
    (a, sa), (b, sb) = loops[True], loops[False]
    for i, ((la, ta), (lb, tb)) in enumerate(zip(sa, sb)):
        assert torch.equal(la, lb), f"step {i}: logits differ"
        assert torch.equal(ta, tb), f"step {i}: tokens differ"
    for l in range(SHAPE.layers):
        assert torch.equal(a.cache.key[l], b.cache.key[l]), f"layer {l}: key cache differs"
        assert torch.equal(a.cache.value[l], b.cache.value[l]), f"layer {l}: value cache differs"
    assert torch.equal(a.generated, b.generated)
