"""GPU test of the config-4 decode loop at its real workload.

Model: random-init Qwen2.5-7B shape (28 layers, hidden 3584, 28 q / 4 kv heads, head_dim 128,
FFN 18944, vocab 152064; 15.2 GB of bf16 weights).  B = 32 sequences of 8192 random prompt ids,
INT8 KV cache over all layers (7.6 GB), two eager decode steps, then two HIP-graph replays of
the same steps.  The reference measures this loop with (T128 - T1) / 127
(bench/benchmark_decode_tpot.py:64-68); here its results are checked:

* prefill: for layers 0, 13 and 27, 4096 seeded rows of the K/V the prefill wrote (of 262,144
  per layer) sit at the slots the block table names for their positions, bit-exact to the
  oracle's static quantisation of the values the model produced;
* decode steps: every row each step wrote (32 per layer, all 28 layers), likewise;
* each step's attention output for layers 0, 13 and 27 against the fp32 oracle over the cache
  at length position + 1, on sequences 0, 9, 22 and 31 (max-abs <= 2e-2, cos >= 0.9999);
* two graph replays from the post-prefill state equal the two eager steps bit for bit (logits
  and tokens), with eager work and synchronisations between the replays.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import MAX_ABS, MIN_COS, metrics
from int8kv import decode_loop as DL
from oracle import int8kv_oracle as O

pytestmark = pytest.mark.gpu

B, S, NEW, STEPS = 32, 8192, 4, 2
CHECK_LAYERS = (0, 13, 27)
CHECK_SEQS = (0, 9, 22, 31)
ROWS_PER_WRITE = 512  # sampled rows of each prefill write call (8 calls of 32,768 rows per layer)


class _Recorder:
    """Keeps samples of what the loop's cache writes and attention calls were given (eager)."""

    def __init__(self, loop):
        self.loop, self.prefill_rows, self.step_rows, self.attends = loop, [], [], []
        cache = loop.cache
        self._write, self._attend, self._rw = cache.write, cache.attend, cache.rotary_write
        gen = torch.Generator().manual_seed(17)
        shape = loop.shape

        calls = {}

        def write(layer, k, v, slots):
            if layer in CHECK_LAYERS:
                j = calls[layer] = calls.get(layer, -1) + 1  # prefill chunk index
                idx = torch.randperm(k.shape[0], generator=gen)[:ROWS_PER_WRITE]
                d = idx.to(k.device)
                self.prefill_rows.append((layer, k[d].clone(), v[d].clone(), slots[d].clone(), j, idx))
            self._write(layer, k, v, slots)

        def rotary_write(layer, qkv, positions, cos, sin, bt):
            self._rw(layer, qkv, positions, cos, sin, bt)
            _, k, v = DL._split_qkv(qkv, shape)  # k rotated in place by the fused kernel
            pos = positions.long()
            slots = bt.long().gather(1, (pos // 16).view(-1, 1)).view(-1) * 16 + pos % 16
            self.step_rows.append((layer, k.clone(), v.clone(), slots))

        def attend(layer, q, bt, sl, out, ws):
            r = self._attend(layer, q, bt, sl, out, ws)
            if layer in CHECK_LAYERS:
                self.attends.append((layer, q.clone(), sl.clone(), r.clone()))
            return r

        cache.write, cache.attend, cache.rotary_write = write, attend, rotary_write

    def detach(self):
        c = self.loop.cache
        c.write, c.attend, c.rotary_write = self._write, self._attend, self._rw


@pytest.fixture(scope="module")
def run(cuda):
    shape = DL.QWEN25_7B
    print(f"cfg4: building {shape}", flush=True)
    w = DL.random_weights(shape, cuda, seed=0)
    calib = torch.randint(0, shape.vocab, (4, 512), generator=torch.Generator().manual_seed(3))
    scales = DL.calibrate_static_scales(w, calib)
    prompt = torch.randint(0, shape.vocab, (B, S), generator=torch.Generator().manual_seed(7))
    loop = DL.DecodeLoop(w, B, S, NEW, "int8", scales=scales)
    rec = _Recorder(loop)
    loop.prefill(prompt)
    torch.cuda.synchronize()
    print("cfg4: prefill done", flush=True)
    after_prefill = loop.state()
    eager = []
    for _ in range(STEPS):
        loop.step_eager()
        eager.append((loop.logits.clone(), loop.tokens.clone()))
    torch.cuda.synchronize()
    rec.detach()
    print("cfg4: eager steps done", flush=True)
    yield loop, rec, after_prefill, eager
    del loop, w
    torch.cuda.empty_cache()


def _check_rows(loop, rows, what):
    shape = loop.shape
    Hkv, D = shape.kv_heads, shape.head_dim
    ks = loop.cache.k_scale.cpu().numpy()
    vs = loop.cache.v_scale.cpu().numpy()
    for layer, k, v, slots, *_ in rows:
        kc = loop.cache.key[layer].view(-1, Hkv, D)[slots].cpu().numpy()
        vc = loop.cache.value[layer].view(-1, Hkv, D)[slots].cpu().numpy()
        kq = O.quant_kv_static_per_head(k.float().cpu().numpy(), ks[layer][None, :, None])
        vq = O.quant_kv_static_per_head(v.float().cpu().numpy(), vs[layer][None, :, None])
        assert np.array_equal(kc, kq), f"{what}, layer {layer}: K rows differ from the oracle"
        assert np.array_equal(vc, vq), f"{what}, layer {layer}: V rows differ from the oracle"


def test_prefill_rows_at_table_slots_bit_exact(run):
    loop, rec, _, _ = run
    per_chunk = 32768 // S  # sequences per prefill chunk (DecodeLoop.prefill's chunk_tokens)
    assert len(rec.prefill_rows) == len(CHECK_LAYERS) * (B // per_chunk)
    bt = loop.block_tables.cpu().long()
    for layer, k, v, slots, chunk, idx in rec.prefill_rows:
        b = chunk * per_chunk + idx // S  # row r of a chunk is token r % S of its r // S-th sequence
        t = idx % S
        want = bt[b, t // 16] * 16 + t % 16
        assert torch.equal(slots.cpu().long(), want), f"layer {layer} chunk {chunk}: prefill slots"
    _check_rows(loop, rec.prefill_rows, "prefill")


def test_step_rows_at_table_slots_bit_exact(run):
    loop, rec, _, _ = run
    shape = loop.shape
    assert len(rec.step_rows) == STEPS * shape.layers
    bt = loop.block_tables.cpu().long()
    for i, (layer, k, v, slots) in enumerate(rec.step_rows):
        pos = S + i // shape.layers
        want = bt[:, pos // 16] * 16 + pos % 16
        assert torch.equal(slots.cpu(), want), f"step {i // shape.layers} layer {layer}: slots"
    _check_rows(loop, rec.step_rows, "decode step")


def test_step_attention_matches_oracle(run):
    loop, rec, _, _ = run
    assert len(rec.attends) == STEPS * len(CHECK_LAYERS)
    bt = loop.block_tables.cpu().numpy()
    ks = loop.cache.k_scale.cpu().numpy()
    vs = loop.cache.v_scale.cpu().numpy()
    caches = {l: (loop.cache.key[l].cpu().numpy(), loop.cache.value[l].cpu().numpy())
              for l in CHECK_LAYERS}
    seqs = list(CHECK_SEQS)
    for i, (layer, q, sl, out) in enumerate(rec.attends):
        step = i // len(CHECK_LAYERS)
        assert sl.cpu().tolist() == [S + 1 + step] * B
        kc, vc = caches[layer]
        ref = O.paged_attention_ref(q[seqs].float().cpu().numpy(), kc, vc, bt[seqs],
                                    np.full(len(seqs), S + 1 + step), ks[layer], vs[layer])
        err, cos, _ = metrics(out[seqs].float().cpu().numpy(), ref)
        print(f"step {step} layer {layer}: max|diff|={err:.2e} cos={cos:.7f}", flush=True)
        assert err <= MAX_ABS and cos >= MIN_COS, (step, layer, err, cos)


def test_graph_replays_equal_eager_steps(run):
    loop, _, after_prefill, eager = run
    loop.restore(after_prefill)
    loop.capture()
    for i in range(STEPS):
        loop.replay()
        torch.cuda.synchronize()
        _ = (loop.logits.float() * 2).sum().item()  # eager work between replays
        assert torch.equal(loop.logits, eager[i][0]), f"replay {i}: logits differ from the eager step"
        assert torch.equal(loop.tokens, eager[i][1]), f"replay {i}: tokens differ"
    assert loop.positions.cpu().tolist() == [S + STEPS] * B
