"""Greedy decode loop of a random-init Qwen2.5-7B-shaped model whose attention runs on libint8kv.

This is the caller one step above the operators, in the role the reference gives vLLM plus its
patches (bench/run_qwen_case_final.py, vllm_int8/vllm_shadow_cache_patch.py,
vllm_int8/vllm_int8_attention_patch.py in "int8_only" mode):

* prefill runs the whole prompt through the model with torch GEMMs and torch SDPA on the
  unquantised bf16 K/V, and writes every layer's K/V into the paged caches: with static per-head
  INT8 scales through ``int8kv_cache_write`` (mode "int8"), or as bf16 (mode "bf16");
* every decode step appends one token per sequence to the caches (the same HIP write, or a bf16
  scatter) and attends with ``int8kv_paged_decode`` over the INT8 or the BF16 cache;
* a decode step is one HIP graph: the sequence state (next token, position, length, slot) lives
  in device buffers updated inside the graph, so a replay is one step with no host work.

Model (Qwen2 architecture, random weights, no checkpoint): token embedding; per layer RMSNorm,
QKV projection with bias, rotary embedding (rotate-half form, theta 1e6), GQA attention
(28 query heads over 4 kv heads, head_dim 128, scale 1/sqrt(128)), output projection, residual,
RMSNorm, SwiGLU MLP (18944), residual; final RMSNorm; untied LM head over 152064 tokens; greedy
argmax.  The shape is README.md:198-207 of the reference.

Static scales follow scripts/04_calibrate_static_scale.py:26-56 of the reference: absmax/127 of
the post-rotary K and of V per (layer, kv head) over separate calibration sequences, floored
at 1e-6.

Timing follows bench/benchmark_decode_tpot.py:64-68 of the reference: T1 = prefill plus the
first token, T128 = T1 plus 127 decode steps, TPOT = (T128 - T1) / 127.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field
from pathlib import Path

import torch
import torch.nn.functional as F

from . import _decode, _lib
from .int8_cache_write import int8_kv_cache_write


@dataclass(frozen=True)
class QwenShape:
    hidden: int = 3584
    layers: int = 28
    q_heads: int = 28
    kv_heads: int = 4
    head_dim: int = 128
    ffn: int = 18944
    vocab: int = 152064
    rope_theta: float = 1.0e6
    rms_eps: float = 1.0e-6

    @property
    def qkv_width(self) -> int:
        return (self.q_heads + 2 * self.kv_heads) * self.head_dim


QWEN25_7B = QwenShape()
BLOCK_SIZE = 16
# Decode step with the fused kernels (rotary + cache write in one launch, the HIP argmax); False
# runs the unfused sequence (rotary, slot arithmetic, cache write, torch argmax) for comparison.
FUSED_STEP = True
MODES = ("int8", "bf16")

# hipBLASLt solutions chosen by torch's TunableOp for the decode step's GEMMs (M = batch rows)
# on MI355X; written by ``configure_gemm_tuning("tune", ...)`` and read back with "use".
GEMM_TUNING_FILE = Path(__file__).resolve().parent / "gemm_tuning_mi355x.csv"
GEMM_TUNING_MODES = ("off", "use", "tune")


def configure_gemm_tuning(mode: str, path: Path | str = GEMM_TUNING_FILE) -> bool:
    """Selects how the decode loop's torch GEMMs pick their hipBLASLt/rocBLAS solutions.

    "off": torch's default heuristics.  "use": TunableOp with the solutions recorded in ``path``
    (shapes not in the file keep the default; nothing is tuned).  "tune": TunableOp tunes each
    new GEMM shape the first time it runs eagerly (``DecodeLoop`` tunes only during the decode
    warm-up step) against a 1 GB rotating buffer, so the timings see cold weights as the model
    does; the results are written to ``path`` when the process exits.  A file whose validators
    (torch, HIP, hipBLASLt, rocBLAS versions, GPU arch) do not match is ignored by torch.
    Returns whether TunableOp is on.
    """
    import torch.cuda.tunable as tunable

    if mode not in GEMM_TUNING_MODES:
        raise ValueError(f"gemm tuning mode must be one of {GEMM_TUNING_MODES}, got {mode!r}")
    if mode == "off":
        tunable.enable(False)
        return False
    path = Path(path)
    tunable.enable(True)
    tunable.tuning_enable(False)
    tunable.set_filename(str(path), insert_device_ordinal=False)
    if mode == "tune":
        tunable.set_rotating_buffer_size(1024)
        tunable.set_max_tuning_duration(100)
    if path.exists():
        tunable.read_file(str(path))
    _TUNING["tune"] = mode == "tune"
    return True


_TUNING = {"tune": False}


def blocks_per_sequence(max_len: int, block_size: int = BLOCK_SIZE) -> int:
    return -(-max_len // block_size)


def kv_cache_bytes(shape: QwenShape, num_blocks: int, mode: str, block_size: int = BLOCK_SIZE) -> dict:
    """Bytes of the paged K+V caches of all layers (and of the INT8 scales)."""
    elems = 2 * shape.layers * num_blocks * block_size * shape.kv_heads * shape.head_dim
    if mode == "int8":
        return {"kv_bytes": elems, "scale_bytes": 2 * shape.layers * shape.kv_heads * 4}
    if mode == "bf16":
        return {"kv_bytes": 2 * elems, "scale_bytes": 0}
    raise ValueError(f"mode must be one of {MODES}, got {mode!r}")


def rope_tables(shape: QwenShape, max_len: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [max_len, head_dim] float32 of the rotate-half rotary embedding."""
    half = shape.head_dim // 2
    inv_freq = 1.0 / (shape.rope_theta ** (torch.arange(half, dtype=torch.float64) * 2.0 / shape.head_dim))
    ang = torch.arange(max_len, dtype=torch.float64)[:, None] * inv_freq[None, :]
    ang = torch.cat([ang, ang], dim=1)
    return ang.cos().float().to(device), ang.sin().float().to(device)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [..., T, H, D] (any float) with cos/sin [T, D] -> rotated, in x's dtype (fp32 math)."""
    xf = x.float()
    half = xf.shape[-1] // 2
    rot = torch.cat([-xf[..., half:], xf[..., :half]], dim=-1)
    c = cos.unsqueeze(-2)
    s = sin.unsqueeze(-2)
    return (xf * c + rot * s).to(x.dtype)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return weight * xf.to(x.dtype)


def _bf16_rows(t: torch.Tensor, what: str) -> None:
    if t.dtype != torch.bfloat16 or t.dim() != 2 or t.stride(-1) != 1 or not t.is_cuda:
        raise ValueError(f"{what}: expected a CUDA bf16 [rows, n] tensor with unit inner stride")


def hip_add_rms_norm(residual: torch.Tensor, delta: torch.Tensor | None, weight: torch.Tensor,
                     out: torch.Tensor, eps: float) -> torch.Tensor:
    """residual += delta (bf16, in place, skipped when delta is None); out = RMSNorm(residual)."""
    _bf16_rows(residual, "residual")
    _bf16_rows(out, "out")
    if delta is not None:
        _bf16_rows(delta, "delta")
        assert delta.shape == residual.shape
    assert out.shape == residual.shape and weight.is_contiguous() and weight.dtype == torch.bfloat16
    rows, hidden = residual.shape
    status = _lib.load().int8kv_add_rms_norm(
        residual.data_ptr(), None if delta is None else delta.data_ptr(), weight.data_ptr(),
        out.data_ptr(), rows, hidden, residual.stride(0), 0 if delta is None else delta.stride(0),
        out.stride(0), eps, _lib.stream_handle(residual.device))
    _lib.check(status, "int8kv_add_rms_norm")
    return out


def hip_rotary_(qkv: torch.Tensor, num_heads: int, head_dim: int, positions: torch.Tensor,
                cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotates the first ``num_heads`` heads of every row of qkv [rows, width] in place."""
    _bf16_rows(qkv, "qkv")
    assert positions.dtype == torch.int64 and positions.is_contiguous()
    assert positions.numel() == qkv.shape[0]
    assert cos.dtype == sin.dtype == torch.float32 and cos.is_contiguous() and sin.is_contiguous()
    assert cos.shape == sin.shape and cos.shape[1] == head_dim
    status = _lib.load().int8kv_rotary_inplace(
        qkv.data_ptr(), qkv.shape[0], qkv.stride(0), num_heads, head_dim, positions.data_ptr(),
        cos.data_ptr(), sin.data_ptr(), cos.shape[0], _lib.stream_handle(qkv.device))
    _lib.check(status, "int8kv_rotary_inplace")
    return qkv


def hip_rotary_cache_write_(qkv: torch.Tensor, shape: QwenShape, positions: torch.Tensor,
                            cos: torch.Tensor, sin: torch.Tensor, block_tables: torch.Tensor,
                            key_cache: torch.Tensor, value_cache: torch.Tensor,
                            k_scale: torch.Tensor | None, v_scale: torch.Tensor | None) -> torch.Tensor:
    """Rotates the q and k heads of every qkv row in place and writes the row's k and v to the
    paged caches at its position's slot (one decode token per row; the fused form of
    ``hip_rotary_`` followed by the cache write, with the same results)."""
    _bf16_rows(qkv, "qkv")
    assert positions.dtype == torch.int64 and positions.is_contiguous()
    assert positions.numel() == qkv.shape[0] == block_tables.shape[0]
    assert block_tables.dtype == torch.int32 and block_tables.stride(1) == 1
    assert cos.dtype == sin.dtype == torch.float32 and cos.is_contiguous() and sin.is_contiguous()
    assert cos.shape == sin.shape and cos.shape[1] == shape.head_dim
    int8 = key_cache.dtype == torch.int8
    assert key_cache.dtype == value_cache.dtype and (int8 or key_cache.dtype == torch.bfloat16)
    num_blocks, block_size = key_cache.shape[0], key_cache.shape[1]
    status = _lib.load().int8kv_rotary_cache_write(
        qkv.data_ptr(), qkv.shape[0], qkv.stride(0), shape.q_heads, shape.kv_heads, shape.head_dim,
        positions.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.shape[0], block_tables.data_ptr(),
        block_tables.shape[1], block_tables.stride(0), num_blocks, block_size,
        _lib.I8 if int8 else _lib.BF16, key_cache.data_ptr(), value_cache.data_ptr(),
        _lib.strides(key_cache), _lib.strides(value_cache),
        k_scale.data_ptr() if int8 else None, v_scale.data_ptr() if int8 else None,
        _lib.stream_handle(qkv.device))
    _lib.check(status, "int8kv_rotary_cache_write")
    return qkv


def hip_argmax_rows(logits: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out[r] = argmax(logits[r]) (int64, first maximum; bf16 logits [rows, vocab])."""
    assert logits.dtype == torch.bfloat16 and logits.stride(1) == 1
    assert out.dtype == torch.int64 and out.is_contiguous() and out.numel() == logits.shape[0]
    status = _lib.load().int8kv_argmax_rows(logits.data_ptr(), logits.shape[0], logits.shape[1],
                                            logits.stride(0), out.data_ptr(),
                                            _lib.stream_handle(logits.device))
    _lib.check(status, "int8kv_argmax_rows")
    return out


def hip_silu_mul(gate_up: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out = silu(gate_up[:, :ffn]) * gate_up[:, ffn:] (bf16)."""
    _bf16_rows(gate_up, "gate_up")
    _bf16_rows(out, "out")
    rows, ffn = out.shape
    assert gate_up.shape == (rows, 2 * ffn)
    status = _lib.load().int8kv_silu_mul(gate_up.data_ptr(), out.data_ptr(), rows, ffn,
                                         gate_up.stride(0), out.stride(0),
                                         _lib.stream_handle(gate_up.device))
    _lib.check(status, "int8kv_silu_mul")
    return out


@dataclass
class LayerWeights:
    ln1: torch.Tensor
    wqkv: torch.Tensor  # [qkv_width, hidden]
    bqkv: torch.Tensor  # [qkv_width]
    wo: torch.Tensor  # [hidden, q_heads * head_dim]
    ln2: torch.Tensor
    w_gate_up: torch.Tensor  # [2 * ffn, hidden]
    w_down: torch.Tensor  # [hidden, ffn]


@dataclass
class ModelWeights:
    shape: QwenShape
    embed: torch.Tensor  # [vocab, hidden]
    layers: list = field(default_factory=list)
    ln_f: torch.Tensor | None = None
    lm_head: torch.Tensor | None = None  # [vocab, hidden]

    def nbytes(self) -> int:
        ts = [self.embed, self.ln_f, self.lm_head]
        for lw in self.layers:
            ts += [lw.ln1, lw.wqkv, lw.bqkv, lw.wo, lw.ln2, lw.w_gate_up, lw.w_down]
        return sum(t.numel() * t.element_size() for t in ts)


def random_weights(shape: QwenShape, device, seed: int = 0, std: float = 0.02,
                   dtype=torch.bfloat16) -> ModelWeights:
    """Seeded N(0, std) weights (norm weights 1) of the given shape, generated on ``device``."""
    g = torch.Generator(device=device).manual_seed(seed)

    def normal(*size):
        return torch.empty(*size, dtype=dtype, device=device).normal_(0.0, std, generator=g)

    def ones(n):
        return torch.ones(n, dtype=dtype, device=device)

    H, D = shape.hidden, shape.head_dim
    w = ModelWeights(shape=shape, embed=normal(shape.vocab, H))
    for _ in range(shape.layers):
        w.layers.append(LayerWeights(
            ln1=ones(H),
            wqkv=normal(shape.qkv_width, H),
            bqkv=normal(shape.qkv_width),
            wo=normal(H, shape.q_heads * D),
            ln2=ones(H),
            w_gate_up=normal(2 * shape.ffn, H),
            w_down=normal(H, shape.ffn),
        ))
    w.ln_f = ones(H)
    w.lm_head = normal(shape.vocab, H)
    return w


def prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Causal GQA attention over [c, H, S, D] bf16 with torch SDPA (flash / memory-efficient).

    The math backend is excluded on purpose: in bf16 it runs batched products on transposed
    views, which this platform does not run reliably.
    """
    from torch.nn.attention import SDPBackend, sdpa_kernel

    group = q.shape[1] // k.shape[1]
    k = k.repeat_interleave(group, dim=1)
    v = v.repeat_interleave(group, dim=1)
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        return F.scaled_dot_product_attention(q, k, v, is_causal=True)


def _split_qkv(qkv: torch.Tensor, shape: QwenShape):
    Hq, Hkv, D = shape.q_heads, shape.kv_heads, shape.head_dim
    lead = qkv.shape[:-1]
    q = qkv[..., : Hq * D].unflatten(-1, (Hq, D))
    k = qkv[..., Hq * D:(Hq + Hkv) * D].unflatten(-1, (Hkv, D))
    v = qkv[..., (Hq + Hkv) * D:].unflatten(-1, (Hkv, D))
    assert q.shape[:-2] == lead
    return q, k, v


class PagedKVCache:
    """Paged K/V caches of every layer: [L, num_blocks, 16, Hkv, D] int8 (+ scales) or bf16."""

    def __init__(self, shape: QwenShape, num_blocks: int, mode: str, device,
                 k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None):
        if mode not in MODES:
            raise ValueError(f"mode must be one of {MODES}, got {mode!r}")
        self.shape, self.mode, self.num_blocks = shape, mode, num_blocks
        dtype = torch.int8 if mode == "int8" else torch.bfloat16
        size = (shape.layers, num_blocks, BLOCK_SIZE, shape.kv_heads, shape.head_dim)
        self.key = torch.zeros(size, dtype=dtype, device=device)
        self.value = torch.zeros(size, dtype=dtype, device=device)
        if mode == "int8":
            assert k_scale is not None and v_scale is not None, "int8 caches need static scales"
            assert k_scale.shape == (shape.layers, shape.kv_heads) == v_scale.shape
            self.k_scale = k_scale.to(device=device, dtype=torch.float32).contiguous()
            self.v_scale = v_scale.to(device=device, dtype=torch.float32).contiguous()
        else:
            self.k_scale = self.v_scale = None

    def nbytes(self) -> dict:
        return kv_cache_bytes(self.shape, self.num_blocks, self.mode)

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor, slots: torch.Tensor) -> None:
        """k, v [N, Hkv, D] bf16; slots [N] int64 (block * 16 + offset)."""
        if self.mode == "int8":
            int8_kv_cache_write(k, v, self.key[layer], self.value[layer], slots,
                                self.k_scale[layer], self.v_scale[layer])
        else:
            Hkv, D = self.shape.kv_heads, self.shape.head_dim
            self.key[layer].view(-1, Hkv, D).index_copy_(0, slots, k.to(torch.bfloat16))
            self.value[layer].view(-1, Hkv, D).index_copy_(0, slots, v.to(torch.bfloat16))

    def rotary_write(self, layer: int, qkv: torch.Tensor, positions: torch.Tensor, cos, sin,
                     block_tables: torch.Tensor) -> None:
        """Rotary on the q/k heads of the decode rows of qkv (in place) fused with the cache write
        of their k (rotated) and v at each row's position."""
        ks = self.k_scale[layer] if self.mode == "int8" else None
        vs = self.v_scale[layer] if self.mode == "int8" else None
        hip_rotary_cache_write_(qkv, self.shape, positions, cos, sin, block_tables, self.key[layer],
                                self.value[layer], ks, vs)

    def attend(self, layer: int, q: torch.Tensor, block_tables: torch.Tensor, seq_lens: torch.Tensor,
               out: torch.Tensor, workspace: torch.Tensor) -> torch.Tensor:
        """q [B, Hq, D] bf16 -> out [B, Hq, D] through the HIP paged decode kernel."""
        ks = self.k_scale[layer] if self.mode == "int8" else None
        vs = self.v_scale[layer] if self.mode == "int8" else None
        return _decode.paged_decode(q, self.key[layer], self.value[layer], block_tables, seq_lens,
                                    ks, vs, out, workspace=workspace)


def _layer_prefill(x, lw: LayerWeights, shape: QwenShape, cos, sin, c, S, on_kv):
    """One layer over x [c*S, H]; on_kv(k, v) receives post-rotary k and v [c*S, Hkv, D]."""
    h = rms_norm(x, lw.ln1, shape.rms_eps)
    qkv = F.linear(h, lw.wqkv, lw.bqkv).view(c, S, shape.qkv_width)
    q, k, v = _split_qkv(qkv, shape)
    q = apply_rope(q, cos, sin)
    k = apply_rope(k, cos, sin)
    on_kv(k.reshape(c * S, shape.kv_heads, shape.head_dim), v.reshape(c * S, shape.kv_heads, shape.head_dim))
    attn = prefill_attention(q.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous(),
                             v.transpose(1, 2).contiguous())
    attn = attn.transpose(1, 2).reshape(c * S, shape.q_heads * shape.head_dim)
    x = x + F.linear(attn, lw.wo)
    h = rms_norm(x, lw.ln2, shape.rms_eps)
    gu = F.linear(h, lw.w_gate_up)
    act = F.silu(gu[:, : shape.ffn]) * gu[:, shape.ffn:]
    return x + F.linear(act, lw.w_down)


def calibrate_static_scales(weights: ModelWeights, calib_ids: torch.Tensor):
    """absmax/127 of post-rotary K and of V per (layer, kv head) over ``calib_ids`` [n, S].

    Same statistic as scripts/04_calibrate_static_scale.py:26-56 of the reference (amax over
    batch, tokens and head_dim, floored at 1e-6); returns (k_scale, v_scale) [L, Hkv] float32.
    """
    shape = weights.shape
    dev = weights.embed.device
    n, S = calib_ids.shape
    cos, sin = rope_tables(shape, S, dev)
    k_amax = torch.zeros(shape.layers, shape.kv_heads, dtype=torch.float32, device=dev)
    v_amax = torch.zeros_like(k_amax)
    with torch.inference_mode():
        x = F.embedding(calib_ids.to(dev).reshape(-1), weights.embed)
        for l, lw in enumerate(weights.layers):
            def on_kv(k, v, l=l):
                k_amax[l] = torch.maximum(k_amax[l], k.float().abs().amax(dim=(0, 2)))
                v_amax[l] = torch.maximum(v_amax[l], v.float().abs().amax(dim=(0, 2)))
            x = _layer_prefill(x, lw, shape, cos, sin, n, S, on_kv)
    return (k_amax / 127.0).clamp_min(1e-6), (v_amax / 127.0).clamp_min(1e-6)


class DecodeLoop:
    """Prefill + graph-captured greedy decode for one cache mode over a fixed batch."""

    def __init__(self, weights: ModelWeights, batch: int, prompt_len: int, new_tokens: int, mode: str,
                 scales=None, seed: int = 2, device=None):
        shape = weights.shape
        dev = weights.embed.device if device is None else torch.device(device)
        assert batch >= 1 and prompt_len >= 1 and new_tokens >= 1
        self.w, self.shape, self.mode, self.dev = weights, shape, mode, dev
        self.batch, self.prompt_len, self.new_tokens = batch, prompt_len, new_tokens
        self.max_len = prompt_len + new_tokens
        width = blocks_per_sequence(self.max_len)
        self.num_blocks = batch * width
        # Shuffled physical blocks shared by all sequences, as a paged allocator hands them out.
        g = torch.Generator().manual_seed(seed)
        pool = torch.randperm(self.num_blocks, generator=g).to(torch.int32)
        self.block_tables = pool.view(batch, width).to(dev)
        ks, vs = scales if scales is not None else (None, None)
        self.cache = PagedKVCache(shape, self.num_blocks, mode, dev, ks, vs)
        self.cos, self.sin = rope_tables(shape, self.max_len, dev)
        lib = _lib.load()
        ws_bytes = lib.int8kv_decode_workspace_bytes(shape.q_heads, shape.kv_heads, shape.head_dim,
                                                     BLOCK_SIZE, 0)
        self.workspace = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
        # Device state of the decode step (graph inputs/outputs).
        B = batch
        self.tokens = torch.zeros(B, dtype=torch.int64, device=dev)
        self.positions = torch.zeros(B, dtype=torch.int64, device=dev)
        self.seq_lens = torch.zeros(B, dtype=torch.int32, device=dev)
        self.step_idx = torch.zeros(1, dtype=torch.int64, device=dev)
        self.generated = torch.zeros(B, new_tokens, dtype=torch.int64, device=dev)
        self.logits = torch.zeros(B, shape.vocab, dtype=torch.bfloat16, device=dev)
        self.attn_out = torch.empty(B, shape.q_heads, shape.head_dim, dtype=torch.bfloat16, device=dev)
        self.resid = torch.empty(B, shape.hidden, dtype=torch.bfloat16, device=dev)
        self.normed = torch.empty_like(self.resid)
        self.act = torch.empty(B, shape.ffn, dtype=torch.bfloat16, device=dev)
        self.graph = None

    # -- prefill --------------------------------------------------------------------------------
    def prefill_slots(self, seqs: slice) -> torch.Tensor:
        t = torch.arange(self.prompt_len, device=self.dev)
        bt = self.block_tables[seqs].to(torch.int64)
        return (bt[:, t // BLOCK_SIZE] * BLOCK_SIZE + t % BLOCK_SIZE).reshape(-1)

    def prefill(self, prompt_ids: torch.Tensor, chunk_tokens: int = 32768) -> torch.Tensor:
        """Runs the prompt [B, S] through the model, fills the caches, returns the first tokens."""
        shape, B, S = self.shape, self.batch, self.prompt_len
        Hq, Hkv, D, L = shape.q_heads, shape.kv_heads, shape.head_dim, shape.layers
        assert prompt_ids.shape == (B, S)
        ids = prompt_ids.to(self.dev)
        c = max(1, min(B, chunk_tokens // S))
        last = torch.empty(B, shape.hidden, dtype=torch.bfloat16, device=self.dev)
        with torch.inference_mode():
            for b0 in range(0, B, c):
                sl = slice(b0, min(B, b0 + c))
                n = sl.stop - sl.start
                slots = self.prefill_slots(sl)
                pos = torch.arange(S, device=self.dev).repeat(n)
                x = F.embedding(ids[sl].reshape(-1), self.w.embed)
                h = torch.empty_like(x)
                hip_add_rms_norm(x, None, self.w.layers[0].ln1, h, shape.rms_eps)
                for l, lw in enumerate(self.w.layers):
                    qkv = F.linear(h, lw.wqkv, lw.bqkv)
                    hip_rotary_(qkv, Hq + Hkv, D, pos, self.cos, self.sin)
                    q, k, v = _split_qkv(qkv, shape)
                    self.cache.write(l, k, v, slots)
                    attn = prefill_attention(*(t.view(n, S, -1, D).transpose(1, 2).contiguous()
                                               for t in (q, k, v)))
                    attn = attn.transpose(1, 2).reshape(n * S, Hq * D)
                    hip_add_rms_norm(x, F.linear(attn, lw.wo), lw.ln2, h, shape.rms_eps)
                    gu = F.linear(h, lw.w_gate_up)
                    act = hip_silu_mul(gu, torch.empty(n * S, shape.ffn, dtype=x.dtype, device=self.dev))
                    del gu
                    nxt = self.w.layers[l + 1].ln1 if l + 1 < L else self.w.ln_f
                    hip_add_rms_norm(x, F.linear(act, lw.w_down), nxt, h, shape.rms_eps)
                last[sl] = h.view(n, S, shape.hidden)[:, -1]
            logits = F.linear(last, self.w.lm_head)
            first = logits.argmax(-1)
        self.prefill_logits = logits
        self.tokens.copy_(first)
        self.generated[:, 0].copy_(first)
        self.positions.fill_(S)
        self.seq_lens.fill_(S + 1)
        self.step_idx.fill_(1)
        return first

    # -- decode ---------------------------------------------------------------------------------
    def _step(self) -> None:
        """One greedy step for every sequence: reads/writes only the device state buffers."""
        shape, B = self.shape, self.batch
        Hq, D, L = shape.q_heads, shape.head_dim, shape.layers
        pos = self.positions
        if not FUSED_STEP:
            slots = self.block_tables.gather(1, (pos // BLOCK_SIZE).view(B, 1)).view(B).to(torch.int64)
            slots = slots * BLOCK_SIZE + pos % BLOCK_SIZE
        x, h = self.resid, self.normed
        torch.index_select(self.w.embed, 0, self.tokens, out=x)
        hip_add_rms_norm(x, None, self.w.layers[0].ln1, h, shape.rms_eps)
        for l, lw in enumerate(self.w.layers):
            qkv = F.linear(h, lw.wqkv, lw.bqkv)
            if FUSED_STEP:
                self.cache.rotary_write(l, qkv, pos, self.cos, self.sin, self.block_tables)
                q, _, _ = _split_qkv(qkv, shape)
            else:
                hip_rotary_(qkv, Hq + shape.kv_heads, D, pos, self.cos, self.sin)
                q, k, v = _split_qkv(qkv, shape)
                self.cache.write(l, k, v, slots)
            self.cache.attend(l, q, self.block_tables, self.seq_lens, self.attn_out, self.workspace)
            hip_add_rms_norm(x, F.linear(self.attn_out.view(B, Hq * D), lw.wo), lw.ln2, h, shape.rms_eps)
            hip_silu_mul(F.linear(h, lw.w_gate_up), self.act)
            nxt = self.w.layers[l + 1].ln1 if l + 1 < L else self.w.ln_f
            hip_add_rms_norm(x, F.linear(self.act, lw.w_down), nxt, h, shape.rms_eps)
        torch.mm(h, self.w.lm_head.t(), out=self.logits)
        if FUSED_STEP:
            hip_argmax_rows(self.logits, self.tokens)
        else:
            self.tokens.copy_(self.logits.argmax(-1))
        col = self.step_idx.clamp(max=self.new_tokens - 1).view(1, 1).expand(B, 1)
        self.generated.scatter_(1, col, self.tokens.view(B, 1))
        self.positions.add_(1)
        self.seq_lens.add_(1)
        self.step_idx.add_(1)

    def state(self):
        return [t.clone() for t in (self.tokens, self.positions, self.seq_lens, self.step_idx, self.generated)]

    def restore(self, saved) -> None:
        for dst, src in zip((self.tokens, self.positions, self.seq_lens, self.step_idx, self.generated), saved):
            dst.copy_(src)

    def step_eager(self) -> None:
        with torch.inference_mode():
            self._step()

    def capture(self) -> None:
        """Records one decode step as a HIP graph (after one eager warm-up step that is undone).

        The warm-up writes the same cache slot the first replay writes again, with the same value.
        """
        saved = self.state()
        side = torch.cuda.Stream(self.dev)
        side.wait_stream(torch.cuda.current_stream(self.dev))
        if _TUNING["tune"]:
            import torch.cuda.tunable as tunable

            tunable.tuning_enable(True)
        with torch.cuda.stream(side):
            self.step_eager()
        if _TUNING["tune"]:
            tunable.tuning_enable(False)
        torch.cuda.current_stream(self.dev).wait_stream(side)
        self.restore(saved)
        torch.cuda.synchronize(self.dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.inference_mode(), torch.cuda.graph(self.graph):
            self._step()
        torch.cuda.synchronize(self.dev)

    def replay(self) -> None:
        self.graph.replay()

    def decode(self, steps: int | None = None) -> None:
        """Runs ``steps`` (default new_tokens - 1) graph replays."""
        steps = self.new_tokens - 1 if steps is None else steps
        if self.graph is None:
            self.capture()
        for _ in range(steps):
            self.graph.replay()


def run_tpot(weights: ModelWeights, batch: int, prompt_len: int, new_tokens: int, mode: str,
             scales=None, seed: int = 0, log=print) -> dict:
    """Prefill + new_tokens greedy tokens for one mode; returns the reference's TPOT record."""
    dev = weights.embed.device
    g = torch.Generator().manual_seed(seed + 7)
    prompt = torch.randint(0, weights.shape.vocab, (batch, prompt_len), generator=g)
    loop = DecodeLoop(weights, batch, prompt_len, new_tokens, mode, scales=scales, device=dev)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    loop.prefill(prompt)
    torch.cuda.synchronize(dev)
    t1 = time.perf_counter() - t0
    log(f"[{mode}] prefill + first token: {t1 * 1e3:.1f} ms", flush=True)
    after_prefill = loop.state()
    loop.capture()
    steps = new_tokens - 1
    stream = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(dev)
    w0 = time.perf_counter()
    e0.record(stream)
    loop.decode(steps)
    e1.record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - w0
    dev_ms = e0.elapsed_time(e1)
    tpot = wall / max(steps, 1) * 1e3
    kv = loop.cache.nbytes()
    rec = {
        "mode": mode,
        "batch": batch,
        "context": prompt_len,
        "new_tokens": new_tokens,
        "t1_ms": t1 * 1e3,
        "t128_ms": (t1 + wall) * 1e3,
        "decode_tpot_ms": tpot,
        "decode_tpot_device_ms": dev_ms / max(steps, 1),
        "decode_tok_s": batch * 1e3 / tpot,
        "kv_cache_bytes": kv["kv_bytes"],
        "kv_scale_bytes": kv["scale_bytes"],
        "weight_bytes": weights.nbytes(),
        "peak_allocated_bytes": torch.cuda.max_memory_allocated(dev),
    }
    log(f"[{mode}] TPOT {tpot:.3f} ms (device {rec['decode_tpot_device_ms']:.3f} ms), "
        f"{rec['decode_tok_s']:.0f} tok/s, KV {kv['kv_bytes'] / 1e9:.3f} GB", flush=True)
    # First decode step again from the post-prefill state (it rewrites the same cache slot with
    # the same value): its logits compare the cache modes on an identical prefix.
    rec["_generated"] = loop.generated.clone()
    loop.restore(after_prefill)
    loop.replay()
    torch.cuda.synchronize(dev)
    rec["_step1_logits"] = loop.logits.float().clone()
    rec["_first_tokens"] = loop.generated[:, 0].clone()
    rec["_loop"] = loop
    return rec

