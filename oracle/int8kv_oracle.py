"""CPU oracle for the INT8 KV-cache hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module,
and only as the checker (or the timed CPU baseline); the product (int8kv, libint8kv.so) never
calls it.  It is a numpy restatement of the reference's PyTorch math (cjsmt/Int8-kvcache):

    quant_kv_static_per_head     src/quant.py:37-40
    int8_kv_cache_write          src/triton_ops/int8_cache_write.py:152-183 (torch reference,
                                 round-half-even) + the kernel's scale floor (:50-51) and
                                 slot < 0 skip (:44-49, :165-168)
    make_paged_cache             src/paged_cache.py:4-36
    gather_from_paged_cache      src/paged_cache.py:39-59 (plus a ragged per-sequence form)
    expand_kv_for_gqa            src/attention_ref.py:11-16
    decode_attention_ref         src/attention_ref.py:19-28
    paged_attention_ref          src/triton_ops/int8_paged_attention.py:776-814 (fp32 output kept;
                                 the reference casts to query.dtype at :814)
    dequantize_paged_cache       src/triton_ops/int8_cache_write.py:186-189
    reshape_and_cache_int8       vllm_int8/vllm_int8_cache_ops.py:13-131 (dynamic per-(token, head)
                                 scales, clamp then round half away from zero)

How each function is pinned (tests/test_oracle.py): known-answer tests for the rounding,
clamping, scale floor and slot mapping; brute-force pure-Python loops on tiny inputs; closed
forms (one-token sequences, constant keys); invariants (physical block permutation, GQA head
mapping); and torch's scaled_dot_product_attention in float64 as an independent library
routine.  The reference ships no golden vectors for this path.

Arrays: 16-bit inputs are passed as float32 arrays holding the exact bf16/fp16 values.
"""

from __future__ import annotations

import math

import numpy as np

SCALE_FLOOR = np.float32(1e-6)


# --------------------------------------------------------------------------- quantisation
def quant_kv_static_per_head(x: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """round(x / scale) (half to even), clamp to [-127, 127], int8.  src/quant.py:37-40.

    ``x`` and ``scale`` are promoted to float32 and divided in IEEE float32, as torch does for a
    bf16 tensor divided by an fp32 tensor.
    """
    q = np.rint(np.asarray(x, np.float32) / np.asarray(scale, np.float32))
    return np.clip(q, -127, 127).astype(np.int8)


def dequantize_paged_cache(cache: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """int8 [NB, BS, Hkv, D] * scale[Hkv] -> float32.  src/triton_ops/int8_cache_write.py:186-189."""
    return cache.astype(np.float32) * np.asarray(scale, np.float32)[None, None, :, None]


def int8_kv_cache_write(
    key: np.ndarray,
    value: np.ndarray,
    key_cache: np.ndarray,
    value_cache: np.ndarray,
    slot_mapping: np.ndarray,
    k_scale: np.ndarray,
    v_scale: np.ndarray,
) -> None:
    """In-place static per-head INT8 write into paged caches [NB, BS, Hkv, D].

    For every token t with slot s = slot_mapping[t] >= 0 (src/triton_ops/int8_cache_write.py:
    165-170): cache[s // BS, s % BS, h, :] = quant(x[t, h, :], max(scale[h], 1e-6)).  Slots at or
    beyond NB * BS are skipped (the HIP kernel's bounds rule; the reference leaves them undefined).
    """
    nb, bs, hkv, d = key_cache.shape
    slots = np.asarray(slot_mapping, np.int64).reshape(-1)
    ok = (slots >= 0) & (slots < nb * bs)
    ks = np.maximum(np.asarray(k_scale, np.float32), SCALE_FLOOR)
    vs = np.maximum(np.asarray(v_scale, np.float32), SCALE_FLOOR)
    kq = quant_kv_static_per_head(np.asarray(key, np.float32)[ok], ks[None, :, None])
    vq = quant_kv_static_per_head(np.asarray(value, np.float32)[ok], vs[None, :, None])
    flat_k = key_cache.reshape(nb * bs, hkv, d)
    flat_v = value_cache.reshape(nb * bs, hkv, d)
    flat_k[slots[ok]] = kq
    flat_v[slots[ok]] = vq


def reshape_and_cache_int8(
    key: np.ndarray,
    value: np.ndarray,
    key_cache: np.ndarray,
    value_cache: np.ndarray,
    k_scale_cache: np.ndarray,
    v_scale_cache: np.ndarray,
    slot_mapping: np.ndarray,
) -> None:
    """In-place dynamic INT8 write (vllm_int8/vllm_int8_cache_ops.py:13-131).

    Per token t with slot s >= 0 and head h: scale = max(absmax(x[t, h]) / 127, 1e-6) in
    float32 (:70-79); code = round_half_away(clamp(x / scale, -127, 127)) (:80-92); codes to
    cache[s // BS, s % BS, h] and the scale to scale_cache[s // BS, s % BS, h] (:93-131).
    """
    nb, bs, hkv, d = key_cache.shape
    slots = np.asarray(slot_mapping, np.int64).reshape(-1)
    ok = (slots >= 0) & (slots < nb * bs)
    for src, dst, sdst in ((key, key_cache, k_scale_cache), (value, value_cache, v_scale_cache)):
        x = np.asarray(src, np.float32)[ok]  # [n, Hkv, D]
        scale = np.maximum(np.abs(x).max(axis=-1) / np.float32(127.0), SCALE_FLOOR)  # [n, Hkv]
        q = np.clip(x / scale[..., None], np.float32(-127), np.float32(127))
        code = np.where(q >= 0, np.floor(q + np.float32(0.5)), np.ceil(q - np.float32(0.5)))
        dst.reshape(nb * bs, hkv, d)[slots[ok]] = code.astype(np.int8)
        sdst.reshape(nb * bs, hkv)[slots[ok]] = scale.astype(np.float32)


# --------------------------------------------------------------------------- paged layout
def make_paged_cache(k: np.ndarray, v: np.ndarray, block_size: int = 16):
    """k/v [B, Hkv, T, D] -> caches [B * ceil(T/BS), BS, Hkv, D], tables, seq_lens.

    Sequential allocation as src/paged_cache.py:4-36 (sequence b owns blocks b*n .. b*n+n-1).
    """
    B, hkv, T, d = k.shape
    n = (T + block_size - 1) // block_size
    kc = np.zeros((B * n, block_size, hkv, d), k.dtype)
    vc = np.zeros_like(kc)
    tables = np.arange(B * n, dtype=np.int32).reshape(B, n)
    for b in range(B):
        for lb in range(n):
            s, e = lb * block_size, min((lb + 1) * block_size, T)
            kc[tables[b, lb], : e - s] = k[b, :, s:e, :].transpose(1, 0, 2)
            vc[tables[b, lb], : e - s] = v[b, :, s:e, :].transpose(1, 0, 2)
    return kc, vc, tables, np.full((B,), T, np.int32)


def gather_sequence(cache: np.ndarray, table_row: np.ndarray, T: int) -> np.ndarray:
    """Logical token order of one sequence: [T, Hkv, D] (src/paged_cache.py:45-58)."""
    bs = cache.shape[1]
    n = (T + bs - 1) // bs
    blocks = np.asarray(table_row[:n], np.int64)
    return cache[blocks].reshape(n * bs, *cache.shape[2:])[:T]


def gather_from_paged_cache(kc, vc, block_tables, seq_lens):
    """Uniform-T gather back to [B, Hkv, T, D] (src/paged_cache.py:39-59)."""
    ks = [gather_sequence(kc, block_tables[b], int(seq_lens[b])).transpose(1, 0, 2)
          for b in range(len(seq_lens))]
    vs = [gather_sequence(vc, block_tables[b], int(seq_lens[b])).transpose(1, 0, 2)
          for b in range(len(seq_lens))]
    return np.stack(ks), np.stack(vs)


# --------------------------------------------------------------------------- attention
def expand_kv_for_gqa(x: np.ndarray, num_query_heads: int) -> np.ndarray:
    """[B, Hkv, T, D] -> [B, Hq, T, D], kv head g repeated Hq/Hkv times (src/attention_ref.py:11-16)."""
    hkv = x.shape[1]
    assert num_query_heads % hkv == 0
    return np.repeat(x, num_query_heads // hkv, axis=1)


def _softmax_attend(q: np.ndarray, k: np.ndarray, v: np.ndarray, dtype) -> np.ndarray:
    """q [H, D], k/v [T, D] (one kv head) -> [H, D]: softmax(q k^T / sqrt(D)) v."""
    d = q.shape[-1]
    scores = (q.astype(dtype) @ k.astype(dtype).T) / dtype(math.sqrt(d))
    scores = scores - scores.max(axis=-1, keepdims=True)
    p = np.exp(scores)
    p /= p.sum(axis=-1, keepdims=True)
    return p @ v.astype(dtype)


def decode_attention_ref(q: np.ndarray, k: np.ndarray, v: np.ndarray, dtype=np.float32):
    """q [B, Hq, D], k/v [B, Hkv, T, D] -> [B, Hq, D] (src/attention_ref.py:19-28)."""
    B, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    out = np.zeros((B, hq, d), dtype)
    for b in range(B):
        for h in range(hkv):
            out[b, h * g:(h + 1) * g] = _softmax_attend(q[b, h * g:(h + 1) * g], k[b, h], v[b, h], dtype)
    return out


def paged_attention_ref(
    query: np.ndarray,
    key_cache: np.ndarray,
    value_cache: np.ndarray,
    block_tables: np.ndarray,
    seq_lens: np.ndarray,
    k_scale: np.ndarray | None = None,
    v_scale: np.ndarray | None = None,
    dtype=np.float32,
    quantize_q: bool = False,
) -> np.ndarray:
    """Decode attention over a paged cache -> [B, Hq, D] in ``dtype``.

    Follows src/triton_ops/int8_paged_attention.py:776-814: q head h reads kv head h // (Hq/Hkv)
    (:796), tokens t < seq_len[b] gathered through the block table (:804-807), dequantised with
    the per-head scales (:808-809), softmax(q.k / sqrt(D)) (:810-811), weighted sum of v (:812).
    With k_scale/v_scale None the cache is used as is (the BF16 path,
    src/triton_ops/bf16_paged_attention.py:64-111).  Scales are floored at 1e-6 like the
    kernels (:150-151).  An empty sequence yields zeros (the reference asserts len > 0).
    quantize_q=True first replaces each query row by its int8 quantisation, dequantised
    (:798-802): q_scale = max(absmax / 127, 1e-6), q = clamp(round_half_away(q / q_scale)) * q_scale.
    """
    B, hq, d = query.shape
    hkv = key_cache.shape[2]
    g = hq // hkv
    out = np.zeros((B, hq, d), dtype)
    ks = None if k_scale is None else np.maximum(np.asarray(k_scale, np.float32), SCALE_FLOOR)
    vs = None if v_scale is None else np.maximum(np.asarray(v_scale, np.float32), SCALE_FLOOR)
    for b in range(B):
        T = int(seq_lens[b])
        if T <= 0:
            continue
        k = gather_sequence(key_cache, block_tables[b], T).astype(np.float32)
        v = gather_sequence(value_cache, block_tables[b], T).astype(np.float32)
        if ks is not None:
            k = k * ks[None, :, None]
        if vs is not None:
            v = v * vs[None, :, None]
        for h in range(hkv):
            qh = np.asarray(query[b, h * g:(h + 1) * g], np.float32)
            if quantize_q:
                qh = quantize_query_rows(qh)
            out[b, h * g:(h + 1) * g] = _softmax_attend(qh, k[:, h], v[:, h], dtype)
    return out


def round_half_away(x: np.ndarray) -> np.ndarray:
    """Round half away from zero (src/triton_ops/int8_paged_attention.py:772-773)."""
    x = np.asarray(x, np.float32)
    return np.where(x >= 0, np.floor(x + np.float32(0.5)), -np.floor(-x + np.float32(0.5)))


def quantize_query_rows(q: np.ndarray) -> np.ndarray:
    """Per-row int8 quantise + dequantise of q [H, D] in float32 (int8_paged_attention.py:798-802)."""
    q = np.asarray(q, np.float32)
    qs = np.maximum(np.abs(q).max(axis=-1, keepdims=True) / np.float32(127.0), SCALE_FLOOR)
    q8 = np.clip(round_half_away(q / qs), -127, 127)
    return (q8 * qs).astype(np.float32)


def decode_bytes(seq_lens, num_kv_heads: int, head_dim: int, cache_elem: int, batch: int,
                 num_q_heads: int, q_elem: int = 2, block_size: int = 16) -> int:
    """Algorithmic HBM bytes of one decode call (K+V read once, tables, q in, out, scales)."""
    lens = np.maximum(np.asarray(seq_lens, np.int64), 0)
    kv = int(lens.sum()) * num_kv_heads * head_dim * cache_elem * 2
    tables = int(((lens + block_size - 1) // block_size).sum()) * 4
    qo = 2 * batch * num_q_heads * head_dim * q_elem
    return kv + tables + qo + batch * 4 + (2 * num_kv_heads * 4 if cache_elem == 1 else 0)
