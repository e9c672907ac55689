"""CPU checks of the Python operator layer: reference-compatible validation and errors, and
that nothing computes without the GPU library (no CPU fallback)."""

from __future__ import annotations

import pytest
import torch

import int8kv
from int8kv import _decode, _ext
from int8kv import synthetic as syn


@pytest.fixture(autouse=True, params=["extension", "ctypes"])
def host_path(request):
    """Every check here runs on both host paths: the torch extension (the default when built)
    and the ctypes binding of the same C ABI."""
    if request.param == "extension":
        if _ext.module() is None:
            pytest.skip("the torch extension is not built")
        yield request.param
    else:
        with _ext.use_ctypes():
            yield request.param


def test_extension_is_built_and_default(host_path):
    assert _ext.EXT_PATH.exists(), "build() makes int8kv/_int8kv_torch.so"
    assert (_ext.module() is not None) == (host_path == "extension")


def _attn_args(**over):
    a = dict(
        query=torch.zeros(2, 28, 128, dtype=torch.bfloat16),
        key_cache=torch.zeros(8, 16, 4, 128, dtype=torch.int8),
        value_cache=torch.zeros(8, 16, 4, 128, dtype=torch.int8),
        block_tables=torch.zeros(2, 4, dtype=torch.int32),
        seq_lens=torch.ones(2, dtype=torch.int32),
        k_scale=torch.ones(4),
        v_scale=torch.ones(4),
    )
    a.update(over)
    return a


@pytest.mark.parametrize("bad", [
    dict(query=torch.zeros(2, 28, 128, dtype=torch.int32)),
    dict(key_cache=torch.zeros(8, 16, 4, 128, dtype=torch.bfloat16)),
    dict(block_tables=torch.zeros(2, 4, dtype=torch.float32)),
    dict(seq_lens=torch.ones(3, dtype=torch.int32)),
    dict(k_scale=torch.ones(3)),
    dict(query=torch.zeros(2, 30, 128, dtype=torch.bfloat16)),
    dict(key_cache=torch.zeros(8, 16, 4, 64, dtype=torch.int8)),
    dict(block_tables=torch.zeros(4, dtype=torch.int32)),
])
def test_int8_attention_validation_matches_reference(bad):
    """Same AssertionError conditions as src/triton_ops/int8_paged_attention.py:698-719."""
    with pytest.raises(AssertionError):
        int8kv.int8_paged_attention(**_attn_args(**bad))


def test_int8_attention_needs_gpu_tensors():
    with pytest.raises(AssertionError, match="GPU"):
        int8kv.int8_paged_attention(**_attn_args())


def test_bf16_attention_needs_gpu_tensors():
    a = _attn_args(key_cache=torch.zeros(8, 16, 4, 128, dtype=torch.bfloat16),
                   value_cache=torch.zeros(8, 16, 4, 128, dtype=torch.bfloat16))
    a.pop("k_scale")
    a.pop("v_scale")
    with pytest.raises(AssertionError, match="GPU"):
        int8kv.bf16_paged_attention(**a)


def test_write_validation_and_gpu_requirement():
    k = torch.zeros(3, 4, 128, dtype=torch.bfloat16)
    kc = torch.zeros(2, 16, 4, 128, dtype=torch.int8)
    s = torch.ones(4)
    slots = torch.zeros(3, dtype=torch.int64)
    with pytest.raises(AssertionError):
        int8kv.int8_kv_cache_write(k, k, kc.float(), kc, slots, s, s)
    with pytest.raises(AssertionError):
        int8kv.int8_kv_cache_write(k, k, kc, kc, slots[:2], s, s)
    with pytest.raises(AssertionError):
        int8kv.int8_kv_cache_write(k, k, kc, kc, slots.float(), s, s)
    with pytest.raises(AssertionError, match="GPU"):
        int8kv.int8_kv_cache_write(k, k, kc, kc, slots, s, s)


def test_dequantize_debug_helper():
    c = torch.tensor([[[[1, -2], [3, 4]]]], dtype=torch.int8)  # [1, 1, 2, 2]
    out = int8kv.dequantize_paged_cache_for_debug(c, torch.tensor([0.5, 2.0]))
    assert out.tolist() == [[[[0.5, -1.0], [6.0, 8.0]]]]


def test_split_request_maps_num_splits():
    """num_splits of the reference (None automatic, 1 a single pass, S splits per sequence) as
    the library's (num_ranges, flags)."""
    from int8kv import _lib

    assert _decode.split_request(64, None) == (0, 0)
    assert _decode.split_request(64, 1) == (0, _lib.DECODE_PER_SEQUENCE)
    assert _decode.split_request(64, 0) == (0, _lib.DECODE_PER_SEQUENCE)
    assert _decode.split_request(3, 4) == (12, _lib.DECODE_SPLIT_SEQUENCES)
    assert _decode.split_request(0, 4) == (4, _lib.DECODE_SPLIT_SEQUENCES)
    assert _decode.split_request(5, 100) == (5 * 64, _lib.DECODE_SPLIT_SEQUENCES)  # at most 64
    assert _decode.split_request(1 << 20, 8) == (1 << 20, _lib.DECODE_SPLIT_SEQUENCES)


def test_synthetic_generators():
    g = torch.Generator().manual_seed(0)
    dist = syn.make_distribution(0)
    k, v = syn.sample_kv(4096, dist, g)
    assert k.dtype == torch.bfloat16 and k.shape == (4096, 4, 128)
    # outlier channels are ~8x wider than the rest
    std = k.float().std(dim=0)
    for h in range(4):
        mask = torch.zeros(128, dtype=torch.bool)
        mask[dist.outlier_channels[h]] = True
        assert std[h, mask].min() > 5 * std[h, ~mask].max()
    assert abs(float(v.float().std()) - 0.5) < 0.02
    ks, vs = syn.calibrate_scales(dist, seed=1)
    assert ks.shape == (4,) and (ks > 0).all() and (vs > 0).all()
    lens = [5, 16, 17]
    bt = syn.random_block_tables(lens, 10, g)
    assert bt.shape == (3, 2)
    used = torch.cat([bt[0, :1], bt[1, :1], bt[2, :2]])
    assert len(set(used.tolist())) == 4
    slots = syn.slot_mapping_for(bt, lens)
    assert slots.shape == (38,)
    assert int(slots[21]) == int(bt[2, 0]) * 16 + 0 and int(slots[37]) == int(bt[2, 1]) * 16 + 0
    r = syn.ragged_lengths(64, 32768, 3)
    assert r.min() >= 1 and r.max() <= 32768


def test_reference_module_aliases():
    """Unmodified reference callers import the operators from src.triton_ops.* (see
    vllm_int8/vllm_int8_attention_patch.py:8-10); the aliases must bind those names here."""
    import sys

    from int8kv import compat

    saved = {k: sys.modules.get(k) for k in ("src", "src.triton_ops", *compat.ALIASES)}
    try:
        names = compat.install_reference_aliases()
        assert sorted(names) == sorted(compat.ALIASES)
        from src.triton_ops.bf16_paged_attention import bf16_paged_attention
        from src.triton_ops.int8_cache_write import int8_kv_cache_write
        from src.triton_ops.int8_paged_attention import int8_paged_attention

        assert int8_paged_attention is int8kv.int8_paged_attention
        assert int8_kv_cache_write is int8kv.int8_kv_cache_write
        assert bf16_paged_attention is int8kv.bf16_paged_attention
    finally:
        for k, v in saved.items():
            if v is None:
                sys.modules.pop(k, None)
            else:
                sys.modules[k] = v


def test_vllm_int8_module_aliases():
    import sys

    from int8kv import compat

    names = ("vllm_int8", *compat.ALIASES, *compat.VLLM_INT8_ALIASES, "src", "src.triton_ops")
    saved = {k: sys.modules.get(k) for k in names}
    try:
        compat.install_reference_aliases(include_vllm_int8=True)
        from vllm_int8.cache_manager import allocate_layer_cache
        from vllm_int8.vllm_int8_cache_ops import runtime_int8_cache_write

        from int8kv.vllm_int8 import cache_manager, vllm_int8_cache_ops

        assert allocate_layer_cache is cache_manager.allocate_layer_cache
        assert runtime_int8_cache_write is vllm_int8_cache_ops.runtime_int8_cache_write
    finally:
        for k, v in saved.items():
            if v is None:
                sys.modules.pop(k, None)
            else:
                sys.modules[k] = v


def test_debug_slot_check():
    """INT8KV_DEBUG's slot_mapping check: duplicates and out-of-cache slots are rejected on the
    host (before any launch); -1 padding and distinct in-range slots pass."""
    import pytest
    import torch

    from int8kv import _decode

    _decode.debug_check_slots(torch.tensor([3, -1, 7, -1, 0]), num_blocks=1, block_size=16)
    with pytest.raises(AssertionError, match="repeats"):
        _decode.debug_check_slots(torch.tensor([3, 5, 3]), num_blocks=1, block_size=16)
    with pytest.raises(AssertionError, match="beyond"):
        _decode.debug_check_slots(torch.tensor([3, 16]), num_blocks=1, block_size=16)
