"""The benchmark's algorithmic byte counts (int8kv.roofline) against the oracle's count and
against hand-computed cases."""

from __future__ import annotations

import numpy as np
import pytest

from int8kv import roofline as R
from oracle import int8kv_oracle as O


def test_decode_bytes_known_answer():
    # lens 16, 1, 0 (2 blocks); 4 kv heads x 128, INT8: 17 tokens * 1024 B of K+V, 2 table
    # entries, q + out of 3 x 28 x 128 bf16, 3 lengths, 2 x 4 fp32 scales.
    assert R.decode_bytes([16, 1, 0], 4, 128, 1, 3, 28) == 17 * 1024 + 8 + 43008 + 12 + 32
    # the same lengths in a BF16 cache: twice the K/V bytes and no scales
    assert R.decode_bytes([16, 1, 0], 4, 128, 2, 3, 28) == 17 * 2048 + 8 + 43008 + 12
    assert R.decode_bytes([-5, 33], 2, 64, 1, 2, 8, q_elem=4, block_size=32) == \
        33 * 256 + 2 * 4 + 2 * 8 * 64 * 4 * 2 + 8 + 16


@pytest.mark.parametrize("e", [1, 2])
def test_decode_bytes_match_the_oracle(e):
    g = np.random.default_rng(e)
    for _ in range(50):
        B = int(g.integers(1, 80))
        lens = g.integers(0, 40000, B)
        bs = int(2 ** g.integers(4, 8))
        assert R.decode_bytes(lens, 4, 128, e, B, 28, block_size=bs) == \
            O.decode_bytes(lens, 4, 128, e, B, 28, block_size=bs)


def test_write_bytes_of_the_benchmark_workloads():
    # config 1: 16,384 tokens + 512 padding slots; the HBM-sized write: 262,144 tokens
    assert R.write_bytes(16384, 16896, 4, 128) == 50_466_848
    assert R.write_bytes(16384, 16896, 4, 128, dynamic=True) == 50_991_104
    assert R.write_bytes(262144, 262144, 4, 128) == 807_403_552
    assert R.write_bytes(262144, 262144, 4, 128, dynamic=True) == 815_792_128
    # fp32 sources read 4 bytes per element; int32 slots 4 bytes per row
    assert R.write_bytes(10, 12, 2, 64, src_elem=4, slot_elem=4) == 10 * 128 * 2 * 5 + 48 + 16
