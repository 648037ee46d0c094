"""Input generator (reference benchmarks/data.py:8-43 recipe) and the
algorithmic byte count used by the benchmark."""
from __future__ import annotations

import math

import torch

from attention_amd.cases import CONFIGS, algorithmic_bytes, make_decode_case


def test_recipe_is_deterministic_and_padded():
    a = make_decode_case(lengths=[5, 0, 33], q_heads=4, kv_heads=2, head_dim=8, block_size=16, seed=3)
    b = make_decode_case(lengths=[5, 0, 33], q_heads=4, kv_heads=2, head_dim=8, block_size=16, seed=3)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    q, k, v, table, lens = a
    assert table.shape == (3, 3) and table.dtype == torch.int32
    assert table[0, 1:].eq(-1).all() and table[1].eq(-1).all() and table[2].ge(0).all()
    assert k.shape == (9, 16, 2, 8)                      # B * max_pages blocks


def test_draw_order_q_k_v_then_permutation():
    gen = torch.Generator().manual_seed(42)
    q = torch.randn(2, 4, 8, generator=gen)
    k = torch.randn(2, 16, 2, 8, generator=gen)
    v = torch.randn(2, 16, 2, 8, generator=gen)
    order = torch.randperm(2, generator=gen)
    q2, k2, v2, t2, _ = make_decode_case(lengths=[16, 16], q_heads=4, kv_heads=2, head_dim=8, seed=42)
    assert torch.equal(q, q2) and torch.equal(k, k2) and torch.equal(v, v2)
    assert torch.equal(order.view(2, 1).int(), t2)


def test_exact_pool_uses_every_block_once():
    lengths = [17, 100, 255, 512]
    q, k, v, table, lens = make_decode_case(lengths=lengths, block_size=16, exact_pool=True, seed=42)
    used = [int(x) for row in table for x in row if x >= 0]
    assert sorted(used) == list(range(k.shape[0])) and k.shape[0] == 57
    for b, L in enumerate(lengths):
        assert (table[b] >= 0).sum() == math.ceil(L / 16)


def test_config_properties():
    assert CONFIGS["cfg1"].lengths() == [17, 100, 255, 512]
    l2 = CONFIGS["cfg2"].lengths()
    assert len(l2) == 32 and min(l2) >= 512 and max(l2) <= 4096
    l3 = CONFIGS["cfg3"].lengths()
    assert len(l3) == 64 and l3.count(1) >= 2 and max(l3) <= 8192
    assert sum(1 for x in l3 if x % 16) >= 0.25 * len(l3)
    l4 = CONFIGS["cfg4"].lengths()
    assert len(l4) == 8 and min(l4) >= 32768 and max(l4) <= 131072
    assert CONFIGS["cfg4"].k_scale == 3.0
    l5 = CONFIGS["cfg5"].lengths()
    assert len(l5) == 256 and min(l5) >= 128 and max(l5) <= 1024
    assert CONFIGS["cfg5"].block_size == 32 and CONFIGS["cfg5"].dtype == torch.float16


def test_algorithmic_bytes_cfg1_exact():
    # K+V 884 tokens * 2 * 2 * 64 * 2 + q,out 2*4*8*64*2 + lens 16 + 57 table entries * 4
    assert algorithmic_bytes([17, 100, 255, 512], 4, 8, 2, 64, 16, 2) == 461_044


def test_k_scale_applies_before_cast():
    a = make_decode_case(lengths=[16], q_heads=2, kv_heads=1, head_dim=8, seed=1, k_scale=3.0)
    b = make_decode_case(lengths=[16], q_heads=2, kv_heads=1, head_dim=8, seed=1)
    torch.testing.assert_close(a[1], 3.0 * b[1])
    assert torch.equal(a[2], b[2])
