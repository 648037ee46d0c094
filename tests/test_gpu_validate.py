"""GPU parity of the device-side metadata validator (reference
attention/validation.py:5-39) against the CPU oracle: the same first failure
message, or none, on random metadata with injected failures of every kind.
Every case prints its name first."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from attention_amd.validation import validate_paged_metadata
from oracle.gqa_oracle import oracle_validate_metadata

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def _random_meta(rng, B, P, max_pages):
    """Valid metadata: distinct pages, lengths within capacity, append
    positions at each sequence's end (distinct destinations)."""
    n_blocks = B * max_pages + 3
    table = rng.permutation(n_blocks)[:B * max_pages].reshape(B, max_pages).astype(np.int32)
    lens = rng.integers(0, (max_pages - 1) * P, B).astype(np.int32)   # room to append
    for b in range(B):
        table[b, -(-int(lens[b]) // P) + 1:] = -1       # padding beyond the next page
    pos = lens.copy()
    return table, lens, pos, n_blocks


def _run(table, lens, P, n_blocks, pos):
    try:
        validate_paged_metadata(torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda(),
                                block_size=P, num_blocks=n_blocks,
                                positions=None if pos is None else torch.from_numpy(pos).cuda())
        return None
    except ValueError as exc:
        return str(exc)


INJECT = ["none", "length", "negative_length", "block", "position", "append_page", "conflict", "many"]


@pytest.mark.parametrize("B", [1, 5, 64, 300])
@pytest.mark.parametrize("kind", INJECT)
def test_validator_matches_oracle(gpu, B, kind):
    rng = np.random.default_rng(B * 31 + INJECT.index(kind))
    P, max_pages = 16, 6
    table, lens, pos, n_blocks = _random_meta(rng, B, P, max_pages)
    b = int(rng.integers(0, B))
    if kind == "length":
        lens[b] = max_pages * P + 1
    elif kind == "negative_length":
        lens[b] = -3
    elif kind == "block":
        lens[b] = max(lens[b], 1)
        table[b, int(rng.integers(0, -(-int(lens[b]) // P)))] = n_blocks + 5
    elif kind == "position":
        pos[b] = max_pages * P
    elif kind == "append_page":
        lens[b] = min(lens[b], (max_pages - 2) * P)
        pos[b] = (max_pages - 1) * P            # page max_pages-1 of row b is padding (-1)
        table[b, max_pages - 1] = -1
    elif kind == "conflict" and B > 1:
        b2 = (b + 1) % B
        lo, hi = min(b, b2), max(b, b2)
        pos[hi] = pos[lo]
        table[hi, pos[lo] // P] = table[lo, pos[lo] // P]
    elif kind == "many":
        for j in rng.choice(B, size=min(B, 4), replace=False):
            lens[j] = -1 if rng.random() < 0.5 else max_pages * P + 7
    say(f"validator B={B} inject={kind}")
    for positions in (None, pos):
        expect = oracle_validate_metadata(table, lens, P, n_blocks, positions)
        got = _run(table, lens, P, n_blocks, positions)
        assert got == expect, (positions is not None, got, expect)


def test_validator_empty_table_columns_and_batch(gpu):
    say("validator with no table capacity / no batch")
    t0 = torch.zeros(3, 0, dtype=torch.int32, device=gpu)
    validate_paged_metadata(t0, torch.zeros(3, dtype=torch.int32, device=gpu), block_size=16, num_blocks=4)
    with pytest.raises(ValueError, match="invalid length at batch 1"):
        validate_paged_metadata(t0, torch.tensor([0, 2, 0], dtype=torch.int32, device=gpu), block_size=16,
                                num_blocks=4)
    with pytest.raises(ValueError, match="invalid append position at batch 0"):
        validate_paged_metadata(t0, torch.zeros(3, dtype=torch.int32, device=gpu), block_size=16, num_blocks=4,
                                positions=torch.zeros(3, dtype=torch.int32, device=gpu))
    validate_paged_metadata(torch.zeros(0, 4, dtype=torch.int32, device=gpu),
                            torch.zeros(0, dtype=torch.int32, device=gpu), block_size=16, num_blocks=4)


def test_validator_accepts_benchmark_configs(gpu):
    from attention_amd.cases import CONFIGS
    for name in ("cfg1", "cfg2", "cfg3", "cfg5"):
        say(f"validator on {name} metadata")
        cfg = CONFIGS[name]
        _, k, _, table, lens = cfg.make(device="cpu")
        validate_paged_metadata(table.to(gpu), lens.to(gpu), block_size=cfg.block_size, num_blocks=k.shape[0])
