"""Host-side validate_paged_metadata (CPU metadata, reference
attention/validation.py:5-39): the first failure message equals the CPU
oracle's on random metadata with injected failures of every kind, and on
unconstrained random metadata; it needs neither a GPU nor the native
library."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from attention_amd import core
from attention_amd.validation import validate_paged_metadata
from oracle.gqa_oracle import oracle_validate_metadata
from tests.test_gpu_validate import INJECT, _random_meta


def _run(table, lens, P, n_blocks, pos):
    try:
        validate_paged_metadata(torch.from_numpy(table), torch.from_numpy(lens), block_size=P,
                                num_blocks=n_blocks, positions=None if pos is None else torch.from_numpy(pos))
        return None
    except ValueError as exc:
        return str(exc)


@pytest.fixture
def no_library(monkeypatch):
    """The host path must not need the op library: pretend it failed to load."""
    monkeypatch.setattr(core, "_LOAD_ERROR", OSError("library absent (test)"))


@pytest.mark.parametrize("B", [1, 5, 64, 300])
@pytest.mark.parametrize("kind", INJECT)
def test_host_validator_matches_oracle(no_library, B, kind):
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
        pos[b] = (max_pages - 1) * P
        table[b, max_pages - 1] = -1
    elif kind == "conflict" and B > 1:
        b2 = (b + 1) % B
        lo, hi = min(b, b2), max(b, b2)
        pos[hi] = pos[lo]
        table[hi, pos[lo] // P] = table[lo, pos[lo] // P]
    elif kind == "many":
        for j in rng.choice(B, size=min(B, 4), replace=False):
            lens[j] = -1 if rng.random() < 0.5 else max_pages * P + 7
    for positions in (None, pos):
        assert _run(table, lens, P, n_blocks, positions) == oracle_validate_metadata(
            table, lens, P, n_blocks, positions)


def test_host_validator_random_metadata(no_library):
    """Unconstrained random metadata (every check and their order), tiny
    block sizes and empty tables included."""
    rng = np.random.default_rng(7)
    for _ in range(600):
        B = int(rng.integers(1, 24))
        P = int(rng.choice([1, 3, 16]))
        mp = int(rng.integers(0, 6))
        n = int(rng.integers(1, B * mp + 5))
        table = rng.integers(-2, n + 2, (B, mp)).astype(np.int32)
        lens = rng.integers(-2, mp * P + 3, B).astype(np.int32)
        pos = rng.integers(-1, mp * P + 2, B).astype(np.int32)
        if rng.random() < 0.5:
            table = np.clip(table, 0, n - 1).astype(np.int32)
            lens = np.clip(lens, 0, mp * P).astype(np.int32)
        for positions in (None, pos):
            assert _run(table, lens, P, n, positions) == oracle_validate_metadata(table, lens, P, n, positions)


def test_host_validator_argument_checks(no_library):
    t = torch.zeros(2, 3, dtype=torch.int32)
    ln = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="block_size and num_blocks must be positive"):
        validate_paged_metadata(t, ln, block_size=0, num_blocks=4)
    with pytest.raises(ValueError, match=r"metadata shapes must be \[B,MaxPages\] and \[B\]"):
        validate_paged_metadata(t[0], ln, block_size=16, num_blocks=4)
    with pytest.raises(ValueError, match="metadata must be int32"):
        validate_paged_metadata(t.long(), ln, block_size=16, num_blocks=4)
    with pytest.raises(ValueError, match=r"positions must be int32 \[B\]"):
        validate_paged_metadata(t, ln, block_size=16, num_blocks=4, positions=ln.long())
    validate_paged_metadata(torch.zeros(0, 4, dtype=torch.int32), torch.zeros(0, dtype=torch.int32),
                            block_size=16, num_blocks=4)
    # Non-contiguous views are read as they are.
    wide = torch.zeros(2, 6, dtype=torch.int32)
    validate_paged_metadata(wide[:, ::2], torch.tensor([16, 48], dtype=torch.int32), block_size=16,
                            num_blocks=4)
