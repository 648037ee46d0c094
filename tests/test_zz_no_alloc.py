"""The no-allocation entry point (qd_gqa_decode_auto_noalloc): the same
output as the automatic entry point with a caller workspace, bit for bit,
on two calls in a row (the second with a smaller input, so the scratch
holds the first call's leftovers), and a clear error, before anything is
enqueued, for shapes whose scratch does not fit."""
from __future__ import annotations

import math

import pytest
import torch

from attention_amd import cabi
from attention_amd.cases import CONFIGS, make_decode_case


def say(msg):
    print(f"[case] {msg}", flush=True)


def test_noalloc_rejects_oversized_shapes():
    # 4096 sequences x 64 heads x 8192 pages need far more than the scratch.
    rc = cabi.lib().qd_gqa_decode_auto_noalloc(1, 1, 1, 1, 1, 1, 4096, 64, 8, 128, 16, 8192, 1 << 20,
                                               cabi.DTYPE[torch.bfloat16], 0.1, None)
    assert rc == 1
    assert "more than the no-allocation scratch holds" in cabi.error_string(rc)
    assert cabi.lib().qd_gqa_decode_noalloc_scratch_bytes() == 16 << 20


@pytest.mark.gpu
def test_noalloc_matches_auto_entry_point(gpu):
    cfg = CONFIGS["cfg2"]
    cases = [("cfg2", cfg.make(device="cpu")),
             ("small", make_decode_case(lengths=[1, 300, 0, 17, 2000], q_heads=32, kv_heads=8, head_dim=128,
                                        block_size=16, dtype=torch.bfloat16, seed=3))]
    for name, case_cpu in cases:
        q, k, v, table, lens = (x.to(gpu) for x in case_cpu)
        B, Hq, D = q.shape
        _, P, Hkv, _ = k.shape
        need = cabi.auto_workspace_bytes(B, Hq, Hkv, D, P, table.shape[1], cabi.DTYPE[q.dtype])
        say(f"no-alloc vs auto: {name} B={B} workspace {need} bytes")
        assert need <= cabi.lib().qd_gqa_decode_noalloc_scratch_bytes()
        ws = cabi.auto_workspace(B, Hq, Hkv, D, P, table.shape[1], cabi.DTYPE[q.dtype], gpu, fill=0xFF)
        ref = torch.full_like(q, float("nan"))
        rc = cabi.auto_launch(q, k, v, table, lens, ref, scale=1 / math.sqrt(D), workspace=ws)
        assert rc == 0, cabi.error_string(rc)
        out = torch.full_like(q, float("nan"))
        rc = cabi.auto_noalloc_launch(q, k, v, table, lens, out, scale=1 / math.sqrt(D))
        assert rc == 0, cabi.error_string(rc)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), name
