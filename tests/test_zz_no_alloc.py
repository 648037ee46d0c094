"""The no-allocation entry point (qd_gqa_decode_auto_noalloc): the same
output as the automatic entry point with a caller workspace, bit for bit,
on two calls in a row (the second with a smaller input, so the scratch
holds the first call's leftovers), also when its first call on the device is
made inside a HIP graph capture and the graph is replayed between other
calls, and a clear error, before anything is enqueued, for shapes whose
scratch does not fit."""
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


def _decode_case(lengths, seed, gpu):
    case = make_decode_case(lengths=lengths, q_heads=32, kv_heads=8, head_dim=128, block_size=16,
                            dtype=torch.bfloat16, seed=seed)
    return [x.to(gpu) for x in case]


def _auto_reference(q, k, v, table, lens, gpu):
    B, Hq, D = q.shape
    _, P, Hkv, _ = k.shape
    ws = cabi.auto_workspace(B, Hq, Hkv, D, P, table.shape[1], cabi.DTYPE[q.dtype], gpu, fill=0xFF)
    ref = torch.full_like(q, float("nan"))
    rc = cabi.auto_launch(q, k, v, table, lens, ref, scale=1 / math.sqrt(D), workspace=ws)
    assert rc == 0, cabi.error_string(rc)
    torch.cuda.synchronize()
    return ref


# Placed first among this file's GPU tests, which hold the only no-alloc
# calls of the suite: in a full run (and alone) the call captured here is the
# process's first on the device, the one that looks up the scratch address.
@pytest.mark.gpu
def test_noalloc_first_call_inside_graph_capture(gpu):
    q, k, v, table, lens = _decode_case([1, 700, 0, 33, 2500, 129], seed=11, gpu=gpu)
    D = q.shape[2]
    out = torch.full_like(q, float("nan"))
    say(f"no-alloc captured in a graph: B={q.shape[0]}")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = cabi.auto_noalloc_launch(q, k, v, table, lens, out, scale=1 / math.sqrt(D))
    assert rc == 0, cabi.error_string(rc)
    # Other work between replays: eager no-alloc calls on another shape
    # (which leave their partials in the shared scratch), and new queries
    # written into the captured input.
    other = _decode_case([5000, 1, 900], seed=12, gpu=gpu)
    other_out = torch.full_like(other[0], float("nan"))
    gen = torch.Generator(device="cpu").manual_seed(13)
    for replay in range(4):
        if replay:
            q.copy_(torch.randn(q.shape, generator=gen).to(q.dtype))
        ref = _auto_reference(q, k, v, table, lens, gpu)
        rc = cabi.auto_noalloc_launch(*other, other_out, scale=1 / math.sqrt(D))
        assert rc == 0, cabi.error_string(rc)
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        say(f"replay {replay}")
        assert torch.equal(out, ref), f"replay {replay}"
        assert torch.equal(other_out, _auto_reference(*other, gpu)), f"eager call after replay {replay}"


@pytest.mark.gpu
def test_noalloc_matches_auto_entry_point(gpu):
    cfg = CONFIGS["cfg2"]
    held = [int(x) for x in torch.randint(1, 600, (300,), generator=torch.Generator().manual_seed(4))]
    cases = [("cfg2", cfg.make(device="cpu")),
             ("small", make_decode_case(lengths=[1, 300, 0, 17, 2000], q_heads=32, kv_heads=8, head_dim=128,
                                        block_size=16, dtype=torch.bfloat16, seed=3)),
             # 300 short sequences: the plan holds result rows in LDS
             ("held", make_decode_case(lengths=held, q_heads=40, kv_heads=8, head_dim=128, block_size=16,
                                       dtype=torch.float16, seed=5))]
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
