"""GPU parity of kv_append (reference csrc/cuda/cache/kv_append.cu:11-56)
against the CPU oracle: bitwise (it is a copy), on both the 16-byte vector
path and the element path, with invalid metadata skipped, plus an
append-then-decode round trip.  Every case prints its name first."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import attention_amd
from attention_amd import cabi
from attention_amd.cases import make_decode_case
from oracle.gqa_oracle import oracle_decode, oracle_kv_append

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def _case(B, Hkv, D, P, dtype, seed, extra_pages=0):
    """Caches with distinct pages per sequence (so destinations are distinct),
    positions inside each row's capacity, random key/value rows."""
    gen = torch.Generator().manual_seed(seed)
    max_pages = 3
    N = B * max_pages + extra_pages
    kc = torch.randn(N, P, Hkv, D, generator=gen).to(dtype)
    vc = torch.randn(N, P, Hkv, D, generator=gen).to(dtype)
    table = torch.randperm(N, generator=gen)[:B * max_pages].view(B, max_pages).int().contiguous()
    pos = torch.randint(0, max_pages * P, (B,), generator=gen, dtype=torch.int32)
    key = torch.randn(B, Hkv, D, generator=gen).to(dtype)
    value = torch.randn(B, Hkv, D, generator=gen).to(dtype)
    return key, value, kc, vc, table, pos


def _np(x):
    return x.view(torch.int16).numpy() if x.dtype in (torch.float16, torch.bfloat16) else x.numpy()


def _check(dev_kc, dev_vc, key, value, kc, vc, table, pos):
    ref_k, ref_v = oracle_kv_append(_np(key), _np(value), _np(kc), _np(vc), table.numpy(), pos.numpy())
    got_k, got_v = _np(dev_kc.cpu()), _np(dev_vc.cpu())
    assert np.array_equal(got_k, ref_k), "k_cache differs from the oracle"
    assert np.array_equal(got_v, ref_v), "v_cache differs from the oracle"


SHAPES = [
    # (B, Hkv, D, P, dtype)            path
    (7, 8, 128, 16, torch.bfloat16),   # 16-byte vectors
    (256, 8, 128, 32, torch.float16),  # 16-byte vectors, high batch
    (5, 3, 17, 5, torch.float16),      # 102-byte rows: element path
    (4, 1, 3, 7, torch.float32),       # 12-byte rows: element path, fp32
    (3, 4, 64, 16, torch.float32),     # fp32 vectors
    (1, 2, 256, 16, torch.bfloat16),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"B{s[0]}-Hkv{s[1]}-D{s[2]}-P{s[3]}-{str(s[4])[6:]}")
def test_kv_append_matches_oracle(gpu, shape):
    B, Hkv, D, P, dtype = shape
    say(f"kv_append {shape}")
    key, value, kc, vc, table, pos = _case(B, Hkv, D, P, dtype, seed=B + D)
    dkc, dvc = kc.to(gpu), vc.to(gpu)
    attention_amd.kv_append(key.to(gpu), value.to(gpu), dkc, dvc, table.to(gpu), pos.to(gpu))
    torch.cuda.synchronize()
    _check(dkc, dvc, key, value, kc, vc, table, pos)


def test_kv_append_unaligned_pointers_take_element_path(gpu):
    say("kv_append with key/value/cache not 16-byte aligned")
    B, Hkv, D, P = 6, 8, 128, 16
    key, value, kc, vc, table, pos = _case(B, Hkv, D, P, torch.bfloat16, seed=11)
    kbig = torch.empty(key.numel() + 1, dtype=key.dtype, device=gpu)
    vbig = torch.empty(value.numel() + 1, dtype=key.dtype, device=gpu)
    kbig[1:] = key.reshape(-1).to(gpu)
    vbig[1:] = value.reshape(-1).to(gpu)
    kcb = torch.empty(kc.numel() + 1, dtype=kc.dtype, device=gpu)
    vcb = torch.empty(vc.numel() + 1, dtype=vc.dtype, device=gpu)
    kcb[1:] = kc.reshape(-1).to(gpu)
    vcb[1:] = vc.reshape(-1).to(gpu)
    dk, dv = kbig[1:].view(B, Hkv, D), vbig[1:].view(B, Hkv, D)
    dkc, dvc = kcb[1:].view(kc.shape), vcb[1:].view(vc.shape)
    assert dk.data_ptr() % 16 != 0
    attention_amd.kv_append(dk, dv, dkc, dvc, table.to(gpu), pos.to(gpu))
    torch.cuda.synchronize()
    _check(dkc, dvc, key, value, kc, vc, table, pos)


def test_kv_append_invalid_metadata_is_skipped(gpu):
    say("kv_append skips out-of-range positions and page ids")
    B, Hkv, D, P = 6, 2, 64, 16
    key, value, kc, vc, table, pos = _case(B, Hkv, D, P, torch.float16, seed=5)
    N = kc.shape[0]
    pos[0] = -1                       # before the row
    pos[1] = 3 * P                    # past the row's capacity
    table[2, :] = -1                  # page id -1
    table[3, :] = N                   # page id past the pool
    dkc, dvc = kc.to(gpu), vc.to(gpu)
    attention_amd.kv_append(key.to(gpu), value.to(gpu), dkc, dvc, table.to(gpu), pos.to(gpu))
    torch.cuda.synchronize()
    _check(dkc, dvc, key, value, kc, vc, table, pos)   # oracle skips the same rows


def test_append_then_decode_round_trip(gpu):
    """Appending token L then decoding L+1 tokens equals decoding the oracle's
    updated cache: kv_append writes exactly the row decode reads."""
    say("append then decode")
    lengths = [15, 16, 40, 1, 100]
    q, k, v, table, lens = make_decode_case(lengths=lengths, q_heads=16, kv_heads=8, head_dim=128,
                                            block_size=16, dtype=torch.bfloat16, seed=13)
    gen = torch.Generator().manual_seed(1)
    key = torch.randn(len(lengths), 8, 128, generator=gen).bfloat16()
    value = torch.randn(len(lengths), 8, 128, generator=gen).bfloat16()
    # Token L goes to slot L % 16 of page L // 16; a sequence whose length is
    # a multiple of 16 needs a fresh page (one new block per sequence, and
    # one more table column for the longest).
    N0 = k.shape[0]
    k = torch.cat([k, torch.zeros(len(lengths), *k.shape[1:], dtype=k.dtype)])
    v = torch.cat([v, torch.zeros(len(lengths), *v.shape[1:], dtype=v.dtype)])
    table = torch.cat([table, torch.full((len(lengths), 1), -1, dtype=torch.int32)], dim=1)
    for b, L in enumerate(lengths):
        if table[b, L // 16] < 0:
            table[b, L // 16] = N0 + b
    pos = torch.tensor(lengths, dtype=torch.int32)
    dk, dv = k.cuda(), v.cuda()
    attention_amd.kv_append(key.cuda(), value.cuda(), dk, dv, table.cuda(), pos.cuda())
    lens2 = (lens + 1).cuda()
    out = attention_amd.gqa_decode(q.cuda(), dk, dv, table.cuda(), lens2)
    torch.cuda.synchronize()
    nk, nv = oracle_kv_append(key.float().numpy(), value.float().numpy(), k.float().numpy(), v.float().numpy(),
                              table.numpy(), pos.numpy())
    ref = oracle_decode(q.float().numpy(), nk, nv, table.numpy(), (lens + 1).numpy(), out_dtype="bf16")
    got = out.float().cpu().numpy()
    err = np.abs(got - ref)
    assert np.all(err <= 2e-3 + 1e-2 * np.abs(ref)), f"max abs err {err.max():.3e}"


def test_kv_append_validation_messages_on_device(gpu):
    say("kv_append validation messages")
    key, value, kc, vc, table, pos = (x.to(gpu) for x in _case(4, 2, 64, 16, torch.float16, seed=2))
    with pytest.raises(RuntimeError, match="dtype mismatch"):
        attention_amd.kv_append(key.float(), value, kc, vc, table, pos)
    with pytest.raises(RuntimeError, match="metadata must be int32"):
        attention_amd.kv_append(key, value, kc, vc, table.long(), pos)
    with pytest.raises(RuntimeError, match="all tensors must be contiguous CUDA tensors"):
        attention_amd.kv_append(key, value, kc.transpose(1, 2), vc, table, pos)
    with pytest.raises(RuntimeError, match=r"key/value must be \[B, Hkv, D\]"):
        attention_amd.kv_append(key, value[:, :1].contiguous(), kc, vc, table, pos)
    attention_amd.kv_append(key[:0], value[:0], kc, vc, table[:0], pos[:0])   # batch 0: no-op


def test_kv_append_cabi_matches_op(gpu):
    say("kv_append C ABI vs op")
    key, value, kc, vc, table, pos = (x.to(gpu) for x in _case(9, 8, 128, 16, torch.bfloat16, seed=8))
    a_k, a_v, b_k, b_v = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    attention_amd.kv_append(key, value, a_k, a_v, table, pos)
    rc = cabi.kv_append_launch(key, value, b_k, b_v, table, pos)
    assert rc == 0, cabi.error_string(rc)
    torch.cuda.synchronize()
    assert torch.equal(a_k, b_k) and torch.equal(a_v, b_v)


def test_kv_append_graph_capture_replays(gpu):
    """kv_append captured in a HIP graph: each replay writes the rows and
    positions then held in the captured input buffers, so after every replay
    (with new inputs copied in, and an eager append to other caches between
    replays) both caches equal the oracle applied replay by replay, bit for
    bit."""
    say("kv_append graph capture: replays vs oracle")
    key, value, kc, vc, table, pos = _case(7, 8, 128, 16, torch.bfloat16, seed=21)
    dkey, dval, dkc, dvc, dtable, dpos = (x.to(gpu) for x in (key, value, kc, vc, table, pos))
    okey, oval, okc, ovc, otable, opos = (x.to(gpu) for x in _case(3, 8, 128, 16, torch.bfloat16, seed=22))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        attention_amd.kv_append(dkey, dval, dkc, dvc, dtable, dpos)
    torch.cuda.synchronize()
    state_k, state_v = kc, vc
    gen = torch.Generator().manual_seed(23)
    for i in range(3):
        say(f"graph replay {i}")
        k_i = torch.randn(key.shape, generator=gen).to(key.dtype)
        v_i = torch.randn(value.shape, generator=gen).to(value.dtype)
        p_i = torch.randint(0, table.shape[1] * kc.shape[1], pos.shape, generator=gen, dtype=torch.int32)
        dkey.copy_(k_i)
        dval.copy_(v_i)
        dpos.copy_(p_i)
        graph.replay()
        torch.cuda.synchronize()
        ref_k, ref_v = oracle_kv_append(_np(k_i), _np(v_i), _np(state_k), _np(state_v), table.numpy(), p_i.numpy())
        assert np.array_equal(_np(dkc.cpu()), ref_k), f"replay {i}: k_cache differs from the oracle"
        assert np.array_equal(_np(dvc.cpu()), ref_v), f"replay {i}: v_cache differs from the oracle"
        state_k, state_v = dkc.cpu(), dvc.cpu()
        attention_amd.kv_append(okey, oval, okc, ovc, otable, opos)   # eager work between replays
        torch.cuda.synchronize()
