"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

The reference ships no golden vectors and its CUDA sources cannot be built
here, so each oracle function is fixed by: an independent float64 brute
force that is itself checked against torch's scaled_dot_product_attention
(a library routine; the reference's own parity precedent,
benchmarks/bench_all_operators.py:61-72), closed forms, index invariants,
a second (C) restatement, and rounding checks against library casts.
``test_planted_mutants_are_caught`` plants plausible mistakes in copies of
the oracle and requires each to fail one of these checks.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from attention_amd.cases import make_decode_case
from oracle import gqa_oracle as O
from oracle.cpu_path import reference_cpu_path


def case_np(lengths, hq=8, hkv=2, d=16, p=4, dtype=torch.float32, seed=0, exact=False):
    q, k, v, t, l = make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=d,
                                     block_size=p, dtype=dtype, seed=seed, exact_pool=exact)
    return q.float().numpy(), k.float().numpy(), v.float().numpy(), t.numpy(), l.numpy()


SMALL = [
    dict(lengths=[1, 5, 8, 13], hq=8, hkv=2, d=16, p=4),
    dict(lengths=[7, 0, 3], hq=6, hkv=3, d=8, p=5),
    dict(lengths=[9, 2], hq=4, hkv=4, d=12, p=3),       # MHA
    dict(lengths=[11, 4], hq=5, hkv=1, d=6, p=2),       # MQA, odd group
    dict(lengths=[16, 17], hq=4, hkv=2, d=32, p=16),
]


def sdpa_f64(q, k, v, table, lens, scale=None):
    """torch SDPA (enable_gqa) on K/V gathered by the table, float64, per sequence."""
    q_t = torch.from_numpy(np.asarray(q, dtype=np.float64))
    k_t = torch.from_numpy(np.asarray(k, dtype=np.float64))
    v_t = torch.from_numpy(np.asarray(v, dtype=np.float64))
    bsz, hq, d = q_t.shape
    _, p, hkv, _ = k_t.shape
    out = torch.zeros(bsz, hq, d, dtype=torch.float64)
    for b in range(bsz):
        L = int(lens[b])
        if L <= 0:
            continue
        n = -(-L // p)
        ids = torch.from_numpy(np.asarray(table[b, :n], dtype=np.int64))
        kk = k_t[ids].reshape(-1, hkv, d)[:L].transpose(0, 1).unsqueeze(0)   # [1,Hkv,L,D]
        vv = v_t[ids].reshape(-1, hkv, d)[:L].transpose(0, 1).unsqueeze(0)
        qq = q_t[b].unsqueeze(0).unsqueeze(2)                                # [1,Hq,1,D]
        o = F.scaled_dot_product_attention(qq, kk, vv, scale=scale, enable_gqa=True)
        out[b] = o[0, :, 0]
    return out.numpy()


@pytest.mark.parametrize("kw", SMALL)
def test_brute_force_matches_library_sdpa(kw):
    q, k, v, t, l = case_np(**kw, seed=1)
    np.testing.assert_allclose(O.brute_force_f64(q, k, v, t, l), sdpa_f64(q, k, v, t, l),
                               rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("kw", SMALL)
@pytest.mark.parametrize("scale", [None, 0.37])
def test_oracle_matches_brute_force(kw, scale):
    q, k, v, t, l = case_np(**kw, seed=2)
    got = O.oracle_decode(q, k, v, t, l, scale=scale, return_f32=True)
    np.testing.assert_allclose(got, O.brute_force_f64(q, k, v, t, l, scale=scale),
                               rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("dtype,name", [(torch.float32, "f32"), (torch.float16, "f16"),
                                        (torch.bfloat16, "bf16")])
def test_c_restatement_matches_numpy(dtype, name):
    q, k, v, t, l = case_np([1, 30, 64, 100, 0], hq=8, hkv=2, d=64, p=16, dtype=dtype, seed=3)
    ref = O.oracle_decode(q, k, v, t, l, out_dtype=name, return_f32=True)
    got = O.c_decode(q, k, v, t, l, dtype=name)
    # Both accumulate in fp32 with different summation orders: equal to within
    # fp32 noise before rounding, hence within one output ulp after it.
    ulp = {"f32": 1e-6, "f16": 2.0 ** -10, "bf16": 2.0 ** -7}[name]
    np.testing.assert_allclose(got, O.round_to(ref, name), rtol=ulp, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_torch_cpu_path_matches_oracle(dtype):
    q, k, v, t, l = make_decode_case(lengths=[3, 40, 17, 0], q_heads=8, kv_heads=2, head_dim=32,
                                     block_size=16, dtype=dtype, seed=4)
    got = reference_cpu_path(q, k, v, t, l).float().numpy()
    name = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}[dtype]
    ref = O.oracle_decode(q.float().numpy(), k.float().numpy(), v.float().numpy(), t.numpy(),
                          l.numpy(), out_dtype=name)
    tol = {"f16": 2.0 ** -10, "bf16": 2.0 ** -7, "f32": 1e-5}[name]
    np.testing.assert_allclose(got, ref, rtol=tol, atol=1e-6)


# ----------------------------------------------------------------------------
# Closed forms and special cases
# ----------------------------------------------------------------------------

def test_zero_length_gives_zeros_and_len1_gives_value():
    q, k, v, t, l = case_np([0, 1, 1], hq=4, hkv=2, d=8, p=4, seed=5)
    out = O.oracle_decode(q, k, v, t, l)
    assert not out[0].any()
    for b in (1, 2):
        for h in range(4):
            np.testing.assert_array_equal(out[b, h], v[t[b, 0], 0, h // 2])


def test_identical_keys_give_mean_of_values():
    q, k, v, t, l = case_np([10, 7], hq=4, hkv=2, d=8, p=4, seed=6)
    k[:] = k[0, 0, 0]                                   # every key equal
    out = O.oracle_decode(q, k, v, t, l, return_f32=True)
    for b, L in enumerate(l):
        toks = [(t[b, i // 4], i % 4) for i in range(L)]
        for h in range(4):
            mean = np.mean([v[p_, s, h // 2] for p_, s in toks], axis=0)
            np.testing.assert_allclose(out[b, h], mean, rtol=1e-5, atol=1e-6)


def test_dominant_key_selects_its_value():
    q, k, v, t, l = case_np([9], hq=2, hkv=1, d=8, p=4, seed=7)
    q[0, :] = 0.0
    q[0, :, 0] = 1.0
    k[:, :, :, 0] = 0.0
    tok = 6
    k[t[0, tok // 4], tok % 4, 0, 0] = 1e3
    out = O.oracle_decode(q, k, v, t, l, scale=1.0, return_f32=True)
    for h in range(2):
        np.testing.assert_allclose(out[0, h], v[t[0, tok // 4], tok % 4, 0], rtol=1e-6)


def test_head_map_is_h_div_group():
    # V constant per kv-head: q-head h must return the constant of kv-head h // g
    # (reference gqa_decode.cu:31, repeat_interleave in gqa.py:38-39).
    q, k, v, t, l = case_np([5, 9], hq=12, hkv=3, d=4, p=4, seed=8)
    for kvh in range(3):
        v[:, :, kvh, :] = 10.0 * (kvh + 1)
    out = O.oracle_decode(q, k, v, t, l, return_f32=True)
    for h in range(12):
        np.testing.assert_allclose(out[:, h], 10.0 * (h // 4 + 1), rtol=1e-6)


def test_mha_and_mqa_reduce_to_plain_attention():
    for hq, hkv in [(4, 4), (4, 1)]:
        q, k, v, t, l = case_np([6, 3], hq=hq, hkv=hkv, d=8, p=4, seed=9)
        out = O.oracle_decode(q, k, v, t, l, return_f32=True)
        for b, L in enumerate(l):
            keys = np.stack([k[t[b, i // 4], i % 4] for i in range(L)])   # [L, Hkv, D]
            vals = np.stack([v[t[b, i // 4], i % 4] for i in range(L)])
            for h in range(hq):
                kh = keys[:, h if hkv == hq else 0].astype(np.float64)
                vh = vals[:, h if hkv == hq else 0].astype(np.float64)
                s = kh @ q[b, h] / math.sqrt(8)
                w = np.exp(s - s.max())
                np.testing.assert_allclose(out[b, h], (w / w.sum()) @ vh, rtol=1e-5, atol=1e-6)


def test_default_scale_is_inverse_sqrt_head_dim():
    q, k, v, t, l = case_np([7, 12], hq=4, hkv=2, d=9, p=4, seed=10)
    np.testing.assert_array_equal(O.oracle_decode(q, k, v, t, l),
                                  O.oracle_decode(q, k, v, t, l, scale=1.0 / 3.0))
    assert not np.array_equal(O.oracle_decode(q, k, v, t, l),
                              O.oracle_decode(q, k, v, t, l, scale=1.0))


# ----------------------------------------------------------------------------
# Index invariants (bit-exact)
# ----------------------------------------------------------------------------

def test_physical_permutation_is_bitwise_invariant():
    q, k, v, t, l = case_np([5, 13, 16, 1], hq=8, hkv=2, d=16, p=4, seed=11)
    rng = np.random.default_rng(0)
    perm = rng.permutation(k.shape[0])
    inv = np.empty_like(perm)
    inv[perm] = np.arange(perm.size)
    t2 = np.where(t >= 0, inv[np.clip(t, 0, None)], -1).astype(np.int32)
    a = O.oracle_decode(q, k, v, t, l)
    b = O.oracle_decode(q, k[perm], v[perm], t2, l)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(O.c_decode(q, k, v, t, l), O.c_decode(q, k[perm], v[perm], t2, l))


def test_unused_slots_poisoned_and_padding_never_read():
    q, k, v, t, l = case_np([5, 13, 0, 1], hq=8, hkv=2, d=16, p=4, seed=12)
    used = np.zeros(k.shape[:2], dtype=bool)
    for b, L in enumerate(l):
        for i in range(L):
            used[t[b, i // 4], i % 4] = True
    kp, vp = k.copy(), v.copy()
    kp[~used] = np.nan
    vp[~used] = np.inf
    assert (t == -1).any()
    for fn in (O.oracle_decode, O.c_decode):
        a = fn(q, k, v, t, l)
        b = fn(q, kp, vp, t, l)
        assert np.isfinite(b).all()
        np.testing.assert_array_equal(a, b)


# ----------------------------------------------------------------------------
# Split partials and merge
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("splits", [1, 2, 3, 4, 7, 16])
def test_split_merge_equals_unsplit(splits):
    q, k, v, t, l = case_np([1, 5, 13, 40, 0], hq=8, hkv=2, d=16, p=4, seed=13)
    ref = O.oracle_decode(q, k, v, t, l, return_f32=True)
    merged = O.merge_partials(O.split_partials(q, k, v, t, l, splits=splits))
    np.testing.assert_allclose(merged, ref, rtol=2e-5, atol=2e-6)
    maxp = t.shape[1]
    page = lambda b, z: O.page_split_range(int(l[b]), 4, maxp, splits, 0, z)
    merged2 = O.merge_partials(O.split_partials(q, k, v, t, l, splits=splits, ranges=page))
    np.testing.assert_allclose(merged2, ref, rtol=2e-5, atol=2e-6)


def test_empty_partials_are_skipped():
    q, k, v, t, l = case_np([2, 3], hq=4, hkv=2, d=8, p=4, seed=14)
    part = O.split_partials(q, k, v, t, l, splits=8)      # most splits empty (len < S)
    assert (part[..., 1] == 0).any()
    assert np.all(part[part[..., 1] == 0][:, 0] == -np.inf)
    np.testing.assert_allclose(O.merge_partials(part), O.oracle_decode(q, k, v, t, l, return_f32=True),
                               rtol=2e-5, atol=2e-6)


def test_reference_split_ranges_cover_tokens_once():
    for L in [0, 1, 5, 16, 17, 1000]:
        for S in [1, 2, 3, 16]:
            r = [O.reference_split_range(L, S, z) for z in range(S)]
            assert r[0][0] == 0 and r[-1][1] == L
            assert all(r[i][1] == r[i + 1][0] for i in range(S - 1))


def test_page_split_ranges_are_page_aligned_and_cover():
    for L in [1, 15, 16, 17, 100, 513]:
        for S, c in [(1, 0), (3, 0), (8, 0), (40, 1), (2, 4)]:
            P, maxp = 16, 40
            if c and S * c < -(-L // P):
                continue
            r = [O.page_split_range(L, P, maxp, S, c, z) for z in range(S)]
            covered = [x for tb, te in r for x in range(tb, te)]
            assert covered == list(range(L))
            assert all(tb % P == 0 for tb, te in r if te > tb)


# ----------------------------------------------------------------------------
# Rounding
# ----------------------------------------------------------------------------

def test_bf16_rounding_matches_torch_including_ties():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(100_000).astype(np.float32) * 10
    base = (np.arange(1000, dtype=np.uint32) << 16) | 0x3F800000
    ties = (base | 0x8000).view(np.float32)           # exactly halfway cases
    x = np.concatenate([x, ties, -ties, np.array([0.0, -0.0, 1e-40, 3.4e38], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.bf16_round(x), want)
    lib = O.c_library()
    lib.oracle_f32_to_bf16.restype = __import__("ctypes").c_uint16
    lib.oracle_f32_to_bf16.argtypes = [__import__("ctypes").c_float]
    got = np.array([lib.oracle_f32_to_bf16(float(a)) for a in x[::97]], dtype=np.uint32) << 16
    np.testing.assert_array_equal(got.view(np.float32), want[::97])


def test_f16_rounding_matches_torch_and_c():
    import ctypes

    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(20_000).astype(np.float32) * 100,
                        rng.standard_normal(2_000).astype(np.float32) * 1e-6,   # subnormals
                        np.array([65504, 65519.99, 65520, 70000, 6e-8, 2.0 ** -25, 0.0],
                                 np.float32)])
    want = torch.from_numpy(x).half().float().numpy()
    np.testing.assert_array_equal(O.f16_round(x), want)
    lib = O.c_library()
    lib.oracle_f32_to_f16.restype = ctypes.c_uint16
    lib.oracle_f32_to_f16.argtypes = [ctypes.c_float]
    lib.oracle_f16_to_f32.restype = ctypes.c_float
    lib.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    bits = np.array([lib.oracle_f32_to_f16(float(a)) for a in x], dtype=np.uint16)
    np.testing.assert_array_equal(bits.view(np.float16).astype(np.float32), want)
    back = np.array([lib.oracle_f16_to_f32(int(b)) for b in bits[::13]], dtype=np.float32)
    np.testing.assert_array_equal(back, want[::13])


# ----------------------------------------------------------------------------
# Planted mistakes: each mutant of the oracle must fail a pinning check
# ----------------------------------------------------------------------------

def _mutant(kind):
    def run(q, k, v, table, lens, scale=None):
        bsz, hq, d = q.shape
        _, P, hkv, _ = k.shape
        g = hq // hkv
        scale = 1 / math.sqrt(d) if scale is None else scale
        out = np.zeros((bsz, hq, d), np.float64)
        for b in range(bsz):
            L = int(lens[b]) + (1 if kind == "len_off_by_one" else 0)
            if L <= 0:
                continue
            for h in range(hq):
                kvh = (h % hkv) if kind == "head_mod" else h // g
                rows_k, rows_v = [], []
                for t_ in range(L):
                    page = t_ // P
                    slot = (t_ // P) if kind == "slot_div" else t_ % P
                    phys = table[b, min(t_, table.shape[1] - 1) if kind == "table_by_token" else page]
                    if phys < 0:
                        phys = 0
                    rows_k.append(k[phys, slot, kvh])
                    rows_v.append(v[phys, slot, kvh])
                K = np.array(rows_k, np.float64)
                V = np.array(rows_v, np.float64)
                if kind == "swap_kv":
                    K, V = V, K
                s = K @ q[b, h]
                if kind != "no_scale":
                    s = s * scale
                w = np.exp(s - s.max())
                if kind == "unnormalized":
                    out[b, h] = w @ V
                else:
                    out[b, h] = (w / w.sum()) @ V
        return out
    return run


MUTANTS = ["head_mod", "slot_div", "table_by_token", "swap_kv", "no_scale", "unnormalized",
           "len_off_by_one"]


@pytest.mark.parametrize("kind", MUTANTS)
def test_planted_mutants_are_caught(kind):
    """The pin (agreement with library SDPA on a ragged, permuted, GQA case)
    rejects each planted mistake."""
    q, k, v, t, l = case_np([3, 6, 9], hq=8, hkv=2, d=8, p=4, seed=15)
    ref = sdpa_f64(q, k, v, t, l)
    np.testing.assert_allclose(O.brute_force_f64(q, k, v, t, l), ref, rtol=1e-10, atol=1e-12)
    got = _mutant(kind)(q, k, v, t, l)
    assert not np.allclose(got, ref, rtol=1e-3, atol=1e-4), f"mutant {kind} not detected"


# ----------------------------------------------------------------------------
# kv_append oracle (reference csrc/cuda/cache/kv_append.cu:11-19)
# ----------------------------------------------------------------------------

def test_kv_append_oracle_matches_torch_indexed_assignment():
    """The reference's own check (benchmarks/bench_all_operators.py:100-104):
    k[page, slot] = key with page = table[b, pos // P], slot = pos % P."""
    gen = torch.Generator().manual_seed(3)
    B, Hkv, D, P, maxP, N = 6, 3, 5, 4, 4, 40
    kc = torch.randn(N, P, Hkv, D, generator=gen)
    vc = torch.randn(N, P, Hkv, D, generator=gen)
    table = torch.randperm(N, generator=gen)[:B * maxP].view(B, maxP).int()
    pos = torch.tensor([0, 3, 4, 15, 7, 9], dtype=torch.int32)
    key = torch.randn(B, Hkv, D, generator=gen)
    value = torch.randn(B, Hkv, D, generator=gen)
    got_k, got_v = O.oracle_kv_append(key.numpy(), value.numpy(), kc.numpy(), vc.numpy(), table.numpy(),
                                      pos.numpy())
    idx = torch.arange(B)
    page = table[idx, (pos // P).long()].long()
    slot = (pos % P).long()
    ref_k, ref_v = kc.clone(), vc.clone()
    ref_k[page, slot] = key
    ref_v[page, slot] = value
    assert np.array_equal(got_k, ref_k.numpy()) and np.array_equal(got_v, ref_v.numpy())


def test_kv_append_oracle_touches_only_destinations_and_skips_invalid():
    rng = np.random.default_rng(0)
    kc = rng.standard_normal((10, 4, 2, 3)).astype(np.float32)
    vc = rng.standard_normal((10, 4, 2, 3)).astype(np.float32)
    table = np.array([[1, 2], [3, -1], [9, 10]], dtype=np.int32)   # 10 is out of the pool
    pos = np.array([5, 4, 4], dtype=np.int32)                      # b1 -> page -1, b2 -> page 10
    key = np.full((3, 2, 3), 7.0, np.float32)
    val = np.full((3, 2, 3), 8.0, np.float32)
    nk, nv = O.oracle_kv_append(key, val, kc, vc, table, pos)
    changed = np.argwhere(np.any(nk != kc, axis=(2, 3)))
    assert changed.tolist() == [[2, 1]]                             # only (table[0][1], 5 % 4)
    assert np.all(nk[2, 1] == 7.0) and np.all(nv[2, 1] == 8.0)
    for bad in ([-1, 8, 100], [8, -5, 9]):                          # all outside [0, maxP*P)
        k2, v2 = O.oracle_kv_append(key, val, kc, vc, table, np.array(bad, np.int32))
        assert np.array_equal(k2, kc) and np.array_equal(v2, vc)


# ----------------------------------------------------------------------------
# Metadata validation oracle (reference attention/validation.py:5-39): each
# failure kind built by hand, and the order between them.
# ----------------------------------------------------------------------------

def _meta():
    table = np.array([[0, 1, -1], [2, 3, 4], [5, -1, -1]], dtype=np.int32)
    lens = np.array([20, 33, 1], dtype=np.int32)   # P = 16: 2, 3 and 1 used pages
    return table, lens


def test_validation_oracle_accepts_valid_metadata():
    table, lens = _meta()
    assert O.oracle_validate_metadata(table, lens, 16, 6) is None
    assert O.oracle_validate_metadata(table, lens, 16, 6, positions=np.array([20, 33, 1])) is None


@pytest.mark.parametrize("edit,expected", [
    (lambda t, l, p: l.__setitem__(1, 49), "invalid length at batch 1"),          # 49 > 3*16
    (lambda t, l, p: l.__setitem__(0, -1), "invalid length at batch 0"),
    (lambda t, l, p: t.__setitem__((1, 2), 6), "invalid block at batch 1, page 2"),
    (lambda t, l, p: t.__setitem__((0, 1), -1), "invalid block at batch 0, page 1"),
    (lambda t, l, p: t.__setitem__((0, 2), 99), None),                              # unused page never read
    (lambda t, l, p: p.__setitem__(2, 48), "invalid append position at batch 2"),  # 48 = 3*16
    (lambda t, l, p: p.__setitem__(2, 16), "invalid append page at batch 2"),      # row 2, page 1 is -1
])
def test_validation_oracle_failure_kinds(edit, expected):
    table, lens = _meta()
    pos = np.array([20, 33, 1], dtype=np.int32)
    edit(table, lens, pos)
    assert O.oracle_validate_metadata(table, lens, 16, 6, positions=pos) == expected


def test_validation_oracle_conflict_is_reported_at_the_later_sequence():
    table = np.array([[0, 1, -1], [2, 3, 4], [5, 3, -1]], dtype=np.int32)
    lens = np.array([20, 33, 17], dtype=np.int32)
    # b1 writes (page 3, slot 1) at position 17; b2 at position 17 writes the same slot.
    assert O.oracle_validate_metadata(table, lens, 16, 6, positions=np.array([20, 17, 17])) == \
        "conflicting append destinations"
    # Same page, different slot: no conflict.
    assert O.oracle_validate_metadata(table, lens, 16, 6, positions=np.array([20, 17, 18])) is None
    # An earlier failure wins over the conflict.
    assert O.oracle_validate_metadata(table, np.array([20, 99, 17]), 16, 6,
                                      positions=np.array([20, 17, 17])) == "invalid length at batch 1"


def test_validation_oracle_reports_first_sequence_and_check_order():
    table, lens = _meta()
    pos = np.array([20, 33, 1], dtype=np.int32)
    table[2, 0] = 9                    # b2: bad block
    lens[1] = 100                      # b1: bad length (earlier sequence wins)
    assert O.oracle_validate_metadata(table, lens, 16, 6, positions=pos) == "invalid length at batch 1"
    lens[1] = 33
    pos[1] = 99                        # b1: bad position, but b1's pages are checked first
    table[1, 0] = -3
    assert O.oracle_validate_metadata(table, lens, 16, 6, positions=pos) == "invalid block at batch 1, page 0"
