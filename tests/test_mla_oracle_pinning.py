"""Pins the MLA oracle (oracle/mla_oracle.py) before it is trusted as the
checker of the MLA kernels.

The reference ships no golden vectors for MLA (its benchmarks compare the
CUDA ops with torch expressions at runtime, bench_attention_primitives.py:
46-85), so each oracle function is fixed by:
  * an independent evaluation order: the non-absorbed (direct) form with
    per-head up-projected keys and values on contiguous latent sequences,
    which the reference's own reference computes next to the absorbed one
    (attention/reference/mla.py:11-16, :30-34);
  * a reduction to the GQA oracle (already pinned against torch SDPA): latent
    attention is multi-query attention over [latent | rope] keys and
    [latent | 0] values;
  * closed forms (one visible token, identical rows, empty rows), causal
    and index-list identities, brute-force loops on tiny inputs, and the
    reference benchmark's indexed-assignment definition of the cache write
    (bench_attention_primitives.py:52-53).
``test_planted_mutants_are_caught`` plants plausible mistakes and requires
each to fail one of these checks.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from attention_amd.cases import make_mla_case
from oracle import gqa_oracle as G
from oracle import mla_oracle as M
from oracle.cpu_path import reference_mla_cpu_path


def case(lengths, q_len=1, heads=4, dn=8, dc=16, dr=8, dv=8, p=4, seed=0, num_indices=None):
    c = make_mla_case(lengths=lengths, q_len=q_len, heads=heads, nope_dim=dn, latent_dim=dc, rope_dim=dr,
                      value_dim=dv, block_size=p, dtype=torch.float32, seed=seed, num_indices=num_indices)
    return {k: (None if v is None else v.numpy()) for k, v in c.items()}


def contiguous_latent(c, dc):
    """[B, Lmax, Dc] latent and [B, Lmax, Dr] rope keys read back through the
    page table (zeros past each length)."""
    cache, table, lens = c["cache"], c["table"], c["lens"]
    bsz = len(lens)
    lmax = max(1, int(lens.max()))
    lat = np.zeros((bsz, lmax, dc))
    rope = np.zeros((bsz, lmax, cache.shape[-1] - dc))
    for b in range(bsz):
        toks = np.arange(int(lens[b]))
        rows = M.gather_rows(cache, table[b], toks)
        lat[b, :len(toks)] = rows[:, :dc]
        rope[b, :len(toks)] = rows[:, dc:]
    return lat, rope


def ends_of(c, causal=True):
    cap = c["table"].shape[1] * c["cache"].shape[1]
    return np.array([[M.attend_end(int(c["lens"][b]), int(c["positions"][b, t]), causal, cap)
                      for t in range(c["positions"].shape[1])] for b in range(len(c["lens"]))])


DECODE_CASES = [
    dict(lengths=[1, 5, 8, 13], q_len=1),
    dict(lengths=[7, 0, 16], q_len=3, heads=3, dn=6, dc=10, dr=2, dv=5, p=5),
    dict(lengths=[20, 9], q_len=2, heads=2, dn=16, dc=32, dr=16, dv=16, p=8),
]


@pytest.mark.parametrize("kw", DECODE_CASES)
@pytest.mark.parametrize("sparse", [False, True])
def test_absorbed_oracle_matches_direct_form(kw, sparse):
    c = case(num_indices=4 if sparse else None, **kw)
    dc = c["w_uk"].shape[-1]
    scale = M.default_mla_scale(c["q_nope"].shape[-1], c["q_rope"].shape[-1])
    got = M.oracle_mla_decode(c["q_nope"], c["q_rope"], c["cache"], c["table"], c["lens"], c["positions"],
                              c["w_uk"], c["w_uv"], scale=scale, indices=c["indices"], out_dtype="f32")
    lat, rope = contiguous_latent(c, dc)
    ref = M.direct_mla_f64(c["q_nope"], c["q_rope"], lat, rope, c["w_uk"], c["w_uv"], ends_of(c), scale,
                           indices=c["indices"])
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-6)


def test_direct_form_matches_torch_sdpa_per_head():
    """The direct form itself against torch SDPA on explicit per-head K/V."""
    c = case([9, 4], q_len=1, heads=3, dn=5, dc=7, dr=3, dv=4, p=3)
    dc = 7
    lat, rope = contiguous_latent(c, dc)
    scale = 0.3
    ref = M.direct_mla_f64(c["q_nope"], c["q_rope"], lat, rope, c["w_uk"], c["w_uv"], ends_of(c), scale)
    for b, L in enumerate(c["lens"]):
        L = int(L)
        k = np.einsum("sc,hdc->hsd", lat[b, :L], c["w_uk"])                       # [H, L, Dn]
        k = np.concatenate([k, np.broadcast_to(rope[b, :L], (3, L, 3))], axis=-1)
        v = np.einsum("sc,hvc->hsv", lat[b, :L], c["w_uv"])
        q = np.concatenate([c["q_nope"][b, 0], c["q_rope"][b, 0]], axis=-1)[:, None, :].astype(np.float64)
        o = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(q), torch.from_numpy(k),
                                                             torch.from_numpy(np.ascontiguousarray(v)),
                                                             scale=scale)
        np.testing.assert_allclose(ref[b, 0], o[:, 0].numpy(), rtol=1e-10, atol=1e-12)


def test_latent_attention_is_mqa_over_latent_rows():
    """mla_attend == the (pinned) GQA oracle with one kv-head: keys are whole
    cache rows, values are the rows with the rope part zeroed."""
    c = case([13, 6, 1, 25], q_len=1, heads=6, dc=12, dr=4, p=4)
    dc = 12
    qa = np.random.default_rng(0).standard_normal((4, 1, 6, dc)).astype(np.float32)
    got = M.oracle_mla_attend(qa, c["q_rope"], c["cache"], c["table"], c["lens"], c["positions"], 0.2, causal=False,
                              out_dtype="f32")
    k = c["cache"][:, :, None, :]
    v = k.copy()
    v[..., dc:] = 0
    q = np.concatenate([qa[:, 0], c["q_rope"][:, 0]], axis=-1)
    ref = G.oracle_decode(q, k, v, c["table"], c["lens"], scale=0.2)
    np.testing.assert_allclose(got[:, 0], ref[..., :dc], rtol=2e-5, atol=2e-6)


def test_causal_equals_shortened_lengths_and_negative_positions_give_zeros():
    c = case([10, 10, 10], q_len=2, heads=2, p=4)
    qa = np.random.default_rng(1).standard_normal((3, 2, 2, 16)).astype(np.float32)
    pos = np.array([[3, 9], [0, 20], [-1, -5]], dtype=np.int32)
    got = M.oracle_mla_attend(qa, c["q_rope"], c["cache"], c["table"], c["lens"], pos, 0.3, causal=True)
    for b in range(3):
        for t in range(2):
            lens2 = np.array([min(10, max(0, pos[b, t] + 1))])
            ref = M.oracle_mla_attend(qa[b:b + 1, t:t + 1], c["q_rope"][b:b + 1, t:t + 1], c["cache"],
                                      c["table"][b:b + 1], lens2, pos[b:b + 1, t:t + 1], 0.3, causal=False)
            np.testing.assert_array_equal(got[b, t], ref[0, 0])
    assert not got[2].any()                                   # no visible token: zeros
    noncausal = M.oracle_mla_attend(qa, c["q_rope"], c["cache"], c["table"], c["lens"], pos, 0.3, causal=False)
    np.testing.assert_array_equal(noncausal[1, 1], got[1, 1])   # pos beyond len: full length


def test_index_lists_match_dense_and_brute_force():
    c = case([11, 7], q_len=1, heads=3, dc=8, dr=4, p=3)
    qa = np.random.default_rng(2).standard_normal((2, 1, 3, 8)).astype(np.float32)
    dense = M.oracle_mla_attend(qa, c["q_rope"], c["cache"], c["table"], c["lens"], c["positions"], 0.4)
    full = np.full((2, 1, 14), -1, dtype=np.int32)
    full[0, 0, :11] = np.arange(11)[::-1]
    full[1, 0, :7] = np.arange(7)
    full[1, 0, 7:9] = [7, 100]                                # past the length: ignored
    np.testing.assert_allclose(M.oracle_mla_attend(qa, c["q_rope"], c["cache"], c["table"], c["lens"],
                                                   c["positions"], 0.4, indices=full), dense, rtol=1e-6, atol=1e-7)
    # A subset by brute force (plain loops over the listed tokens).
    sub = np.array([[[5, -1, 0, 9]], [[6, 2, 2, -3]]], dtype=np.int32)   # repeated 2 counts twice
    got = M.oracle_mla_attend(qa, c["q_rope"], c["cache"], c["table"], c["lens"], c["positions"], 0.4, indices=sub)
    for b in range(2):
        rows = []
        for tok in sub[b, 0]:
            if 0 <= tok < c["lens"][b]:
                page = c["table"][b, tok // 3]
                rows.append(c["cache"][page, tok % 3].astype(np.float64))
        for h in range(3):
            s = [0.4 * (float(np.dot(qa[b, 0, h], r[:8])) + float(np.dot(c["q_rope"][b, 0, h], r[8:]))) for r in rows]
            w = np.exp(np.array(s) - max(s))
            w /= w.sum()
            ref = sum(wi * r[:8] for wi, r in zip(w, rows))
            np.testing.assert_allclose(got[b, 0, h], ref, rtol=1e-6, atol=1e-7)


def test_closed_forms():
    c = case([1, 6], q_len=1, heads=2, dc=8, dr=4, p=3)
    qa = np.random.default_rng(3).standard_normal((2, 1, 2, 8)).astype(np.float32)
    got = M.oracle_mla_attend(qa, c["q_rope"], c["cache"], c["table"], c["lens"], c["positions"], 0.5,
                              out_dtype="bf16")
    row0 = c["cache"][c["table"][0, 0], 0, :8]
    np.testing.assert_array_equal(got[0, 0, 0], G.bf16_round(row0))     # one token: its latent, rounded once
    same = c["cache"].copy()
    for i in range(6):                                                   # identical rows: that row
        same[c["table"][1, i // 3], i % 3] = same[c["table"][1, 0], 0]
    got = M.oracle_mla_attend(qa, c["q_rope"], same, c["table"], c["lens"], c["positions"], 0.5)
    np.testing.assert_allclose(got[1, 0, 1], same[c["table"][1, 0], 0, :8], rtol=1e-6)


def test_projection_identities():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 3, 4, 5)).astype(np.float32)
    eye = np.broadcast_to(np.eye(5, dtype=np.float32), (4, 5, 5))
    np.testing.assert_array_equal(M.oracle_mla_project(x, eye, True), x)
    np.testing.assert_array_equal(M.oracle_mla_project(x, eye, False), x)
    w = rng.standard_normal((4, 5, 7)).astype(np.float32)
    got = M.oracle_mla_project(x, w, True)
    for b, t, h, o in [(0, 0, 0, 0), (1, 2, 3, 6), (0, 1, 2, 3)]:
        ref = sum(float(x[b, t, h, k]) * float(w[h, k, o]) for k in range(5))
        assert abs(got[b, t, h, o] - ref) < 1e-5
    wv = rng.standard_normal((4, 7, 5)).astype(np.float32)               # value layout: w[h, o, k]
    got = M.oracle_mla_project(x, wv, False)
    ref = sum(float(x[1, 0, 2, k]) * float(wv[2, 6, k]) for k in range(5))
    assert abs(got[1, 0, 2, 6] - ref) < 1e-5


def test_latent_write_matches_indexed_assignment():
    rng = np.random.default_rng(5)
    cache = rng.standard_normal((5, 4, 7)).astype(np.float32)
    lat = rng.standard_normal((6, 5)).astype(np.float32)
    rope = rng.standard_normal((6, 2)).astype(np.float32)
    slots = np.array([19, 0, 7, 3, 12, 8], dtype=np.int64)
    got = M.oracle_latent_kv_write(lat, rope, cache, slots)
    ref = cache.copy().reshape(-1, 7)
    ref[slots] = np.concatenate([lat, rope], axis=1)      # bench_attention_primitives.py:53
    np.testing.assert_array_equal(got.reshape(-1, 7), ref)
    bad = slots.copy()
    bad[[1, 4]] = [-1, 20]
    got = M.oracle_latent_kv_write(lat, rope, cache, bad)
    keep = np.ones(6, dtype=bool)
    keep[[1, 4]] = False
    ref = cache.copy().reshape(-1, 7)
    ref[bad[keep]] = np.concatenate([lat, rope], axis=1)[keep]
    np.testing.assert_array_equal(got.reshape(-1, 7), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_torch_mla_cpu_path_matches_oracle(dtype):
    """The timed MLA CPU baseline (oracle/cpu_path.reference_mla_cpu_path, the
    torch CPU expressions of reference attention/reference/mla.py:6-34 read
    through the page table) computes the attention of the pinned oracle:
    fp32 within fp32 accumulation error; bf16 within one rounding of the
    output, since the CPU path rounds once at the end where the oracle, fed
    fp32 here, rounds nowhere before it.  Empty rows, causal queries (3 per
    row, the first ones seeing fewer tokens) and a permuted page pool."""
    c = make_mla_case(lengths=[0, 1, 7, 33, 20], q_len=3, heads=4, nope_dim=8, latent_dim=16, rope_dim=8,
                      value_dim=8, block_size=4, dtype=dtype, seed=5)
    scale = M.default_mla_scale(8, 8)
    got = reference_mla_cpu_path(c["q_nope"], c["q_rope"], c["cache"], c["table"], c["lens"], c["positions"],
                                 c["w_uk"], c["w_uv"], scale=scale)
    assert got.dtype == dtype and got.shape == (5, 3, 4, 8)
    got = got.float().numpy()
    f = lambda x: x.float().numpy()
    ref = M.oracle_mla_decode(f(c["q_nope"]), f(c["q_rope"]), f(c["cache"]), c["table"].numpy(), c["lens"].numpy(),
                              c["positions"].numpy(), f(c["w_uk"]), f(c["w_uv"]), scale, out_dtype="f32")
    assert np.all(got[0] == 0.0)                                  # length 0: zeros
    if dtype == torch.float32:
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)
    else:
        ref16 = torch.from_numpy(ref).to(torch.bfloat16).float().numpy()
        assert np.all(np.abs(got - ref16) <= 2.0 ** -7 * np.abs(ref16) + 1e-6)


def test_default_scale():
    assert M.default_mla_scale(128, 64) == pytest.approx(1 / np.sqrt(192))


# ---- planted mutants --------------------------------------------------------


def _mutant(kind):
    """A copy of oracle_mla_attend / oracle_mla_project with one plausible mistake."""
    def attend(q, q_rope, cache, table, lens, positions, scale, causal=True, indices=None, out_dtype="f32",
               return_f64=False):
        q = np.asarray(q, dtype=np.float64)
        qr = np.asarray(q_rope, dtype=np.float64)
        cache = np.asarray(cache, dtype=np.float64)
        bsz, tq, heads, dc = q.shape
        page = cache.shape[1]
        out = np.zeros((bsz, tq, heads, dc))
        for b in range(bsz):
            for t in range(tq):
                L = int(lens[b])
                pos = int(positions[b, t])
                if causal:
                    end = min(L, max(0, pos)) if kind == "causal_off_by_one" else min(L, max(0, pos + 1))
                else:
                    end = L
                toks = M.row_tokens(end, None if indices is None else indices[b, t])
                if toks.size == 0:
                    continue
                phys = table[b][toks // page]
                slot = toks // page if kind == "slot_swap" else toks % page
                rows = cache.reshape(-1, cache.shape[-1])[phys * page + slot]
                s = q[b, t] @ rows[:, :dc].T
                if kind != "no_rope":
                    s = s + qr[b, t] @ rows[:, dc:].T
                s = s * (scale if kind != "no_scale" else 1.0)
                s -= s.max(axis=1, keepdims=True)
                p = np.exp(s)
                p /= p.sum(axis=1, keepdims=True)
                vals = rows[:, :dc] if kind != "value_from_tail" else rows[:, -dc:]
                out[b, t] = p @ vals
        return out.astype(np.float32)
    return attend


MUTANTS = ["causal_off_by_one", "slot_swap", "no_rope", "no_scale", "value_from_tail"]


@pytest.mark.parametrize("kind", MUTANTS)
def test_planted_mutants_are_caught(kind, monkeypatch):
    monkeypatch.setattr(M, "oracle_mla_attend", _mutant(kind))
    failures = 0
    for test in (lambda: test_absorbed_oracle_matches_direct_form(DECODE_CASES[2], False),
                 lambda: test_absorbed_oracle_matches_direct_form(DECODE_CASES[1], False),
                 test_latent_attention_is_mqa_over_latent_rows,
                 test_index_lists_match_dense_and_brute_force):
        try:
            test()
        except AssertionError:
            failures += 1
    assert failures > 0, f"mutant {kind} passed every check"


def test_unmutated_oracle_passes_the_mutant_harness():
    assert _mutant("none") is not None
    test_absorbed_oracle_matches_direct_form(DECODE_CASES[2], False)
