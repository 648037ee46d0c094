"""GPU parity of the paged MLA decode operators (reference
csrc/cuda/mla/mla.cu:16-198, attention/mla.py:16-53) against the CPU oracle
(oracle/mla_oracle.py).  Every case prints its name first.

Tolerance (north_star, 16-bit): |got - ref| <= 2e-3 + 1e-2 |ref|; fp32:
1e-4 + 1e-4 |ref| (the reference's MLA benchmark tolerance, 1e-4 to 5e-4).
Copies (latent_kv_write) are bitwise.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import attention_amd
from attention_amd import cabi
from attention_amd.cases import make_mla_case
from oracle.mla_oracle import (default_mla_scale, oracle_latent_kv_write, oracle_mla_attend, oracle_mla_decode,
                               oracle_mla_project)

pytestmark = pytest.mark.gpu

QD_FLAG_FORCE_GENERIC = 1
QD_FLAG_MLA_STAGED = 2
QD_FLAG_MLA_WAVE = 4
TOL = {torch.bfloat16: (2e-3, 1e-2), torch.float16: (2e-3, 1e-2), torch.float32: (1e-4, 1e-4)}
ODT = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def say(msg):
    print(f"[case] {msg}", flush=True)


def _np(x):
    return None if x is None else x.float().cpu().numpy() if x.is_floating_point() else x.cpu().numpy()


def _close(got, ref, dtype, what):
    atol, rtol = TOL[dtype]
    got = got.float().cpu().numpy()
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} outside tolerance, max abs err {err.max():.3e} "
                           f"at {np.unravel_index(err.argmax(), err.shape)}")


def _case(gpu, **kw):
    return make_mla_case(device=gpu, **kw)


def _absorbed(c, dtype):
    """The absorbed query as the oracle computes it (rounded to dtype)."""
    return torch.from_numpy(oracle_mla_project(_np(c["q_nope"]), _np(c["w_uk"]), True, ODT[dtype]))


def _oracle_attend(c, qa, scale, causal=True, indices=None, dtype=torch.bfloat16):
    return oracle_mla_attend(_np(qa), _np(c["q_rope"]), _np(c["cache"]), _np(c["table"]), _np(c["lens"]),
                             _np(c["positions"]), scale, causal, _np(indices), ODT[dtype])


# (name, case kwargs)
ATTEND_SHAPES = [
    ("ref-bench-fp32", dict(lengths=[64], q_len=4, heads=4, nope_dim=16, latent_dim=32, rope_dim=8, value_dim=16,
                            block_size=16, dtype=torch.float32)),
    ("ref-bench-bf16", dict(lengths=[512, 1024], q_len=1, heads=4, nope_dim=32, latent_dim=64, rope_dim=16,
                            value_dim=32, block_size=16, dtype=torch.bfloat16)),
    ("deepseek-h16", dict(lengths=[1, 17, 300, 1031], q_len=1, heads=16, block_size=64, dtype=torch.bfloat16)),
    ("deepseek-h16-t3-empty", dict(lengths=[0, 16, 2500, 33], q_len=3, heads=16, block_size=16,
                                   dtype=torch.bfloat16)),
    ("deepseek-h12-fp16", dict(lengths=[700, 64, 1, 129, 4000], q_len=1, heads=12, block_size=32,
                               dtype=torch.float16)),
    ("deepseek-h128", dict(lengths=[0, 65, 777, 2048], q_len=1, heads=128, block_size=64, dtype=torch.bfloat16)),
    ("deepseek-h64-fp16-t2", dict(lengths=[0, 40, 1500, 3000], q_len=2, heads=64, block_size=16,
                                  dtype=torch.float16)),
    ("h20-fp16-p16", dict(lengths=[5, 200, 33], q_len=2, heads=20, block_size=16, dtype=torch.float16)),
    ("deepseek-h64-fp16-p32", dict(lengths=[0, 40, 1500, 3000, 31, 32, 33], q_len=2, heads=64, block_size=32,
                                   dtype=torch.float16)),
    ("deepseek-h96-p64", dict(lengths=[2100, 1, 700], q_len=1, heads=96, block_size=64, dtype=torch.bfloat16)),
    ("dc192-dr32", dict(lengths=[90, 257], q_len=1, heads=24, latent_dim=192, rope_dim=32, block_size=32,
                        dtype=torch.bfloat16)),
]


@pytest.mark.parametrize("name,kw", ATTEND_SHAPES, ids=[s[0] for s in ATTEND_SHAPES])
@pytest.mark.parametrize("variant", ["auto", "split1", "split3", "generic", "staged", "wave"])   # split<n>: forced partition
def test_mla_attend_matches_oracle(gpu, name, kw, variant):
    say(f"mla_attend {name} {variant}")
    dtype = kw["dtype"]
    c = _case(gpu, **kw)
    qa = _absorbed(c, dtype).to(dtype).to(gpu)
    B, T, H, Dc = qa.shape
    scale = default_mla_scale(c["q_nope"].shape[-1], c["q_rope"].shape[-1])
    out = torch.empty_like(qa)
    splits = {"auto": 0, "split1": 1, "split3": 3, "generic": 0, "staged": 0, "wave": 0}[variant]
    flags = {"generic": QD_FLAG_FORCE_GENERIC, "staged": QD_FLAG_MLA_STAGED, "wave": QD_FLAG_MLA_WAVE}.get(variant, 0)
    rc = cabi.mla_attend(qa, c["q_rope"], c["cache"], c["table"], c["lens"], c["positions"], out, scale=scale,
                         splits=splits, flags=flags)
    assert rc == 0, cabi.error_string(rc)
    torch.cuda.synchronize()
    _close(out, _oracle_attend(c, qa, scale, dtype=dtype), dtype, name)


def test_mla_attend_kernel_choice(gpu):
    say("mla_attend plan on the device")
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    kind, wgs, groups = cabi.mla_attend_info(32, 1, 128, 512, 64, 64, 64)
    assert kind == 3 and groups == 2 and wgs * groups == cus      # shared-tile kernel: 2 groups of 64 heads
    kind, wgs, groups = cabi.mla_attend_info(32, 1, 64, 512, 64, 32, 64)
    assert kind == 3 and groups == 1
    assert cabi.mla_attend_info(32, 1, 64, 512, 64, 16, 64)[0] == 2   # 16-token pages: wave-streamed kernel
    assert cabi.mla_attend_info(32, 1, 32, 512, 64, 64, 64)[0] == 2   # 32 heads: wave-streamed kernel
    kind, wgs, groups = cabi.mla_attend_info(32, 1, 128, 512, 64, 64, 64, flags=QD_FLAG_MLA_WAVE)
    assert kind == 2 and groups == 8 and wgs * groups <= 256      # wave-streamed kernel, 8 head groups
    kind, wgs, groups = cabi.mla_attend_info(32, 1, 20, 512, 64, 64, 64)
    assert kind == 2 and groups == 2 and wgs * groups <= 256      # 2 head groups, the second of 4 heads
    kind, wgs, groups = cabi.mla_attend_info(32, 1, 128, 512, 64, 64, 64, flags=QD_FLAG_MLA_STAGED)
    assert kind == 1 and groups >= 1 and wgs * groups <= 2 * 256
    assert cabi.mla_attend_info(128, 1, 16, 512, 64, 64, 64)[0] == 2       # wave-streamed kernel
    assert cabi.mla_attend_info(128, 1, 16, 512, 64, 64, 64, flags=QD_FLAG_MLA_STAGED)[0] == 1
    assert cabi.mla_attend_info(128, 1, 16, 512, 64, 64, 64, nk=32)[0] == 1  # index lists: staged kernel
    assert cabi.mla_attend_info(128, 1, 16, 512, 64, 8, 64)[0] == 1         # pages of 8 tokens
    assert cabi.mla_attend_info(1, 4, 4, 32, 8, 16, 4, dtype=0)[0] == 0      # fp32: VALU kernel
    assert cabi.mla_attend_info(1, 1, 4, 36, 8, 16, 4)[0] == 0              # Dc % 8 != 0


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("kernel", ["mfma", "generic"])
def test_mla_attend_sparse_and_causal(gpu, causal, kernel):
    say(f"mla_attend sparse causal={causal} {kernel}")
    dtype = torch.bfloat16
    c = _case(gpu, lengths=[40, 300, 1, 0, 129], q_len=3, heads=32, block_size=16, dtype=dtype, num_indices=48)
    idx = c["indices"].clone()
    idx[0, 0, :3] = torch.tensor([-1, 10_000, 39], dtype=torch.int32)   # ignored, ignored, last visible
    idx[1, 2, 5] = -7
    qa = _absorbed(c, dtype).to(dtype).to(gpu)
    scale = 0.07
    flags = QD_FLAG_FORCE_GENERIC if kernel == "generic" else 0
    for sparse in (None, idx):
        out = torch.empty_like(qa)
        rc = cabi.mla_attend(qa, c["q_rope"], c["cache"], c["table"], c["lens"], c["positions"], out, scale=scale,
                             indices=sparse, causal=causal, flags=flags, splits=2)
        assert rc == 0, cabi.error_string(rc)
        torch.cuda.synchronize()
        _close(out, _oracle_attend(c, qa, scale, causal, sparse, dtype), dtype, f"sparse={sparse is not None}")


@pytest.mark.parametrize("seed", range(1, 9))
@pytest.mark.parametrize("heads,flags", [(16, 0), (16, QD_FLAG_MLA_STAGED), (64, 0)], ids=["wave", "staged", "shared"])
def test_mla_attend_bf16_accuracy_over_seeds(gpu, heads, flags, seed):
    """Random DeepSeek-shaped inputs with short rows in bf16: with one bf16
    rounding of the softmax weights in the PV product, 3 of these 8 seeds
    landed past the 16-bit bar (worst 1.23x); the kernels carry the weights
    as hi + lo and stay under 0.5x."""
    say(f"mla_attend bf16 accuracy seed {seed} heads {heads} flags {flags}")
    dtype = torch.bfloat16
    c = _case(gpu, lengths=[3, 300, 1031, 2500], q_len=1, heads=heads, block_size=64, dtype=dtype, seed=seed)
    qa = _absorbed(c, dtype).to(dtype).to(gpu)
    scale = default_mla_scale(c["q_nope"].shape[-1], c["q_rope"].shape[-1])
    out = torch.empty_like(qa)
    rc = cabi.mla_attend(qa, c["q_rope"], c["cache"], c["table"], c["lens"], c["positions"], out, scale=scale,
                         flags=flags)
    assert rc == 0, cabi.error_string(rc)
    torch.cuda.synchronize()
    _close(out, _oracle_attend(c, qa, scale, dtype=dtype), dtype, f"seed {seed}")


@pytest.mark.parametrize("dtype,mag", [(torch.bfloat16, 1e4), (torch.bfloat16, 1e-4), (torch.float16, 8e3),
                                       (torch.float16, 1e-3)], ids=["bf16-1e4", "bf16-1e-4", "f16-8e3", "f16-1e-3"])
@pytest.mark.parametrize("heads,flags,splits", [(64, 0, 0), (64, 0, 3), (16, 0, 3), (64, QD_FLAG_MLA_WAVE, 3),
                                                (64, QD_FLAG_MLA_STAGED, 3), (64, QD_FLAG_FORCE_GENERIC, 3)],
                         ids=["shared-auto", "shared-split3", "wave-h16", "wave-h64", "staged", "generic"])
def test_mla_attend_latent_magnitude(gpu, dtype, mag, heads, flags, splits):
    """Latent rows scaled by ``mag`` and the absorbed query by ``1/mag``: the
    scores stay put and the output scales by ``mag``.  The split rows' partial
    results pass through 16-bit storage in some kernels, so values far above
    the fp16 range (1e4 latent rows summed over thousands of tokens) and far
    below it must come back with the 16-bit tolerance relative to ``mag``."""
    say(f"mla_attend latent magnitude {mag} {ODT[dtype]} heads={heads} flags={flags} splits={splits}")
    c = _case(gpu, lengths=[3000, 700, 1, 1500], q_len=1, heads=heads, block_size=64, dtype=dtype, seed=11)
    Dc = c["w_uk"].shape[-1]
    c["cache"][..., :Dc] = (c["cache"][..., :Dc].float() * mag).to(dtype)
    qa = (_absorbed(c, dtype).float() / mag).to(dtype).to(gpu)
    scale = default_mla_scale(c["q_nope"].shape[-1], c["q_rope"].shape[-1])
    out = torch.empty_like(qa)
    rc = cabi.mla_attend(qa, c["q_rope"], c["cache"], c["table"], c["lens"], c["positions"], out, scale=scale,
                         splits=splits, flags=flags)
    assert rc == 0, cabi.error_string(rc)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    ref = _oracle_attend(c, qa, scale, dtype=dtype)
    _close(out.float() / mag, ref / mag, dtype, f"magnitude {mag}")


@pytest.mark.parametrize("heads,flags", [(64, 0), (64, QD_FLAG_MLA_WAVE), (64, QD_FLAG_MLA_STAGED), (16, 0)],
                         ids=["shared-h64", "wave-h64", "staged-h64", "wave-h16"])
def test_mla_attend_page_permutation_and_poison_bitwise(gpu, heads, flags):
    """Physical page order and unreferenced cache contents do not change a bit
    of the output (index handling is exact)."""
    say(f"mla_attend permutation + poison invariance heads={heads} flags={flags}")
    dtype = torch.bfloat16
    c = _case(gpu, lengths=[100, 513, 64], q_len=1, heads=heads, block_size=64, dtype=dtype)
    qa = _absorbed(c, dtype).to(dtype).to(gpu)
    scale = 0.05

    def run(cache, table):
        out = torch.empty_like(qa)
        rc = cabi.mla_attend(qa, c["q_rope"], cache, table, c["lens"], c["positions"], out, scale=scale, splits=2,
                             flags=flags)
        assert rc == 0, cabi.error_string(rc)
        torch.cuda.synchronize()
        return out

    base = run(c["cache"], c["table"])
    N = c["cache"].shape[0]
    perm = torch.randperm(N + 3, generator=torch.Generator().manual_seed(3)).to(gpu)
    big = torch.full((N + 3, *c["cache"].shape[1:]), float("nan"), dtype=dtype, device=gpu)
    big[perm[:N]] = c["cache"]
    table = c["table"].clone()
    used = table >= 0
    table[used] = perm[table[used].long()].int()
    # Poison the slots past each sequence's end inside its last page.
    flat = big.view(-1, big.shape[-1])
    for b, L in enumerate(c["lens"].tolist()):
        if L % 64:
            page = int(table[b, L // 64])
            flat[page * 64 + L % 64:(page + 1) * 64] = float("inf")
    table[~used] = 10 ** 6                                  # never read
    got = run(big, table)
    assert torch.equal(got.view(torch.int16), base.view(torch.int16))


PROJ_SHAPES = [
    ("deepseek-absorb", True, (3, 1, 128, 128), 512, torch.bfloat16),
    ("deepseek-value", False, (3, 1, 128, 512), 128, torch.bfloat16),
    ("rows70-fp16-absorb", True, (35, 2, 8, 64), 96, torch.float16),
    ("rows70-fp16-value", False, (35, 2, 8, 96), 40, torch.float16),
    ("long-k-absorb", True, (4, 1, 8, 512), 64, torch.bfloat16),           # 16-row tiles, 4 chunks a wave
    ("big-value", False, (256, 1, 128, 512), 128, torch.bfloat16),         # 512 workgroups: 64-row tiles
    ("big-absorb", True, (64, 1, 128, 128), 512, torch.bfloat16),          # 512 workgroups: 64-row tiles
    ("odd-generic", True, (2, 3, 4, 16), 32, torch.bfloat16),
    ("fp32", False, (1, 4, 4, 32), 16, torch.float32),
]


@pytest.mark.parametrize("name,absorb,xshape,dout,dtype", PROJ_SHAPES, ids=[s[0] for s in PROJ_SHAPES])
def test_mla_project_matches_oracle(gpu, name, absorb, xshape, dout, dtype):
    say(f"mla_project {name}")
    gen = torch.Generator().manual_seed(len(name))
    B, T, H, di = xshape
    x = torch.randn(*xshape, generator=gen).to(dtype)
    w = (torch.randn(H, di, dout, generator=gen) if absorb else torch.randn(H, dout, di, generator=gen))
    w = (w / di ** 0.5).to(dtype)
    ref = oracle_mla_project(_np(x), _np(w), absorb, ODT[dtype])
    fn = attention_amd.mla_query_absorb if absorb else attention_amd.mla_value_project
    got = fn(x.to(gpu), w.to(gpu))
    torch.cuda.synchronize()
    assert got.shape == (B, T, H, dout) and got.dtype == dtype
    _close(got, ref, dtype, name)
    if dtype != torch.float32:
        out = torch.empty(B, T, H, dout, dtype=dtype, device=gpu)
        assert cabi.mla_project(x.to(gpu), w.to(gpu), out, absorb, flags=QD_FLAG_FORCE_GENERIC) == 0
        torch.cuda.synchronize()
        _close(out, ref, dtype, name + " generic")


@pytest.mark.parametrize("dtype,dc,dr", [(torch.bfloat16, 512, 64), (torch.float16, 20, 4),
                                         (torch.float32, 32, 8)])
def test_latent_kv_write_bitwise(gpu, dtype, dc, dr):
    say(f"latent_kv_write {dtype} Dc={dc} Dr={dr}")
    gen = torch.Generator().manual_seed(dc)
    N, P, n = 6, 16, 40
    cache = torch.randn(N, P, dc + dr, generator=gen).to(dtype)
    latent = torch.randn(n, dc, generator=gen).to(dtype)
    rope = torch.randn(n, dr, generator=gen).to(dtype)
    slots = torch.randperm(N * P, generator=gen)[:n].to(torch.int64)
    slots[3] = N * P + 5                       # outside the cache: skipped
    slots[7] = -2
    ref = oracle_latent_kv_write(latent.view(torch.int16 if dtype != torch.float32 else torch.int32).numpy(),
                                 rope.view(torch.int16 if dtype != torch.float32 else torch.int32).numpy(),
                                 cache.view(torch.int16 if dtype != torch.float32 else torch.int32).numpy(),
                                 slots.numpy())
    dcache = cache.to(gpu)
    attention_amd.latent_kv_write(latent.to(gpu), rope.to(gpu), dcache, slots.to(gpu))
    torch.cuda.synchronize()
    got = dcache.cpu().view(torch.int16 if dtype != torch.float32 else torch.int32).numpy()
    assert np.array_equal(got, ref)


DECODE_SHAPES = [
    ("deepseek-h128-t1", dict(lengths=[33, 700, 2049], q_len=1, heads=128, block_size=64, dtype=torch.bfloat16)),
    # One query per row, so the C ABI's fused op runs: the value projection
    # merges the split rows itself (wave kernel; shared-tile kernel in fp16
    # with every workgroup range non-empty).
    ("deepseek-h16-t1-b40", dict(lengths=[(37 * i * i + 11 * i) % 3001 + 1 for i in range(40)], q_len=1, heads=16,
                                 block_size=64, dtype=torch.bfloat16)),
    ("deepseek-h16-t1-fp16-b20", dict(lengths=[(53 * i + 7) % 2500 + 1 for i in range(20)], q_len=1, heads=16,
                                      block_size=64, dtype=torch.float16)),
    ("deepseek-h128-t1-fp16-long", dict(lengths=[3000, 2500, 1, 4000, 2047, 64, 3333, 1800], q_len=1, heads=128,
                                        block_size=64, dtype=torch.float16)),
    # 256 rows x 128 heads: the value projection takes 64-row tiles, so the
    # fused op runs the merge kernel and the plain projection.
    ("deepseek-h128-t1-b256", dict(lengths=[(13 * i) % 97 + 1 for i in range(256)], q_len=1, heads=128,
                                   block_size=64, dtype=torch.bfloat16)),
    ("deepseek-h16-t2", dict(lengths=[5, 1000], q_len=2, heads=16, block_size=64, dtype=torch.bfloat16)),
    ("ref-bench-bf16", dict(lengths=[4096], q_len=1, heads=4, nope_dim=32, latent_dim=64, rope_dim=16,
                            value_dim=32, block_size=16, dtype=torch.bfloat16)),
    ("ref-bench-fp32", dict(lengths=[64, 1024], q_len=1, heads=4, nope_dim=16, latent_dim=32, rope_dim=8,
                            value_dim=16, block_size=16, dtype=torch.float32)),
    ("sparse-h32", dict(lengths=[300, 64, 2000], q_len=1, heads=32, block_size=64, dtype=torch.bfloat16,
                        num_indices=64)),
]

# The decode chain rounds twice before its output (absorbed query, latent
# output).  Where a value sits near a rounding boundary, fp32 and float64
# sums round it to neighbouring 16-bit values; a 1-ulp step of the absorbed
# query moves the scores by ~ulp * |c| * scale and the sharp softmax carries
# that into the output (observed up to ~2 bf16 ulps at |out| ~ 0.5).  So
# every stage is checked at the 16-bit tolerance with the GPU's previous
# stage as its input, the fused op must equal the composed GPU stages bit
# for bit, and the chain end to end is held to CHAIN_TOL.  That loosened bar
# covers a few elements moved by the intermediate roundings; a systematic
# mistake (a dropped term, a wrong index) moves most of them, so at most
# CHAIN_OUTSIDE of the outputs may lie past the 16-bit bar (measured on
# MI355X: none, in every case below).
CHAIN_TOL = (1.5e-2, 2e-2)
CHAIN_OUTSIDE = 0.002


def _chain_close(got, ref, dtype, name):
    err = np.abs(got.float().cpu().numpy() - ref)
    atol, rtol = CHAIN_TOL if dtype != torch.float32 else TOL[dtype]
    assert (err <= atol + rtol * np.abs(ref)).all(), f"{name}: chain max abs err {err.max():.3e}"
    a16, r16 = TOL[dtype]
    outside = float((err > a16 + r16 * np.abs(ref)).mean())
    say(f"{name}: {outside:.4%} of the outputs past the {ODT[dtype]} bar")
    assert outside <= CHAIN_OUTSIDE, f"{name}: {outside:.3%} of the outputs past the 16-bit bar"


@pytest.mark.parametrize("name,kw", DECODE_SHAPES, ids=[s[0] for s in DECODE_SHAPES])
def test_mla_decode_matches_oracle(gpu, name, kw):
    say(f"mla_decode {name}")
    kw = dict(kw)
    dtype = kw["dtype"]
    nk = kw.pop("num_indices", None)
    c = _case(gpu, num_indices=nk, **kw)
    idx = c["indices"]
    scale = default_mla_scale(c["q_nope"].shape[-1], c["q_rope"].shape[-1])
    meta = (c["cache"], c["table"], c["lens"], c["positions"])
    # Stage by stage, each from the GPU's previous stage.
    qa = attention_amd.mla_query_absorb(c["q_nope"], c["w_uk"])
    _close(qa, oracle_mla_project(_np(c["q_nope"]), _np(c["w_uk"]), True, ODT[dtype]), dtype, name + " absorb")
    latent = attention_amd.mla_latent_attention(qa, c["q_rope"], *meta, scale=scale, indices=idx)
    _close(latent, oracle_mla_attend(_np(qa), _np(c["q_rope"]), *(_np(x) for x in meta), scale, True, _np(idx),
                                     ODT[dtype]), dtype, name + " attend")
    composed = attention_amd.mla_value_project(latent, c["w_uv"])
    _close(composed, oracle_mla_project(_np(latent), _np(c["w_uv"]), False, ODT[dtype]), dtype, name + " value")
    # The public entry point (fused op for one query per row) equals the
    # composition bit for bit, and the whole chain is within CHAIN_TOL.
    got = attention_amd.mla_decode(c["q_nope"], c["q_rope"], *meta, c["w_uk"], c["w_uv"], indices=idx)
    torch.cuda.synchronize()
    assert got.dtype == dtype and got.shape == composed.shape
    assert torch.equal(got, composed)
    ref = oracle_mla_decode(_np(c["q_nope"]), _np(c["q_rope"]), *(_np(x) for x in meta), _np(c["w_uk"]),
                            _np(c["w_uv"]), indices=_np(idx), out_dtype=ODT[dtype])
    _chain_close(got, ref, dtype, "mla_decode " + name)


@pytest.mark.parametrize("heads,lengths", [(16, [(37 * i * i + 11 * i) % 3001 + 1 for i in range(40)]),
                                           (128, [33, 700, 2049, 1, 1500])], ids=["wave-h16", "shared-h128"])
def test_mla_decode_graph_capture_replays_match_eager(gpu, heads, lengths):
    """mla_decode (fused op: absorption, latent attention with rows split
    across workgroups, value projection merging them) captured in a HIP
    graph: the workspace comes from the graph's pool and nothing in the op
    clears memory, so every replay, with eager calls and synchronizations
    between replays, equals the eager output bit for bit."""
    say(f"mla_decode graph capture {heads} heads: replays vs eager")
    c = _case(gpu, lengths=lengths, q_len=1, heads=heads, block_size=64, dtype=torch.bfloat16)
    args = (c["q_nope"], c["q_rope"], c["cache"], c["table"], c["lens"], c["positions"], c["w_uk"], c["w_uv"])
    ref = attention_amd.mla_decode(*args)
    o = _case(gpu, lengths=[90, 2500], q_len=1, heads=heads, block_size=64, dtype=torch.bfloat16, seed=5)
    other = (o["q_nope"], o["q_rope"], o["cache"], o["table"], o["lens"], o["positions"], o["w_uk"], o["w_uv"])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            attention_amd.mla_decode(*args)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = attention_amd.mla_decode(*args)
    torch.cuda.synchronize()
    for i in range(3):
        say(f"graph replay {i}")
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}"
        attention_amd.mla_decode(*other)   # eager work on the same stream between replays
        torch.cuda.synchronize()


def test_sparse_mla_is_mla_decode_with_indices(gpu):
    say("sparse_mla entry point")
    c = _case(gpu, lengths=[300, 64], q_len=1, heads=32, block_size=64, dtype=torch.bfloat16, num_indices=16)
    args = (c["q_nope"], c["q_rope"], c["cache"], c["table"], c["lens"], c["positions"], c["w_uk"], c["w_uv"])
    a = attention_amd.sparse_mla(*args, c["indices"])
    b = attention_amd.mla_decode(*args, indices=c["indices"])
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_mla_decode_cabi_generic_matches_mfma(gpu):
    say("mla_decode C ABI: VALU kernels vs MFMA kernels")
    dtype = torch.bfloat16
    c = _case(gpu, lengths=[77, 1500], q_len=1, heads=32, block_size=64, dtype=dtype)
    args = (c["q_nope"], c["q_rope"], c["cache"], c["table"], c["lens"], c["positions"], c["w_uk"], c["w_uv"])
    outs = []
    for flags in (0, QD_FLAG_FORCE_GENERIC):
        out = torch.empty(2, 1, 32, 128, dtype=dtype, device=gpu)
        rc = cabi.mla_decode(*args, out, scale=default_mla_scale(128, 64), flags=flags)
        assert rc == 0, cabi.error_string(rc)
        outs.append(out)
    torch.cuda.synchronize()
    ref = oracle_mla_decode(*(_np(x) for x in args), out_dtype="bf16")
    for i, out in enumerate(outs):
        _chain_close(out, ref, torch.bfloat16, f"mla_decode flags-variant {i}")


def test_mla_validation_messages_on_device(gpu):
    say("MLA validation messages")
    c = _case(gpu, lengths=[20, 40], q_len=1, heads=4, nope_dim=16, latent_dim=32, rope_dim=8, value_dim=16,
              block_size=16, dtype=torch.float16)
    qa = torch.randn(2, 1, 4, 32, device=gpu).half()
    args = [qa, c["q_rope"], c["cache"], c["table"], c["lens"], c["positions"]]
    with pytest.raises(RuntimeError, match="q_rope must be contiguous and on the same CUDA device"):
        attention_amd.mla_latent_attention(qa, c["q_rope"].transpose(2, 3), *args[2:], scale=0.1)
    with pytest.raises(RuntimeError, match="dtype mismatch"):
        attention_amd.mla_latent_attention(qa.float(), c["q_rope"].float(), *args[2:], scale=0.1)
    with pytest.raises(RuntimeError, match="metadata must be int32"):
        attention_amd.mla_latent_attention(qa, c["q_rope"], c["cache"], c["table"].long(), c["lens"],
                                           c["positions"], scale=0.1)
    with pytest.raises(RuntimeError, match="scale must be positive and finite"):
        attention_amd.mla_latent_attention(*args, scale=0.0)
    with pytest.raises(RuntimeError, match=r"indices must be int32 \[B,T,K\]"):
        attention_amd.mla_latent_attention(*args, scale=0.1, indices=c["lens"].view(2, 1, 1).long())
    with pytest.raises(RuntimeError, match="invalid dimensions"):
        attention_amd.mla_decode(c["q_nope"], c["q_rope"], c["cache"], c["table"], c["lens"], c["positions"],
                                 c["w_uk"][:, :8].contiguous(), c["w_uv"])
    with pytest.raises(RuntimeError, match="projection dimension mismatch"):
        attention_amd.mla_value_project(c["q_nope"], c["w_uv"])
    with pytest.raises(RuntimeError, match="slots must be int64 and tensors must share dtype"):
        attention_amd.latent_kv_write(torch.zeros(2, 32, device=gpu).half(), torch.zeros(2, 8, device=gpu).half(),
                                      c["cache"], torch.zeros(2, dtype=torch.int32, device=gpu))
    empty = attention_amd.mla_latent_attention(qa[:0], c["q_rope"][:0], c["cache"], c["table"][:0],
                                               c["lens"][:0], c["positions"][:0], scale=0.1)
    assert empty.shape == (0, 1, 4, 32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("heads,flags", [(64, 0), (64, QD_FLAG_MLA_WAVE), (16, 0)], ids=["shared-h64", "wave-h64", "wave-h16"])
def test_mla_attend_subnormal_partial_block(gpu, dtype, heads, flags):
    """Split rows stored as half-precision blocks scaled by each block's
    largest |value|: here the tokens that carry the softmax (even ones) have
    an all-zero first 128-column latent block, and the only nonzero values
    of that block come from tokens weighted about 2^-140 below them, so the
    block's accumulator maximum is subnormal (or flushed to zero).  The scale
    must keep 1/scale finite: the output is finite and matches the oracle."""
    say(f"mla_attend subnormal partial block {ODT[dtype]} heads={heads} flags={flags}")
    c = _case(gpu, lengths=[3000, 1700], q_len=1, heads=heads, block_size=64, dtype=dtype, seed=13)
    Dc = c["w_uk"].shape[-1]
    Dr = c["q_rope"].shape[-1]
    scale = default_mla_scale(c["q_nope"].shape[-1], Dr)
    # Scores from the rope part only: q_rope = e_0 for every head, rope key
    # dim 0 = `high` for even tokens and 0 for odd ones, 140 / log2(e) apart
    # after scaling; the latent query is zero.
    high = float(torch.tensor(140.0 / (scale * 1.4426950408889634)).to(dtype))
    cache = c["cache"].float()
    ids = torch.arange(cache.shape[0] * cache.shape[1], device=cache.device).view(cache.shape[0], cache.shape[1])
    even = (ids % 2 == 0)
    cache[..., Dc:] = 0.0
    cache[..., Dc] = torch.where(even, torch.full_like(cache[..., Dc], high), torch.zeros_like(cache[..., Dc]))
    block0 = cache[..., :128]
    cache[..., :128] = torch.where(even[..., None], torch.zeros_like(block0), block0 * 0.01)
    c["cache"] = cache.to(dtype)
    qr = torch.zeros_like(c["q_rope"].float())
    qr[..., 0] = 1.0
    c["q_rope"] = qr.to(dtype)
    qa = torch.zeros(c["q_nope"].shape[:3] + (Dc,), dtype=dtype, device=gpu)
    out = torch.empty_like(qa)
    rc = cabi.mla_attend(qa, c["q_rope"], c["cache"], c["table"], c["lens"], c["positions"], out, scale=scale,
                         splits=3, flags=flags)
    assert rc == 0, cabi.error_string(rc)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    _close(out, _oracle_attend(c, qa, scale, dtype=dtype), dtype, "subnormal partial block")


@pytest.mark.parametrize("heads,flags", [(64, 0), (64, QD_FLAG_MLA_WAVE), (16, 0)], ids=["shared-h64", "wave-h64", "wave-h16"])
def test_mla_attend_fp16_partial_error_bound(gpu, heads, flags):
    """The half-precision partials keep each value to 2^-12 of its
    128-column block's largest |value|, so on fp16 the split run (rows over
    three workgroups, merged from fp16 partials) may differ from the unsplit
    run (no partials) by 2^-12 of each row's block maximum, weighted; the
    rows' block maxima exceed the merged block's by about sqrt(3) on these
    random inputs, so the test allows 4 * 2^-12 of the merged block's
    largest |output| per element, plus the two outputs' own rounding (half
    an fp16 ulp each)."""
    say(f"mla_attend fp16 partial error bound heads={heads} flags={flags}")
    c = _case(gpu, lengths=[3000, 700, 2000, 1500], q_len=1, heads=heads, block_size=64, dtype=torch.float16, seed=17)
    qa = _absorbed(c, torch.float16).to(torch.float16).to(gpu)
    scale = default_mla_scale(c["q_nope"].shape[-1], c["q_rope"].shape[-1])
    outs = {}
    for splits in (1, 3):
        out = torch.empty_like(qa)
        rc = cabi.mla_attend(qa, c["q_rope"], c["cache"], c["table"], c["lens"], c["positions"], out, scale=scale,
                             splits=splits, flags=flags)
        assert rc == 0, cabi.error_string(rc)
        torch.cuda.synchronize()
        outs[splits] = out.float().cpu()
    one, three = outs[1], outs[3]
    blocks = one.view(*one.shape[:-1], -1, 128)
    bmax = blocks.abs().amax(dim=-1, keepdim=True).expand_as(blocks).reshape(one.shape)
    ulp = lambda x: 2.0 ** (torch.floor(torch.log2(x.abs().clamp_min(2.0 ** -14))) - 10)  # noqa: E731
    bound = 4 * 2.0 ** -12 * bmax + 0.5 * ulp(one) + 0.5 * ulp(three) + 2.0 ** -24
    diff = (three - one).abs()
    assert torch.all(diff <= bound), f"max excess {(diff - bound).max().item():.3e}"
