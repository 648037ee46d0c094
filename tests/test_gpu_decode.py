"""GPU parity of the HIP decode path against the CPU oracle.

Tolerance: |err| <= 2e-3 + 1e-2*|ref| for
bf16/fp16 caches with fp32 accumulation; fp32 caches use 1e-5 + 1e-4*|ref|.
Index handling (page permutation, poisoned unused slots, -1 padding) must be
bit-exact.  Every case prints its name before touching the GPU.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import attention_amd
from attention_amd.cases import CONFIGS, make_decode_case
from oracle.gqa_oracle import oracle_decode, page_split_range, split_partials
from attention_amd import cabi

pytestmark = pytest.mark.gpu

DT_NAME = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}
TOL = {"f32": (1e-5, 1e-4), "f16": (2e-3, 1e-2), "bf16": (2e-3, 1e-2)}


def say(msg):
    print(f"[case] {msg}", flush=True)


def subcase(case, batches):
    """Compact CPU copy of the selected sequences (pages remapped 0..n-1)."""
    q, k, v, table, lens = case
    P = k.shape[1]
    lens_c = lens.cpu()
    tab_c = table.cpu()
    sel_pages, rows, offset = [], [], 0
    for b in batches:
        n = max(0, math.ceil(int(lens_c[b]) / P))
        sel_pages.append(tab_c[b, :n].long())
        rows.append(list(range(offset, offset + n)))
        offset += n
    ids = torch.cat(sel_pages) if sel_pages else torch.zeros(0, dtype=torch.long)
    if ids.numel() == 0:
        ids = torch.zeros(1, dtype=torch.long)
    k_s = k[ids.to(k.device)].float().cpu().numpy()
    v_s = v[ids.to(v.device)].float().cpu().numpy()
    maxp = max(1, max(len(r) for r in rows))
    t_s = np.full((len(batches), maxp), -1, dtype=np.int32)
    for i, r in enumerate(rows):
        t_s[i, :len(r)] = r
    q_s = q[list(batches)].float().cpu().numpy()
    l_s = lens_c[list(batches)].numpy()
    return q_s, k_s, v_s, t_s, l_s


def oracle_rows(case, batches=None, scale=None):
    q = case[0]
    bsz = q.shape[0]
    batches = list(range(bsz)) if batches is None else list(batches)
    q_s, k_s, v_s, t_s, l_s = subcase(case, batches)
    return oracle_decode(q_s, k_s, v_s, t_s, l_s, scale=scale, out_dtype=DT_NAME[q.dtype]), batches


def assert_close(out, ref, dtype_name, rows=None, what=""):
    got = out.float().cpu().numpy()
    if rows is not None:
        got = got[rows]
    atol, rtol = TOL[dtype_name]
    err = np.abs(got - ref)
    bad = ~(err <= atol + rtol * np.abs(ref))
    assert not bad.any(), (f"{what}: {bad.sum()} mismatches, max abs err {np.nanmax(err):.3e} "
                           f"at {np.argwhere(bad)[:3].tolist()}")


def to_dev(case, dev):
    return tuple(x.to(dev) for x in case)


# ----------------------------------------------------------------------------
# Benchmark configurations
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["cfg1", "cfg2", "cfg3", "cfg5"])
def test_config_matches_oracle(gpu, name):
    cfg = CONFIGS[name]
    say(f"config {name} full oracle")
    case = to_dev(cfg.make(device="cpu"), gpu)
    out = attention_amd.gqa_decode(*case)
    torch.cuda.synchronize()
    ref, rows = oracle_rows(case)
    assert out.shape == case[0].shape and out.dtype == case[0].dtype
    assert_close(out, ref, DT_NAME[cfg.dtype], rows, name)


def test_cfg4_long_context(gpu):
    """cfg4 from the CPU-seeded recipe (the same q/K/V as the CPU path would
    see), every sequence compared with the oracle, one at a time so the
    fp32 copies stay near 1 GB of host memory."""
    cfg = CONFIGS["cfg4"]
    say("config cfg4 (CPU-seeded recipe, oracle on all 8 sequences)")
    case_cpu = cfg.make(device="cpu")
    case = to_dev(case_cpu, gpu)
    del case_cpu
    out = attention_amd.gqa_decode(*case)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    for b in range(cfg.batch):
        say(f"cfg4 sequence {b} (len {int(case[4][b])})")
        ref, rows = oracle_rows(case, [b])
        assert_close(out, ref, "bf16", rows, f"cfg4 sequence {b}")


# ----------------------------------------------------------------------------
# Both kernels, through the C ABI
# ----------------------------------------------------------------------------

SHAPES = [
    # (dtype, Hq, Hkv, D, P, lengths)
    (torch.bfloat16, 32, 8, 128, 16, [1, 15, 16, 17, 300, 1024, 0, 33]),
    (torch.float16, 28, 4, 128, 16, [5, 700, 4097, 1]),
    (torch.float16, 40, 8, 128, 32, [128, 31, 32, 33, 1000]),
    (torch.bfloat16, 8, 2, 64, 16, [17, 100, 255, 512]),
    (torch.bfloat16, 16, 1, 256, 16, [1, 90, 513]),
    (torch.float16, 16, 16, 64, 48, [47, 48, 49, 200]),
    (torch.bfloat16, 17, 1, 128, 16, [40, 1, 300]),
    (torch.float32, 32, 8, 128, 16, [1, 300, 1025]),
    (torch.float32, 6, 3, 100, 7, [1, 6, 7, 8, 100]),
    (torch.float16, 12, 4, 17, 5, [3, 19, 64]),
    (torch.bfloat16, 4, 4, 1, 1, [1, 2, 9]),
    (torch.float16, 64, 8, 128, 16, [2000, 1]),
    (torch.bfloat16, 32, 32, 96, 16, [1, 300, 2049]),    # head_dim 96 (loads ending inside a K row, 12-byte V rows)
    (torch.float16, 32, 8, 96, 32, [17, 1000, 0, 33]),
    # fp32 on the balanced path (fp32 MFMA; B * max_pages * P >= 65536): head_dim 64
    # on 32-token pages, a group of 16
    (torch.float32, 16, 4, 64, 32, [17, 1000, 0, 16400]),
    (torch.float32, 16, 1, 128, 16, [1, 700, 33, 16384]),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{DT_NAME[s[0]]}-Hq{s[1]}-Hkv{s[2]}-D{s[3]}-P{s[4]}")
@pytest.mark.parametrize("flags", [0, cabi.QD_FLAG_FORCE_GENERIC], ids=["auto", "generic"])
def test_shapes_cabi(gpu, shape, flags):
    dtype, hq, hkv, d, p, lengths = shape
    kind = cabi.lib().qd_gqa_decode_kernel_kind(hq, hkv, d, p, cabi.DTYPE[dtype], flags)
    say(f"shape {shape[1:5]} {DT_NAME[dtype]} kernel={'mfma' if kind else 'generic'}")
    case = to_dev(make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=d,
                                   block_size=p, dtype=dtype, seed=7), gpu)
    q, k, v, table, lens = case
    scale = 1.0 / math.sqrt(d)
    ref, rows = oracle_rows(case)
    for splits, chunk in [(1, 0), (3, 0), (table.shape[1], 1)]:
        out = torch.full_like(q, float("nan"))
        ws = torch.empty(max(1, q.shape[0] * hq * splits * (d + 2)), device=gpu, dtype=torch.float32)
        rc = cabi.launch(q, k, v, table, lens, out, scale=scale, splits=splits, chunk_pages=chunk,
                         workspace=ws if splits > 1 else None, flags=flags)
        assert rc == 0, cabi.error_string(rc)
        torch.cuda.synchronize()
        assert_close(out, ref, DT_NAME[dtype], rows, f"splits={splits} chunk={chunk}")


# ----------------------------------------------------------------------------
# Split API, workspace contents
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_split_merge_alignments(gpu, dtype):
    """The split layout's merge with a 16-byte aligned output and 8-byte
    aligned workspace (combine_rows_kernel: four lane groups per head, 16
    partials per round trip each) and with the output or the workspace one
    element off that alignment (combine_kernel): every form matches the
    oracle, with 1 to 300 partials per head (several round trips per lane
    group at 300)."""
    hq, hkv, d, p = 32, 8, 128, 16
    lengths = [1, 16, 17, 1000, 4800, 0]
    case = to_dev(make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=d, block_size=p,
                                   dtype=dtype, seed=29), gpu)
    q, k, v, table, lens = case
    ref, rows = oracle_rows(case)
    B, maxp = len(lengths), table.shape[1]
    for splits, chunk in [(maxp, 1), (7, 0), (65, 0)]:
        n = B * hq * splits * (d + 2)
        for out_off, ws_off in [(0, 0), (1, 0), (0, 1)]:
            say(f"split merge {DT_NAME[dtype]} splits={splits} chunk={chunk} out+{out_off} ws+{ws_off}")
            obuf = torch.full((q.numel() + 8,), float("nan"), dtype=dtype, device=gpu)
            out = obuf[out_off:out_off + q.numel()].view(q.shape)
            ws = torch.full((n + 4,), float("nan"), dtype=torch.float32, device=gpu)[ws_off:ws_off + n]
            rc = cabi.launch(q, k, v, table, lens, out, scale=1 / math.sqrt(d), splits=splits, chunk_pages=chunk,
                             workspace=ws)
            assert rc == 0, cabi.error_string(rc)
            torch.cuda.synchronize()
            assert_close(out, ref, DT_NAME[dtype], rows, f"splits={splits} out+{out_off} ws+{ws_off}")


@pytest.mark.parametrize("splits", [1, 2, 3, 4, 8, 16, 64])
def test_split_api(gpu, splits):
    say(f"gqa_decode_split splits={splits}")
    case = to_dev(make_decode_case(lengths=[1, 17, 300, 1000, 64, 0], q_heads=32, kv_heads=8,
                                   head_dim=128, block_size=16, dtype=torch.bfloat16, seed=3), gpu)
    ref, rows = oracle_rows(case)
    out = attention_amd.gqa_decode_split(*case, splits=splits)
    torch.cuda.synchronize()
    assert_close(out, ref, "bf16", rows, f"split {splits}")
    if splits > 1:
        ws = torch.full((6, 32, splits, 130), float("nan"), device=gpu)
        out2 = attention_amd.gqa_decode_split(*case, splits=splits, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(out, out2)


def test_workspace_partials_match_oracle(gpu):
    say("workspace partial contents vs oracle split_partials")
    splits = 4
    case_cpu = make_decode_case(lengths=[300, 1000, 64], q_heads=8, kv_heads=2, head_dim=64,
                                block_size=16, dtype=torch.float16, seed=11)
    case = to_dev(case_cpu, gpu)
    ws = torch.full((3, 8, splits, 66), float("nan"), device=gpu)
    attention_amd.gqa_decode_split(*case, splits=splits, workspace=ws)
    torch.cuda.synchronize()
    q, k, v, table, lens = (x.float().numpy() if x.is_floating_point() else x.numpy() for x in case_cpu)
    maxp = table.shape[1]
    ranges = lambda b, z: page_split_range(int(lens[b]), 16, maxp, splits, 0, z)
    part = split_partials(q, k, v, table, lens, splits=splits, ranges=ranges)
    got = ws.cpu().numpy()
    for b in range(3):
        n = math.ceil(int(lens[b]) / 16)
        nch = min(splits, math.ceil(n / math.ceil(n / splits)))
        if nch <= 1:
            continue
        np.testing.assert_allclose(got[b, :, :nch, 0], part[b, :, :nch, 0], rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(got[b, :, :nch, 1], part[b, :, :nch, 1], rtol=2e-3)
        np.testing.assert_allclose(got[b, :, :nch, 2:], part[b, :, :nch, 2:], rtol=2e-2, atol=2e-2)


# ----------------------------------------------------------------------------
# Bit-exact index handling
# ----------------------------------------------------------------------------

def _poisoned_case(dev, dtype=torch.bfloat16, lengths=(1, 17, 31, 300, 0, 64), hq=32, hkv=8, d=128, p=16,
                   seed=5):
    """A case on a pool larger than the used blocks (the recipe's
    B*max_pages pool), and the same case with every cache slot no sequence
    uses set to NaN (K) and Inf (V): unused blocks, and the slots past each
    sequence's length in its last page."""
    q, k, v, table, lens = make_decode_case(lengths=list(lengths), q_heads=hq, kv_heads=hkv,
                                            head_dim=d, block_size=p, dtype=dtype, seed=seed)
    used = torch.zeros(k.shape[0], p, dtype=torch.bool)
    for b, L in enumerate(lengths):
        if L <= 0:
            continue
        t = torch.arange(L)
        used[table[b, t // p].long(), t % p] = True
    kp, vp = k.clone(), v.clone()
    kp[~used] = float("nan")
    vp[~used] = float("inf")
    return (q, k, v, table, lens), (q, kp, vp, table, lens)


def _ragged_lengths(n, hi, seed):
    """cfg3-style ragged lengths: uniform in [1, hi], with lengths 1, 16,
    17, a page boundary minus one and a zero mixed in."""
    rng = np.random.default_rng(seed)
    lens = [int(x) for x in rng.integers(1, hi + 1, n)]
    for i, x in enumerate((1, 16, 17, 255, 0)):
        lens[(i * 7) % n] = x
    return lens


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("wide", [False, True], ids=["narrow-table", "wide-table"])
def test_poisoned_unused_slots_bitwise_product_path(gpu, dtype, wide):
    """The product path (attention_amd.gqa_decode: decode_mfma_sk_kernel and
    merge_sk_kernel) on ragged lengths whose sequences split across
    workgroups: NaN/Inf in every unused slot and -1 table padding change no
    output bit.  A narrow page table runs one kv-head per wave, a wide
    -1-padded one (8192 pages) two kv-heads per wave; the C entry point
    with a NaN-filled scratch must give the same bits.  fp32: the narrow
    table's capacity (below 65536 tokens) takes the split layout, the wide
    one the fp32 balanced kernel."""
    hq, hkv, d, p = 32, 8, 128, 16
    lengths = _ragged_lengths(12, 3000, seed=17)
    clean, poison = _poisoned_case("cpu", dtype=dtype, lengths=lengths, hq=hq, hkv=hkv, d=d, p=p, seed=27)
    maxp = 8192 if wide else clean[3].shape[1]
    kind, waves, _, _ = cabi.auto_info(len(lengths), hq, hkv, d, p, maxp, cabi.DTYPE[dtype])
    say(f"poisoned slots, product path: {DT_NAME[dtype]} max_pages={maxp} kind={kind} waves={waves}")
    assert kind == (0 if dtype == torch.float32 and not wide else 1)
    outs = []
    for case in (clean, poison):
        q, k, v, table, lens = case
        tpad = torch.full((len(lengths), maxp), -1, dtype=torch.int32)
        tpad[:, :table.shape[1]] = table
        dev_case = to_dev((q, k, v, tpad, lens), gpu)
        out = attention_amd.gqa_decode(*dev_case)
        ws = cabi.auto_workspace(len(lengths), hq, hkv, d, p, maxp, cabi.DTYPE[dtype], gpu,
                                 fill=0xFF)   # NaN / -1 scratch past the counters
        out_c = torch.full_like(dev_case[0], float("nan"))
        rc = cabi.auto_launch(*dev_case, out_c, scale=1 / math.sqrt(d), workspace=ws)
        assert rc == 0, cabi.error_string(rc)
        torch.cuda.synchronize()
        assert torch.equal(out, out_c)
        outs.append(out)
    assert torch.isfinite(outs[1]).all()
    assert torch.equal(outs[0], outs[1])
    ref, rows = oracle_rows(to_dev(clean, gpu))
    assert_close(outs[0], ref, DT_NAME[dtype], rows, "clean")


@pytest.mark.parametrize("variant", ["aligned", "offset-table", "wide-table"])
def test_auto_table_layouts(gpu, variant):
    """The product path on a ragged batch (sequences split over workgroups,
    several sequences per workgroup, -1 padding) with the block
    table at a 4-byte offset inside a larger buffer and with a -1-padded
    table wider than the lengths need: the same bits as the aligned table,
    and the oracle's values."""
    hq, hkv, d, p = 32, 8, 128, 16
    lengths = _ragged_lengths(24, 2000, seed=31)
    q, k, v, table, lens = make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=d,
                                            block_size=p, dtype=torch.bfloat16, seed=32)
    maxp = 400 if variant == "wide-table" else 128
    tpad = torch.full((len(lengths), maxp), -1, dtype=torch.int32)
    tpad[:, :table.shape[1]] = table
    base = to_dev((q, k, v, tpad, lens), gpu)
    t_dev = base[3]
    if variant == "offset-table":
        buf = torch.full((tpad.numel() + 1,), -7, dtype=torch.int32, device=gpu)
        t_dev = buf[1:].view(tpad.shape)
        t_dev.copy_(base[3])
        assert t_dev.data_ptr() % 16 != 0
    say(f"table layout {variant}: max_pages={maxp}")
    out = attention_amd.gqa_decode(base[0], base[1], base[2], t_dev, base[4])
    ref_out = attention_amd.gqa_decode(*to_dev((q, k, v, tpad[:, :128], lens), gpu))
    torch.cuda.synchronize()
    if variant != "wide-table":   # a wider table may change the grid, so the split points
        assert torch.equal(out, ref_out)
    ref, rows = oracle_rows(to_dev((q, k, v, tpad, lens), gpu))
    assert_close(out, ref, "bf16", rows, variant)


def test_auto_long_and_short_poisoned(gpu):
    """One long sequence split over most workgroups, next to short ones
    that share workgroups with its ends; every cache slot no sequence uses
    is NaN/Inf: the outputs match the oracle, stay finite and equal the
    clean case bit for bit."""
    hq, hkv, d, p = 32, 8, 128, 16
    lengths = [12345, 17, 1, 1000, 33, 2049]
    clean, poison = _poisoned_case("cpu", dtype=torch.bfloat16, lengths=lengths, hq=hq, hkv=hkv, d=d, p=p,
                                   seed=44)
    say(f"long and short sequences, poisoned: {lengths}")
    out0 = attention_amd.gqa_decode(*to_dev(clean, gpu))
    out1 = attention_amd.gqa_decode(*to_dev(poison, gpu))
    torch.cuda.synchronize()
    assert torch.isfinite(out1).all()
    assert torch.equal(out0, out1)
    ref, rows = oracle_rows(to_dev(clean, gpu))
    assert_close(out0, ref, "bf16", rows, "long and short")


def test_auto_batch_beyond_register_lengths(gpu):
    """Batches above 256 sequences: the prologue holds the lengths of
    sequences 0..255 in registers and re-reads the rest from memory, for the
    partition scan and when a workgroup enters them; empty sequences on both
    sides of 256."""
    hq, hkv, d, p = 8, 2, 128, 16
    rng = np.random.default_rng(41)
    lengths = [int(x) for x in rng.integers(1, 160, size=300)]
    for i in (0, 5, 255, 256, 257, 299):
        lengths[i] = 0
    say(f"batch {len(lengths)} beyond staged lengths")
    case = to_dev(make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=d, block_size=p,
                                   dtype=torch.float16, seed=42), gpu)
    kind, _, _, _ = cabi.auto_info(len(lengths), hq, hkv, d, p, case[3].shape[1], cabi.DTYPE[torch.float16])
    assert kind in (1, 2)
    out = attention_amd.gqa_decode(*case)
    torch.cuda.synchronize()
    ref, rows = oracle_rows(case)
    assert_close(out, ref, "f16", rows, "B300")


def test_poisoned_cfg3_bitwise_product_path(gpu):
    """cfg3's own lengths (B64, Hq28/Hkv4, up to 8192 tokens, many not a
    multiple of 16) on a pool with unused blocks, poisoned versus clean
    through attention_amd.gqa_decode."""
    cfg = CONFIGS["cfg3"]
    lengths = cfg.lengths()
    say("poisoned slots, cfg3 lengths, product path")
    clean, poison = _poisoned_case("cpu", dtype=cfg.dtype, lengths=lengths, hq=cfg.q_heads, hkv=cfg.kv_heads,
                                   d=cfg.head_dim, p=cfg.block_size, seed=cfg.seed)
    out0 = attention_amd.gqa_decode(*to_dev(clean, gpu))
    out1 = attention_amd.gqa_decode(*to_dev(poison, gpu))
    torch.cuda.synchronize()
    assert torch.isfinite(out1).all()
    assert torch.equal(out0, out1)


@pytest.mark.parametrize("flags", [0, cabi.QD_FLAG_FORCE_GENERIC], ids=["auto", "generic"])
def test_poisoned_unused_slots_bitwise(gpu, flags):
    say(f"poisoned unused slots flags={flags}")
    clean, poison = _poisoned_case("cpu")
    outs = []
    for case in (clean, poison):
        q, k, v, table, lens = to_dev(case, gpu)
        out = torch.empty_like(q)
        ws = torch.empty(q.shape[0] * q.shape[1] * 4 * (q.shape[2] + 2), device=gpu)
        rc = cabi.launch(q, k, v, table, lens, out, scale=1 / math.sqrt(q.shape[2]), splits=4,
                         chunk_pages=0, workspace=ws, flags=flags)
        assert rc == 0, cabi.error_string(rc)
        torch.cuda.synchronize()
        outs.append(out)
    assert torch.isfinite(outs[1]).all()
    assert torch.equal(outs[0], outs[1])


def test_physical_permutation_bitwise(gpu):
    say("physical block permutation invariance")
    q, k, v, table, lens = make_decode_case(lengths=[1, 77, 500, 1024], q_heads=32, kv_heads=8,
                                            head_dim=128, block_size=16, dtype=torch.bfloat16, seed=9)
    perm = torch.randperm(k.shape[0], generator=torch.Generator().manual_seed(1))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    k2, v2 = k[perm], v[perm]                      # new block i holds old block perm[i]
    t2 = torch.where(table >= 0, inv[table.clamp(min=0).long()].int(), table)
    out1 = attention_amd.gqa_decode(*to_dev((q, k, v, table, lens), gpu))
    out2 = attention_amd.gqa_decode(*to_dev((q, k2, v2, t2, lens), gpu))
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)


def test_len_one_is_exact_value(gpu):
    say("len=1 -> exactly v")
    for dtype in (torch.bfloat16, torch.float16, torch.float32):
        q, k, v, table, lens = make_decode_case(lengths=[1, 1, 1], q_heads=16, kv_heads=4,
                                                head_dim=128, block_size=16, dtype=dtype, seed=2)
        out = attention_amd.gqa_decode(*to_dev((q, k, v, table, lens), gpu)).cpu()
        for b in range(3):
            for h in range(16):
                assert torch.equal(out[b, h], v[table[b, 0], 0, h // 4]), (dtype, b, h)


def test_zero_and_negative_lengths_give_zeros(gpu):
    say("len <= 0 -> zeros")
    case = make_decode_case(lengths=[0, 5, 0], q_heads=8, kv_heads=2, head_dim=64, block_size=16,
                            dtype=torch.float16, seed=4)
    q, k, v, table, lens = to_dev(case, gpu)
    lens[2] = -7
    out = attention_amd.gqa_decode(q, k, v, table, lens)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[0]) == 0 and torch.count_nonzero(out[2]) == 0
    assert torch.count_nonzero(out[1]) > 0


def test_batch_zero(gpu):
    say("batch 0")
    q = torch.empty(0, 8, 64, device=gpu, dtype=torch.float16)
    k = torch.randn(4, 16, 2, 64, device=gpu).half()
    out = attention_amd.gqa_decode(q, k, k.clone(), torch.empty(0, 3, dtype=torch.int32, device=gpu),
                                   torch.empty(0, dtype=torch.int32, device=gpu))
    assert out.shape == (0, 8, 64)


def test_large_pool_64bit_offsets(gpu):
    say("pool > 2^31 bytes, pages at the end")
    hkv, d, p = 8, 128, 16
    nblocks = (1 << 31) // (p * hkv * d * 2) + 64       # K pool just above 2 GiB
    k = torch.empty(nblocks, p, hkv, d, device=gpu, dtype=torch.bfloat16)
    v = torch.empty_like(k)
    lengths = [700, 33]
    pages = [list(range(nblocks - 44, nblocks - 44 + 44))[:44], [nblocks - 1, nblocks - 2, nblocks - 3]]
    table = torch.full((2, 44), -1, dtype=torch.int32)
    table[0, :44] = torch.tensor(pages[0], dtype=torch.int32)
    table[1, :3] = torch.tensor(pages[1], dtype=torch.int32)
    gen = torch.Generator(device=gpu).manual_seed(0)
    used = sorted(set(pages[0] + pages[1]))
    for blk in used:
        k[blk].normal_(generator=gen)
        v[blk].normal_(generator=gen)
    q = torch.randn(2, 32, d, device=gpu, generator=gen).bfloat16()
    lens = torch.tensor(lengths, dtype=torch.int32, device=gpu)
    out = attention_amd.gqa_decode(q, k, v, table.to(gpu), lens)
    torch.cuda.synchronize()
    ref, rows = oracle_rows((q, k, v, table.to(gpu), lens))
    assert_close(out, ref, "bf16", rows, "large pool")
    del k, v
    torch.cuda.empty_cache()


# ----------------------------------------------------------------------------
# Boundary behaviour on device tensors
# ----------------------------------------------------------------------------

def test_validation_messages_on_device(gpu):
    say("validation messages")
    q, k, v, table, lens = to_dev(make_decode_case(lengths=[3, 5], q_heads=8, kv_heads=2,
                                                   head_dim=64, dtype=torch.float16), gpu)
    with pytest.raises(RuntimeError, match="q/k/v dtype must match"):
        attention_amd.gqa_decode(q.float(), k, v, table, lens)
    with pytest.raises(RuntimeError, match="k_cache must be contiguous"):
        attention_amd.gqa_decode(q, k.transpose(1, 2), v, table, lens)
    with pytest.raises(RuntimeError, match="block_table and context_lens must be int32"):
        attention_amd.gqa_decode(q, k, v, table.long(), lens)
    with pytest.raises(RuntimeError, match="batch sizes must match"):
        attention_amd.gqa_decode(q[:1], k, v, table, lens)
    with pytest.raises(RuntimeError, match="scale must be positive and finite"):
        attention_amd.gqa_decode(q, k, v, table, lens, scale=-1.0)
    with pytest.raises(RuntimeError, match=r"splits must be in \[1, 65535\]"):
        attention_amd.gqa_decode_split(q, k, v, table, lens, splits=0)
    ws = torch.empty(2, 8, 2, 66, device=gpu)
    with pytest.raises(RuntimeError, match="workspace requires splits > 1"):
        attention_amd.gqa_decode_split(q, k, v, table, lens, splits=1, workspace=ws[:, :, :1].contiguous())
    with pytest.raises(RuntimeError, match=r"workspace shape must be \[B,Hq,splits,D\+2\]"):
        attention_amd.gqa_decode_split(q, k, v, table, lens, splits=4, workspace=ws)
    with pytest.raises(RuntimeError, match="workspace must be contiguous float32 on q device"):
        attention_amd.gqa_decode_split(q, k, v, table, lens, splits=2, workspace=ws.double())


def test_cabi_matches_torch_op_bitwise(gpu):
    say("C ABI automatic path vs torch op")
    cfg = CONFIGS["cfg2"]
    q, k, v, table, lens = to_dev(cfg.make(device="cpu"), gpu)
    out_op = attention_amd.gqa_decode(q, k, v, table, lens)
    ws = cabi.auto_workspace(32, 32, 8, 128, 16, table.shape[1], cabi.DTYPE[q.dtype], gpu)
    out = torch.empty_like(q)
    rc = cabi.auto_launch(q, k, v, table, lens, out, scale=1 / math.sqrt(128), workspace=ws)
    assert rc == 0, cabi.error_string(rc)
    torch.cuda.synchronize()
    assert torch.equal(out, out_op)


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{DT_NAME[s[0]]}-Hq{s[1]}-Hkv{s[2]}-D{s[3]}-P{s[4]}")
def test_shapes_auto_cabi(gpu, shape):
    dtype, hq, hkv, d, p, lengths = shape
    kind, waves, splits, chunk = cabi.auto_info(len(lengths), hq, hkv, d, p,
                                                max(1, -(-max(lengths) // p)), cabi.DTYPE[dtype])
    say(f"auto shape {shape[1:5]} {DT_NAME[dtype]} kind={kind} waves={waves} splits={splits}")
    if dtype == torch.float32 and d in (64, 128) and p % 16 == 0 and hq // hkv <= 16:
        # fp32 takes the balanced (fp32 MFMA) path exactly when the capacity reaches 65536 tokens
        assert (kind == 1) == (len(lengths) * -(-max(lengths) // p) * p >= 65536), kind
    case = to_dev(make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=d,
                                   block_size=p, dtype=dtype, seed=8), gpu)
    q, k, v, table, lens = case
    ref, rows = oracle_rows(case)
    ws = cabi.auto_workspace(q.shape[0], hq, hkv, d, p, table.shape[1], cabi.DTYPE[dtype], gpu,
                             fill=0xFF)  # NaN / -1 scratch past the counters
    out = torch.full_like(q, float("nan"))
    rc = cabi.auto_launch(q, k, v, table, lens, out, scale=1 / math.sqrt(d), workspace=ws)
    assert rc == 0, cabi.error_string(rc)
    torch.cuda.synchronize()
    assert_close(out, ref, DT_NAME[dtype], rows, "auto")


def test_auto_workspace_reuse_across_length_mixes(gpu):
    """One workspace, three calls whose lengths split the items differently:
    an item held whole by one wave in a later call must not be merged from
    an earlier call's leftovers."""
    hq, hkv, d, p = 32, 8, 128, 16
    mixes = [[4096, 4096, 1, 3000, 17, 2048], [16, 4096, 4096, 1, 0, 5000], [300, 1, 1, 1, 1, 6000]]
    maxp = -(-max(max(m) for m in mixes) // p)
    ws = cabi.auto_workspace(6, hq, hkv, d, p, maxp, cabi.DTYPE[torch.bfloat16], gpu, fill=0x7F)
    for i, lengths in enumerate(mixes):
        say(f"workspace reuse mix {i}: {lengths}")
        q, k, v, table, lens = make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=d,
                                                block_size=p, dtype=torch.bfloat16, seed=20 + i)
        tpad = torch.full((6, maxp), -1, dtype=torch.int32)
        tpad[:, :table.shape[1]] = table
        case = to_dev((q, k, v, tpad, lens), gpu)
        ref, rows = oracle_rows(case)
        out = torch.full_like(case[0], float("nan"))
        rc = cabi.auto_launch(*case, out, scale=1 / math.sqrt(d), workspace=ws)
        assert rc == 0, cabi.error_string(rc)
        torch.cuda.synchronize()
        assert_close(out, ref, "bf16", rows, f"mix {i}")
    

@pytest.mark.parametrize("lengths", [[40, 0], [48, 20], [1, 200, 3], [17] * 5], ids=["3g", "3g+2g", "1g+13g+1g", "5x2g"])
def test_auto_few_groups_wide_table(gpu, lengths):
    """A wide page table (256 pages) sizes the stream-K grid for long
    sequences; with only a few 16-token groups in the batch most workgroups
    get no group.  No workgroup between the first and the last holder of a
    sequence may be left without one: the merge folds every slot in that
    span, and the scratch here is NaN, so an unwritten slot shows."""
    hq, hkv, d, p, maxp = 32, 8, 128, 16, 256
    B = len(lengths)
    kind, waves, _, _ = cabi.auto_info(B, hq, hkv, d, p, maxp, cabi.DTYPE[torch.bfloat16])
    say(f"few groups, wide table: lengths {lengths} kind={kind} waves={waves}")
    q, k, v, table, lens = make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=d,
                                            block_size=p, dtype=torch.bfloat16, seed=41)
    tpad = torch.full((B, maxp), -1, dtype=torch.int32)
    tpad[:, :table.shape[1]] = table
    case = to_dev((q, k, v, tpad, lens), gpu)
    ref, rows = oracle_rows(case)
    ws = cabi.auto_workspace(B, hq, hkv, d, p, maxp, cabi.DTYPE[torch.bfloat16], gpu, fill=0xFF)
    out = torch.full_like(case[0], float("nan"))
    rc = cabi.auto_launch(*case, out, scale=1 / math.sqrt(d), workspace=ws)
    assert rc == 0, cabi.error_string(rc)
    torch.cuda.synchronize()
    assert_close(out, ref, "bf16", rows, "few groups")


_BIG_MIX = [int(x) for x in np.random.default_rng(5).integers(0, 120, 520)]
for _i in range(0, 520, 37):
    _BIG_MIX[_i] = 0


@pytest.mark.parametrize("lengths", [[1] * 300, [0] * 5 + [33], [16] * 64, [1, 0, 2, 0, 15, 16, 17],
                                     _BIG_MIX],
                         ids=["ones", "zeros-then-one", "one-group-each", "tiny-mix", "b520-with-zeros"])
def test_auto_tiny_items(gpu, lengths):
    say(f"auto tiny items {lengths[:8]}... (B={len(lengths)})")
    case = to_dev(make_decode_case(lengths=lengths, q_heads=16, kv_heads=2, head_dim=64, block_size=16,
                                   dtype=torch.float16, seed=31), gpu)
    ref, rows = oracle_rows(case)
    out = attention_amd.gqa_decode(*case)
    torch.cuda.synchronize()
    assert_close(out, ref, "f16", rows, "tiny")


@pytest.mark.parametrize("shape", [
    # one head per wave (B*Hq <= 2048); the one sequence spans every
    # workgroup, so each of a wave's four row groups folds 64 rows in
    # several round trips
    (torch.bfloat16, 8, 2, 128, 16, [20000]),
    # four heads per wave (B*Hq > 2048); about 28 workgroups per sequence,
    # more than one 8-row round trip per head
    (torch.float16, 256, 16, 64, 16, [3000, 2900, 3100, 2999, 3001, 17, 2800, 3050, 2950]),
    # fp32 output rows from both merge layouts
    (torch.float32, 8, 2, 128, 16, [65600]),
    (torch.float32, 256, 16, 64, 16, [8000, 1100, 1000, 17, 800, 950, 1, 1020, 990]),
], ids=["one-head-many-rows", "four-heads-many-rows", "f32-one-head", "f32-four-heads"])
def test_auto_merge_layouts(gpu, shape):
    dt, hq, hkv, d, p, lengths = shape
    say(f"merge layouts: {DT_NAME[dt]} Hq{hq} Hkv{hkv} D{d} lengths {lengths[:3]}... (B={len(lengths)})")
    case = to_dev(make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=d, block_size=p,
                                   dtype=dt, seed=23, exact_pool=True), gpu)
    assert cabi.auto_info(len(lengths), hq, hkv, d, p, case[3].shape[1], cabi.DTYPE[dt])[0] == 1
    ref, rows = oracle_rows(case)
    out = attention_amd.gqa_decode(*case)
    torch.cuda.synchronize()
    assert_close(out, ref, DT_NAME[dt], rows, "merge layouts")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_auto_wave_shapes_by_capacity(gpu, dtype):
    """The automatic path serves two kv-heads per wave when the batch's
    static capacity (B * max_pages * block_size) is large, else one.  The
    same lengths under a narrow and under a wide (-1 padded) page table run
    both wave shapes; each must match the oracle."""
    hq, hkv, d, p = 32, 8, 128, 16
    lengths = [3000, 1, 4097, 2000, 17, 0, 5000, 700]
    B = len(lengths)
    q, k, v, table, lens = make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=d,
                                            block_size=p, dtype=dtype, seed=19, exact_pool=True)
    for maxp in (table.shape[1], 8192):
        kind, waves, _, _ = cabi.auto_info(B, hq, hkv, d, p, maxp, cabi.DTYPE[dtype])
        say(f"wave shapes: {DT_NAME[dtype]} max_pages={maxp} kind={kind} waves={waves}")
        tpad = torch.full((B, maxp), -1, dtype=torch.int32)
        tpad[:, :table.shape[1]] = table
        case = to_dev((q, k, v, tpad, lens), gpu)
        ref, rows = oracle_rows(case)
        out = attention_amd.gqa_decode(*case)
        torch.cuda.synchronize()
        assert_close(out, ref, DT_NAME[dtype], rows, f"max_pages={maxp}")


def test_auto_wave_layout_on_device(gpu):
    """Resident waves of the automatic path on the device: one workgroup per
    CU in every layout.  8 kv-heads: 8 one-kv-head waves (two per SIMD), or
    4 two-kv-head waves for large capacities; 4 kv-heads at head_dim 128: 4
    waves with one per SIMD (3 groups in flight), not two 4-wave workgroups
    per CU."""
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    bf16 = cabi.DTYPE[torch.bfloat16]
    say(f"wave layout on device: {cus} CUs")
    assert cabi.auto_info(32, 32, 8, 128, 16, 256, bf16)[:2] == (1, cus * 8)     # cfg2
    assert cabi.auto_info(8, 64, 8, 128, 16, 8192, bf16)[:2] == (1, cus * 4)     # cfg4
    assert cabi.auto_info(64, 28, 4, 128, 16, 512, bf16)[:2] == (1, cus * 4)     # cfg3
    assert cabi.auto_info(64, 28, 4, 64, 16, 512, bf16)[1] > cus * 4             # D 64: 4-wave groups share CUs


def test_repeat_calls_deterministic(gpu):
    say("determinism across calls")
    case = to_dev(CONFIGS["cfg3"].make(device="cpu"), gpu)
    a = attention_amd.gqa_decode(*case)
    b = attention_amd.gqa_decode(*case)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("seed", range(1, 9))
def test_bf16_accuracy_over_seeds(gpu, seed):
    """Random lengths with short, peaked rows in bf16.  With one bf16 rounding
    of the softmax weights in the PV product some of these seeds landed past
    the 16-bit bar (worst 1.3x of it); the MFMA kernels carry the weights as
    hi + lo (MfmaOps::kSplitWeights) and stay near 0.6x."""
    rng = np.random.default_rng(seed)
    lengths = [int(x) for x in rng.integers(1, 700, size=6)] + [1, 2, 3, 17]
    say(f"bf16 accuracy seed {seed} lengths {lengths}")
    case = to_dev(make_decode_case(lengths=lengths, q_heads=32, kv_heads=8, head_dim=128, block_size=16,
                                   dtype=torch.bfloat16, seed=seed), gpu)
    out = attention_amd.gqa_decode(*case)
    torch.cuda.synchronize()
    ref, rows = oracle_rows(case)
    assert_close(out, ref, "bf16", rows, f"seed {seed}")


def test_graph_capture_replays_match_eager(gpu):
    """attention_amd.gqa_decode captured in a HIP graph: its per-call
    workspace comes from the graph's pool, so every replay (with eager calls
    and synchronizations between replays) reproduces the eager output bit
    for bit."""
    say("graph capture: replays vs eager")
    case = to_dev(make_decode_case(lengths=[700, 1, 2049, 0, 333, 1500], q_heads=32, kv_heads=8, head_dim=128,
                                   block_size=16, dtype=torch.bfloat16, seed=12), gpu)
    ref = attention_amd.gqa_decode(*case)
    other = to_dev(make_decode_case(lengths=[40, 900], q_heads=32, kv_heads=8, head_dim=128, block_size=16,
                                    dtype=torch.bfloat16, seed=13), gpu)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            attention_amd.gqa_decode(*case)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = attention_amd.gqa_decode(*case)
    torch.cuda.synchronize()
    for i in range(3):
        say(f"graph replay {i}")
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}"
        attention_amd.gqa_decode(*other)   # eager work on the same stream between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("hq,hkv,dtype", [(32, 8, torch.bfloat16), (40, 8, torch.float16), (28, 4, torch.bfloat16),
                                          (64, 8, torch.bfloat16)], ids=["g4-bf16", "g5-f16", "g7-bf16", "g8-bf16"])
def test_valu_comparison_variant_matches_oracle(gpu, hq, hkv, dtype):
    """The VALU math variant of the balanced decode kernel (QD_STAGE_VALU,
    kept for the MFMA-versus-VALU measurement) on group sizes 4, 5, 7 and 8,
    with ragged lengths, a zero length and sequences split across
    workgroups."""
    lengths = [1, 17, 300, 0, 2049, 1000, 16, 4000]
    say(f"VALU variant g={hq // hkv} {DT_NAME[dtype]}")
    case = to_dev(make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=128, block_size=16,
                                   dtype=dtype, seed=29), gpu)
    q, k, v, table, lens = case
    ref, rows = oracle_rows(case)
    ws = cabi.auto_workspace(len(lengths), hq, hkv, 128, 16, table.shape[1], cabi.DTYPE[dtype], gpu, fill=0xFF)
    out = torch.full_like(q, float("nan"))
    rc = cabi.auto_launch(q, k, v, table, lens, out, scale=1 / math.sqrt(128), workspace=ws,
                          stages=cabi.QD_STAGE_ALL | cabi.QD_STAGE_VALU)
    assert rc == 0, cabi.error_string(rc)
    torch.cuda.synchronize()
    assert_close(out, ref, DT_NAME[dtype], rows, "VALU variant")


# ----------------------------------------------------------------------------
# Fused merge: split sequences merged inside the decode kernel by the wave
# that arrives last at each (sequence, kv-head) counter.
# ----------------------------------------------------------------------------

def _fused_lengths(n, lo, hi, seed):
    rng = np.random.default_rng(seed)
    return [int(x) for x in rng.integers(lo, hi + 1, size=n)]


FUSED_SHAPES = [
    # cfg2's shape: one kv-head per wave, 4 heads, ~9 rows per merge
    (torch.bfloat16, 32, 8, 128, 16, _fused_lengths(32, 512, 4096, 51)),
    # cfg5's shape: 5 heads (two passes), block_size 32, mostly 1-2 rows
    (torch.float16, 40, 8, 128, 32, _fused_lengths(96, 128, 1024, 52)),
    # cfg3's shape: 4 kv-heads (one wave per SIMD, 3 groups in flight), 7 heads
    (torch.bfloat16, 28, 4, 128, 16, [1, 8192, 17, 5000, 0, 16, 3001, 4096, 2, 7000]),
    # head_dim 64 and 256 (8 rows per round trip at 256)
    (torch.float16, 16, 2, 64, 16, [3000, 1, 2500, 0, 4000]),
    (torch.bfloat16, 16, 4, 256, 16, [6000, 300, 4100]),
    # two kv-heads per wave (wide table), 16 heads per merging wave, one
    # sequence over every workgroup: many passes and row batches
    (torch.bfloat16, 64, 8, 128, 16, [60000]),
]


@pytest.mark.parametrize("shape", FUSED_SHAPES,
                         ids=lambda s: f"{DT_NAME[s[0]]}-Hq{s[1]}-Hkv{s[2]}-D{s[3]}-P{s[4]}-B{len(s[5])}")
def test_fused_merge_matches_unfused_and_oracle(gpu, shape):
    """QD_STAGE_FUSED (merge by the last-arriving wave, sc1 partials) and
    QD_STAGE_UNFUSED (merge_sk_kernel) on one workspace whose bytes past the
    counters are NaN: both match the oracle, match each other to fp32
    rounding of the fold order, and the counters are all zero afterwards."""
    dtype, hq, hkv, d, p, lengths = shape
    B = len(lengths)
    case = to_dev(make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=d, block_size=p,
                                   dtype=dtype, seed=61, exact_pool=True), gpu)
    q, k, v, table, lens = case
    maxp = table.shape[1]
    kind, waves, _, _ = cabi.auto_info(B, hq, hkv, d, p, maxp, cabi.DTYPE[dtype])
    say(f"fused vs unfused: {DT_NAME[dtype]} Hq{hq} Hkv{hkv} D{d} P{p} B{B} kind={kind} waves={waves}")
    assert kind in (1, 2)
    ref, rows = oracle_rows(case)
    ws = cabi.auto_workspace(B, hq, hkv, d, p, maxp, cabi.DTYPE[dtype], gpu, fill=0xFF)
    outs = {}
    for name, flag in (("fused", cabi.QD_STAGE_FUSED), ("unfused", cabi.QD_STAGE_UNFUSED),
                       ("fused-again", cabi.QD_STAGE_FUSED)):
        out = torch.full_like(q, float("nan"))
        rc = cabi.auto_launch(q, k, v, table, lens, out, scale=1 / math.sqrt(d), workspace=ws,
                              stages=cabi.QD_STAGE_ALL | flag)
        assert rc == 0, cabi.error_string(rc)
        torch.cuda.synchronize()
        assert_close(out, ref, DT_NAME[dtype], rows, name)
        outs[name] = out
    assert torch.equal(outs["fused"], outs["fused-again"])
    # Same partials, folded in another order: within one output rounding.
    diff = (outs["fused"].float() - outs["unfused"].float()).abs()
    assert torch.all(diff <= 1e-2 * outs["unfused"].float().abs() + 1e-6), diff.max().item()
    nc = cabi.auto_counter_bytes()
    assert int(torch.count_nonzero(ws[:nc])) == 0, "arrival counters not left at zero"


def test_fused_counters_reused_across_shapes(gpu):
    """One workspace through fused calls of different batches, head counts
    and lengths: every call starts from and leaves zero counters, and every
    output matches the oracle."""
    specs = [(32, 8, [4096, 3000, 1, 2048] * 8), (40, 8, [700, 0, 1024, 129] * 16), (28, 4, [8192, 1, 5000, 33]),
             (32, 8, [17, 4000, 4000, 4000, 3])]
    maxp = 512
    nbytes = max(cabi.auto_workspace_bytes(len(l), hq, hkv, 128, 16, maxp, cabi.DTYPE[torch.bfloat16])
                 for hq, hkv, l in specs)
    ws = torch.full((nbytes,), 0x7F, device=gpu, dtype=torch.uint8)
    ws[:cabi.auto_counter_bytes()].zero_()
    for i, (hq, hkv, lengths) in enumerate(specs):
        say(f"fused counters reuse {i}: Hq{hq} Hkv{hkv} B{len(lengths)}")
        q, k, v, table, lens = make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=128,
                                                block_size=16, dtype=torch.bfloat16, seed=70 + i)
        tpad = torch.full((len(lengths), maxp), -1, dtype=torch.int32)
        tpad[:, :table.shape[1]] = table
        case = to_dev((q, k, v, tpad, lens), gpu)
        ref, rows = oracle_rows(case)
        out = torch.full_like(case[0], float("nan"))
        rc = cabi.auto_launch(*case, out, scale=1 / math.sqrt(128), workspace=ws,
                              stages=cabi.QD_STAGE_ALL | cabi.QD_STAGE_FUSED)
        assert rc == 0, cabi.error_string(rc)
        torch.cuda.synchronize()
        assert_close(out, ref, "bf16", rows, f"reuse {i}")
        assert int(torch.count_nonzero(ws[:cabi.auto_counter_bytes()])) == 0


def test_torch_op_on_concurrent_streams(gpu):
    """attention_amd.gqa_decode on two streams at once: each stream has its
    own workspace (and counters), so interleaved calls give the same bits as
    calls made one at a time."""
    say("torch op on two concurrent streams")
    cases = [to_dev(make_decode_case(lengths=_fused_lengths(32, 512, 4096, 80 + i), q_heads=32, kv_heads=8,
                                     head_dim=128, block_size=16, dtype=torch.bfloat16, seed=80 + i), gpu)
             for i in range(2)]
    refs = [attention_amd.gqa_decode(*c) for c in cases]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outs = [[], []]
    for _ in range(4):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                outs[i].append(attention_amd.gqa_decode(*cases[i]))
    torch.cuda.synchronize()
    for i in range(2):
        for j, o in enumerate(outs[i]):
            assert torch.equal(o, refs[i]), (i, j)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_held_results_flush_when_full(gpu, dtype):
    """Batches with at least one sequence per two workgroups hold each
    wave's result rows in LDS until its range ends.  3000 one- and
    two-group sequences (and some empty ones) give every wave more items
    than its LDS area and record table hold, so the area is flushed
    early, repeatedly; every row must match the oracle, and the -1 padded
    wide table must not matter."""
    rng = np.random.default_rng(91)
    lengths = [int(x) for x in rng.integers(1, 33, size=3000)]
    for i in (0, 7, 1500, 2999):
        lengths[i] = 0
    say(f"held results, many items per wave: {DT_NAME[dtype]} B={len(lengths)}")
    q, k, v, table, lens = make_decode_case(lengths=lengths, q_heads=32, kv_heads=8, head_dim=128, block_size=16,
                                            dtype=dtype, seed=92, exact_pool=True)
    case = to_dev((q, k, v, table, lens), gpu)
    kind, waves, _, _ = cabi.auto_info(len(lengths), 32, 8, 128, 16, table.shape[1], cabi.DTYPE[dtype])
    assert kind == 1
    ref, rows = oracle_rows(case)
    out = attention_amd.gqa_decode(*case)
    torch.cuda.synchronize()
    assert_close(out, ref, DT_NAME[dtype], rows, "held results")
    # Same bits through the C ABI on a NaN-filled workspace.
    ws = cabi.auto_workspace(len(lengths), 32, 8, 128, 16, table.shape[1], cabi.DTYPE[dtype], gpu, fill=0xFF)
    out_c = torch.full_like(case[0], float("nan"))
    rc = cabi.auto_launch(*case, out_c, scale=1 / math.sqrt(128), workspace=ws)
    assert rc == 0, cabi.error_string(rc)
    torch.cuda.synchronize()
    assert torch.equal(out, out_c)


# (q_heads, kv_heads, head_dim, dtype, waves per workgroup of the plan, lengths)
HELD_LAYOUTS = [
    # head_dim 64, 2 kv-heads: 2 single-kv-head waves per workgroup, several workgroups per CU
    (16, 2, 64, torch.float16, 2, _fused_lengths(1200, 1, 300, 93)),
    # head_dim 256: 4 waves, one per SIMD, two kv-heads of a sequence per wave (with one
    # kv-head per wave, as for 4 kv-heads at head_dim 128, the rows are stored after each item)
    (16, 8, 256, torch.bfloat16, 4, _fused_lengths(300, 1, 200, 94)),
    # two kv-heads per wave: a wide table (one long sequence) among short ones
    (32, 8, 128, torch.float16, 4, [3500] + _fused_lengths(299, 1, 100, 96)),
    # head_dim 96: 8 single-kv-head waves, 12-byte output pieces
    (32, 8, 96, torch.bfloat16, 8, _fused_lengths(300, 1, 200, 135)),
    # fp32 caches: head_dim 128 with 4 waves (one per SIMD), head_dim 64 with 4 of up to 8
    (32, 8, 128, torch.float32, 4, [240] + _fused_lengths(299, 1, 200, 136)),
    (16, 4, 64, torch.float32, 4, _fused_lengths(600, 1, 300, 137)),
]


LARGE_GROUP_SHAPES = [
    # (dtype, Hq, Hkv, D, P, lengths): groups above 16 q-heads, served as equal chunks of <= 16
    (torch.bfloat16, 48, 1, 128, 16, [1, 17, 300, 2048, 0, 5000]),          # 3 x 16, 3 waves
    (torch.float16, 32, 1, 64, 32, [33, 1000, 4097, 2]),                    # 2 x 16, D 64
    (torch.bfloat16, 64, 2, 128, 16, [700, 1, 3000]),                       # 4 virtual kv-heads: one wave per SIMD
    (torch.bfloat16, 40, 1, 128, 16, [129, 2500]),                          # 14 + 14 + 12: a short last chunk
    (torch.bfloat16, 71, 1, 64, 16, [1, 500, 2100]),                        # 4 x 15 + 11, D 64
    (torch.float16, 128, 1, 128, 16, [40, 3000]),                           # 8 x 16, 8 waves
    (torch.bfloat16, 64, 1, 64, 16, [17, 1500, 3000]),                      # 4 x 16, D 64
    (torch.bfloat16, 64, 1, 128, 16, [700, 1, 3000]),                       # 4 x 16: one wave per SIMD
    (torch.bfloat16, 48, 1, 96, 16, [1, 700, 2500]),                        # 3 x 16 at head_dim 96
    (torch.float16, 96, 2, 256, 16, [900, 31, 2000]),                       # D 256, 3 x 16
    (torch.bfloat16, 384, 8, 128, 16, [300, 1200]),                         # 24 virtual kv-heads, 6 waves
    (torch.bfloat16, 48, 1, 128, 16, _fused_lengths(300, 1, 200, 131)),     # held result rows
    (torch.float16, 40, 1, 64, 16, _fused_lengths(300, 1, 120, 132)),      # held rows, short last chunk
]


@pytest.mark.parametrize("shape", LARGE_GROUP_SHAPES,
                         ids=lambda s: f"{DT_NAME[s[0]]}-Hq{s[1]}-Hkv{s[2]}-D{s[3]}-P{s[4]}-B{len(s[5])}")
def test_large_groups_balanced_path(gpu, shape):
    """Groups of more than 16 q-heads per kv-head on the balanced MFMA path:
    each kv-head is served as equal chunks of at most 16 q-heads by waves of
    one workgroup reading the same K/V rows.  The plan takes the path (kind
    1), every row matches the oracle, and the torch op and the C ABI on a
    NaN-filled workspace give the same bits."""
    dtype, hq, hkv, d, p, lengths = shape
    B = len(lengths)
    case = to_dev(make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=d, block_size=p,
                                   dtype=dtype, seed=133, exact_pool=True), gpu)
    q, k, v, table, lens = case
    kind, waves, _, _ = cabi.auto_info(B, hq, hkv, d, p, table.shape[1], cabi.DTYPE[dtype])
    say(f"large group: {DT_NAME[dtype]} Hq{hq} Hkv{hkv} D{d} P{p} B{B} kind={kind} waves={waves}")
    assert kind == 1
    ref, rows = oracle_rows(case)
    out = attention_amd.gqa_decode(*case)
    torch.cuda.synchronize()
    assert_close(out, ref, DT_NAME[dtype], rows, "large group")
    ws = cabi.auto_workspace(B, hq, hkv, d, p, table.shape[1], cabi.DTYPE[dtype], gpu, fill=0xFF)
    out_c = torch.full_like(q, float("nan"))
    rc = cabi.auto_launch(*case, out_c, scale=1 / math.sqrt(d), workspace=ws)
    assert rc == 0, cabi.error_string(rc)
    torch.cuda.synchronize()
    assert torch.equal(out, out_c)


def test_group_above_128_generic_path(gpu):
    """A group of 136 q-heads (more than 8 chunks of 16) stays on the split
    layout's generic kernel and matches the oracle."""
    hq, hkv, d, p, lengths = 136, 1, 64, 16, [1, 500, 2100]
    case = to_dev(make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=d, block_size=p,
                                   dtype=torch.bfloat16, seed=134), gpu)
    kind = cabi.auto_info(len(lengths), hq, hkv, d, p, case[3].shape[1], cabi.DTYPE[torch.bfloat16])[0]
    say(f"group 136: kind={kind}")
    assert kind == 0
    ref, rows = oracle_rows(case)
    out = attention_amd.gqa_decode(*case)
    torch.cuda.synchronize()
    assert_close(out, ref, "bf16", rows, "group 136")


@pytest.mark.parametrize("shape", HELD_LAYOUTS,
                         ids=lambda s: f"{DT_NAME[s[3]]}-Hq{s[0]}-Hkv{s[1]}-D{s[2]}-B{len(s[5])}")
def test_held_results_every_layout(gpu, shape):
    """The held-results kernels (result rows kept in LDS until a range ends,
    chosen when the batch has at least one sequence per two workgroups) in
    each wave layout the plan can pair them with: the batch is large enough
    for the hold (2 B >= W), every row matches the oracle, and the torch op
    and the C ABI on a NaN-filled workspace give the same bits."""
    hq, hkv, d, dtype, wg_waves, lengths = shape
    B = len(lengths)
    case = to_dev(make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=d, block_size=16,
                                   dtype=dtype, seed=97, exact_pool=True), gpu)
    q, k, v, table, lens = case
    kind, waves, _, _ = cabi.auto_info(B, hq, hkv, d, 16, table.shape[1], cabi.DTYPE[dtype])
    say(f"held results: {DT_NAME[dtype]} Hq{hq} Hkv{hkv} D{d} B{B} kind={kind} waves={waves}")
    assert kind == 1 and waves % wg_waves == 0
    assert 2 * B >= waves // wg_waves, "the batch does not take the held-results kernel"
    ref, rows = oracle_rows(case)
    out = attention_amd.gqa_decode(*case)
    torch.cuda.synchronize()
    assert_close(out, ref, DT_NAME[dtype], rows, "held results")
    ws = cabi.auto_workspace(B, hq, hkv, d, 16, table.shape[1], cabi.DTYPE[dtype], gpu, fill=0xFF)
    out_c = torch.full_like(q, float("nan"))
    rc = cabi.auto_launch(*case, out_c, scale=1 / math.sqrt(d), workspace=ws)
    assert rc == 0, cabi.error_string(rc)
    torch.cuda.synchronize()
    assert torch.equal(out, out_c)


@pytest.mark.parametrize("merge", ["unfused", "fused"])
@pytest.mark.parametrize("shape", [(32, 8, 128, torch.bfloat16, _fused_lengths(32, 512, 4096, 98)),
                                   (40, 8, 128, torch.float16, _fused_lengths(300, 1, 600, 99))],
                         ids=["cfg2-like", "held-results"])
def test_stages_separately_match_whole_call(gpu, shape, merge):
    """qd_gqa_decode_auto_stages as the header documents it: QD_STAGE_DECODE
    then QD_STAGE_MERGE (same arguments and workspace, same stream) give the
    bits of one QD_STAGE_ALL call; with the fused merge the decode stage is
    the whole call and QD_STAGE_MERGE alone changes nothing."""
    hq, hkv, d, dtype, lengths = shape
    B = len(lengths)
    case = to_dev(make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=d, block_size=16,
                                   dtype=dtype, seed=100, exact_pool=True), gpu)
    q = case[0]
    maxp = case[3].shape[1]
    flag = cabi.QD_STAGE_FUSED if merge == "fused" else cabi.QD_STAGE_UNFUSED
    say(f"stages separately: {DT_NAME[dtype]} Hq{hq} Hkv{hkv} B{B} merge={merge}")
    ws = cabi.auto_workspace(B, hq, hkv, d, 16, maxp, cabi.DTYPE[dtype], gpu, fill=0xFF)

    def run(stages, out):
        rc = cabi.auto_launch(*case, out, scale=1 / math.sqrt(d), workspace=ws, stages=stages | flag)
        assert rc == 0, cabi.error_string(rc)

    whole = torch.full_like(q, float("nan"))
    run(cabi.QD_STAGE_ALL, whole)
    parts = torch.full_like(q, float("nan"))
    run(cabi.QD_STAGE_DECODE, parts)
    if merge == "fused":
        torch.cuda.synchronize()
        before = parts.clone()
        run(cabi.QD_STAGE_MERGE, parts)
        torch.cuda.synchronize()
        assert torch.equal(parts, before), "QD_STAGE_MERGE alone changed a fused call's output"
    else:
        run(cabi.QD_STAGE_MERGE, parts)
    torch.cuda.synchronize()
    assert torch.equal(parts, whole)
    ref, rows = oracle_rows(case)
    assert_close(whole, ref, DT_NAME[dtype], rows, "whole call")


# (dtype, Hq, Hkv, D, P, lengths): sequences over many 64-page table windows
# of the generic kernel, window edges inside 4-token steps, both head-chunk
# widths (4 heads per wave for groups of at most 4, else 8).
GENERIC_WINDOW_SHAPES = [
    (torch.float32, 6, 2, 128, 1, [700, 1, 130, 65]),     # P=1: a window is 64 tokens
    (torch.float32, 40, 5, 100, 3, [1000, 194, 2]),      # 8 heads per group, D not a power of two
    (torch.bfloat16, 8, 2, 64, 7, [900, 449, 450, 451]),  # 4 heads per group, 7-token pages
    (torch.float16, 20, 4, 256, 16, [3000, 1025, 17]),   # head_dim 256: one step at a time
]


@pytest.mark.parametrize("shape", GENERIC_WINDOW_SHAPES,
                         ids=lambda s: f"{DT_NAME[s[0]]}-Hq{s[1]}-Hkv{s[2]}-D{s[3]}-P{s[4]}")
def test_generic_kernel_table_windows(gpu, shape):
    """The generic kernel's page-table window (64 pages in the lanes of a
    wave) and its two steps in flight: every row matches the oracle with one
    split (a sequence crosses many windows) and with three."""
    dtype, hq, hkv, d, p, lengths = shape
    say(f"generic windows {DT_NAME[dtype]} Hq{hq} Hkv{hkv} D{d} P{p} lengths {lengths}")
    case = to_dev(make_decode_case(lengths=lengths, q_heads=hq, kv_heads=hkv, head_dim=d, block_size=p,
                                   dtype=dtype, seed=101), gpu)
    q, k, v, table, lens = case
    ref, rows = oracle_rows(case)
    for splits in (1, 3):
        out = torch.full_like(q, float("nan"))
        ws = torch.empty(max(1, q.shape[0] * hq * splits * (d + 2)), device=gpu, dtype=torch.float32)
        rc = cabi.launch(q, k, v, table, lens, out, scale=1 / math.sqrt(d), splits=splits, chunk_pages=0,
                         workspace=ws if splits > 1 else None, flags=cabi.QD_FLAG_FORCE_GENERIC)
        assert rc == 0, cabi.error_string(rc)
        torch.cuda.synchronize()
        assert_close(out, ref, DT_NAME[dtype], rows, f"splits={splits}")
