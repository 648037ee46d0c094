"""CPU tests of the drop-in boundary: the C ABI library loads and exports
every declared symbol, host-side validation reproduces the reference's
checks in order (reference csrc/cuda/dense/gqa_decode.cu:103-138, :148-152),
the launch plan, launch argument errors (reported before anything is
enqueued), the torch op schemas, and the Python API's error behaviour
(reference attention/core.py:30-35, :48-49, :86-87).  No kernel runs here.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

import attention_amd
from attention_amd import cabi, core
from attention_amd.cases import CONFIGS

F32, F16, BF16, I32 = 0, 1, 2, 3


def test_library_exports_every_header_symbol():
    names = cabi.header_functions()
    assert len(names) >= 8
    L = ctypes.CDLL(cabi.LIB_PATH)
    for n in names:
        assert hasattr(L, n), n
    assert cabi.lib().qd_abi_version() == 2


def good():
    return [cabi.desc([4, 8, 64], F16), cabi.desc([57, 16, 2, 64], F16),
            cabi.desc([57, 16, 2, 64], F16), cabi.desc([4, 32], I32), cabi.desc([4], I32)]


def test_validate_accepts_good_shapes():
    assert cabi.validate(*good()) == (0, "")


def _case(mutate, scale=0.125, splits=1):
    d = good()
    mutate(d)
    return cabi.validate(*d, scale=scale, splits=splits)


def _set(i, **kw):
    def f(d):
        for key, val in kw.items():
            if key == "sizes":
                d[i] = cabi.desc(val, d[i].dtype, d[i].is_device, d[i].device_index, d[i].contiguous)
            else:
                setattr(d[i], key, val)
    return f


VALIDATION_ORDER = [
    # (mutation, scale, splits, expected message)
    (lambda d: None, 0.125, 0, "splits must be in [1, 65535]"),
    (lambda d: None, 0.125, 65536, "splits must be in [1, 65535]"),
    (_set(0, is_device=0), 0.125, 1, "q must be a CUDA tensor"),
    (_set(0, contiguous=0), 0.125, 1, "q must be contiguous"),
    (_set(1, is_device=0), 0.125, 1, "k_cache must be a CUDA tensor"),
    (_set(2, contiguous=0), 0.125, 1, "v_cache must be contiguous"),
    (_set(3, is_device=0), 0.125, 1, "block_table must be a CUDA tensor"),
    (_set(4, contiguous=0), 0.125, 1, "context_lens must be contiguous"),
    (_set(0, sizes=[4, 8]), 0.125, 1, "q must be [B, Hq, D]"),
    (_set(1, sizes=[57, 16, 128]), 0.125, 1, "k_cache must be [Nblocks, BlockSize, Hkv, D]"),
    (_set(2, sizes=[57, 16, 2, 32]), 0.125, 1, "v_cache shape mismatch"),
    (_set(3, sizes=[4, 32, 1]), 0.125, 1, "block_table must be [B, MaxPages]"),
    (_set(4, sizes=[4, 1]), 0.125, 1, "context_lens must be [B]"),
    (_set(2, device_index=1), 0.125, 1, "all tensors must use one CUDA device"),
    (_set(1, dtype=BF16), 0.125, 1, "q/k/v dtype must match"),
    (lambda d: [setattr(x, "dtype", 5) for x in d[:3]], 0.125, 1,
     "q/k/v must be float32/float16/bfloat16"),
    (_set(3, dtype=5), 0.125, 1, "block_table and context_lens must be int32"),
    (_set(4, sizes=[3]), 0.125, 1, "batch sizes must match"),
    (lambda d: (_set(1, sizes=[57, 16, 2, 32])(d), _set(2, sizes=[57, 16, 2, 32])(d)), 0.125, 1,
     "q head_dim and cache head_dim must match"),
    (lambda d: (_set(1, sizes=[57, 16, 3, 64])(d), _set(2, sizes=[57, 16, 3, 64])(d)), 0.125, 1,
     "Hq must be divisible by Hkv"),
    (lambda d: [_set(i, sizes=s)(d) for i, s in
                [(0, [4, 8, 300]), (1, [57, 16, 2, 300]), (2, [57, 16, 2, 300])]], 0.125, 1,
     "supported head_dim is [1, 256]"),
    (lambda d: (_set(1, sizes=[0, 16, 2, 64])(d), _set(2, sizes=[0, 16, 2, 64])(d)), 0.125, 1,
     "cache must have positive blocks and block_size"),
    (_set(3, sizes=[4, 0]), 0.125, 1, "block_table must have at least one page"),
    (lambda d: None, 0.0, 1, "scale must be positive and finite"),
    (lambda d: None, float("inf"), 1, "scale must be positive and finite"),
    (lambda d: None, float("nan"), 1, "scale must be positive and finite"),
    (lambda d: [_set(i, sizes=s)(d) for i, s in
                [(0, [2 ** 31, 8, 64]), (3, [2 ** 31, 32]), (4, [2 ** 31])]], 0.125, 1,
     "tensor sizes exceed int32 CUDA launch limits"),
]


@pytest.mark.parametrize("i", range(len(VALIDATION_ORDER)))
def test_validation_messages_in_reference_order(i):
    mutate, scale, splits, want = VALIDATION_ORDER[i]
    rc, msg = _case(mutate, scale, splits)
    assert rc == 1 and msg == want
    assert cabi.error_string(rc) == want


def test_first_failing_check_wins():
    d = good()
    d[0].is_device = 0           # check 2 (q)
    d[1].dtype = BF16            # check 9
    d[3].sizes[1] = 0            # check 17
    assert cabi.validate(*d)[1] == "q must be a CUDA tensor"


def test_workspace_validation():
    q = cabi.desc([4, 8, 64], F16)
    ok = cabi.desc([4, 8, 4, 66], F32)
    assert cabi.validate_workspace(q, ok, 4) == (0, "")
    assert cabi.validate_workspace(q, ok, 1)[1] == "workspace requires splits > 1"
    bad_dtype = cabi.desc([4, 8, 4, 66], F16)
    assert cabi.validate_workspace(q, bad_dtype, 4)[1] == "workspace must be contiguous float32 on q device"
    other_dev = cabi.desc([4, 8, 4, 66], F32, device=1)
    assert cabi.validate_workspace(q, other_dev, 4)[1] == "workspace must be contiguous float32 on q device"
    assert cabi.validate_workspace(q, cabi.desc([4, 8, 2, 66], F32), 4)[1] == \
        "workspace shape must be [B,Hq,splits,D+2]"
    assert cabi.validate_workspace(q, cabi.desc([4, 8, 4, 64], F32), 4)[1] == \
        "workspace shape must be [B,Hq,splits,D+2]"


# ----------------------------------------------------------------------------
# Plan and workspace size
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("name", list(CONFIGS))
def test_plan_covers_capacity(name):
    cfg = CONFIGS[name]
    max_pages = max(1, -(-max(cfg.lengths()) // cfg.block_size))
    s, c = cabi.plan(cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.block_size, max_pages)
    assert 1 <= s <= 65535 and 1 <= c <= 64 or (s == 1 and c == max_pages)
    assert s * c >= max_pages
    if s > 1:
        assert c * cfg.block_size >= 32 or c == max_pages


def test_plan_values_for_configs():
    # cfg2: 256 (seq, kv-head) items for ~4 waves per CU on 256 CUs, 256-page
    # tables -> 4 splits of 64 pages.
    assert cabi.plan(32, 32, 8, 128, 16, 256) == (4, 64)
    # One sequence: 8 items -> 128 splits of 2 pages (32 tokens at least).
    assert cabi.plan(1, 32, 8, 128, 16, 256) == (128, 2)
    assert cabi.plan(1, 32, 8, 128, 16, 1024) == (128, 8)
    # cfg4: 64 items, 8192-page tables -> 64-page splits.
    assert cabi.plan(8, 64, 8, 128, 16, 8192) == (128, 64)
    # cfg5: 2048 items already fill the GPU -> one pass.
    assert cabi.plan(256, 40, 8, 128, 32, 32) == (1, 32)


@pytest.mark.skipif(torch.cuda.is_available(),
                    reason="wave counts assume the CPU-only occupancy fallback (256 CUs, one workgroup each)")
def test_auto_wave_shape_by_capacity():
    """The automatic path's wave shape follows the batch's static token
    capacity B*max_pages*P: one kv-head per wave (8-wave workgroups for 8
    kv-heads) below 2048 tokens per resident workgroup, two kv-heads per wave
    (4-wave workgroups) at or above it.  Without a GPU the occupancy query
    falls back to 256 CUs and one workgroup each, so 2048 tokens per
    workgroup is a capacity of 524288 tokens."""
    bf16 = cabi.DTYPE[torch.bfloat16]
    # cfg2 (131072 tokens) and cfg5 (262144): one kv-head per wave.
    assert cabi.auto_info(32, 32, 8, 128, 16, 256, bf16)[1] == 256 * 8
    assert cabi.auto_info(256, 40, 8, 128, 32, 32, cabi.DTYPE[torch.float16])[1] == 256 * 8
    # cfg4 (1048576 tokens): two kv-heads per wave.
    assert cabi.auto_info(8, 64, 8, 128, 16, 8192, bf16)[1] == 256 * 4
    # The threshold itself, and just below it.
    assert cabi.auto_info(8, 64, 8, 128, 16, 4096, bf16)[1] == 256 * 4
    assert cabi.auto_info(8, 64, 8, 128, 16, 4095, bf16)[1] == 256 * 8
    # Two kv-heads per wave needs 8+ (an even number of) kv-heads and D <= 128.
    assert cabi.auto_info(8, 28, 4, 128, 16, 8192, bf16)[1] == 256 * 4  # 4 kv-heads: 4 waves
    assert cabi.auto_info(8, 64, 8, 256, 16, 8192, bf16)[1] == 256 * 4  # D 256: 4 waves, one each


@pytest.mark.skipif(torch.cuda.is_available(),
                    reason="wave counts assume the CPU-only occupancy fallback (256 CUs, one workgroup each)")
def test_auto_grid_below_resident():
    """Batches too small to fill the resident grid R: W = min(R, Gmax,
    max(64 B, min(ceil(S / 256 KiB), 128 B))) workgroups, Gmax the 16-token
    groups of the largest batch the shapes allow and S their K/V bytes (64 KiB
    per group at Hkv8/D128 in 16 bits).  At least one group per workgroup, a
    split sequence's partial rows within one merge round trip (64 per head)
    unless the bytes need more workgroups, and at most 128 per sequence.
    8 waves per workgroup here (one kv-head each), 2 for cfg1's 2 kv-heads."""
    bf16, f16 = cabi.DTYPE[torch.bfloat16], cabi.DTYPE[torch.float16]
    cases = [
        ((1, 32, 8, 128, 16, 8), 8),        # B1/L128: one group per workgroup (Gmax = 8)
        ((16, 32, 8, 128, 16, 8), 128),     # B16/L128: Gmax = 128
        ((1, 32, 8, 128, 16, 64), 64),      # B1/L1024: Gmax = 64 = 64 B
        ((1, 32, 8, 128, 16, 256), 64),     # B1/L4096: 64 B (S = 16 MiB is 64 x 256 KiB)
        ((1, 32, 8, 128, 16, 512), 128),    # B1/L8192: S / 256 KiB = 128
        ((1, 32, 8, 128, 16, 2048), 128),   # B1/L32768: capped at 128 B
        ((2, 32, 8, 128, 16, 256), 128),    # B2/L4096: 64 B = S / 256 KiB = 128
        ((4, 32, 8, 128, 16, 64), 256),     # B4/L1024: 64 B = 256 = R
    ]
    for shape, wgs in cases:
        assert cabi.auto_info(*shape, bf16)[:2] == (1, 8 * wgs), shape
    assert cabi.auto_info(4, 8, 2, 64, 16, 32, f16)[:2] == (1, 2 * 128)  # cfg1: Gmax = 128


@pytest.mark.skipif(torch.cuda.is_available(),
                    reason="wave counts assume the CPU-only occupancy fallback (256 CUs, one workgroup each)")
def test_auto_large_groups():
    """Groups above 16 q-heads take the balanced path as c = ceil(g/16)
    virtual kv-heads per kv-head (chunks of ceil(g/c) q-heads, the last one
    shorter), c <= 8, with one kv-head's chunks in one pass of a workgroup's
    waves; larger groups, and fp32, take the split layout (kind 0)."""
    bf16, f32 = cabi.DTYPE[torch.bfloat16], cabi.DTYPE[torch.float32]
    assert cabi.auto_info(32, 48, 1, 128, 16, 128, bf16)[:2] == (1, 256 * 3)    # 3 x 16
    assert cabi.auto_info(32, 40, 1, 128, 16, 64, bf16)[:2] == (1, 256 * 3)     # 14 + 14 + 12
    assert cabi.auto_info(16, 71, 1, 64, 16, 256, bf16)[:2] == (1, 256 * 5)     # 4 x 15 + 11
    assert cabi.auto_info(32, 64, 2, 128, 16, 128, bf16)[:2] == (1, 256 * 4)    # 2 x 2 x 16
    assert cabi.auto_info(8, 384, 8, 128, 16, 256, bf16)[:2] == (1, 256 * 6)    # 24 virtual, passes of 6
    assert cabi.auto_info(4, 128, 1, 128, 16, 64, bf16)[:2] == (1, 256 * 8)     # 8 x 16, the most
    assert cabi.auto_info(4, 136, 1, 128, 16, 64, bf16)[0] == 0                  # 9 chunks would be needed
    assert cabi.auto_info(32, 48, 1, 128, 16, 128, f32)[0] == 0


def test_head_dim_96_takes_the_mfma_kernels():
    """head_dim 96 (K loaded in the MFMA A layout, 12-byte V rows) runs the
    MFMA kernels on both paths; 80 and other head dims the generic one."""
    bf16 = cabi.DTYPE[torch.bfloat16]
    assert cabi.auto_info(32, 32, 32, 96, 16, 128, bf16)[0] == 1
    assert cabi.auto_info(32, 32, 8, 96, 32, 64, bf16)[0] == 1
    assert cabi.lib().qd_gqa_decode_kernel_kind(32, 8, 96, 16, bf16, 0) == 1
    assert cabi.auto_info(32, 32, 32, 80, 16, 128, bf16)[0] == 0
    assert cabi.lib().qd_gqa_decode_kernel_kind(32, 8, 80, 16, bf16, 0) == 0


def test_auto_plan_uses_the_merge_kernel():
    """The automatic plan merges split sequences with the separate merge
    kernel (kind 1) for every benchmark shape; the fused merge is a
    measurement option only (QD_STAGE_FUSED)."""
    bf16, f16 = cabi.DTYPE[torch.bfloat16], cabi.DTYPE[torch.float16]
    for shape in [(32, 32, 8, 128, 16, 256, bf16), (64, 28, 4, 128, 16, 512, bf16), (256, 40, 8, 128, 32, 32, f16),
                  (4, 8, 2, 64, 16, 32, f16), (8, 64, 8, 128, 16, 8192, bf16)]:
        assert cabi.auto_info(*shape)[0] == 1, shape



def test_plan_rejects_bad_shapes():
    s, c = ctypes.c_int(), ctypes.c_int()
    assert cabi.lib().qd_gqa_decode_plan(1, 8, 0, 64, 16, 4, 1, 256, ctypes.byref(s), ctypes.byref(c)) != 0


def test_workspace_bytes():
    assert cabi.lib().qd_gqa_decode_workspace_bytes(32, 32, 128, 8) == 32 * 32 * 8 * 130 * 4
    assert cabi.lib().qd_gqa_decode_workspace_bytes(32, 32, 128, 1) == 0


def test_kernel_kind_selection():
    kind = cabi.lib().qd_gqa_decode_kernel_kind
    assert kind(32, 8, 128, 16, BF16, 0) == 1
    assert kind(40, 8, 128, 32, F16, 0) == 1
    assert kind(8, 2, 64, 16, F16, 0) == 1
    assert kind(32, 8, 128, 16, BF16, cabi.QD_FLAG_FORCE_GENERIC) == 0
    assert kind(32, 8, 128, 16, F32, 0) == 0       # fp32 caches: VALU kernel
    assert kind(32, 8, 100, 16, BF16, 0) == 0      # head_dim not 64/128/256
    assert kind(32, 8, 128, 8, BF16, 0) == 0       # block_size not a multiple of 16
    assert kind(34, 2, 128, 16, BF16, 0) == 0      # group of 17 > 16


# ----------------------------------------------------------------------------
# Launch argument errors (returned before any HIP call)
# ----------------------------------------------------------------------------

def _launch_args(**over):
    a = dict(q=1, k=1, v=1, table=1, lens=1, out=1, ws=None, ws_bytes=0, B=4, Hq=8, Hkv=2, D=64,
             P=16, maxP=32, N=57, dtype=F16, scale=0.125, splits=1, chunk=0, flags=0, stream=None)
    a.update(over)
    return [a[k] for k in ["q", "k", "v", "table", "lens", "out", "ws", "ws_bytes", "B", "Hq", "Hkv",
                           "D", "P", "maxP", "N", "dtype", "scale", "splits", "chunk", "flags",
                           "stream"]]


@pytest.mark.parametrize("over,msg", [
    (dict(Hkv=3), "Hq must be divisible by Hkv"),
    (dict(D=0), "supported head_dim is [1, 256]"),
    (dict(P=0), "cache must have positive blocks and block_size"),
    (dict(maxP=0), "block_table must have at least one page"),
    (dict(dtype=3), "q/k/v must be float32/float16/bfloat16"),
    (dict(scale=-1.0), "scale must be positive and finite"),
    (dict(splits=0), "splits must be in [1, 65535]"),
    (dict(splits=4, chunk=2), "splits * chunk_pages must cover max_pages"),
    (dict(splits=4), "workspace too small for [B,Hq,splits,D+2] float32"),
    (dict(B=70000), "gqa_decode kernel launch failed: invalid configuration argument"),
    (dict(Hq=70000, Hkv=70000), "gqa_decode kernel launch failed: invalid configuration argument"),
    (dict(q=None), "null tensor pointer"),
])
def test_launch_argument_errors(over, msg):
    rc = cabi.lib().qd_gqa_decode_launch(*_launch_args(**over))
    # Argument errors are hipErrorInvalidValue (1); a grid beyond the launch
    # limits is the launch error itself, hipErrorInvalidConfiguration (9).
    assert rc == (9 if msg.startswith("gqa_decode kernel launch failed") else 1)
    assert cabi.error_string(rc) == msg


def test_launch_batch_zero_is_a_no_op():
    assert cabi.lib().qd_gqa_decode_launch(*_launch_args(B=0, q=None)) == 0


# ----------------------------------------------------------------------------
# Automatic path (qd_gqa_decode_auto*): plan, workspace layout, argument errors
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("name", list(CONFIGS))
def test_auto_plan_for_configs(name):
    cfg = CONFIGS[name]
    max_pages = max(1, -(-max(cfg.lengths()) // cfg.block_size))
    dt = {torch.float16: F16, torch.bfloat16: BF16}[cfg.dtype]
    kind, waves, splits, chunk = cabi.auto_info(cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim,
                                                cfg.block_size, max_pages, dt)
    assert kind in (1, 2)                              # every benchmark config takes the MFMA path
    assert waves > 0 and waves % min(cfg.kv_heads, 8) == 0
    nbytes = cabi.auto_workspace_bytes(cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim,
                                       cfg.block_size, max_pages, dt)
    wgs = waves // min(cfg.kv_heads, 8)
    slots = (wgs + cfg.batch) * cfg.q_heads * (cfg.head_dim + 2) * 4
    assert cabi.auto_counter_bytes() == 256 << 10
    assert nbytes >= cabi.auto_counter_bytes() + slots + 8 * cfg.batch


def test_auto_plan_falls_back_to_splits():
    # fp32 caches at head dims other than 64 and 128, or with pages that do
    # not hold whole 16-token groups, take the split layout with the split plan.
    for d, p in [(100, 16), (256, 16), (128, 8)]:
        kind, waves, splits, chunk = cabi.auto_info(32, 32, 8, d, p, 1024, F32)
        assert (kind, waves) == (0, 0) and (splits, chunk) == cabi.plan(32, 32, 8, d, p, 1024), (d, p)
    assert cabi.auto_info(32, 48, 2, 128, 16, 256, F32)[0] == 0   # more than 16 q-heads per kv-head
    assert cabi.auto_info(4, 8, 3, 64, 16, 4, F16)[0] == -1   # Hq % Hkv != 0


def test_auto_plan_f32_balanced_path():
    # fp32 caches at head_dim 64 and 128 take the balanced kernel on the fp32
    # matrix cores once the batch's static capacity (B * max_pages * P) is
    # 65536 tokens: 8-wave workgroups at 64, 4-wave ones (one wave per SIMD)
    # at 128, so the wave count is a multiple of the workgroup's.
    k64 = cabi.auto_info(32, 32, 8, 64, 16, 256, F32)
    k128 = cabi.auto_info(32, 32, 8, 128, 16, 256, F32)
    assert k64[0] == 1 and k64[1] % 8 == 0 and k64[1] > 0
    assert k128[0] == 1 and k128[1] % 4 == 0 and k128[1] > 0
    assert cabi.auto_info(4, 8, 2, 128, 32, 512, F32)[0] == 1    # 32-token pages
    assert cabi.auto_info(4, 16, 1, 128, 16, 1024, F32)[0] == 1  # 16 q-heads per kv-head
    # One token short of the capacity: the split layout.
    assert cabi.auto_info(4, 16, 1, 128, 16, 1023, F32)[0] == 0
    assert cabi.auto_info(16, 32, 8, 128, 16, 64, F32)[0] == 0


def test_auto_waves_per_workgroup_divide_kv_heads():
    for hkv, per_wg in [(1, 1), (2, 2), (4, 4), (8, 8), (12, 6), (16, 8), (7, 7), (9, 3)]:
        kind, waves, _, _ = cabi.auto_info(4, hkv, hkv, 64, 16, 64, F16)
        assert kind in (1, 2) and waves % per_wg == 0, (hkv, waves)


def _auto_args(**over):
    a = dict(q=1, k=1, v=1, table=1, lens=1, out=1, ws=None, ws_bytes=0, B=4, Hq=8, Hkv=2, D=64,
             P=16, maxP=32, N=57, dtype=F16, scale=0.125, stages=cabi.QD_STAGE_ALL, stream=None)
    a.update(over)
    return [a[k] for k in ["q", "k", "v", "table", "lens", "out", "ws", "ws_bytes", "B", "Hq", "Hkv",
                           "D", "P", "maxP", "N", "dtype", "scale", "stages", "stream"]]


@pytest.mark.parametrize("over,msg", [
    (dict(Hkv=3), "Hq must be divisible by Hkv"),
    (dict(scale=float("inf")), "scale must be positive and finite"),
    (dict(stages=0), "stages must be a non-empty mask of QD_STAGE_*"),
    (dict(stages=4), "stages must be a non-empty mask of QD_STAGE_*"),
    (dict(q=None), "null tensor pointer"),
    (dict(), "workspace smaller than qd_gqa_decode_auto_workspace_bytes()"),
    (dict(dtype=F32, ws=16, ws_bytes=1 << 30, stages=cabi.QD_STAGE_DECODE),
     "stages apply to the balanced MFMA path only"),
])
def test_auto_argument_errors(over, msg):
    rc = cabi.lib().qd_gqa_decode_auto_stages(*_auto_args(**over))
    assert rc == 1
    assert cabi.error_string(rc) == msg


def test_auto_fused_stage_refused_for_f32():
    # An fp32 plan on the balanced path (aligned pointers, capacity >= 65536
    # tokens) refuses QD_STAGE_FUSED before anything is launched.
    args = _auto_args(q=16, k=16, v=16, table=16, lens=16, out=16, ws=16, ws_bytes=1 << 30, B=16, Hq=32,
                      Hkv=8, D=128, P=16, maxP=256, N=4096, dtype=F32, stages=cabi.QD_STAGE_ALL | cabi.QD_STAGE_FUSED)
    assert cabi.auto_info(16, 32, 8, 128, 16, 256, F32)[0] == 1
    rc = cabi.lib().qd_gqa_decode_auto_stages(*args)
    assert rc == 1
    assert cabi.error_string(rc).startswith("QD_STAGE_FUSED needs 16-bit MFMA math")


def test_auto_batch_zero_is_a_no_op():
    assert cabi.lib().qd_gqa_decode_auto_stages(*_auto_args(B=0, q=None)) == 0


# ----------------------------------------------------------------------------
# kv_append boundary (reference csrc/cuda/cache/kv_append.cu:32-45)
# ----------------------------------------------------------------------------

def kv_good():
    return [cabi.desc([4, 2, 64], BF16), cabi.desc([4, 2, 64], BF16), cabi.desc([57, 16, 2, 64], BF16),
            cabi.desc([57, 16, 2, 64], BF16), cabi.desc([4, 32], I32), cabi.desc([4], I32)]


def _kv(mutate):
    d = kv_good()
    mutate(d)
    return cabi.validate_kv_append(*d)


KV_ORDER = [
    (lambda d: None, ""),
    (_set(0, is_device=0), "all tensors must be contiguous CUDA tensors"),
    (_set(3, contiguous=0), "all tensors must be contiguous CUDA tensors"),
    (_set(5, device_index=1), "all tensors must share a device"),
    (_set(0, sizes=[4, 2]), "key/value must be [B, Hkv, D]"),
    (_set(1, sizes=[4, 2, 32]), "key/value must be [B, Hkv, D]"),
    (_set(2, sizes=[57, 16, 2]), "cache must be [Nblocks, P, Hkv, D]"),
    (_set(3, sizes=[57, 16, 2, 32]), "cache must be [Nblocks, P, Hkv, D]"),
    (lambda d: (_set(2, sizes=[57, 16, 4, 64])(d), _set(3, sizes=[57, 16, 4, 64])(d)), "cache head shape mismatch"),
    (lambda d: (_set(2, sizes=[0, 16, 2, 64])(d), _set(3, sizes=[0, 16, 2, 64])(d)), "invalid dimensions"),
    (_set(4, sizes=[3, 32]), "invalid metadata shape"),
    (_set(4, sizes=[4, 0]), "invalid metadata shape"),
    (_set(5, sizes=[4, 1]), "invalid metadata shape"),
    (_set(4, dtype=5), "metadata must be int32"),
    (_set(2, dtype=F16), "dtype mismatch"),
    (lambda d: [setattr(x, "dtype", 5) for x in d[:4]], "unsupported dtype"),
]


@pytest.mark.parametrize("i", range(len(KV_ORDER)))
def test_kv_append_validation_in_reference_order(i):
    mutate, msg = KV_ORDER[i]
    rc, got = _kv(mutate)
    assert (rc == 0) == (msg == "")
    assert got == msg


def test_kv_append_launch_argument_errors():
    L = cabi.lib()
    args = [1, 1, 1, 1, 1, 1, 4, 2, 64, 16, 32, 57, BF16, None]
    assert L.qd_kv_append_launch(*args[:12], 5, None) == 1
    assert cabi.error_string(1) == "unsupported dtype"
    bad = list(args)
    bad[10] = 0
    assert L.qd_kv_append_launch(*bad) == 1 and cabi.error_string(1) == "invalid dimensions"
    zero = list(args)
    zero[6] = 0
    assert L.qd_kv_append_launch(*zero) == 0                     # batch 0: nothing enqueued


# ----------------------------------------------------------------------------
# Torch op surface and Python API
# ----------------------------------------------------------------------------

def test_op_schemas_match_reference():
    ops = torch.ops.qd_attention
    assert str(ops.gqa_decode.default._schema) == (
        "qd_attention::gqa_decode(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_table, "
        "Tensor context_lens, float scale) -> Tensor")
    assert str(ops.gqa_decode_split.default._schema) == (
        "qd_attention::gqa_decode_split(Tensor q, Tensor k_cache, Tensor v_cache, "
        "Tensor block_table, Tensor context_lens, float scale, int splits) -> Tensor")
    assert str(ops.gqa_decode_split_workspace.default._schema) == (
        "qd_attention::gqa_decode_split_workspace(Tensor q, Tensor k, Tensor v, Tensor table, "
        "Tensor lengths, float scale, int splits, Tensor(a!) workspace) -> Tensor")
    assert str(ops.kv_append.default._schema) == (
        "qd_attention::kv_append(Tensor key, Tensor value, Tensor(a!) k_cache, Tensor(b!) v_cache, "
        "Tensor block_table, Tensor positions) -> ()")


def test_cpu_tensors_have_no_kernel():
    q = torch.zeros(1, 8, 64, dtype=torch.float16)
    k = torch.zeros(4, 16, 2, 64, dtype=torch.float16)
    t = torch.zeros(1, 4, dtype=torch.int32)
    with pytest.raises(NotImplementedError):
        torch.ops.qd_attention.gqa_decode(q, k, k, t, torch.ones(1, dtype=torch.int32), 0.125)


def test_public_api_surface():
    assert attention_amd.is_cuda_extension_loaded()
    for name in ["gqa_decode", "gqa_decode_split", "gqa_decode_auto", "kv_append", "is_cuda_extension_loaded"]:
        assert name in attention_amd.__all__


def test_missing_extension_raises_runtime_error(monkeypatch):
    monkeypatch.setattr(core, "_LOAD_ERROR", OSError("libqd_attention_torch.so: missing"))
    q = torch.zeros(1, 8, 64)
    # The reference's texts (core.py:31-35, :51, :62): the first sentence is
    # the same, gqa_decode adds a build hint.
    with pytest.raises(RuntimeError, match=r"^qd_attention CUDA extension was not loaded\. Build it in-tree"):
        attention_amd.gqa_decode(q, q, q, q, q)
    with pytest.raises(RuntimeError, match=r"^qd_attention CUDA extension was not loaded$"):
        attention_amd.gqa_decode_split(q, q, q, q, q)
    with pytest.raises(RuntimeError, match=r"^qd_attention CUDA extension was not loaded$"):
        attention_amd.kv_append(q, q, q, q, q, q)
    assert not attention_amd.is_cuda_extension_loaded()


def test_backend_and_dimension_errors():
    q = torch.zeros(1, 8, 64)
    with pytest.raises(ValueError, match="triton"):
        attention_amd.gqa_decode_split(q, q, q, q, q, backend="triton")
    with pytest.raises(ValueError, match="backend must be cuda or triton"):
        attention_amd.gqa_decode_split(q, q, q, q, q, backend="cpu")
    with pytest.raises(ValueError, match="invalid decode input dimensions"):
        attention_amd.gqa_decode_auto(q, q, q, q, q)


def test_validate_paged_metadata_argument_errors():
    from attention_amd.validation import validate_paged_metadata as vpm
    t = torch.zeros(2, 3, dtype=torch.int32)
    l = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="block_size and num_blocks must be positive"):
        vpm(t, l, block_size=0, num_blocks=4)
    with pytest.raises(ValueError, match=r"metadata shapes must be \[B,MaxPages\] and \[B\]"):
        vpm(t, l[:1], block_size=16, num_blocks=4)
    with pytest.raises(ValueError, match="metadata must be int32"):
        vpm(t.long(), l, block_size=16, num_blocks=4)
    with pytest.raises(ValueError, match=r"positions must be int32 \[B\]"):
        vpm(t, l, block_size=16, num_blocks=4, positions=l.long())
