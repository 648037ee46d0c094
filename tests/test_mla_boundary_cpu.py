"""CPU checks of the MLA boundary: the C ABI validators reproduce the
reference's checks in order with its messages (csrc/cuda/mla/mla.cu:139-142,
:152-155, :162-171, :185-191), the op schemas match the reference's
(csrc/binding/torch_ops.cpp:47-50), and the Python surface mirrors
attention/mla.py.  No kernel runs here."""
from __future__ import annotations

import pytest
import torch

import attention_amd
from attention_amd import cabi
from attention_amd.cabi import desc

BF16, F16, F32, I32, I64 = 2, 1, 0, 3, 4


def attend_descs(B=2, T=1, H=4, Dc=32, Dr=8, N=6, P=16, maxP=4, dt=BF16):
    return dict(q=desc([B, T, H, Dc], dt), qr=desc([B, T, H, Dr], dt), cache=desc([N, P, Dc + Dr], dt),
                table=desc([B, maxP], I32), lens=desc([B], I32), pos=desc([B, T], I32))


def run_attend(d, indices=None, scale=0.1):
    return cabi.validate_mla_attend(d["q"], d["qr"], d["cache"], d["table"], d["lens"], d["pos"], indices, scale)


ATTEND_FAILURES = [
    # (edit, message) in the reference's order
    (lambda d: d.update(q=desc([2, 1, 4, 32], BF16, contiguous=0)), "q must be contiguous and on the same CUDA device"),
    (lambda d: d.update(qr=desc([2, 1, 4, 8], BF16, device=1)), "q_rope must be contiguous and on the same CUDA device"),
    (lambda d: d.update(cache=desc([6, 16, 40], BF16, is_device=0)),
     "cache must be contiguous and on the same CUDA device"),
    (lambda d: d.update(table=desc([2, 4], I32, contiguous=0)), "table must be contiguous and on the same CUDA device"),
    (lambda d: d.update(lens=desc([2], I32, device=3)), "lengths must be contiguous and on the same CUDA device"),
    (lambda d: d.update(pos=desc([2, 1], I32, contiguous=0)), "positions must be contiguous and on the same CUDA device"),
    (lambda d: [d[k].__setattr__("dtype", 5) for k in ("q", "qr", "cache")], "dtype must be float32/float16/bfloat16"),
    (lambda d: d.update(pos=desc([2], I32)), "invalid tensor ranks"),
    (lambda d: d.update(qr=desc([2, 1, 3, 8], BF16)), "shape mismatch"),
    (lambda d: d.update(pos=desc([2, 2], I32)), "shape mismatch"),
    (lambda d: d.update(q=desc([2, 1, 4, 520], BF16), cache=desc([6, 16, 528], BF16)), "invalid dimensions"),
    (lambda d: d.update(cache=desc([6, 16, 41], BF16)), "invalid dimensions"),
    (lambda d: d.update(table=desc([2, 0], I32)), "invalid dimensions"),
    (lambda d: d.update(q=desc([70000, 1, 4, 32], BF16), qr=desc([70000, 1, 4, 8], BF16),
                        table=desc([70000, 4], I32), lens=desc([70000], I32), pos=desc([70000, 1], I32)),
     "CUDA grid limit"),
    (lambda d: d.update(cache=desc([6, 16, 40], F16)), "dtype mismatch"),
    (lambda d: d.update(lens=desc([2], I64)), "metadata must be int32"),
]


@pytest.mark.parametrize("i", range(len(ATTEND_FAILURES)))
def test_mla_attend_validation_order_and_messages(i):
    d = attend_descs()
    edit, message = ATTEND_FAILURES[i]
    edit(d)
    rc, msg = run_attend(d)
    assert rc == 1 and msg == message


def test_mla_attend_validation_scale_and_indices():
    d = attend_descs()
    assert run_attend(d) == (0, "")
    assert run_attend(d, scale=0.0)[1] == "scale must be positive and finite"
    assert run_attend(d, scale=float("inf"))[1] == "scale must be positive and finite"
    assert run_attend(d, indices=desc([2, 1, 8], I32, contiguous=0))[1] == \
        "indices must be contiguous and on the same CUDA device"
    assert run_attend(d, indices=desc([2, 2, 8], I32))[1] == "indices must be int32 [B,T,K]"
    assert run_attend(d, indices=desc([2, 1, 8], I64))[1] == "indices must be int32 [B,T,K]"
    assert run_attend(d, indices=desc([2, 1, 0], I32)) == (0, "")
    assert run_attend(d, indices=desc([2, 1, 8], I32, defined=0)) == (0, "")
    # scale is checked before indices, dimensions before dtype (reference order)
    assert run_attend(d, indices=desc([2, 2, 8], I32), scale=-1.0)[1] == "scale must be positive and finite"


def decode_descs(B=2, T=1, H=4, Dn=16, Dc=32, Dr=8, Dv=16, dt=BF16):
    return dict(q=desc([B, T, H, Dn], dt), qr=desc([B, T, H, Dr], dt), cache=desc([6, 16, Dc + Dr], dt),
                table=desc([B, 4], I32), lens=desc([B], I32), pos=desc([B, T], I32),
                wk=desc([H, Dn, Dc], dt), wv=desc([H, Dv, Dc], dt))


def run_decode(d, indices=None, scale=0.1):
    return cabi.validate_mla_decode(*(d[k] for k in ("q", "qr", "cache", "table", "lens", "pos", "wk", "wv")),
                                    indices, scale)


DECODE_FAILURES = [
    (lambda d: d.update(wv=desc([4, 16, 32], BF16, contiguous=0)), "input must be contiguous and on the same CUDA device"),
    (lambda d: d.update(q=desc([2, 1, 4, 16], I32)), "dtype must be float32/float16/bfloat16"),
    (lambda d: d.update(wk=desc([4, 16], BF16)), "invalid tensor ranks"),
    (lambda d: d.update(lens=desc([3], I32)), "shape mismatch"),
    (lambda d: d.update(wk=desc([4, 16, 600], BF16), wv=desc([4, 16, 600], BF16), cache=desc([6, 16, 608], BF16)),
     "invalid dimensions"),
    (lambda d: d.update(wk=desc([4, 8, 32], BF16)), "invalid dimensions"),
    (lambda d: d.update(wv=desc([4, 16, 16], BF16)), "invalid dimensions"),
    (lambda d: d.update(wv=desc([4, 16, 32], F16)), "dtype mismatch"),
    (lambda d: d.update(pos=desc([2, 1], I64)), "invalid metadata or scale"),
]


@pytest.mark.parametrize("i", range(len(DECODE_FAILURES)))
def test_mla_decode_validation_order_and_messages(i):
    d = decode_descs()
    edit, message = DECODE_FAILURES[i]
    edit(d)
    rc, msg = run_decode(d)
    assert rc == 1 and msg == message


def test_mla_decode_validation_scale_and_indices():
    d = decode_descs()
    assert run_decode(d) == (0, "")
    assert run_decode(d, scale=float("nan"))[1] == "invalid metadata or scale"
    assert run_decode(d, indices=desc([2, 1, 4], I64))[1] == "invalid indices"
    assert run_decode(d, indices=desc([2, 1, 4], I32, device=2))[1] == \
        "indices must be contiguous and on the same CUDA device"


def test_mla_project_validation():
    x = desc([2, 1, 4, 16], BF16)
    assert cabi.validate_mla_project(x, desc([4, 16, 32], BF16), True) == (0, "")
    assert cabi.validate_mla_project(x, desc([4, 32, 16], BF16), False) == (0, "")
    assert cabi.validate_mla_project(desc([2, 1, 4, 16], BF16, contiguous=0), desc([4, 16, 32], BF16), True)[1] == \
        "x must be contiguous and on the same CUDA device"
    assert cabi.validate_mla_project(x, desc([4, 16, 32], BF16, device=1), True)[1] == \
        "w must be contiguous and on the same CUDA device"
    assert cabi.validate_mla_project(desc([2, 1, 4, 16], I32), desc([4, 16, 32], I32), True)[1] == \
        "dtype must be float32/float16/bfloat16"
    assert cabi.validate_mla_project(x, desc([4, 16, 32], F16), True)[1] == "dtype mismatch"
    assert cabi.validate_mla_project(x, desc([5, 16, 32], BF16), True)[1] == \
        "x [B,T,H,D], weight [H,Dn,Dc] or [H,Dv,Dc]"
    assert cabi.validate_mla_project(x, desc([4, 8, 32], BF16), True)[1] == "projection dimension mismatch"
    assert cabi.validate_mla_project(x, desc([4, 16, 32], BF16), False)[1] == "projection dimension mismatch"


def test_latent_kv_write_validation():
    lat, rope, cache, slots = desc([5, 32], BF16), desc([5, 8], BF16), desc([3, 16, 40], BF16), desc([5], I64)
    assert cabi.validate_latent_kv_write(lat, rope, cache, slots) == (0, "")
    assert cabi.validate_latent_kv_write(lat, rope, cache, desc([5], I64, contiguous=0))[1] == \
        "slots must be contiguous and on the same CUDA device"
    assert cabi.validate_latent_kv_write(desc([5, 32], I32), rope, cache, slots)[1] == \
        "dtype must be float32/float16/bfloat16"
    assert cabi.validate_latent_kv_write(lat, desc([4, 8], BF16), cache, slots)[1] == \
        "invalid latent/rope/cache/slots shape"
    assert cabi.validate_latent_kv_write(lat, rope, desc([3, 16, 41], BF16), slots)[1] == "invalid cache width"
    assert cabi.validate_latent_kv_write(lat, rope, cache, desc([5], I32))[1] == \
        "slots must be int64 and tensors must share dtype"
    assert cabi.validate_latent_kv_write(lat, desc([5, 8], F16), cache, slots)[1] == \
        "slots must be int64 and tensors must share dtype"


REFERENCE_SCHEMAS = {
    "mla_decode_fused": "qd_attention::mla_decode_fused(Tensor q, Tensor qr, Tensor cache, Tensor table, "
                        "Tensor lens, Tensor positions, Tensor wk, Tensor wv, Tensor? indices, float scale, "
                        "bool causal) -> Tensor",
    "mla_project": "qd_attention::mla_project(Tensor x, Tensor weight, bool absorb) -> Tensor",
    "latent_kv_write": "qd_attention::latent_kv_write(Tensor latent, Tensor rope, Tensor(a!) cache, "
                       "Tensor slots) -> ()",
    "mla_attend": "qd_attention::mla_attend(Tensor q, Tensor q_rope, Tensor cache, Tensor table, Tensor lens, "
                  "Tensor positions, Tensor? indices, float scale, bool causal) -> Tensor",
}


@pytest.mark.parametrize("name", sorted(REFERENCE_SCHEMAS))
def test_mla_op_schemas_match_reference(name):
    assert attention_amd.is_cuda_extension_loaded()
    op = getattr(torch.ops.qd_attention, name).default
    assert str(op._schema) == REFERENCE_SCHEMAS[name]


def test_python_surface_mirrors_reference():
    for name in ("latent_kv_write", "mla_query_absorb", "mla_value_project", "mla_latent_attention",
                 "mla_decode", "mla_prefill", "sparse_mla"):
        assert callable(getattr(attention_amd, name)) and name in attention_amd.__all__
    with pytest.raises(NotImplementedError):
        attention_amd.mla_prefill()


def test_attend_plan_queries():
    # VALU kernel for fp32 and for latent widths that are not a multiple of 8.
    assert cabi.mla_attend_info(1, 4, 4, 32, 8, 16, 4, dtype=F32)[0] == 0
    assert cabi.mla_attend_info(1, 1, 4, 36, 8, 16, 4)[0] == 0
    assert cabi.mla_attend_info(1, 1, 4, 32, 8, 16, 4, splits=5)[1] == 5
    assert cabi.mla_attend_info(0, 1, 4, 32, 8, 16, 4, nk=-2)[0] == -1
    ws = cabi.lib().qd_mla_attend_workspace_bytes
    # VALU kernel (fp32): [R, H, splits, Dc+2] fp32, none for one split.
    assert ws(2, 1, 4, 32, 8, 16, 4, -1, F32, 3, 0) == 2 * 4 * 3 * 34 * 4
    assert ws(2, 1, 4, 32, 8, 16, 4, -1, F32, 1, 0) == 0
    # MFMA kernel: (workgroups + rows) partial slots, then G and the row spans.
    assert cabi.mla_attend_info(2, 1, 4, 32, 8, 16, 4, splits=3)[0] == 1
    r256 = lambda x: (x + 255) // 256 * 256
    assert ws(2, 1, 4, 32, 8, 16, 4, -1, BF16, 3, 0) == r256((3 + 2) * 4 * 34 * 4) + r256(8 + 2 * 2 * 4)
    total = cabi.lib().qd_mla_decode_workspace_bytes(2, 1, 4, 32, 8, 16, 4, -1, BF16, 3, 0)
    assert total == 512 + 512 + ws(2, 1, 4, 32, 8, 16, 4, -1, BF16, 3, 0)   # qa, latent ([2,1,4,32] bf16), then those
