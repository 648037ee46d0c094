"""ctypes binding of the C ABI in include/qd_attention.h.

For Python callers that want the C entry points without the torch op layer
(explicit split/chunk plans, kernel choice, caller-owned output and
workspace), and the same stub a ctypes user of the reference would add.
``launch`` takes torch device tensors and enqueues on the current stream.
"""
from __future__ import annotations

import ctypes
import os
import re

import torch  # noqa: F401  (loads torch's HIP runtime before the library)

PKG = os.path.dirname(os.path.abspath(__file__))
HEADER = os.path.join(os.path.dirname(PKG), "include", "qd_attention.h")
LIB_PATH = os.path.join(PKG, "lib", "libqd_attention.so")

DTYPE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.int32: 3, torch.int64: 4}
QD_FLAG_FORCE_GENERIC = 1
QD_FLAG_MLA_STAGED = 2
QD_FLAG_MLA_WAVE = 4
QD_STAGE_DECODE, QD_STAGE_MERGE, QD_STAGE_ALL = 1, 2, 3
QD_STAGE_VALU = 4   # measurement option: VALU math in the balanced decode kernel
QD_STAGE_UNFUSED, QD_STAGE_FUSED = 8, 16   # measurement options: where split sequences are merged


class TensorDesc(ctypes.Structure):
    _fields_ = [("defined", ctypes.c_int32), ("is_device", ctypes.c_int32),
                ("device_index", ctypes.c_int32), ("contiguous", ctypes.c_int32),
                ("dtype", ctypes.c_int32), ("ndim", ctypes.c_int32),
                ("sizes", ctypes.c_int64 * 8)]


def desc(sizes, dtype=0, is_device=1, device=0, contiguous=1, defined=1) -> TensorDesc:
    d = TensorDesc()
    d.defined, d.is_device, d.device_index, d.contiguous, d.dtype = (
        defined, is_device, device, contiguous, dtype)
    d.ndim = len(sizes)
    for i, s in enumerate(list(sizes)[:8]):
        d.sizes[i] = s
    return d


def header_functions() -> list[str]:
    text = open(HEADER).read()
    return re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\*?\s+(qd_[a-z_0-9]+)\(", text, re.M)


_lib = None


def lib():
    global _lib
    if _lib is None:
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER(TensorDesc)
        L.qd_abi_version.restype = ctypes.c_int
        L.qd_error_string.restype = ctypes.c_char_p
        L.qd_error_string.argtypes = [ctypes.c_int]
        L.qd_gqa_decode_validate.restype = ctypes.c_int
        L.qd_gqa_decode_validate.argtypes = [P, P, P, P, P, ctypes.c_double, ctypes.c_int64,
                                             ctypes.c_char_p, ctypes.c_size_t]
        L.qd_gqa_decode_validate_workspace.restype = ctypes.c_int
        L.qd_gqa_decode_validate_workspace.argtypes = [P, P, ctypes.c_int64, ctypes.c_char_p,
                                                       ctypes.c_size_t]
        L.qd_gqa_decode_plan.restype = ctypes.c_int
        L.qd_gqa_decode_plan.argtypes = [ctypes.c_int] * 8 + [ctypes.POINTER(ctypes.c_int)] * 2
        L.qd_gqa_decode_workspace_bytes.restype = ctypes.c_size_t
        L.qd_gqa_decode_workspace_bytes.argtypes = [ctypes.c_int] * 4
        L.qd_gqa_decode_kernel_kind.restype = ctypes.c_int
        L.qd_gqa_decode_kernel_kind.argtypes = [ctypes.c_int] * 6
        L.qd_gqa_decode_launch.restype = ctypes.c_int
        L.qd_gqa_decode_launch.argtypes = (
            [ctypes.c_void_p] * 7 + [ctypes.c_size_t] + [ctypes.c_int] * 6 + [ctypes.c_int64]
            + [ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int,
               ctypes.c_void_p])
        L.qd_gqa_decode_auto_workspace_bytes.restype = ctypes.c_size_t
        L.qd_gqa_decode_auto_workspace_bytes.argtypes = [ctypes.c_int] * 7
        L.qd_gqa_decode_auto.restype = ctypes.c_int
        L.qd_gqa_decode_auto.argtypes = (
            [ctypes.c_void_p] * 7 + [ctypes.c_size_t] + [ctypes.c_int] * 6 + [ctypes.c_int64]
            + [ctypes.c_int, ctypes.c_float, ctypes.c_void_p])
        L.qd_gqa_decode_noalloc_scratch_bytes.restype = ctypes.c_size_t
        L.qd_gqa_decode_noalloc_scratch_bytes.argtypes = []
        L.qd_gqa_decode_auto_noalloc.restype = ctypes.c_int
        L.qd_gqa_decode_auto_noalloc.argtypes = (
            [ctypes.c_void_p] * 6 + [ctypes.c_int] * 6 + [ctypes.c_int64] + [ctypes.c_int, ctypes.c_float, ctypes.c_void_p])
        L.qd_gqa_decode_auto_stages.restype = ctypes.c_int
        L.qd_gqa_decode_auto_stages.argtypes = (
            [ctypes.c_void_p] * 7 + [ctypes.c_size_t] + [ctypes.c_int] * 6 + [ctypes.c_int64]
            + [ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_void_p])
        L.qd_kv_append_validate.restype = ctypes.c_int
        L.qd_kv_append_validate.argtypes = [P] * 6 + [ctypes.c_char_p, ctypes.c_size_t]
        L.qd_kv_append_launch.restype = ctypes.c_int
        L.qd_kv_append_launch.argtypes = ([ctypes.c_void_p] * 6 + [ctypes.c_int] * 5 + [ctypes.c_int64]
                                          + [ctypes.c_int, ctypes.c_void_p])
        L.qd_validate_paged_metadata.restype = ctypes.c_int
        L.qd_validate_paged_metadata.argtypes = ([ctypes.c_void_p] * 3 + [ctypes.c_int] * 3
                                                 + [ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p])
        L.qd_gqa_decode_auto_info.restype = ctypes.c_int
        L.qd_gqa_decode_auto_counter_bytes.restype = ctypes.c_size_t
        L.qd_gqa_decode_auto_counter_bytes.argtypes = []
        L.qd_gqa_decode_auto_info.argtypes = [ctypes.c_int] * 7 + [ctypes.POINTER(ctypes.c_int)] * 3
        V, I, I64, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
        MSG = [ctypes.c_char_p, ctypes.c_size_t]
        L.qd_latent_kv_write_validate.restype = I
        L.qd_latent_kv_write_validate.argtypes = [P] * 4 + MSG
        L.qd_latent_kv_write.restype = I
        L.qd_latent_kv_write.argtypes = [V] * 4 + [I64, I, I, I64, I, V]
        L.qd_mla_project_validate.restype = I
        L.qd_mla_project_validate.argtypes = [P, P, I] + MSG
        L.qd_mla_project.restype = I
        L.qd_mla_project.argtypes = [V] * 3 + [I64] + [I] * 6 + [V]
        L.qd_mla_attend_validate.restype = I
        L.qd_mla_attend_validate.argtypes = [P] * 7 + [ctypes.c_double] + MSG
        L.qd_mla_attend_workspace_bytes.restype = ctypes.c_size_t
        L.qd_mla_attend_workspace_bytes.argtypes = [I] * 11
        L.qd_mla_attend_info.restype = I
        L.qd_mla_attend_info.argtypes = [I] * 11 + [ctypes.POINTER(I)] * 2
        L.qd_mla_attend.restype = I
        L.qd_mla_attend.argtypes = ([V] * 9 + [ctypes.c_size_t] + [I] * 7 + [I64] + [I] * 3 + [F]
                                    + [I, I, V])
        L.qd_mla_decode_validate.restype = I
        L.qd_mla_decode_validate.argtypes = [P] * 9 + [ctypes.c_double] + MSG
        L.qd_mla_decode_workspace_bytes.restype = ctypes.c_size_t
        L.qd_mla_decode_workspace_bytes.argtypes = [I] * 11
        L.qd_mla_decode.restype = I
        L.qd_mla_decode.argtypes = ([V] * 11 + [ctypes.c_size_t] + [I] * 9 + [I64] + [I] * 3 + [F]
                                    + [I, I, V])
        _lib = L
    return _lib


def validate(q, k, v, table, lens, scale=0.125, splits=1):
    buf = ctypes.create_string_buffer(256)
    rc = lib().qd_gqa_decode_validate(ctypes.byref(q), ctypes.byref(k), ctypes.byref(v),
                                      ctypes.byref(table), ctypes.byref(lens), scale, splits,
                                      buf, 256)
    return rc, buf.value.decode()


def validate_workspace(q, ws, splits):
    buf = ctypes.create_string_buffer(256)
    rc = lib().qd_gqa_decode_validate_workspace(ctypes.byref(q), ctypes.byref(ws), splits, buf, 256)
    return rc, buf.value.decode()


def plan(batch, q_heads, kv_heads, head_dim, block_size, max_pages, dtype=2, cu_count=256):
    s, c = ctypes.c_int(), ctypes.c_int()
    rc = lib().qd_gqa_decode_plan(batch, q_heads, kv_heads, head_dim, block_size, max_pages, dtype,
                                  cu_count, ctypes.byref(s), ctypes.byref(c))
    assert rc == 0, lib().qd_error_string(rc)
    return s.value, c.value


def launch(q, k, v, table, lens, out, *, scale, splits=1, chunk_pages=0, workspace=None,
           flags=0, stream=None):
    """Calls qd_gqa_decode_launch on torch device tensors (no validation)."""
    B, Hq, D = q.shape
    _, P, Hkv, _ = k.shape
    if stream is None:
        stream = torch.cuda.current_stream(q.device).cuda_stream if q.is_cuda else 0
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * 4 if workspace is not None else 0
    rc = lib().qd_gqa_decode_launch(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr(), lens.data_ptr(),
        out.data_ptr(), ws_ptr, ws_bytes, B, Hq, Hkv, D, P, table.shape[1], k.shape[0],
        DTYPE[q.dtype], float(scale), splits, chunk_pages, flags, stream)
    return rc


def error_string(rc: int) -> str:
    return lib().qd_error_string(rc).decode()


def auto_workspace_bytes(batch, q_heads, kv_heads, head_dim, block_size, max_pages, dtype=2):
    return lib().qd_gqa_decode_auto_workspace_bytes(batch, q_heads, kv_heads, head_dim, block_size,
                                                    max_pages, dtype)


def auto_counter_bytes() -> int:
    """Bytes of arrival counters at the start of every automatic-path workspace."""
    return lib().qd_gqa_decode_auto_counter_bytes()


def auto_workspace(batch, q_heads, kv_heads, head_dim, block_size, max_pages, dtype, device, fill=0):
    """A workspace for auto_launch: auto_workspace_bytes() bytes whose arrival
    counters (the first auto_counter_bytes()) are zero, as they must be before
    first use, and whose other bytes all hold `fill`."""
    n = max(16, auto_workspace_bytes(batch, q_heads, kv_heads, head_dim, block_size, max_pages, dtype))
    ws = torch.full((n,), fill, dtype=torch.uint8, device=device)
    ws[:min(n, auto_counter_bytes())].zero_()
    return ws


def auto_info(batch, q_heads, kv_heads, head_dim, block_size, max_pages, dtype=2):
    """(kind, waves, splits, chunk_pages); kind 2 = balanced MFMA path with the
    fused merge, 1 = balanced MFMA path with the merge kernel, 0 = split path."""
    w, s, c = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    kind = lib().qd_gqa_decode_auto_info(batch, q_heads, kv_heads, head_dim, block_size, max_pages,
                                         dtype, ctypes.byref(w), ctypes.byref(s), ctypes.byref(c))
    return kind, w.value, s.value, c.value


def auto_launch(q, k, v, table, lens, out, *, scale, workspace=None, stream=None, stages=QD_STAGE_ALL):
    """Calls qd_gqa_decode_auto on torch device tensors (no validation).

    ``workspace`` (any dtype, contiguous) must hold auto_workspace_bytes();
    its first auto_counter_bytes() must be zero before first use (every call
    leaves them zero: see auto_workspace), the rest needs no initialization."""
    B, Hq, D = q.shape
    _, P, Hkv, _ = k.shape
    if stream is None:
        stream = torch.cuda.current_stream(q.device).cuda_stream if q.is_cuda else 0
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    return lib().qd_gqa_decode_auto_stages(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr(), lens.data_ptr(), out.data_ptr(),
        ws_ptr, ws_bytes, B, Hq, Hkv, D, P, table.shape[1], k.shape[0], DTYPE[q.dtype], float(scale),
        stages, stream)


def auto_noalloc_launch(q, k, v, table, lens, out, *, scale, stream=None):
    """Calls qd_gqa_decode_auto_noalloc (the library's own scratch, no
    workspace argument) on torch device tensors (no validation)."""
    B, Hq, D = q.shape
    _, P, Hkv, _ = k.shape
    if stream is None:
        stream = torch.cuda.current_stream(q.device).cuda_stream if q.is_cuda else 0
    return lib().qd_gqa_decode_auto_noalloc(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr(), lens.data_ptr(), out.data_ptr(),
        B, Hq, Hkv, D, P, table.shape[1], k.shape[0], DTYPE[q.dtype], float(scale), stream)


def validate_kv_append(key, value, kc, vc, table, pos):
    buf = ctypes.create_string_buffer(256)
    rc = lib().qd_kv_append_validate(*(ctypes.byref(d) for d in (key, value, kc, vc, table, pos)), buf, 256)
    return rc, buf.value.decode()


def kv_append_launch(key, value, kc, vc, table, pos, stream=None):
    """Calls qd_kv_append_launch on torch device tensors (no validation)."""
    B, Hkv, D = key.shape
    if stream is None:
        stream = torch.cuda.current_stream(key.device).cuda_stream if key.is_cuda else 0
    return lib().qd_kv_append_launch(key.data_ptr(), value.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                     table.data_ptr(), pos.data_ptr(), B, Hkv, D, kc.shape[1],
                                     table.shape[1], kc.shape[0], DTYPE[key.dtype], stream)


# ---- Paged MLA decode ------------------------------------------------------


def _stream(t, stream):
    if stream is None:
        return torch.cuda.current_stream(t.device).cuda_stream if t.is_cuda else 0
    return stream


def _msg_call(fn, *args):
    buf = ctypes.create_string_buffer(256)
    rc = fn(*args, buf, 256)
    return rc, buf.value.decode()


def _ref(d):
    return None if d is None else ctypes.byref(d)


def validate_latent_kv_write(latent, rope, cache, slots):
    return _msg_call(lib().qd_latent_kv_write_validate, *(ctypes.byref(d) for d in (latent, rope, cache, slots)))


def validate_mla_project(x, w, absorb):
    return _msg_call(lib().qd_mla_project_validate, ctypes.byref(x), ctypes.byref(w), int(absorb))


def validate_mla_attend(q, qr, cache, table, lens, pos, indices=None, scale=0.1):
    return _msg_call(lib().qd_mla_attend_validate, *(ctypes.byref(d) for d in (q, qr, cache, table, lens, pos)),
                     _ref(indices), scale)


def validate_mla_decode(q, qr, cache, table, lens, pos, wk, wv, indices=None, scale=0.1):
    return _msg_call(lib().qd_mla_decode_validate,
                     *(ctypes.byref(d) for d in (q, qr, cache, table, lens, pos, wk, wv)), _ref(indices), scale)


def mla_attend_info(B, T, H, Dc, Dr, P, maxP, nk=-1, dtype=2, splits=0, flags=0):
    """(kind, splits, head_groups); kind 1 = MFMA kernel, 0 = VALU kernel."""
    s, g = ctypes.c_int(), ctypes.c_int()
    kind = lib().qd_mla_attend_info(B, T, H, Dc, Dr, P, maxP, nk, dtype, splits, flags, ctypes.byref(s),
                                    ctypes.byref(g))
    return kind, s.value, g.value


def latent_kv_write(latent, rope, cache, slots, stream=None):
    return lib().qd_latent_kv_write(latent.data_ptr(), rope.data_ptr(), cache.data_ptr(), slots.data_ptr(),
                                    latent.shape[0], latent.shape[1], rope.shape[1],
                                    cache.shape[0] * cache.shape[1], DTYPE[latent.dtype], _stream(latent, stream))


def mla_project(x, w, out, absorb, flags=0, stream=None):
    B, T, H, di = x.shape
    dout = out.shape[-1]
    return lib().qd_mla_project(x.data_ptr(), w.data_ptr(), out.data_ptr(), B * T, H, di, dout, int(absorb),
                                DTYPE[x.dtype], flags, _stream(x, stream))


def mla_attend(q, qr, cache, table, lens, pos, out, *, scale, indices=None, causal=True, splits=0, flags=0,
               workspace=None, stream=None):
    """Calls qd_mla_attend on torch device tensors (no validation); allocates
    the split workspace when none is given."""
    B, T, H, Dc = q.shape
    Dr = qr.shape[-1]
    nk = -1 if indices is None else indices.shape[-1]
    need = lib().qd_mla_attend_workspace_bytes(B, T, H, Dc, Dr, cache.shape[1], table.shape[1], nk,
                                               DTYPE[q.dtype], splits, flags)
    if workspace is None and need:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    return lib().qd_mla_attend(q.data_ptr(), qr.data_ptr(), cache.data_ptr(), table.data_ptr(), lens.data_ptr(),
                               pos.data_ptr(), None if indices is None else indices.data_ptr(), out.data_ptr(),
                               ws_ptr, ws_bytes, B, T, H, Dc, Dr, cache.shape[1], table.shape[1], cache.shape[0],
                               nk, int(causal), DTYPE[q.dtype], float(scale), splits, flags, _stream(q, stream))


def mla_decode(q, qr, cache, table, lens, pos, wk, wv, out, *, scale, indices=None, causal=True, splits=0,
               flags=0, stream=None):
    """Calls qd_mla_decode on torch device tensors (no validation)."""
    B, T, H, Dn = q.shape
    Dr = qr.shape[-1]
    Dc = wk.shape[-1]
    Dv = wv.shape[1]
    nk = -1 if indices is None else indices.shape[-1]
    need = lib().qd_mla_decode_workspace_bytes(B, T, H, Dc, Dr, cache.shape[1], table.shape[1], nk,
                                               DTYPE[q.dtype], splits, flags)
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=q.device)
    return lib().qd_mla_decode(q.data_ptr(), qr.data_ptr(), cache.data_ptr(), table.data_ptr(), lens.data_ptr(),
                               pos.data_ptr(), wk.data_ptr(), wv.data_ptr(),
                               None if indices is None else indices.data_ptr(), out.data_ptr(), ws.data_ptr(),
                               ws.numel(), B, T, H, Dn, Dc, Dr, Dv, cache.shape[1], table.shape[1], cache.shape[0],
                               nk, int(causal), DTYPE[q.dtype], float(scale), splits, flags, _stream(q, stream))
