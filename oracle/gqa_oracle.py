"""CPU oracle for paged GQA decode (test infrastructure only; see oracle/__init__.py).

Arrays are numpy.  Values of 16-bit inputs are passed as float32 arrays that
hold exactly-representable values; ``out_dtype`` ("f32", "f16", "bf16")
selects the final rounding, done once, round-to-nearest-even, as the
reference's ``.to(q.dtype)`` (reference ``attention/reference/gqa.py:43``)
and the kernel's ``static_cast<scalar_t>`` (``gqa_decode.cu:65``).
"""
from __future__ import annotations

import ctypes
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
C_LIB = os.path.join(HERE, "_build", "libgqa_oracle.so")
DTYPE_CODES = {"f32": 0, "f16": 1, "bf16": 2}

# ----------------------------------------------------------------------------
# Rounding helpers
# ----------------------------------------------------------------------------


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 (ties to even) -> float32.  NaN stays NaN."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).copy()
    nan = np.isnan(x)
    out[nan] = np.nan
    return out


def f16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest float16 (numpy's IEEE conversion, ties to even) -> float32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "f32":
        return np.asarray(x, dtype=np.float32)
    if dtype == "f16":
        return f16_round(x)
    if dtype == "bf16":
        return bf16_round(x)
    raise ValueError(dtype)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    return bf16_round(x).view(np.uint32) >> 16


def from_bf16_bits(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


# ----------------------------------------------------------------------------
# Oracle: numpy restatement of reference attention/reference/gqa.py:21-44
# ----------------------------------------------------------------------------


def default_scale(head_dim: int) -> float:
    """reference attention/core.py:36-37 and gqa.py:26-27."""
    return 1.0 / math.sqrt(head_dim)


def oracle_decode(q, k, v, table, lens, scale=None, out_dtype="f32", return_f32=False,
                  batches=None):
    """Paged GQA decode in fp32, one sequence at a time.

    Steps follow gqa.py: per sequence (``:29``) read the length (``:30``);
    a non-positive length gives a zero row (``:31-33``; negative lengths as
    the kernel, gqa_decode.cu:40-42/65); gather the first ceil(len/P) pages
    (``:34-35``), flatten to tokens and keep ``len`` of them (``:36-37``);
    q-head h reads kv-head h // (Hq/Hkv) (``:38-39`` repeat_interleave);
    fp32 scores times scale (``:40``), softmax (``:41``), weighted sum of V
    (``:42``), one cast (``:43``).  The head repeat is expressed as a grouped
    matmul instead of materializing the repeated K/V.

    ``batches`` restricts the computation to a subset of sequences (other
    rows are returned as zeros).
    """
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    table = np.asarray(table)
    lens = np.asarray(lens)
    bsz, hq, d = q.shape
    nblocks, block_size, hkv, cache_d = k.shape
    assert cache_d == d
    assert v.shape == k.shape
    assert hq % hkv == 0
    if scale is None:
        scale = default_scale(d)
    g = hq // hkv
    out = np.zeros((bsz, hq, d), dtype=np.float32)
    for b in (range(bsz) if batches is None else batches):
        length = int(lens[b])
        if length <= 0:
            continue
        n_pages = (length + block_size - 1) // block_size
        pages = table[b, :n_pages].astype(np.int64)
        keys = k[pages].reshape(-1, hkv, d)[:length]
        values = v[pages].reshape(-1, hkv, d)[:length]
        kh = np.ascontiguousarray(keys.transpose(1, 2, 0))      # [Hkv, D, L]
        vh = np.ascontiguousarray(values.transpose(1, 0, 2))    # [Hkv, L, D]
        qb = q[b].reshape(hkv, g, d)
        scores = np.matmul(qb, kh) * np.float32(scale)          # [Hkv, g, L]
        scores = scores - scores.max(axis=-1, keepdims=True)
        weights = np.exp(scores)
        weights /= weights.sum(axis=-1, keepdims=True)
        out[b] = np.matmul(weights, vh).reshape(hq, d)
    if return_f32:
        return out
    return round_to(out, out_dtype)


# ----------------------------------------------------------------------------
# Float64 brute force: literal loops over (b, h, t) with the kernel's
# addressing (gqa_decode.cu:31 head map; :43-47 page, slot, element offset).
# ----------------------------------------------------------------------------


def brute_force_f64(q, k, v, table, lens, scale=None):
    q = np.asarray(q, dtype=np.float64)
    kf = np.asarray(k, dtype=np.float64).reshape(-1)
    vf = np.asarray(v, dtype=np.float64).reshape(-1)
    table = np.asarray(table)
    bsz, hq, d = q.shape
    _, block_size, hkv, _ = np.asarray(k).shape
    max_pages = table.shape[1]
    flat_table = table.reshape(-1)
    if scale is None:
        scale = default_scale(d)
    out = np.zeros((bsz, hq, d), dtype=np.float64)
    for b in range(bsz):
        length = int(lens[b])
        for h in range(hq):
            kv_head = h // (hq // hkv)
            if length <= 0:
                continue
            scores = np.empty(length)
            rows = []
            for t in range(length):
                page = t // block_size
                slot = t % block_size
                phys = int(flat_table[b * max_pages + page])
                base = ((phys * block_size + slot) * hkv + kv_head) * d
                rows.append(base)
                scores[t] = float(np.dot(q[b, h], kf[base:base + d])) * scale
            m = scores.max()
            e = np.exp(scores - m)
            z = e.sum()
            acc = np.zeros(d)
            for t in range(length):
                acc += e[t] * vf[rows[t]:rows[t] + d]
            out[b, h] = acc / z
    return out


# ----------------------------------------------------------------------------
# Split-context partials and merge
# ----------------------------------------------------------------------------


def reference_split_range(length: int, splits: int, z: int) -> tuple[int, int]:
    """Token range of split z: gqa_decode.cu:40-41 (int64 products, floor)."""
    return (length * z) // splits, (length * (z + 1)) // splits


def page_split_range(length: int, block_size: int, max_pages: int, splits: int,
                     chunk_pages: int, z: int) -> tuple[int, int]:
    """Page-aligned token range of split z used by the HIP kernels: split z
    covers pages [z*c, (z+1)*c) with c = chunk_pages, or c = ceil(n/splits)
    for a sequence of n pages when chunk_pages == 0; lengths are clamped to
    the table capacity max_pages*block_size."""
    length = min(length, max_pages * block_size)
    if length <= 0:
        return 0, 0
    n = -(-length // block_size)
    c = chunk_pages if chunk_pages > 0 else -(-n // splits)
    tb = min(z * c * block_size, length)
    te = min(tb + c * block_size, length) if z * c * block_size < length else tb
    return tb, te


def split_partials(q, k, v, table, lens, scale=None, splits=4, ranges=None):
    """Partials [B, Hq, S, D+2] = {m, l, acc} per split (gqa_decode.cu:66-69).

    m is the max scaled score, l = sum exp(s - m), acc = sum exp(s - m) v
    (unnormalized), i.e. the state SoftmaxState::add (online_softmax.cuh:10-16)
    reaches over the split, evaluated in closed form in float64 and stored as
    float32.  Empty splits hold m = -inf, l = 0, acc = 0.  ``ranges(b, z)``
    overrides the token range (default: the reference's, gqa_decode.cu:40-41).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    table = np.asarray(table)
    bsz, hq, d = q.shape
    _, block_size, hkv, _ = k.shape
    g = hq // hkv
    if scale is None:
        scale = default_scale(d)
    part = np.zeros((bsz, hq, splits, d + 2), dtype=np.float32)
    part[..., 0] = -np.inf
    for b in range(bsz):
        length = int(lens[b])
        for z in range(splits):
            tb, te = ranges(b, z) if ranges else reference_split_range(max(length, 0), splits, z)
            if te <= tb:
                continue
            t = np.arange(tb, te)
            phys = table[b, t // block_size].astype(np.int64)
            slot = t % block_size
            for h in range(hq):
                kvh = h // g
                keys = k[phys, slot, kvh]
                vals = v[phys, slot, kvh]
                s = keys @ q[b, h] * scale
                m = s.max()
                e = np.exp(s - m)
                part[b, h, z, 0] = m
                part[b, h, z, 1] = e.sum()
                part[b, h, z, 2:] = e @ vals
    return part


def merge_partials(part, out_dtype="f32"):
    """Sequential merge of gqa_decode.cu:74-87 with SoftmaxState::merge
    (online_softmax.cuh:17-24): skip l == 0, rescale by exp(m - max)."""
    part = np.asarray(part, dtype=np.float32)
    bsz, hq, splits, dp2 = part.shape
    out = np.zeros((bsz, hq, dp2 - 2), dtype=np.float32)
    for b in range(bsz):
        for h in range(hq):
            m = -np.inf
            l = np.float32(0.0)
            acc = np.zeros(dp2 - 2, dtype=np.float32)
            for s in range(splits):
                om, ol = part[b, h, s, 0], part[b, h, s, 1]
                if ol == 0.0:
                    continue
                nm = max(m, om)
                a = np.float32(0.0) if l == 0.0 else np.float32(math.exp(m - nm))
                be = np.float32(math.exp(om - nm))
                l = a * l + be * ol
                acc = a * acc + be * part[b, h, s, 2:]
                m = nm
            out[b, h] = acc / l if l > 0 else 0.0
    return round_to(out, out_dtype)


# ----------------------------------------------------------------------------
# KV-cache append: reference csrc/cuda/cache/kv_append.cu:11-19
# ----------------------------------------------------------------------------


def oracle_kv_append(key, value, k_cache, v_cache, table, positions):
    """Returns copies of the caches after writing sequence b's [Hkv, D] key and
    value row to (table[b, pos // P], pos % P) (kv_append.cu:12-18).  The
    reference leaves out-of-range metadata to the caller; here, as in the
    HIP kernel, a position outside [0, maxP*P) or a page id outside [0, N)
    writes nothing.  Sequences are applied in order (the reference requires
    distinct destinations, so order does not matter for valid input)."""
    kc = np.array(k_cache, copy=True)
    vc = np.array(v_cache, copy=True)
    table = np.asarray(table)
    positions = np.asarray(positions)
    nblocks, block_size = kc.shape[0], kc.shape[1]
    max_pages = table.shape[1]
    for b in range(positions.shape[0]):
        t = int(positions[b])
        if t < 0 or t >= max_pages * block_size:
            continue
        phys = int(table[b, t // block_size])
        if phys < 0 or phys >= nblocks:
            continue
        kc[phys, t % block_size] = key[b]
        vc[phys, t % block_size] = value[b]
    return kc, vc


# ----------------------------------------------------------------------------
# Metadata validation: reference attention/validation.py:23-38
# ----------------------------------------------------------------------------


def oracle_validate_metadata(table, lens, block_size, num_blocks, positions=None):
    """First failure message of the reference's host loop, or None.

    Per sequence b in order (validation.py:23-38): length in
    [0, maxP*P]; each used page id in [0, num_blocks); then, when appending,
    position in [0, maxP*P), its page id in [0, num_blocks), and a
    (page, slot) destination not seen for an earlier sequence."""
    table = np.asarray(table)
    max_pages = table.shape[1]
    seen = set()
    for b, length in enumerate(np.asarray(lens).tolist()):
        if not 0 <= length <= max_pages * block_size:
            return f'invalid length at batch {b}'
        for p in range((length + block_size - 1) // block_size):
            if not 0 <= int(table[b, p]) < num_blocks:
                return f'invalid block at batch {b}, page {p}'
        if positions is not None:
            t = int(positions[b])
            if not 0 <= t < max_pages * block_size:
                return f'invalid append position at batch {b}'
            page = int(table[b, t // block_size])
            if not 0 <= page < num_blocks:
                return f'invalid append page at batch {b}'
            dest = (page, t % block_size)
            if dest in seen:
                return 'conflicting append destinations'
            seen.add(dest)
    return None


# ----------------------------------------------------------------------------
# C restatement (oracle/gqa_oracle.c) through ctypes
# ----------------------------------------------------------------------------

_c_lib = None


def c_library():
    global _c_lib
    if _c_lib is None:
        lib = ctypes.CDLL(C_LIB)
        lib.oracle_gqa_decode.restype = ctypes.c_int
        lib.oracle_gqa_decode.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int] * 8 + [ctypes.c_float]
        _c_lib = lib
    return _c_lib


def _storage(x, dtype):
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dtype == "f32":
        return x
    if dtype == "f16":
        return x.astype(np.float16)
    return np.ascontiguousarray(to_bf16_bits(x).astype(np.uint16))


def c_decode(q, k, v, table, lens, scale=None, dtype="f32"):
    """Runs oracle_gqa_decode from the C restatement; returns float32 values."""
    q = np.asarray(q, dtype=np.float32)
    bsz, hq, d = q.shape
    _, block_size, hkv, _ = np.asarray(k).shape
    table = np.ascontiguousarray(table, dtype=np.int32)
    lens = np.ascontiguousarray(lens, dtype=np.int32)
    if scale is None:
        scale = default_scale(d)
    qs, ks, vs = (_storage(x, dtype) for x in (q, k, v))
    out = np.zeros_like(qs)
    rc = c_library().oracle_gqa_decode(
        qs.ctypes.data, ks.ctypes.data, vs.ctypes.data, table.ctypes.data, lens.ctypes.data,
        out.ctypes.data, bsz, hq, hkv, d, block_size, table.shape[1], DTYPE_CODES[dtype],
        int(np.asarray(k).shape[0]), float(scale))
    if rc != 0:
        raise RuntimeError(f"oracle_gqa_decode failed: {rc}")
    if dtype == "f32":
        return out
    if dtype == "f16":
        return out.astype(np.float32)
    return from_bf16_bits(out.astype(np.uint32))
