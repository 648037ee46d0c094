"""CPU oracle for paged MLA decode (test infrastructure only; see oracle/__init__.py).

Restates the reference's paged latent-attention operators (paths relative to
the reference tree):

  latent_kv_write    csrc/cuda/mla/mla.cu:28-32, :151-160
  mla_project        csrc/cuda/mla/mla.cu:16-27, :138-150
  mla_attend         csrc/cuda/mla/mla.cu:34-84, :161-181
  mla_decode_fused   csrc/cuda/mla/mla.cu:86-135, :184-198

Arrays are numpy; 16-bit inputs are float32 arrays holding representable
values.  The arithmetic is float64, rounded at the points where the reference
kernels round to the input dtype: the absorbed query (``mla.cu:89``, ``:110``
and the projection's store ``:26``), the latent attention output (``:54``,
``:81``, ``:100``, ``:131``) and the value projection (``:26``, ``:102``,
``:133``).
"""
from __future__ import annotations

import math

import numpy as np

from .gqa_oracle import round_to


def default_mla_scale(nope_dim: int, rope_dim: int) -> float:
    """reference attention/mla.py:44 (and :63): 1/sqrt(Dn + Dr)."""
    return 1.0 / math.sqrt(nope_dim + rope_dim)


def oracle_latent_kv_write(latent, rope, cache, slots):
    """Writes [latent | rope] rows to flat cache rows ``slots`` (mla.cu:29-32).

    ``cache`` is [Nblocks, P, Dc+Dr]; slot s is row s of the flattened
    [Nblocks*P, Dc+Dr] view.  A slot outside [0, Nblocks*P) is skipped (the
    reference does not check; this build does not write outside the cache).
    Works on any dtype (bit patterns are copied).  Returns a new cache.
    """
    cache = np.array(cache, copy=True)
    flat = cache.reshape(-1, cache.shape[-1])
    dc = latent.shape[1]
    for t, s in enumerate(np.asarray(slots, dtype=np.int64)):
        if 0 <= s < flat.shape[0]:
            flat[s, :dc] = latent[t]
            flat[s, dc:] = rope[t]
    return cache


def oracle_mla_project(x, w, absorb, out_dtype="f32"):
    """Per-head projection (mla.cu:16-27).

    absorb:  out[b,t,h,c] = sum_d x[b,t,h,d] * w[h,d,c]   (w [H, Dn, Dc])
    value:   out[b,t,h,v] = sum_c x[b,t,h,c] * w[h,v,c]   (w [H, Dv, Dc])
    fp32-or-better accumulation, one rounding to the dtype.
    """
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    if absorb:
        out = np.einsum("bthd,hdc->bthc", x, w)
    else:
        out = np.einsum("bthc,hvc->bthv", x, w)
    return round_to(out.astype(np.float32), out_dtype)


def attend_end(length: int, position: int, causal: bool, capacity: int) -> int:
    """Visible prefix of a query row (mla.cu:37): min(len, max(0, pos+1)) when
    causal, else len; clamped to the table capacity max_pages*P (longer
    lengths are caller errors that would read past the table row)."""
    end = min(length, max(0, position + 1)) if causal else length
    return max(0, min(end, capacity))


def row_tokens(end: int, selected=None):
    """Logical tokens a query row attends to, in processing order.

    Dense: 0..end-1 (mla.cu:42-44).  Sparse: the listed indices, skipping
    entries outside [0, end) (mla.cu:43-44); a repeated index is counted as
    often as it is listed, as the kernel loop does.
    """
    if selected is None:
        return np.arange(end, dtype=np.int64)
    sel = np.asarray(selected, dtype=np.int64)
    return sel[(sel >= 0) & (sel < end)]


def gather_rows(cache, table_row, tokens):
    """Cache rows of logical tokens through one sequence's page table (mla.cu:45-46)."""
    nblocks, page, width = cache.shape
    flat = cache.reshape(-1, width)
    phys = np.asarray(table_row, dtype=np.int64)[tokens // page]
    return flat[phys * page + tokens % page]


def oracle_mla_attend(q, q_rope, cache, table, lens, positions, scale, causal=True,
                      indices=None, out_dtype="f32", return_f64=False):
    """Paged latent attention (mla.cu:34-55; split form :57-82 is the same softmax).

    q [B,T,H,Dc] (absorbed query), q_rope [B,T,H,Dr], cache [N,P,Dc+Dr].
    Per query row: score_j = (q . c_j[:Dc] + q_rope . c_j[Dc:]) * scale over
    the row's tokens; output = softmax-weighted sum of c_j[:Dc]; a row with
    no tokens is zero (mla.cu:54).
    """
    q = np.asarray(q, dtype=np.float64)
    qr = np.asarray(q_rope, dtype=np.float64)
    cache = np.asarray(cache, dtype=np.float64)
    bsz, tq, heads, dc = q.shape
    capacity = table.shape[1] * cache.shape[1]
    out = np.zeros((bsz, tq, heads, dc), dtype=np.float64)
    for b in range(bsz):
        for t in range(tq):
            end = attend_end(int(lens[b]), int(positions[b, t]), causal, capacity)
            toks = row_tokens(end, None if indices is None else indices[b, t])
            if toks.size == 0:
                continue
            rows = gather_rows(cache, table[b], toks)              # [n, Dc+Dr]
            s = (q[b, t] @ rows[:, :dc].T + qr[b, t] @ rows[:, dc:].T) * scale  # [H, n]
            s -= s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            out[b, t] = p @ rows[:, :dc]
    if return_f64:
        return out
    return round_to(out.astype(np.float32), out_dtype)


def oracle_mla_decode(q_nope, q_rope, cache, table, lens, positions, w_uk, w_uv, scale=None,
                      causal=True, indices=None, out_dtype="f32"):
    """Absorbed paged MLA (mla.cu:86-103, split form :107-134).

    qa = round(q_nope . w_uk)  ->  latent = round(attend(qa, q_rope))  ->
    out = round(latent . w_uv), the rounding points of the reference kernels.
    """
    if scale is None:
        scale = default_mla_scale(q_nope.shape[-1], q_rope.shape[-1])
    qa = oracle_mla_project(q_nope, w_uk, True, out_dtype)
    latent = oracle_mla_attend(qa, q_rope, cache, table, lens, positions, scale, causal, indices,
                               out_dtype)
    return oracle_mla_project(latent, w_uv, False, out_dtype)


def direct_mla_f64(q_nope, q_rope, latent, rope_key, w_uk, w_uv, ends, scale, indices=None):
    """The non-absorbed form of the same attention on contiguous (unpaged)
    latent/rope sequences, in float64: keys and values are up-projected per
    head (k = c . w_uk^T, v = c . w_uv^T) and attended with the plain
    softmax, with the visibility mask given by ``ends`` [B,T] and optional
    index lists.  An independent evaluation order used only to pin the
    absorbed oracle (reference attention/reference/mla.py:6-34 computes both
    forms).
    """
    q = np.asarray(q_nope, dtype=np.float64)
    qr = np.asarray(q_rope, dtype=np.float64)
    c = np.asarray(latent, dtype=np.float64)
    kr = np.asarray(rope_key, dtype=np.float64)
    wk = np.asarray(w_uk, dtype=np.float64)
    wv = np.asarray(w_uv, dtype=np.float64)
    bsz, tq, heads, _ = q.shape
    dv = wv.shape[1]
    keys = np.einsum("bsc,hdc->bshd", c, wk)
    values = np.einsum("bsc,hvc->bshv", c, wv)
    out = np.zeros((bsz, tq, heads, dv))
    for b in range(bsz):
        for t in range(tq):
            end = int(ends[b, t])
            mask = np.zeros(c.shape[1], dtype=bool)
            if indices is None:
                mask[:max(0, end)] = True
            else:
                for i in np.asarray(indices[b, t]):
                    if 0 <= i < end:
                        mask[i] = True
            if not mask.any():
                continue
            s = (np.einsum("hd,shd->hs", q[b, t], keys[b]) + qr[b, t] @ kr[b].T) * scale
            s = np.where(mask[None, :], s, -np.inf)
            s -= s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            out[b, t] = np.einsum("hs,shv->hv", p, values[b])
    return out
