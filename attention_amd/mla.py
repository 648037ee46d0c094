"""Paged MLA (multi-head latent attention) decode operators (drop-in for the
reference's ``attention.mla``: reference ``attention/mla.py:1-53``).

The cache is ``[Nblocks, page_size, Dc+Dr]`` (normalized latent | rotated
rope key per token); page ids, positions, lengths, slots and selected
indices are caller-owned GPU metadata.  Every function forwards to
``torch.ops.qd_attention.*`` from the in-tree HIP library; there is no
fallback.  Forward only.
"""
from __future__ import annotations

import math

import torch

from .core import is_cuda_extension_loaded


def _ready():
    """reference ``mla.py:12-13``."""
    if not is_cuda_extension_loaded():
        raise RuntimeError('CUDA extension unavailable')


def mla_query_absorb(q_nope, w_uk):
    """``q_nope [B,T,H,Dn] . w_uk [H,Dn,Dc] -> [B,T,H,Dc]`` (reference ``mla.py:16-18``)."""
    _ready()
    return torch.ops.qd_attention.mla_project(q_nope, w_uk, True)


def mla_value_project(latent_output, w_uv):
    """``latent [B,T,H,Dc] . w_uv[H,Dv,Dc]^T -> [B,T,H,Dv]`` (reference ``mla.py:21-23``)."""
    _ready()
    return torch.ops.qd_attention.mla_project(latent_output, w_uv, False)


def latent_kv_write(latent, rope_key, cache, slot_mapping):
    """In-place write of ``[N,Dc]`` latent and ``[N,Dr]`` rope rows to flat
    int64 cache slots (reference ``mla.py:26-29``).  Slots must be unique; a
    slot outside the cache is skipped."""
    _ready()
    torch.ops.qd_attention.latent_kv_write(latent, rope_key, cache, slot_mapping)


def mla_latent_attention(q_absorbed, q_rope, cache, block_table, lengths, positions, *, scale, causal=True,
                         indices=None):
    """Latent output ``[B,T,H,Dc]`` (reference ``mla.py:32-39``).

    ``positions`` are absolute int32 ``[B,T]``; with ``causal`` a query sees
    tokens ``[0, min(len, pos+1))``.  ``indices`` are logical int32
    ``[B,T,K]``; entries outside the visible range (e.g. -1) are ignored.
    Empty or fully masked rows are zero.
    """
    _ready()
    return torch.ops.qd_attention.mla_attend(q_absorbed, q_rope, cache, block_table, lengths, positions, indices,
                                             float(scale), causal)


def mla_decode(q_nope, q_rope, cache, block_table, lengths, positions, w_uk, w_uv, *, scale=None, causal=True,
               indices=None):
    """Absorbed paged MLA with pre-applied RoPE (reference ``mla.py:42-53``).

    Single-query rows take the fused operator (absorption, latent attention
    and value projection in one op); other shapes compose the three ops.
    Both round the absorbed query and the latent output to the input dtype.
    """
    if scale is None:
        scale = 1.0 / math.sqrt(q_nope.shape[-1] + q_rope.shape[-1])
    if (q_nope.ndim == 4 and q_nope.shape[1] == 1 and cache.ndim == 3 and block_table.ndim == 2
            and w_uk.ndim == 3 and w_uk.shape[-1] <= 512 and (indices is None or indices.ndim == 3)):
        _ready()
        return torch.ops.qd_attention.mla_decode_fused(q_nope, q_rope, cache, block_table, lengths, positions,
                                                       w_uk, w_uv, indices, float(scale), causal)
    absorbed = mla_query_absorb(q_nope, w_uk)
    latent = mla_latent_attention(absorbed, q_rope, cache, block_table, lengths, positions, scale=scale,
                                  causal=causal, indices=indices)
    return mla_value_project(latent, w_uv)


def sparse_mla(q_nope, q_rope, cache, block_table, lengths, positions, w_uk, w_uv, indices, *, scale=None):
    """MLA decode over selected tokens (reference ``attention/sparse.py:22-23``)."""
    return mla_decode(q_nope, q_rope, cache, block_table, lengths, positions, w_uk, w_uv, scale=scale,
                      indices=indices)


def mla_prefill(*args, **kwargs):
    """Dense MLA prefill (reference ``mla.py:56-65``) is not part of this
    decode build."""
    raise NotImplementedError("mla_prefill: dense MLA prefill is not part of this decode-path build")
