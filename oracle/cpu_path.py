"""The reference's CPU path, timed as the CPU baseline (test infrastructure only).

Restates reference ``attention/reference/gqa.py:21-44`` with the same torch
CPU operations in the same order — per-sequence ``index_select`` of the
used pages, flatten and slice to the length, ``transpose`` +
``repeat_interleave`` of the kv-heads, ``.float()``, ``einsum`` for the
scores times scale, ``softmax``, ``einsum`` with V, ``.to(q.dtype)``,
``stack`` — because the point of this function is to cost exactly that
path on the host cores.  The reference file itself never travels to the GPU
box.
"""
from __future__ import annotations

import math

import torch


def reference_cpu_path(q, k_cache, v_cache, block_table, context_lens, *, scale=None):
    bsz, hq, d = q.shape
    _, block_size, hkv, cache_d = k_cache.shape
    if cache_d != d or v_cache.shape != k_cache.shape or hq % hkv:
        raise ValueError("inconsistent decode shapes")
    group = hq // hkv
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    rows = []
    for b in range(bsz):
        length = int(context_lens[b].item())
        if length <= 0:
            rows.append(torch.zeros_like(q[b]))
            continue
        used = (length + block_size - 1) // block_size
        page_ids = block_table[b, :used].long()
        keys = k_cache.index_select(0, page_ids).reshape(-1, hkv, d)[:length]
        vals = v_cache.index_select(0, page_ids).reshape(-1, hkv, d)[:length]
        keys = keys.transpose(0, 1).repeat_interleave(group, dim=0).float()
        vals = vals.transpose(0, 1).repeat_interleave(group, dim=0).float()
        logits = torch.einsum("hd,hld->hl", q[b].float(), keys) * scale
        probs = torch.softmax(logits, dim=-1)
        rows.append(torch.einsum("hl,hld->hd", probs, vals).to(q.dtype))
    return torch.stack(rows, dim=0)


def reference_mla_cpu_path(q_nope, q_rope, cache, block_table, lengths, positions, w_uk, w_uv, *, scale):
    """The reference's MLA CPU path: attention/reference/mla.py:6-34 with
    ``absorbed=True`` (the same torch CPU einsums, mask and softmax), fed the
    latent and rope keys each sequence reads through its page table."""
    bsz, tq, heads, dn = q_nope.shape
    dc = w_uk.shape[-1]
    block = cache.shape[1]
    out = []
    for b in range(bsz):
        length = int(lengths[b].item())
        if length <= 0:
            out.append(torch.zeros(1, tq, heads, w_uv.shape[1], dtype=q_nope.dtype))
            continue
        used = (length + block - 1) // block
        rows = cache.index_select(0, block_table[b, :used].long()).reshape(-1, cache.shape[-1])[:length]
        c = rows[:, :dc].float()[None]
        kr = rows[:, dc:].float()[None]
        q = q_nope[b:b + 1].float()
        qr = q_rope[b:b + 1].float()
        qa = torch.einsum('bthd,hdc->bthc', q, w_uk.float())
        scores = torch.einsum('bthc,bsc->bths', qa, c)
        scores = (scores + torch.einsum('bthr,bsr->bths', qr, kr)) * scale
        ids = torch.arange(c.shape[1]).view(1, 1, 1, -1)
        mask = (ids < length) & (ids <= positions[b:b + 1, :, None, None])
        scores = scores.masked_fill(~mask, -torch.inf)
        any_valid = mask.any(dim=-1, keepdim=True)
        weights = torch.softmax(torch.where(any_valid, scores, torch.zeros_like(scores)), dim=-1)
        weights = torch.where(any_valid, weights, torch.zeros_like(weights))
        u = torch.einsum('bths,bsc->bthc', weights, c)
        out.append(torch.einsum('bthc,hvc->bthv', u, w_uv.float()).to(q_nope.dtype))
    return torch.cat(out, dim=0)
