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
