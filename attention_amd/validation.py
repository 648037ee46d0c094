"""Opt-in paged-metadata validation (drop-in for the reference's
``attention.validation``: reference ``attention/validation.py:5-39``).

Metadata on the GPU is checked there (``qd_validate_paged_metadata``): one
wave per sequence, the first failure in the reference's order selected with
a 64-bit atomic minimum, then one word read back.  Metadata already on the
host (all of ``block_table``, ``context_lens`` and ``positions`` CPU
tensors) is checked on the host with vectorized array code and needs no GPU
or native library.  Like the reference, this synchronizes and is not meant
for the hot path; the caller still owns page lifetime and cross-stream
ordering.
"""
from __future__ import annotations

import numpy as np
import torch

from . import cabi, core

_MESSAGES = {
    1: "invalid length at batch {b}",
    2: "invalid block at batch {b}, page {p}",
    3: "invalid append position at batch {b}",
    4: "invalid append page at batch {b}",
    5: "conflicting append destinations",
}


def _first_failure_host(table: np.ndarray, lens: np.ndarray, block_size: int, num_blocks: int,
                        positions: np.ndarray | None):
    """(b, check, page) of the first failure in the reference's loop order
    (per sequence: length, used page ids in page order, append position,
    append page, destination already taken by an earlier sequence), or None.

    Every check is evaluated for all sequences at once; the answer is the
    smallest failing sequence and, within it, the first failing check.  A
    destination conflict is decided against earlier sequences only: when the
    first failure is at b, every earlier sequence passed all its checks, so
    its destination is a valid one."""
    batch, max_pages = table.shape
    cap = max_pages * block_size
    lens = lens.astype(np.int64)
    code = np.zeros(batch, dtype=np.int64)
    page_at = np.zeros(batch, dtype=np.int64)
    bad_len = (lens < 0) | (lens > cap)
    used = -(-np.clip(lens, 0, cap) // block_size)
    if max_pages > 0:
        in_use = np.arange(max_pages)[None, :] < used[:, None]
        bad_page = in_use & ((table < 0) | (table >= num_blocks))
        any_bad_page = bad_page.any(axis=1)
        page_at = np.argmax(bad_page, axis=1)
    else:
        any_bad_page = np.zeros(batch, dtype=bool)
    if positions is not None:
        pos = positions.astype(np.int64)
        bad_pos = (pos < 0) | (pos >= cap)
        safe = np.where(bad_pos, 0, pos)
        pg = (table[np.arange(batch), safe // block_size].astype(np.int64) if max_pages > 0
              else np.full(batch, -1, dtype=np.int64))
        bad_apage = ~bad_pos & ((pg < 0) | (pg >= num_blocks))
        # Destinations as one key each; invalid ones get distinct negative
        # keys so they never collide.
        dest = np.where(bad_pos | bad_apage, -1 - np.arange(batch), pg * block_size + safe % block_size)
        _, first_idx, inverse = np.unique(dest, return_index=True, return_inverse=True)
        conflict = first_idx[inverse.reshape(-1)] < np.arange(batch)
        code = np.select([bad_pos, bad_apage, conflict], [3, 4, 5], 0)
    code = np.where(any_bad_page, 2, code)
    code = np.where(bad_len, 1, code)
    failing = np.nonzero(code)[0]
    if failing.size == 0:
        return None
    b = int(failing[0])
    return b, int(code[b]), int(page_at[b])


def validate_paged_metadata(block_table, context_lens, *, block_size, num_blocks, positions=None):
    """Validate page bounds and lengths; if appending, also reject duplicate
    destinations.  Raises ``ValueError`` with the reference's messages
    (``validation.py:11-38``).  All-CPU metadata is checked on the host;
    otherwise CPU tensors are copied to the GPU of the other ones (or the
    current GPU) and checked there."""
    if block_size <= 0 or num_blocks <= 0:
        raise ValueError('block_size and num_blocks must be positive')
    if block_table.ndim != 2 or context_lens.ndim != 1 or block_table.shape[0] != context_lens.numel():
        raise ValueError('metadata shapes must be [B,MaxPages] and [B]')
    if block_table.dtype != torch.int32 or context_lens.dtype != torch.int32:
        raise ValueError('metadata must be int32')
    if positions is not None and (positions.shape != context_lens.shape or positions.dtype != torch.int32):
        raise ValueError('positions must be int32 [B]')
    if not any(t.is_cuda for t in (block_table, context_lens, positions) if t is not None):
        fail = _first_failure_host(block_table.detach().numpy(), context_lens.detach().numpy(),
                                   int(block_size), int(num_blocks),
                                   None if positions is None else positions.detach().numpy())
        if fail is not None:
            b, check, page = fail
            raise ValueError(_MESSAGES[check].format(b=b, p=page))
        return
    core._require_extension()
    batch, max_pages = block_table.shape
    if batch == 0:
        return
    if max_pages == 0:
        # No capacity: every length must be 0 and no position is valid
        # (validation.py:24-32 with an empty table row).
        for b, length in enumerate(context_lens.detach().cpu().tolist()):
            if length != 0:
                raise ValueError(_MESSAGES[1].format(b=b))
            if positions is not None:
                raise ValueError(_MESSAGES[3].format(b=b))
        return
    if batch >= (1 << 28):
        raise ValueError('batch too large for device validation')
    dev = block_table.device if block_table.is_cuda else torch.device("cuda", torch.cuda.current_device())
    table = block_table.to(dev).contiguous()
    lens = context_lens.to(dev).contiguous()
    pos = positions.to(dev).contiguous() if positions is not None else None
    result = torch.empty(1, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = cabi.lib().qd_validate_paged_metadata(
        table.data_ptr(), lens.data_ptr(), pos.data_ptr() if pos is not None else None, batch, max_pages,
        int(block_size), int(num_blocks), result.data_ptr(), stream)
    if rc:
        raise RuntimeError(cabi.error_string(rc))
    key = int(result.item()) & ((1 << 64) - 1)   # synchronizes, as the reference does
    if key == (1 << 64) - 1:
        return
    b, check, page = key >> 35, (key >> 32) & 7, key & 0xFFFFFFFF
    raise ValueError(_MESSAGES[check].format(b=b, p=page))
