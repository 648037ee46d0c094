"""Opt-in paged-metadata validation (drop-in for the reference's
``attention.validation``: reference ``attention/validation.py:5-39``).

The checks run on the GPU (``qd_validate_paged_metadata``): one wave per
sequence, the first failure in the reference's order selected with a 64-bit
atomic minimum.  Like the reference, this synchronizes (it reads one result
word back to raise the error) and is not meant for the hot path; the caller
still owns page lifetime and cross-stream ordering.
"""
from __future__ import annotations

import torch

from . import cabi, core

_MESSAGES = {
    1: "invalid length at batch {b}",
    2: "invalid block at batch {b}, page {p}",
    3: "invalid append position at batch {b}",
    4: "invalid append page at batch {b}",
    5: "conflicting append destinations",
}


def validate_paged_metadata(block_table, context_lens, *, block_size, num_blocks, positions=None):
    """Validate page bounds and lengths; if appending, also reject duplicate
    destinations.  Raises ``ValueError`` with the reference's messages
    (``validation.py:11-38``).  CPU tensors are copied to the current GPU."""
    if block_size <= 0 or num_blocks <= 0:
        raise ValueError('block_size and num_blocks must be positive')
    if block_table.ndim != 2 or context_lens.ndim != 1 or block_table.shape[0] != context_lens.numel():
        raise ValueError('metadata shapes must be [B,MaxPages] and [B]')
    if block_table.dtype != torch.int32 or context_lens.dtype != torch.int32:
        raise ValueError('metadata must be int32')
    if positions is not None and (positions.shape != context_lens.shape or positions.dtype != torch.int32):
        raise ValueError('positions must be int32 [B]')
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
