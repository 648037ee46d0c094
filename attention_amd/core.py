"""Python API of the paged GQA decode operator (drop-in for the reference's
``attention.core``: reference ``attention/core.py:1-96``).

Every function forwards to ``torch.ops.qd_attention.*``, registered by the
in-tree HIP library.  There is no fallback: if the library is missing, each
call raises ``RuntimeError`` naming the load error, as the reference does
(``core.py:30-35``).
"""
from __future__ import annotations

import math

import torch

from . import _loader

_LOAD_ERROR: BaseException | None = None


def _try_load() -> None:
    global _LOAD_ERROR
    try:
        _loader.load_ops()
        _LOAD_ERROR = None
    except (OSError, RuntimeError) as exc:  # missing or unloadable library
        _LOAD_ERROR = exc


_try_load()


def reload_extension() -> bool:
    """Retries loading the op library (after an in-process build); returns
    :func:`is_cuda_extension_loaded`."""
    if _LOAD_ERROR is not None:
        _try_load()
    return _LOAD_ERROR is None


def is_cuda_extension_loaded() -> bool:
    """True when the HIP op library is registered (reference ``core.py:13-14``)."""
    return _LOAD_ERROR is None


def _require_extension(detail: bool = False) -> None:
    """The reference's missing-extension errors (``core.py:31-35`` for
    ``gqa_decode``, ``:51`` and ``:62`` for the others): a ``RuntimeError``
    with the reference's first sentence (PyTorch-ROCm calls the HIP device
    "CUDA") and the load error as its cause.  ``detail`` adds the build hint,
    in place of the reference's pip/nvcc one."""
    if _LOAD_ERROR is not None:
        msg = "qd_attention CUDA extension was not loaded"
        if detail:
            msg += (". Build it in-tree with `python -m attention_amd._build` on a machine with hipcc "
                    "and a ROCm-enabled PyTorch build.")
        raise RuntimeError(msg) from _LOAD_ERROR


def gqa_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    context_lens: torch.Tensor,
    *,
    scale: float | None = None,
) -> torch.Tensor:
    """Paged single-token MHA/MQA/GQA decode (reference ``core.py:17-40``).

    q ``[B, Hq, D]``; caches ``[blocks, block_size, Hkv, D]``; int32
    ``block_table [B, max_pages]`` and ``context_lens [B]``; all contiguous on
    one GPU, q/k/v of one dtype (fp32/fp16/bf16).  Returns ``[B, Hq, D]`` in
    q's dtype.  The context-split count comes from the library's launch plan
    (static shapes only, no host synchronization); forward only.
    """
    _require_extension(detail=True)
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    return torch.ops.qd_attention.gqa_decode(
        q, k_cache, v_cache, block_table, context_lens, float(scale)
    )


def gqa_decode_split(q, k_cache, v_cache, block_table, context_lens, *, splits=4, scale=None,
                     workspace=None, backend="cuda"):
    """Split-context decode with an fp32 log-sum-exp merge (reference ``core.py:43-56``).

    ``backend`` keeps the reference's keyword: ``"cuda"`` (PyTorch's device
    name on ROCm) and ``"hip"`` select this native path.  The reference's
    ``"triton"`` backend is not part of this build and raises ``ValueError``.
    ``workspace``, if given, must be float32 ``[B, Hq, splits, D + 2]``.
    """
    if backend == "triton":
        raise ValueError("backend 'triton' is not available: this build has only the native HIP path")
    if backend not in ("cuda", "hip"):
        raise ValueError("backend must be cuda or triton")
    _require_extension()
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    if workspace is not None:
        return torch.ops.qd_attention.gqa_decode_split_workspace(
            q, k_cache, v_cache, block_table, context_lens, float(scale), splits, workspace)
    return torch.ops.qd_attention.gqa_decode_split(
        q, k_cache, v_cache, block_table, context_lens, float(scale), splits)


def gqa_decode_auto(q, k_cache, v_cache, block_table, context_lens, *, scale=None):
    """Split choice from static shapes, without synchronizing lengths
    (reference ``core.py:80-96``).

    The reference picks a Triton split count on the host; here the native
    launch plan inside :func:`gqa_decode` already does that (from batch,
    kv-heads, table capacity and the CU count), so this forwards to it after
    the reference's dimension check.
    """
    if q.ndim != 3 or k_cache.ndim != 4 or block_table.ndim != 2:
        raise ValueError('invalid decode input dimensions')
    return gqa_decode(q, k_cache, v_cache, block_table, context_lens, scale=scale)


def kv_append(key, value, k_cache, v_cache, block_table, positions):
    """Writes one token per sequence into the paged caches (reference
    ``core.py:59-63``): ``key``/``value`` ``[B, Hkv, D]`` go to row
    ``(block_table[b, pos // P], pos % P)``.  Destinations are caller-owned
    and must be distinct; a position or page id outside the table or the
    pool is skipped rather than written."""
    _require_extension()
    torch.ops.qd_attention.kv_append(key, value, k_cache, v_cache, block_table, positions)
