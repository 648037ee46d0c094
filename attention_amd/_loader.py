"""Locates and loads the in-tree native libraries.

``libqd_attention_torch.so`` registers ``torch.ops.qd_attention.*`` when it
is loaded; it pulls in ``libqd_attention.so`` (the HIP kernels and C ABI)
through its RUNPATH.  torch must be imported first so that the process uses
torch's HIP runtime for both libraries.
"""
from __future__ import annotations

import os

import torch

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
HIP_LIB = os.path.join(LIB_DIR, "libqd_attention.so")
TORCH_LIB = os.path.join(LIB_DIR, "libqd_attention_torch.so")

_loaded: list[str] = []


def load_ops() -> None:
    """Load the op library once; raises OSError if it was not built."""
    if _loaded:
        return
    if not os.path.exists(TORCH_LIB):
        raise OSError(f"{TORCH_LIB} not found; run attention_amd._build.build()")
    torch.ops.load_library(TORCH_LIB)
    _loaded.append(TORCH_LIB)


def loaded_libraries() -> list[str]:
    return list(_loaded)
