"""MI355X-native paged grouped-query decode attention.

Drop-in for the reference package's decode surface (reference
``attention/__init__.py:2-20``): ``gqa_decode``, ``gqa_decode_split``,
``gqa_decode_auto``, ``kv_append`` and ``is_cuda_extension_loaded``, backed
by hand-written gfx950 HIP kernels registered as ``torch.ops.qd_attention.*``.
"""
from . import validation
from .core import gqa_decode, gqa_decode_auto, gqa_decode_split, is_cuda_extension_loaded, kv_append

__all__ = ["gqa_decode", "gqa_decode_split", "gqa_decode_auto", "kv_append", "is_cuda_extension_loaded"]
__version__ = "0.1.0"
