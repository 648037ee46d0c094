"""MI355X-native paged grouped-query decode attention.

Drop-in for the reference package's decode surface (reference
``attention/__init__.py:2-20``): ``gqa_decode``, ``gqa_decode_split``,
``gqa_decode_auto``, ``kv_append``, ``is_cuda_extension_loaded`` and the
paged MLA decode operators (``latent_kv_write``, ``mla_query_absorb``,
``mla_value_project``, ``mla_latent_attention``, ``mla_decode``,
``sparse_mla``), backed by hand-written gfx950 HIP kernels registered as
``torch.ops.qd_attention.*``.
"""
from . import validation
from .core import gqa_decode, gqa_decode_auto, gqa_decode_split, is_cuda_extension_loaded, kv_append
from .mla import (latent_kv_write, mla_decode, mla_latent_attention, mla_prefill, mla_query_absorb,
                  mla_value_project, sparse_mla)

__all__ = ["gqa_decode", "gqa_decode_split", "gqa_decode_auto", "kv_append", "is_cuda_extension_loaded",
           "latent_kv_write", "mla_query_absorb", "mla_value_project", "mla_latent_attention", "mla_decode",
           "mla_prefill", "sparse_mla"]
__version__ = "0.1.0"
