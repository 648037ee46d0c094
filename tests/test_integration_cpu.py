"""The reference-side integration path (keep the reference's Python, load
this library instead of its CUDA extension): in a fresh interpreter that
loads only ``libqd_attention_torch.so`` with ``torch.ops.load_library`` (no
``attention_amd`` import, none of the reference's code), the library must
register, in the ``qd_attention`` namespace, exactly the decode and MLA op
schemas of reference ``csrc/binding/torch_ops.cpp:47-56`` with kernels on the
CUDA key only (``:59-77``: no CPU kernel, so all-CPU inputs raise
NotImplementedError as with the reference)."""
from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

from attention_amd import _loader

# Reference schema strings (csrc/binding/torch_ops.cpp:47-56), as torch prints them.
REFERENCE_SCHEMAS = {
    "mla_decode_fused": "qd_attention::mla_decode_fused(Tensor q, Tensor qr, Tensor cache, Tensor table, "
                        "Tensor lens, Tensor positions, Tensor wk, Tensor wv, Tensor? indices, float scale, "
                        "bool causal) -> Tensor",
    "mla_project": "qd_attention::mla_project(Tensor x, Tensor weight, bool absorb) -> Tensor",
    "latent_kv_write": "qd_attention::latent_kv_write(Tensor latent, Tensor rope, Tensor(a!) cache, "
                       "Tensor slots) -> ()",
    "mla_attend": "qd_attention::mla_attend(Tensor q, Tensor q_rope, Tensor cache, Tensor table, Tensor lens, "
                  "Tensor positions, Tensor? indices, float scale, bool causal) -> Tensor",
    "kv_append": "qd_attention::kv_append(Tensor key, Tensor value, Tensor(a!) k_cache, Tensor(b!) v_cache, "
                 "Tensor block_table, Tensor positions) -> ()",
    "gqa_decode_split_workspace": "qd_attention::gqa_decode_split_workspace(Tensor q, Tensor k, Tensor v, "
                                  "Tensor table, Tensor lengths, float scale, int splits, "
                                  "Tensor(a!) workspace) -> Tensor",
    "gqa_decode_split": "qd_attention::gqa_decode_split(Tensor q, Tensor k_cache, Tensor v_cache, "
                        "Tensor block_table, Tensor context_lens, float scale, int splits) -> Tensor",
    "gqa_decode": "qd_attention::gqa_decode(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_table, "
                  "Tensor context_lens, float scale) -> Tensor",
}

_PROBE = r"""
import json, sys, torch
torch.ops.load_library(sys.argv[1])
names = sorted(n for n in torch._C._dispatch_get_all_op_names() if n.startswith("qd_attention::"))
out = {"ops": {}, "cpu_call": None}
for n in names:
    op = getattr(torch.ops.qd_attention, n.split("::", 1)[1]).default
    out["ops"][n] = {"schema": str(op._schema),
                     "cuda": torch._C._dispatch_has_kernel_for_dispatch_key(n, "CUDA"),
                     "cpu": torch._C._dispatch_has_kernel_for_dispatch_key(n, "CPU")}
q = torch.zeros(1, 8, 64, dtype=torch.float16)
k = torch.zeros(4, 16, 2, 64, dtype=torch.float16)
try:
    torch.ops.qd_attention.gqa_decode(q, k, k, torch.zeros(1, 4, dtype=torch.int32),
                                      torch.ones(1, dtype=torch.int32), 0.125)
except NotImplementedError:
    out["cpu_call"] = "NotImplementedError"
except Exception as exc:
    out["cpu_call"] = type(exc).__name__
print(json.dumps(out))
"""


@pytest.fixture(scope="module")
def probe():
    if not os.path.exists(_loader.TORCH_LIB):
        pytest.skip("op library not built")
    env = dict(os.environ)
    env.pop("PYTHONPATH", None)
    res = subprocess.run([sys.executable, "-c", _PROBE, _loader.TORCH_LIB], capture_output=True, text=True,
                         timeout=300, cwd="/", env=env)
    assert res.returncode == 0, res.stderr[-2000:]
    return json.loads(res.stdout.strip().splitlines()[-1])


def test_library_alone_registers_exactly_the_reference_schemas(probe):
    got = {n.split("::", 1)[1]: v["schema"] for n, v in probe["ops"].items()}
    assert got == REFERENCE_SCHEMAS


def test_kernels_on_the_cuda_key_only(probe):
    for name, info in probe["ops"].items():
        assert info["cuda"] and not info["cpu"], name


def test_cpu_inputs_raise_not_implemented(probe):
    assert probe["cpu_call"] == "NotImplementedError"
