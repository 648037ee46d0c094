"""CPU oracle for paged GQA decode — TEST INFRASTRUCTURE ONLY.

This package restates the reference algorithm on the CPU so that the HIP
path can be checked against it.  Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg may import, call, link or execute
anything under ``oracle/``, and only as the checker (or, for the CPU
baseline, as the timed reference CPU path) — never as a product code path.
The product (``attention_amd``) fails loudly when its HIP library is missing.

Contents
  gqa_oracle.py   numpy restatement of reference attention/reference/gqa.py:21-44,
                  float64 brute force following csrc/cuda/dense/gqa_decode.cu:31-65,
                  split partials + merge following gqa_decode.cu:40-87 and
                  common/online_softmax.cuh:10-24, bf16/fp16 rounding helpers
  cpu_path.py     the reference CPU path (same torch CPU ops in the same order as
                  gqa.py:29-44), timed as the CPU baseline
  gqa_oracle.c    C restatement (fp32 accumulate), built to oracle/_build/ by
                  oracle/Makefile; a second, independent implementation

Pinning (what fixes each function, tests/test_oracle_pinning.py):
  * float64 brute force vs torch SDPA on gathered K/V (library routine, the
    reference's own parity precedent, bench_all_operators.py:61-72)
  * numpy oracle vs brute force, vs C restatement, vs torch CPU path
  * closed forms: len=0 -> zeros, len=1 -> v exactly, identical keys -> mean
    of V, one dominant key -> its value, MHA/MQA reductions, head map h//g
  * invariants: physical-block permutation (bitwise), poisoned unused
    blocks/slots and -1 padding (bitwise), split count S=1..16 (fp32 rounding)
  * rounding: bf16/fp16 RNE against torch/numpy casts incl. ties
  * planted mutants of the oracle (wrong head map, slot, scale, mask, ...)
    must each fail at least one of the above
There are no golden vectors in the reference (it ships no tests), and its
CUDA sources cannot be built here (no nvcc; CUDA-only), so oracle/_ref is
not built.
"""
