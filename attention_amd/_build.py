"""In-tree build of the native libraries (no setuptools, no hipify).

Outputs, all under ``attention_amd/lib``:

* ``libqd_attention.so``        — gfx950 HIP kernels + the C ABI of
  ``include/qd_attention.h`` (hipcc, device code for gfx950 only).
* ``libqd_attention_torch.so``  — thin PyTorch-ROCm op registration
  (host C++ against torch's headers), linked to the library above.

The reference builds one ``CUDAExtension`` (reference ``setup.py:9-27``);
here hipcc compiles the HIP source directly so nothing is hipified.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "attention_amd")
CSRC = os.path.join(PKG, "csrc")
LIB_DIR = os.path.join(PKG, "lib")
INCLUDE = os.path.join(ROOT, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

HIP_LIB = os.path.join(LIB_DIR, "libqd_attention.so")
TORCH_LIB = os.path.join(LIB_DIR, "libqd_attention_torch.so")
# Diagnostic library, loaded only by bench.py --mode stamps / read /
# mla-stamps: copies of the decode and MLA kernels with per-wave timestamps
# (gqa_decode.hip and mla.hip built with -DQD_STAMPS) and the streaming-read
# probes (stream_probe.hip).
DIAG_LIB = os.path.join(LIB_DIR, "libqd_attention_diag.so")
DIAG_SOURCES = ["gqa_decode", "stream_probe", "mla"]

# Packed-fp32 VALU forms are disabled for every HIP compile.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    path = os.path.join(ROCM, "bin", "hipcc")
    return path if os.path.exists(path) else (shutil.which("hipcc") or "hipcc")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in res.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in line)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


HIP_SOURCES = ["gqa_decode", "kv_append", "validate", "mla"]
OBJ_DIR = os.path.join(ROOT, "_build", "obj")

# Per-source flags.  mla: MFMA accumulators in VGPRs where the register
# budget allows (one wave per SIMD gives 512); with the default AGPR form the
# attention kernels moved hundreds of registers between the two files per
# cache tile.
SOURCE_FLAGS = {"mla": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hip_object_cmd(name: str) -> list[str]:
    return [_hipcc(), *HIP_FLAGS, *SOURCE_FLAGS.get(name, []), f"-I{INCLUDE}", "-c",
            os.path.join(CSRC, f"{name}.hip"), "-o", os.path.join(OBJ_DIR, f"{name}.o")]


def hip_link_cmd() -> list[str]:
    return [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC",
            *[os.path.join(OBJ_DIR, f"{n}.o") for n in HIP_SOURCES],
            "-o", HIP_LIB + ".tmp", f"-Wl,-rpath,{ROCM}/lib"]


def _stale(name: str) -> bool:
    obj = os.path.join(OBJ_DIR, f"{name}.o")
    if not os.path.exists(obj):
        return True
    deps = [os.path.join(CSRC, f"{name}.hip"), os.path.join(CSRC, "qd_device.h"),
            os.path.join(INCLUDE, "qd_attention.h")]
    return any(os.path.getmtime(d) > os.path.getmtime(obj) for d in deps)


def _torch_flags() -> tuple[list[str], str]:
    import torch  # noqa: F401  (paths only)
    from torch.utils.cpp_extension import include_paths, library_paths

    abi = int(getattr(__import__("torch")._C, "_GLIBCXX_USE_CXX11_ABI", True))
    incs = [f"-I{p}" for p in include_paths()] + [f"-I{INCLUDE}", f"-I{ROCM}/include"]
    return (["-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}", *incs],
            library_paths()[0])


def torch_object_cmd() -> list[str]:
    flags, _ = _torch_flags()
    return ["g++", "-O2", "-std=c++17", "-fPIC", *flags, "-c", os.path.join(CSRC, "torch_ops.cpp"),
            "-o", os.path.join(OBJ_DIR, "torch_ops.o")]


def torch_link_cmd() -> list[str]:
    _, torch_lib = _torch_flags()
    return ["g++", "-shared", os.path.join(OBJ_DIR, "torch_ops.o"), "-o", TORCH_LIB + ".tmp",
            f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-lamdhip64",
            f"-L{LIB_DIR}", "-l:libqd_attention.so",
            "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"]


def build(verbose: bool = False, incremental: bool = False) -> None:
    """Compile both libraries (every source unless ``incremental``, which
    recompiles only sources newer than their object): one compiler process
    per source file, concurrently, then the two links."""
    os.makedirs(LIB_DIR, exist_ok=True)
    os.makedirs(OBJ_DIR, exist_ok=True)
    cmds = [hip_object_cmd(n) for n in HIP_SOURCES if not incremental or _stale(n)]
    torch_obj = os.path.join(OBJ_DIR, "torch_ops.o")
    if (not incremental or not os.path.exists(torch_obj)
            or os.path.getmtime(os.path.join(CSRC, "torch_ops.cpp")) > os.path.getmtime(torch_obj)
            or os.path.getmtime(os.path.join(INCLUDE, "qd_attention.h")) > os.path.getmtime(torch_obj)):
        cmds.append(torch_object_cmd())
    with ThreadPoolExecutor(max_workers=max(1, len(cmds))) as ex:
        for f in [ex.submit(_run, c, verbose) for c in cmds]:
            f.result()
    _run(hip_link_cmd(), verbose)
    os.replace(HIP_LIB + ".tmp", HIP_LIB)
    _run(torch_link_cmd(), verbose)
    os.replace(TORCH_LIB + ".tmp", TORCH_LIB)


def build_diag(verbose: bool = False) -> None:
    """The diagnostic library: gqa_decode.hip and mla.hip with -DQD_STAMPS
    and the streaming-read probes."""
    os.makedirs(LIB_DIR, exist_ok=True)
    os.makedirs(OBJ_DIR, exist_ok=True)
    objs = [os.path.join(OBJ_DIR, f"{n}_diag.o") for n in DIAG_SOURCES]
    with ThreadPoolExecutor(max_workers=len(objs)) as ex:
        futs = [ex.submit(_run, [_hipcc(), *HIP_FLAGS, *SOURCE_FLAGS.get(n, []), "-DQD_STAMPS", f"-I{INCLUDE}", "-c",
                                 os.path.join(CSRC, f"{n}.hip"), "-o", o], verbose)
                for n, o in zip(DIAG_SOURCES, objs)]
        for f in futs:
            f.result()
    _run([_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", DIAG_LIB + ".tmp",
          f"-Wl,-rpath,{ROCM}/lib"], verbose)
    os.replace(DIAG_LIB + ".tmp", DIAG_LIB)


def build_parallel(extra: list[list[str]] | None = None, verbose: bool = False) -> None:
    """Build the libraries (and the diagnostic one) and any extra independent
    commands concurrently."""
    os.makedirs(LIB_DIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=4) as ex:
        futs = [ex.submit(build, verbose), ex.submit(build_diag, verbose)]
        for cmd in extra or []:
            futs.append(ex.submit(_run, cmd, verbose))
        for f in futs:
            f.result()


if __name__ == "__main__":
    build(verbose="-v" in sys.argv, incremental="-i" in sys.argv)
    print("built", HIP_LIB, TORCH_LIB)
