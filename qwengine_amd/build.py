"""Build the gfx950 HIP library ``qwengine_amd/_lib/libqwattn.so`` with hipcc (no JIT, no torch extension).

Usage: ``python -m qwengine_amd.build`` (or ``__graft_entry__.build()``).  Every call recompiles.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import tempfile
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_lib")
LIB = os.path.join(OUT_DIR, "libqwattn.so")
ARCH = "gfx950"

SOURCES = ["capi.hip", "kv_append.hip", "attn_decode.hip", "attn_decode_ilp.hip", "attn_simple.hip", "attn_prefill.hip",
           "deltanet.hip", "gemv.hip", "gemv_mc.hip", "gemm.cpp"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed fp32 ops stay disabled (some forms have given wrong results on these boxes)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-rdc",
    "-Wall",
    "-Wno-unused-function",
    "-I", os.path.join(ROOT, "include"),
    "-I", CSRC,
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    return "hipcc"


# per-source flags.  attn_decode.hip: MFMA results in VGPRs wherever the register budget allows.  Its one-wave-per-SIMD
# verify kernels otherwise get their score MFMAs written to accumulation registers, and every block's product is then
# copied out for its scale multiply (the Q8_0 three-tile kernel spilled 77 registers that way).
# attn_decode_ilp.hip (the F16 one-pass three-tile verify kernel): the same, and LLVM's iterative-ILP machine
# scheduler (latency hiding ahead of register economy).  deltanet.hip: that scheduler too (decode 6.1 -> 5.7 us,
# 7-token verify 10.0 -> 9.5 us per layer; prefill unchanged).  The other sources measured the same or slower with it.
ILP_SCHED = ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"]
FILE_FLAGS = {"attn_decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
              "attn_decode_ilp.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1", *ILP_SCHED],
              "deltanet.hip": ILP_SCHED,
              # gemv_mc.hip (IQ4_XS / IQ2_S one-column GEMV): the max-memory-clause scheduler
              "gemv_mc.hip": ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause"]}


def _compile(src: str, extra: list[str], obj_dir: str) -> str:
    obj = os.path.join(obj_dir, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src, []), *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    return obj


def build(verbose: bool = False, extra: list[str] | None = None, out: str | None = None) -> str:
    """Compile every source and link the library (to ``out``, default qwengine_amd/_lib/libqwattn.so)."""
    os.makedirs(OUT_DIR, exist_ok=True)
    extra = extra or []
    workers = min(len(SOURCES), max(1, (os.cpu_count() or 4) // 2), 8)
    target = out or LIB
    obj_dir = tempfile.mkdtemp(prefix="qwattn_obj_")
    with concurrent.futures.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, extra, obj_dir), SOURCES))
    tmp = target + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-L/opt/rocm/lib", "-lhipblaslt",
           "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, target)
    shutil.rmtree(obj_dir, ignore_errors=True)
    if verbose:
        print(f"built {target}")
    return target


SHIM_E2E_SRC = os.path.join(ROOT, "tests", "shim_e2e.cpp")
SHIM_E2E = os.path.join(ROOT, "tests", "_build", "shim_e2e")


def build_shim_e2e(verbose: bool = False) -> str:
    """Host-only C++ program that drives the library through include/q38rt_attn.hpp (the GPU test of the drop-in
    C++ boundary).  Built here, beside the library, so GPU runs only execute it."""
    os.makedirs(os.path.dirname(SHIM_E2E), exist_ok=True)
    cmd = ["g++", "-std=c++17", "-O2", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"), "-I",
           "/opt/rocm/include", SHIM_E2E_SRC, "-o", SHIM_E2E, "-L", OUT_DIR, "-lqwattn", "-L/opt/rocm/lib",
           "-lamdhip64", "-Wl,-rpath,$ORIGIN/../../qwengine_amd/_lib", "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"shim_e2e build failed:\n{r.stderr[-4000:]}")
    if verbose:
        print(f"built {SHIM_E2E}")
    return SHIM_E2E


if __name__ == "__main__":
    build(verbose=True, extra=sys.argv[1:])
    build_shim_e2e(verbose=True)
