"""Build ``libsisa_hip.so`` in-tree from ``sisa_amd/csrc/*.hip`` with hipcc for gfx950.

Objects go to ``sisa_amd/_build/`` (not versioned); the shared library is written next to this package's
``kernels`` directory as ``sisa_amd/libsisa_hip.so``. Every call recompiles.
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libsisa_hip.so")
ARCH = "gfx950"

# -packed-fp32-ops: hipcc never emits v_pk_{add,mul,fma}_f32 for this library.
HIPFLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", f"-I{os.path.join(ROOT, 'include')}",
            f"-I{CSRC}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# Per-source additions, each the fastest of the default, max-ILP, max-memory-clause, iterative-ILP and
# iterative-minreg machine schedulers measured on MI355X: max-ILP for the dkv attention kernel (dependency chains of
# MFMA, exponentials and fp32 row sums), the fused CE forward, the weight-gradient GEMM (all operand fragments of a
# step read ahead of its MFMAs) and the decoder-block kernels (the forward norms 2-5 % faster); iterative-ILP for the
# dq attention kernel (4-6 % faster than under max-ILP, which makes the dkv kernel 1-4 % slower); the default one
# for the forward attention kernel, the CE training kernels and the prep kernels.
_MAX_ILP = ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]
_ITER_ILP = ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"]
EXTRA_FLAGS = {"attention_bwd.hip": _MAX_ILP, "attention_dq.hip": _ITER_ILP, "lmce_fwd.hip": _MAX_ILP,
               "wgrad.hip": _MAX_ILP, "norm.hip": _MAX_ILP}


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(line for line in res.stderr.splitlines() if "packed-fp32-ops' is not a recognized" not in line)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")


def build(verbose: bool = False) -> str:
    """Compile every HIP source and link the library. Returns the library path."""
    hipcc = _hipcc()
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    objs = [os.path.join(BUILD, os.path.basename(s)[:-4] + ".o") for s in srcs]

    def compile_one(pair):
        src, obj = pair
        if verbose:
            print(f"[build] {os.path.relpath(src, ROOT)}", flush=True)
        _run([hipcc, *HIPFLAGS, *EXTRA_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj])

    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(compile_one, zip(srcs, objs)))
    tmp = LIB + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    if verbose:
        print(f"[build] wrote {os.path.relpath(LIB, ROOT)}", flush=True)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
