"""Builds libtbq.so in-tree: the gfx950 HIP kernels + C-ABI shim (hipcc) and
the C11 host layer (gcc -std=c11), linked into one shared library next to
this file.  Run `python -m trailblaze_amd.build` or __graft_entry__.build().
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
HOST = os.path.join(HERE, "host")
OBJ = os.path.join(ROOT, "_build", "tbq")
LIB = os.path.join(HERE, "libtbq.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-I", os.path.join(ROOT, "include"),
]
C_FLAGS = ["-std=c11", "-O2", "-fPIC", "-Wall", "-Wextra", "-ffp-contract=off",
           "-I", os.path.join(ROOT, "include")]

HIP_SOURCES = ["tbq_matvec.hip", "tbq_mv_q4k.hip", "tbq_mv_kq.hip", "tbq_moe.hip", "tbq_moe_q4k.hip", "tbq_moe_prefill.hip", "tbq_dense.hip", "tbq_dense_prefill.hip", "tbq_gemm.hip", "tbq_api.hip",
               "tbq_noalloc.hip"]
C_SOURCES = ["tb_cuda_abi.c", "tbq_moe_host.c", "tbq_gguf.c"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {os.path.basename(cmd[-1])}")
    return r


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    jobs = []
    for src in HIP_SOURCES:
        o = os.path.join(OBJ, src.replace(".hip", ".o"))
        jobs.append([HIPCC, *HIP_FLAGS, "-c", "-o", o, os.path.join(CSRC, src)])
    for src in C_SOURCES:
        o = os.path.join(OBJ, src.replace(".c", ".o"))
        jobs.append(["gcc", *C_FLAGS, "-c", "-o", o, os.path.join(HOST, src)])
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        for r in ex.map(_run, jobs):
            if verbose and (r.stdout or r.stderr):
                sys.stderr.write(r.stdout + r.stderr)
    objs = [j[j.index("-o") + 1] for j in jobs]
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs, "-lpthread"])
    os.replace(tmp, LIB)
    return LIB


def build_oracle(with_reference: bool = True) -> None:
    """Compile the parity oracle (and, where /root/reference exists, the
    compiled reference under oracle/_ref).  Test infrastructure only."""
    odir = os.path.join(ROOT, "oracle")
    _run(["make", "-s", "-C", odir, "all"])
    ref = os.environ.get("TBQ_REFERENCE", "/root/reference")
    if with_reference and os.path.isdir(ref) and shutil.which("make"):
        _run(["make", "-s", "-C", odir, f"REF={ref}", "ref"])


if __name__ == "__main__":
    print(build(verbose=True))
    build_oracle()
