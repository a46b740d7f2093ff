"""Builds libfovi_hip.so (gfx950) in-tree with hipcc.

Usage: ``python -m fovi_amd.build`` (also called by ``__graft_entry__.build``).
The library lands next to this file so it travels with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libfovi_hip.so")
SOURCES = ["abi.hip", "sampler.hip", "knnconv.hip", "knnconv_v5.hip", "knnconv_fp8.hip", "quantize.hip",
           "knnpool.hip", "knnconv_bwd.hip", "knn_tables.hip", "knnconv_dw.hip", "knnconv_fewc.hip",
           "knnconv_fewc_vm.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # no fused multiply-add unless written explicitly: the fixation transform
    # must round every op like the reference's separate tensor ops do
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
    return res.returncode


def build(verbose: bool = False) -> str:
    """Compiles each translation unit to an object in parallel, then links the library."""
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
    objs = [os.path.join(objdir, os.path.splitext(s)[0] + ".o") for s in srcs]
    cmds = [[hipcc, *HIPCC_FLAGS, *inc, "-c", os.path.join(CSRC, s), "-o", o] for s, o in zip(srcs, objs)]
    jobs = max(1, min(len(cmds), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(jobs) as ex:
        codes = list(ex.map(lambda c: _run(c, verbose), cmds))
    for s, rc in zip(srcs, codes):
        if rc != 0:
            raise RuntimeError(f"hipcc failed ({rc}) compiling {s}")
    tmp = LIB + ".tmp"
    if _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp], verbose) != 0:
        raise RuntimeError(f"hipcc failed linking {LIB}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
