"""Build libr9k.so (the gfx950 HIP kernels of the MoE hot path) in-tree.

    python r9700-stack_amd/build.py            # -> r9700-stack_amd/r9700_vllm/kernels/libr9k.so

Every `csrc/*.hip` is compiled for gfx950 only and linked into one shared library exporting the C-ABI declared in
include/r9k.h. Objects go to `_build/` next to this file (not tracked).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "r9700_vllm", "kernels", "libr9k.so")
BUILD = os.path.join(HERE, "_build")

ARCH = "gfx950"
CFLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC",
    "-ffp-contract=off",                                        # arithmetic exactly as written (bit-exact paths)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",  # no packed fp32 VALU ops
    "-Wno-unused-command-line-argument",
]
# Per-source additions. The prefill GEMM interleaves its MFMAs with LDS reads and DMA issue under scheduling
# barriers; machine sinking would move the MFMAs (pure operations) past the loop's wait/barrier branches into one
# block at the end of the loop body and undo that order.
FILE_FLAGS = {"r9k_moe_prefill.hip": ["-mllvm", "-disable-machine-sink"]}


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (ROCm is required to build libr9k.so)")


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    cmd = [hipcc(), *CFLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-I", CSRC, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(out: str = OUT, jobs: int = 8, verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not srcs:
        raise RuntimeError(f"no HIP sources in {CSRC}")
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = out + ".tmp"
    cmd = [hipcc(), "-shared", f"--offload-arch={ARCH}", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out} from {len(srcs)} sources", flush=True)
    return out


if __name__ == "__main__":
    build(jobs=int(sys.argv[1]) if len(sys.argv) > 1 else 8)
