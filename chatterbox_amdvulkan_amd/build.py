"""Builds libcbxops.so (gfx950) in-tree with hipcc.

    python -m chatterbox_amdvulkan_amd.build [--jobs N] [--verbose]

Every HIP translation unit is compiled with:
  -ffp-contract=off                     one rounding per written f32 operation
                                        (the kernels reproduce ggml-cpu's
                                        scalar arithmetic)
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                        no packed f32 VALU ops
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libcbxops.so")

SOURCES = [
    "cbx_api.cpp",
    "cbx_gguf.cpp",
    "cbx_graph.cpp",
    "k_rows.hip",
    "k_norm.hip",
    "k_group_norm.hip",
    "k_rope.hip",
    "k_norm_rope.hip",
    "k_softmax.hip",
    "k_norm_ext.hip",
    "k_conv1d.hip",
    "k_eltwise.hip",
    "k_batch.hip",
    "k_binary.hip",
]
HEADERS = ["cbx_internal.h", "cbx_device.h", "cbx_rowops.h", os.path.join("..", "..", "include", "cbxops.h")]

ARCH = "gfx950"
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
    f"-I{os.path.join(ROOT, 'include')}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libcbxops)")


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    path = os.path.join(CSRC, src)
    cmd = [hipcc()] + COMMON + (["-x", "hip"] if src.endswith(".hip") else []) + ["-c", path, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{r.stdout}\n{r.stderr}")
    if verbose and r.stderr.strip():
        print(r.stderr, file=sys.stderr)
    return obj


def build(jobs: int = 0, verbose: bool = False) -> str:
    """Compiles every source for gfx950 and links libcbxops.so; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=0)
    ap.add_argument("--verbose", action="store_true")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose))
    return 0


if __name__ == "__main__":
    sys.exit(main())
