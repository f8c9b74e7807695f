"""Build the gfx950 HIP library luisaml_amd/liblcml_fp8.so with hipcc.

Each csrc/*.hip is compiled to an object in parallel, then linked into one
shared library next to this file (in-tree, so it travels with the source
tree).  Flags:
  --offload-arch=gfx950                     MI355X only
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                            no v_pk_{add,mul,fma}_f32 generation
  -fvisibility=hidden                       only the LCML_API C symbols export
  -mllvm -amdgpu-kernarg-preload-count=N    (gemm_skinny.hip, quantize.hip,
                                            gemv_valu.hip) the N leading scalar
                                            kernel arguments arrive in SGPRs
                                            at wave start
Usage:  python -m luisaml_amd.build   (or luisaml_amd.build.build())
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
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "liblcml_fp8.so")
ROOT = os.path.dirname(HERE)

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
]


# per-file flags: leading scalar kernel arguments preloaded into SGPRs
# instead of fetched by the first instructions (the small-M GEMM's first
# weight loads depend on eight of them: 0.25-0.4 us per launch on the
# 4096x11008 linear, with its shorter prologue; the quantisers' first loads
# on four: 0.1 us)
EXTRA = {
    "gemm_skinny.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=8"],
    "quantize.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=4"],
    "gemv_valu.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=6"],
}


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [HIPCC, *COMMON, *EXTRA.get(os.path.basename(src), []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile every csrc/*.hip and link liblcml_fp8.so; returns its path."""
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


def clean() -> None:
    shutil.rmtree(OBJ, ignore_errors=True)
    if os.path.exists(LIB):
        os.remove(LIB)


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
