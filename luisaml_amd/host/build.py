"""Build the C++ operator layer (luisaml_amd/host/libluisaml_onnx.so) and its
test drivers (luisaml_amd/host/bin/), linked against liblcml_fp8.so.

The layer is host C++20 (hipcc as the compiler driver for the HIP runtime
headers); it launches no kernels of its own, only the C ABI's.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libluisaml_onnx.so")
BIN = os.path.join(HERE, "bin")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = [HIPCC, "-std=c++20", "-O2", "-fPIC", "-Wall", "-Wno-unused-command-line-argument",
       "-I" + os.path.join(HERE, "include"), "-I" + os.path.join(ROOT, "include")]
DRIVERS = {  # test drivers under tests/cpp
    "test_registry": os.path.join(ROOT, "tests", "cpp", "test_registry.cpp"),
    "test_network": os.path.join(ROOT, "tests", "cpp", "test_network.cpp"),
    # the FP8 QDQ MLP model-file fixture writer (tests/golden/fp8_mlp.*)
    "write_fp8_mlp": os.path.join(ROOT, "tests", "golden", "write_fp8_mlp.cpp"),
}


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.relpath(src, HERE).replace(os.sep, "_") + ".o")
    _run([*CXX, "-c", src, "-o", obj])
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(BIN, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(HERE, "src", "*.cpp")) + glob.glob(os.path.join(HERE, "src", "operators", "*.cpp")))
    with cf.ThreadPoolExecutor(min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    _run([HIPCC, "-shared", "-fPIC", "-o", LIB + ".tmp", *objs, "-L" + PKG, "-llcml_fp8",
          "-Wl,-rpath,$ORIGIN/.."])
    os.replace(LIB + ".tmp", LIB)
    oracle_dir = os.path.join(ROOT, "oracle")
    for name, src in DRIVERS.items():
        _run([*CXX, src, "-o", os.path.join(BIN, name), "-L" + HERE, "-lluisaml_onnx", "-L" + PKG, "-llcml_fp8",
              "-L" + oracle_dir, "-llcml_oracle", "-Wl,-rpath,$ORIGIN/..:$ORIGIN/../..:$ORIGIN/../../../oracle"])
    if verbose:
        print("built", LIB, "and", ", ".join(DRIVERS))
    return LIB


if __name__ == "__main__":
    build(verbose=True)
