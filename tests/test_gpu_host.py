"""The C++ operator layer on the GPU (tests/cpp/test_network.cpp, the
counterpart of the reference's tests/onnx/test_onnx_inference.cpp): the
reference's fp32 MLP fixture end to end, QDQ graphs fused into FP8Linear and
unfused, static/dynamic activation quantisation, standalone Q/DQ/Cast
bit-exactness, error behaviour -- all checked against the oracle."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "luisaml_amd", "host", "bin")

pytestmark = pytest.mark.gpu


def test_network_instance(dev):
    exe = os.path.join(BIN, "test_network")
    assert os.path.exists(exe), "run __graft_entry__.build() first"
    r = subprocess.run([exe, os.path.join(ROOT, "tests", "golden")], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0 and r.stdout.strip().endswith("PASS"), r.stdout + r.stderr
