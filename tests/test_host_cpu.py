"""The C++ operator layer without a GPU: registry, ONNX-JSON import of the
reference's MLP fixture, operator creation, tensor API, error behaviour
(tests/cpp/test_registry.cpp, the counterpart of the reference's
tests/onnx/test_onnx_import.cpp)."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "luisaml_amd", "host", "bin")


def _ensure_built():
    if not os.path.exists(os.path.join(BIN, "test_registry")):
        from luisaml_amd.host import build
        build.build()


def test_registry_and_import():
    _ensure_built()
    r = subprocess.run([os.path.join(BIN, "test_registry"), os.path.join(ROOT, "tests", "golden")],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "PASS" in r.stdout, r.stdout + r.stderr
