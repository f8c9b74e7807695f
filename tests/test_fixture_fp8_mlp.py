"""The FP8 QDQ MLP model-file fixture (tests/golden/fp8_mlp.*), checked
without a GPU:
  * the C++ writer (tests/golden/write_fp8_mlp.cpp, Model::save_to_json +
    WeightBlobWriter) reproduces the committed files byte for byte;
  * the file follows the reference's model format: FP8 initializers are
    4-byte padded at 4-byte offsets (src/onnx/network_instance.cpp:222-224),
    every other initializer is n * sizeof(element) bytes;
  * each per-tensor weight scale is amax/448, so every weight tensor's
    largest code is +-448 (0x7e / 0xfe);
  * the stored output (the oracle's fp32 Gemm chain) agrees with an
    independent float64 evaluation: E4M3 decoded by the closed form
    (-1)^s * (1 + m/8) * 2^(e-7), subnormals m * 2^-9 (fp_quantized.h:226-249),
    within 1e-5 of sum |a*b| per element.
"""
import json
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
WRITER = os.path.join(ROOT, "luisaml_amd", "host", "bin", "write_fp8_mlp")
FILES = ("fp8_mlp.onnx.json", "fp8_mlp.bin", "fp8_mlp_input.bin", "fp8_mlp_output.bin")


def _e4m3_decode_closed_form(q: np.ndarray) -> np.ndarray:
    q = q.astype(np.int64)
    s = np.where(q >> 7, -1.0, 1.0)
    e = (q >> 3) & 15
    m = q & 7
    v = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return s * v


def _load():
    model = json.load(open(os.path.join(GOLDEN, "fp8_mlp.onnx.json")))
    blob = open(os.path.join(GOLDEN, "fp8_mlp.bin"), "rb").read()
    inits = {i["name"]: i for i in model["graph"]["initializer"]}
    return model, blob, inits


def _tensor(blob, init, dtype):
    s, e = init["data_offsets"]
    n = int(np.prod([int(d) for d in init["dims"]]))
    return np.frombuffer(blob[s:e], dtype=dtype)[:n].reshape([int(d) for d in init["dims"]])


def test_writer_reproduces_the_committed_fixture(tmp_path):
    if not os.path.exists(WRITER):
        from luisaml_amd.host import build
        build.build()
    r = subprocess.run([WRITER, str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    for f in FILES:
        assert open(os.path.join(tmp_path, f), "rb").read() == open(os.path.join(GOLDEN, f), "rb").read(), f


def test_fixture_layout_and_scales():
    model, blob, inits = _load()
    assert [n["op_type"] for n in model["graph"]["node"]] == ["DequantizeLinear", "Gemm", "Relu"] * 2 + [
        "DequantizeLinear", "Gemm"]
    for name, init in inits.items():
        s, e = init["data_offsets"]
        n = int(np.prod([int(d) for d in init["dims"]]))
        assert s % 4 == 0 and e <= len(blob)
        if init["data_type"] == "FLOAT8E4M3FN":
            assert e - s == (n + 3) // 4 * 4, name
            assert not any(blob[s + n:e]), name  # zero padding
        else:
            assert init["data_type"] == "FLOAT" and e - s == 4 * n, name
    for l in range(3):
        q = _tensor(blob, inits[f"net.{l}.weight"], np.uint8)
        assert np.max(q & 0x7F) == 0x7E  # amax / 448 maps the largest weight to 448
        assert not np.any((q & 0x7F) == 0x7F)  # no NaN codes
        assert not any(_tensor(blob, inits[f"net.{l}.weight_zero_point"], np.uint8).ravel())


def test_stored_output_matches_float64_evaluation():
    model, blob, inits = _load()
    x = np.fromfile(os.path.join(GOLDEN, "fp8_mlp_input.bin"), np.float32).reshape(64, 784).astype(np.float64)
    y = np.fromfile(os.path.join(GOLDEN, "fp8_mlp_output.bin"), np.float32).reshape(64, 10)
    assert np.all((x >= 0) & (x < 1))  # U(0, 1)
    h, ah = x, np.abs(x)
    for l in range(3):
        w = _e4m3_decode_closed_form(_tensor(blob, inits[f"net.{l}.weight"], np.uint8))
        s = float(_tensor(blob, inits[f"net.{l}.weight_scale"], np.float32)[0])
        b = _tensor(blob, inits[f"net.{l}.bias"], np.float32).astype(np.float64)
        wf = (w * s).astype(np.float32).astype(np.float64)  # DequantizeLinear: one fp32 multiply
        z = h @ wf.T + b
        bound = ah @ np.abs(wf).T + np.abs(b)
        h = np.maximum(z, 0.0) if l < 2 else z
        ah = np.abs(h) + 1e-5 * bound  # the fp32 chain's earlier error, carried as magnitude
    assert np.all(np.abs(y - h) <= 1e-5 * bound + 1e-7), np.max(np.abs(y - h) / bound)
