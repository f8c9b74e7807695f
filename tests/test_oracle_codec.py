"""CPU checks that pin the oracle's E4M3 codec and bf16 rounding.

The oracle restates FP8E4M3FN::from_float / to_float
(reference include/onnx/fp_quantized.h:149-249).  The reference has no
fixture for FP8, so the restatement is pinned by:
  * an independent closed-form encoder (nearest E4M3 grid point, ties to the
    even code, saturation/NaN/signed-zero rules) over all 2^32 fp32 patterns;
  * torch.float8_e4m3fn's cast on every finite fp32 with |x| <= 448 (where
    both are plain round-to-nearest-even);
  * the decode closed form for all 256 codes and known-answer vectors.
"""
import math

import numpy as np
import pytest
import torch

import oracle


def test_restatement_matches_closed_form_spec_on_all_fp32():
    bad, first = oracle.e4m3_sweep_vs_spec(0, 1 << 32)
    assert bad == 0, f"first mismatching pattern 0x{first:08x}"


def _decode_closed_form(c: int) -> float:
    s, e, m = c >> 7, (c >> 3) & 15, c & 7
    if e == 15 and m == 7:
        return math.nan
    v = math.ldexp(m, -9) if e == 0 else math.ldexp(1 + m / 8, e - 7)
    return -v if s else v


def test_decode_table_closed_form():
    t = oracle.e4m3_decode_table()
    for c in range(256):
        want = _decode_closed_form(c)
        if math.isnan(want):
            assert math.isnan(t[c])
        else:
            assert t[c] == want and math.copysign(1, t[c]) == math.copysign(1, want if c != 0x80 else -1.0)
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0 and t[0x01] == 2.0 ** -9 and t[0x08] == 2.0 ** -6


def test_encode_decode_roundtrip_all_codes():
    t = oracle.e4m3_decode_table()
    q = oracle.e4m3_from_float(t)
    for c in range(256):
        if c in (0x7F, 0xFF):
            assert q[c] == 0x7F  # NaN -> canonical 0x7f
        elif c == 0x80:
            assert q[c] == 0x00  # -0.0 -> 0x00 (fp_quantized.h:155-158)
        else:
            assert q[c] == c


KNOWN = [
    (0.0, 0x00), (-0.0, 0x00), (1.0, 0x38), (-1.0, 0xB8), (448.0, 0x7E), (-448.0, 0xFE),
    (449.0, 0x7E), (464.0, 0x7E), (480.0, 0x7E), (1e30, 0x7E), (-1e30, 0xFE),
    (math.inf, 0x7E), (-math.inf, 0xFE), (math.nan, 0x7F), (-math.nan, 0x7F),
    (2.0 ** -9, 0x01), (2.0 ** -10, 0x00), (-(2.0 ** -10), 0x80), (1.5 * 2.0 ** -10, 0x01),
    (1.5 * 2.0 ** -9, 0x02), (2.5 * 2.0 ** -9, 0x02), (3.5 * 2.0 ** -9, 0x04), (2.0 ** -11, 0x00),
    (-(2.0 ** -30), 0x80), (1e-45, 0x00), (-1e-45, 0x80),
    (1.0625, 0x38), (1.0625 + 2.0 ** -20, 0x39), (1.1875, 0x3A), (7.5 * 2.0 ** -9, 0x08),
    (416.0, 0x7D), (432.0, 0x7E), (424.0, 0x7D), (440.0, 0x7E),
]


@pytest.mark.parametrize("x,code", KNOWN)
def test_known_answers(x, code):
    assert int(oracle.e4m3_from_float(np.array([x], np.float32))[0]) == code
    assert oracle.e4m3_spec_encode(np.float32(x)) == code


def test_matches_torch_float8_e4m3fn_on_every_in_range_float():
    """All fp32 patterns with 0 < |x| <= 448, both signs, against torch's RNE cast."""
    lo = np.uint32(0x00000001)
    hi = np.uint32(0x43E00000)  # 448.0
    step = 1 << 24
    for sign in (0, 1):
        for start in range(int(lo), int(hi) + 1, step):
            stop = min(start + step, int(hi) + 1)
            bits = np.arange(start, stop, dtype=np.uint32) | np.uint32(sign << 31)
            x = bits.view(np.float32)
            ours = oracle.e4m3_from_float(x)
            theirs = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            assert np.array_equal(ours, theirs), f"block at 0x{start:08x} sign {sign}"


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(1 << 20).astype(np.float32) * 1e3,
        (rng.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32)).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 3.0e38, 1e-40, -1e-40], np.float32),
    ])
    x = x[~np.isnan(x)]
    ours = oracle.bf16_rne(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    assert np.isnan(torch.from_numpy(oracle.bf16_rne(np.array([np.nan], np.float32)).view(np.int16))
                    .view(torch.bfloat16).float().numpy()).all()


def test_quantize_dequantize_closed_forms():
    x = np.array([[0.5, -3.0, 1000.0], [1e-9, 7.0, -0.0]], np.float32)
    s = np.array([0.25, 2.0, 4.0], np.float32)  # per axis 1
    q = oracle.quantize(x, s, axis=1)
    assert np.array_equal(q, oracle.e4m3_from_float(x / s))
    y = oracle.dequantize(q, s, axis=1)
    assert np.array_equal(y, oracle.e4m3_to_float(q) * s)
    # dynamic scale convention
    assert oracle.scale_from_amax(448.0) == 1.0
    assert oracle.scale_from_amax(0.0) == 1.0
    assert oracle.scale_from_amax(float("inf")) == 1.0
    assert oracle.scale_from_amax(float("nan")) == 1.0
    assert oracle.scale_from_amax(1e-44) == 1.0  # quotient underflows to zero
    assert oracle.amax(np.array([1.0, np.nan, -5.0], np.float32)) == 5.0


@pytest.fixture(scope="module")
def host_lib(tmp_path_factory):
    """luisaml_amd/csrc/lcml_device.hpp's host-callable functions, compiled
    here for the host (tests/cpp/encoder_host.cpp)."""
    import ctypes
    import os
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    src = os.path.join(root, "tests", "cpp", "encoder_host.cpp")
    so = str(tmp_path_factory.mktemp("host") / "libenc_host.so")
    subprocess.run(["/opt/rocm/bin/hipcc", "-O2", "-std=c++17", "-fPIC", "-shared", "-fopenmp",
                    "-I" + os.path.join(root, "luisaml_amd", "csrc"), src, "-o", so], check=True,
                   capture_output=True)
    return ctypes.CDLL(so)


def test_scale_quotient_matches_ieee_division_on_its_range(host_lib):
    """The dynamic scale's amax / 448 (div448_corrected, the corrected
    reciprocal product the device uses for amax in [2^-100, FLT_MAX]) equals
    the IEEE quotient on every fp32 value of that range."""
    import ctypes
    host_lib.div448_mismatches.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
    host_lib.div448_mismatches.restype = ctypes.c_uint64
    first, last = 0x0D800000, 0x7F800000  # 2^-100 .. FLT_MAX
    assert np.float32(2.0 ** -100).view(np.uint32) == first
    assert host_lib.div448_mismatches(first, last) == 0


def test_product_encoder_matches_oracle_on_all_fp32(host_lib):
    """The HIP library's integer encoder (luisaml_amd/csrc/lcml_device.hpp,
    compiled here for the host) against the oracle over all 2^32 patterns."""
    import ctypes
    lib = host_lib
    lib.enc_range.argtypes = [ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p]
    chunk = 1 << 28
    got = np.empty(chunk, np.uint8)
    for c in range((1 << 32) // chunk):
        lib.enc_range(c * chunk, chunk, got.ctypes.data)
        ref = oracle.e4m3_encode_bits(c * chunk, chunk)
        if not np.array_equal(got, ref):
            i = int(np.flatnonzero(got != ref)[0])
            pytest.fail(f"pattern 0x{c * chunk + i:08x}: product 0x{got[i]:02x} oracle 0x{ref[i]:02x}")
