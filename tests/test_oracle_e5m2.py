"""Pins for the oracle's E5M2 codec, half rounding, quantised binary ops and
E5M2 Q/DQ (oracle/lcml_oracle.c):
  * the line-by-line restatement of FP8E5M2::from_float
    (include/onnx/fp_quantized.h:272-346) against an independent closed-form
    encoder over all 2^32 fp32 bit patterns;
  * torch.float8_e5m2's RNE cast on every finite fp32 with |x| <= 57344
    (beyond that torch rounds while the reference encoder returns infinity);
  * the decoder (fp_quantized.h:350-377) against the closed form and
    torch.float8_e5m2 on all 256 codes;
  * binary16 rounding against numpy.float16;
  * the quantised Add/Sub/Mul/Div (binary.cpp:184-285) against an independent
    numpy restatement (float16 arithmetic, numpy broadcasting, the encoders);
  * known answers for the non-saturating overflow, ties and specials.
"""
import numpy as np
import pytest
import torch

import oracle


def test_e5m2_restatement_matches_closed_form_spec_on_all_fp32():
    bad, first = oracle.e5m2_sweep_vs_spec(0, 1 << 32)
    assert bad == 0, f"{bad} mismatches, first pattern 0x{first:08x}"


def test_e5m2_matches_torch_on_every_in_range_float():
    hi = 0x47600000  # 57344.0
    step = 1 << 24
    for sign in (0, 1):
        for start in range(1, hi + 1, step):
            stop = min(start + step, hi + 1)
            x = (np.arange(start, stop, dtype=np.uint32) | np.uint32(sign << 31)).view(np.float32)
            ours = oracle.e5m2_from_float(x)
            theirs = torch.from_numpy(x).to(torch.float8_e5m2).view(torch.uint8).numpy()
            assert np.array_equal(ours, theirs), f"block at 0x{start:08x} sign {sign}"


def test_e5m2_decode_table():
    t = oracle.e5m2_decode_table()
    for c in range(256):
        s, e, m = c >> 7, (c >> 2) & 31, c & 3
        if e == 31:
            if m == 0:
                assert t[c] == (-np.inf if s else np.inf)
            else:
                assert np.isnan(t[c])
            continue
        v = m / 4.0 * 2.0 ** -14 if e == 0 else (1 + m / 4.0) * 2.0 ** (e - 15)
        assert t[c] == np.float32(-v if s else v) and np.signbit(t[c]) == bool(s), hex(c)
    theirs = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e5m2).float().numpy()
    both = ~np.isnan(t)
    assert np.array_equal(np.isnan(t), np.isnan(theirs))
    assert np.array_equal(t[both].view(np.uint32), theirs[both].view(np.uint32))
    # every finite code survives a round trip except -0 (the encoder maps -0 to 0x00)
    codes = np.arange(256, dtype=np.uint8)
    fin = np.isfinite(t) & (codes != 0x80)
    assert np.array_equal(oracle.e5m2_from_float(t[fin]), codes[fin])


@pytest.mark.parametrize("x,code", [
    (57344.0, 0x7b), (-57344.0, 0xfb), (57345.0, 0x7c), (61440.0, 0x7c), (1e30, 0x7c), (-1e30, 0xfc),
    (np.inf, 0x7c), (-np.inf, 0xfc), (np.nan, 0x7f), (-0.0, 0x00), (0.0, 0x00),
    (2.0 ** -17, 0x00), (-(2.0 ** -17), 0x80), (2.0 ** -17 * 1.0000001, 0x01), (3 * 2.0 ** -17, 0x02),
    (2.0 ** -16, 0x01), (1.0, 0x3c), (1.125, 0x3c), (1.1250001, 0x3d), (1.375, 0x3e), (1.875, 0x40),
    (-2.5, 0xc1), (2.0 ** -14 * 0.875, 0x04),
])
def test_e5m2_known_answers(x, code):
    assert int(oracle.e5m2_from_float(np.float32(x)).reshape(-1)[0]) == code


def test_half_round_matches_numpy_float16():
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 2 ** 32, 1 << 22, dtype=np.uint64).astype(np.uint32)
    edge = np.array([65504, 65519.996, 65520, -65520, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001,
                     3 * 2.0 ** -25, 2.0 ** -14, 2049, 2051, -0.0], np.float32)
    x = np.concatenate([bits.view(np.float32), edge])
    ours = oracle.half_round(x)
    with np.errstate(over="ignore", invalid="ignore"):
        theirs = x.astype(np.float16).astype(np.float32)
    nan = np.isnan(theirs)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), theirs[~nan].view(np.uint32))


def _numpy_binary(op, dtype, a, b):
    """Independent restatement: numpy float16 arithmetic on the decoded
    values (numpy rounds each float16 op once), numpy broadcasting."""
    if dtype == oracle.DTYPE_FLOAT:
        f = {0: np.add, 1: np.subtract, 2: np.multiply, 3: np.divide}[op]
        with np.errstate(all="ignore"):
            return f(a, b).astype(np.float32)
    dec = oracle.e4m3_to_float if dtype == oracle.DTYPE_E4M3 else oracle.e5m2_to_float
    enc = oracle.e4m3_from_float if dtype == oracle.DTYPE_E4M3 else oracle.e5m2_from_float
    ha, hb = dec(a).astype(np.float16), dec(b).astype(np.float16)
    f = {0: np.add, 1: np.subtract, 2: np.multiply, 3: np.divide}[op]
    with np.errstate(all="ignore"):
        r = f(ha, hb)
    return enc(r.astype(np.float32))


SHAPES = [((3, 5, 7), (3, 5, 7)), ((4, 1, 6), (5, 1)), ((2, 3), ()), ((), (2, 3)), ((7,), (2, 7)),
          ((1, 9), (4, 1)), ((2, 1, 3, 1), (1, 4, 1, 5))]


@pytest.mark.parametrize("dtype", [oracle.DTYPE_FLOAT, oracle.DTYPE_E4M3, oracle.DTYPE_E5M2])
@pytest.mark.parametrize("op", [0, 1, 2, 3])
def test_fp8_binary_matches_numpy_restatement(dtype, op):
    rng = np.random.default_rng(op * 31 + dtype)
    for sa, sb in SHAPES:
        if dtype == oracle.DTYPE_FLOAT:
            a = rng.normal(size=sa).astype(np.float32)
            b = rng.normal(size=sb).astype(np.float32)
            if b.size:
                b.reshape(-1)[0] = 0.0  # a division by zero
        else:
            a = rng.integers(0, 256, size=sa, dtype=np.uint8)
            b = rng.integers(0, 256, size=sb, dtype=np.uint8)
        got = oracle.fp8_binary(op, dtype, a, b)
        ref = _numpy_binary(op, dtype, a, b)
        assert got.shape == ref.shape
        if dtype == oracle.DTYPE_FLOAT:
            nan = np.isnan(ref)
            assert np.array_equal(np.isnan(got), nan)
            assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
        else:
            assert np.array_equal(got, ref), (sa, sb)


def test_fp8_binary_known_answers():
    E4, E5 = oracle.DTYPE_E4M3, oracle.DTYPE_E5M2
    one4, one5 = 0x38, 0x3c
    assert oracle.fp8_binary(0, E4, np.uint8([one4]), np.uint8([one4]))[0] == 0x40  # 1 + 1 = 2
    assert oracle.fp8_binary(0, E4, np.uint8([0x7e]), np.uint8([0x7e]))[0] == 0x7e  # 448 + 448 saturates
    assert oracle.fp8_binary(0, E5, np.uint8([0x7b]), np.uint8([0x7b]))[0] == 0x7c  # 57344 + 57344 -> inf
    assert oracle.fp8_binary(3, E4, np.uint8([one4]), np.uint8([0x00]))[0] == 0x7e  # 1 / 0 = inf -> 448
    assert oracle.fp8_binary(3, E5, np.uint8([0xbc]), np.uint8([0x00]))[0] == 0xfc  # -1 / 0 -> -inf
    assert oracle.fp8_binary(3, E5, np.uint8([0x00]), np.uint8([0x00]))[0] == 0x7f  # 0 / 0 -> NaN
    assert oracle.fp8_binary(1, E4, np.uint8([one4]), np.uint8([one4]))[0] == 0x00  # 1 - 1 = +0
    # 1 + 2^-9 (the smallest E4M3 subnormal): the half sum 1.001953125 is
    # exact in half, then rounds to 1.0 in E4M3
    assert oracle.fp8_binary(0, E4, np.uint8([one4]), np.uint8([0x01]))[0] == one4


def test_quantize_e5m2_closed_forms():
    x = np.array([1.0, -3.0, 1e6, -1e6, np.inf, -np.inf, np.nan, 0.0, -0.0, 57344.0 * 2], np.float32)
    s = np.float32(2.0)
    sat = oracle.quantize_e5m2(x, s, saturate=1)
    raw = oracle.quantize_e5m2(x, s, saturate=0)
    q = (x / s).astype(np.float32)
    assert np.array_equal(raw, oracle.e5m2_from_float(q))
    clamp = np.where(np.isnan(q), q, np.clip(q, -57344.0, 57344.0)).astype(np.float32)
    assert np.array_equal(sat, oracle.e5m2_from_float(clamp))
    assert sat[2] == 0x7b and sat[3] == 0xfb and sat[4] == 0x7b and sat[5] == 0xfb and raw[4] == 0x7c
    codes = np.arange(256, dtype=np.uint8)
    dq = oracle.dequantize_e5m2(codes, np.float32(0.5))
    ref = (oracle.e5m2_decode_table() * np.float32(0.5)).astype(np.float32)
    assert np.array_equal(np.isnan(dq), np.isnan(ref))
    assert np.array_equal(dq[~np.isnan(dq)], ref[~np.isnan(ref)])
