"""GPU parity of the fp8 data-type entry points against the oracle:
lcml_fp8_cast (FLOAT <-> FLOAT8E4M3FN <-> FLOAT8E5M2, the reference's CPU
codecs, include/onnx/fp_quantized.h:149-249, 272-377), E5M2
QuantizeLinear / DequantizeLinear, and the quantised elementwise ops
(src/onnx/operators/binary.cpp:184-285).  Every result is bit-exact (NaN
compared as NaN)."""
import numpy as np
import pytest
import torch

import oracle
from luisaml_amd import capi

pytestmark = pytest.mark.gpu

F, E4, E5 = capi.DTYPE_FLOAT, capi.DTYPE_FLOAT8E4M3FN, capi.DTYPE_FLOAT8E5M2


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _int32_bits(first, count, dev):
    b = torch.arange(first, first + count, dtype=torch.int64, device=dev)
    b = torch.where(b >= 2**31, b - 2**32, b)
    return b.to(torch.int32)


def f32_equal(got, ref):
    got, ref = np.asarray(got, np.float32), np.asarray(ref, np.float32)
    nan = np.isnan(ref)
    return np.array_equal(np.isnan(got), nan) and np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_cast_to_e5m2_exhaustive_all_fp32_patterns(dev):
    """Every fp32 bit pattern through lcml_fp8_cast FLOAT -> FLOAT8E5M2
    (hardware RNE plus the explicit NaN / overflow selection) against the
    oracle's restatement of FP8E5M2::from_float."""
    chunk = 1 << 28
    y = torch.empty(chunk, dtype=torch.uint8, device=dev)
    for c in range((1 << 32) // chunk):
        first = c * chunk
        x = _int32_bits(first, chunk, dev).view(torch.float32)
        capi.cast(x, F, E5, out=y)
        got = y.cpu().numpy()
        ref = oracle.e5m2_encode_bits(first, chunk)
        if not np.array_equal(got, ref):
            i = int(np.flatnonzero(got != ref)[0])
            pytest.fail(f"pattern 0x{first + i:08x}: gpu 0x{got[i]:02x} oracle 0x{ref[i]:02x}")
        del x


def test_cast_float_to_e4m3_matches_quantize_path(dev):
    rng = np.random.default_rng(1)
    x = rng.integers(0, 2**32, 1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    got = capi.cast(to_dev(x, dev), F, E4).cpu().numpy()
    assert np.array_equal(got, oracle.e4m3_from_float(x))


@pytest.mark.parametrize("fmt,table", [(E4, oracle.e4m3_decode_table), (E5, oracle.e5m2_decode_table)])
def test_cast_decode_all_codes(dev, fmt, table):
    codes = np.tile(np.arange(256, dtype=np.uint8), 6)[:1283]  # odd length: vector body + tail
    got = capi.cast(to_dev(codes, dev), fmt, F).cpu().numpy()
    assert f32_equal(got, table()[codes])


def test_cast_fp8_to_fp8_all_codes(dev):
    codes = np.arange(256, dtype=np.uint8)
    e4_to_e5 = capi.cast(to_dev(codes, dev), E4, E5).cpu().numpy()
    assert np.array_equal(e4_to_e5, oracle.e5m2_from_float(oracle.e4m3_decode_table()))
    e5_to_e4 = capi.cast(to_dev(codes, dev), E5, E4).cpu().numpy()
    assert np.array_equal(e5_to_e4, oracle.e4m3_from_float(oracle.e5m2_decode_table()))
    same = capi.cast(to_dev(codes, dev), E5, E5).cpu().numpy()
    assert np.array_equal(same, oracle.e5m2_from_float(oracle.e5m2_decode_table()))


@pytest.mark.parametrize("saturate", [0, 1])
@pytest.mark.parametrize("s", [1.0, 0.0137, 3.5e-4, 700.0, 2.0 ** -70])
def test_quantize_e5m2_per_tensor(dev, saturate, s):
    rng = np.random.default_rng(int(s * 1e4) % 997 + saturate)
    bits = rng.integers(0, 2**32, (1 << 20) + 3, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    sd = torch.tensor([s], dtype=torch.float32, device=dev)
    got = capi.quantize_e5m2(to_dev(x, dev), sd, saturate=saturate).cpu().numpy()
    ref = oracle.quantize_e5m2(x, np.float32(s), saturate=saturate)
    bad = np.flatnonzero(got != ref)
    assert bad.size == 0, f"{bad.size} mismatches, first x=0x{bits[bad[0]]:08x}: {got[bad[0]]:#x} vs {ref[bad[0]]:#x}"


@pytest.mark.parametrize("shape,axis", [((6, 40, 8), 1), ((5, 7, 3), 1), ((33, 12), 0)])
def test_quantize_dequantize_e5m2_per_axis(dev, shape, axis):
    rng = np.random.default_rng(sum(shape))
    x = (rng.normal(size=shape) * 3000).astype(np.float32)
    s = (rng.random(shape[axis]) * 0.1 + 0.01).astype(np.float32)
    q = capi.quantize_e5m2(to_dev(x, dev), to_dev(s, dev), axis=axis).cpu().numpy()
    qr = oracle.quantize_e5m2(x, s, axis=axis)
    assert np.array_equal(q, qr)
    d = capi.dequantize_e5m2(to_dev(qr, dev), to_dev(s, dev), axis=axis).cpu().numpy()
    assert f32_equal(d, oracle.dequantize_e5m2(qr, s, axis=axis))


SHAPES = [((3, 5, 7), (3, 5, 7)), ((1029,), (1029,)), ((4, 1, 6), (5, 1)), ((2, 3), ()), ((), (2, 3)),
          ((7,), (2, 7)), ((1, 9), (4, 1)), ((2, 1, 3, 1), (1, 4, 1, 5)), ((64, 257), (257,))]


@pytest.mark.parametrize("dtype", [F, E4, E5])
@pytest.mark.parametrize("op", [capi.BINARY_ADD, capi.BINARY_SUB, capi.BINARY_MUL, capi.BINARY_DIV])
def test_binary_matches_oracle(dev, dtype, op):
    rng = np.random.default_rng(op * 7 + dtype)
    for sa, sb in SHAPES:
        if dtype == F:
            a = rng.normal(size=sa).astype(np.float32)
            b = rng.normal(size=sb).astype(np.float32)
            if b.size:
                b.reshape(-1)[0] = 0.0
        else:
            a = rng.integers(0, 256, size=sa, dtype=np.uint8)
            b = rng.integers(0, 256, size=sb, dtype=np.uint8)
        got = capi.binary(op, to_dev(a, dev), to_dev(b, dev), dtype).cpu().numpy()
        ref = oracle.fp8_binary(op, dtype, a, b)
        assert got.shape == ref.shape, (sa, sb)
        if dtype == F:
            assert f32_equal(got, ref), (sa, sb)
        else:
            assert np.array_equal(got, ref), (sa, sb, np.flatnonzero(got.reshape(-1) != ref.reshape(-1))[:5])


def test_binary_all_code_pairs(dev):
    """Every pair of codes (65536) for every op and both fp8 formats."""
    a = np.repeat(np.arange(256, dtype=np.uint8), 256)
    b = np.tile(np.arange(256, dtype=np.uint8), 256)
    for dtype in (E4, E5):
        for op in range(4):
            got = capi.binary(op, to_dev(a, dev), to_dev(b, dev), dtype).cpu().numpy()
            assert np.array_equal(got, oracle.fp8_binary(op, dtype, a, b)), (dtype, op)


def test_argument_errors(dev):
    x = torch.zeros(6, dtype=torch.uint8, device=dev)
    with pytest.raises(capi.LcmlError):
        capi.cast(x, 16, F)  # bf16 source is not an fp8 data type here
    a = torch.zeros((2, 3), device=dev)
    b = torch.zeros((4,), device=dev)
    sh = lambda t: (capi.C.c_int64 * len(t))(*t)
    rc = capi.lib().lcml_fp8_binary(0, F, a.data_ptr(), sh((2, 3)), 2, b.data_ptr(), sh((4,)), 1, a.data_ptr(),
                                    sh((2, 3)), 2, None)
    assert rc == capi.ERR_INVALID_ARG


def test_scalar_paths_unaligned_and_ragged(dev):
    """Pointers that are not 16-byte aligned and axis views with inner % 4 != 0
    take the element-wise code paths; results stay bit-exact."""
    rng = np.random.default_rng(42)
    x = (rng.normal(size=4099) * 100).astype(np.float32)
    xd = to_dev(np.concatenate([[0.0], x]).astype(np.float32), dev)[1:]  # 4-byte aligned, not 16
    assert xd.data_ptr() % 16 != 0
    got = capi.cast(xd, F, E5).cpu().numpy()
    assert np.array_equal(got, oracle.e5m2_from_float(x))
    codes = rng.integers(0, 256, 4099, dtype=np.uint8)
    cd = to_dev(np.concatenate([[0], codes]).astype(np.uint8), dev)[1:]  # odd address
    assert f32_equal(capi.cast(cd, E5, F).cpu().numpy(), oracle.e5m2_decode_table()[codes])
    # per-axis E5M2 with inner = 3 (no groups of four share a scale)
    xs = (rng.normal(size=(5, 7, 3)) * 50).astype(np.float32)
    s = (rng.random(7) + 0.1).astype(np.float32)
    q = capi.quantize_e5m2(to_dev(xs, dev), to_dev(s, dev), axis=1).cpu().numpy()
    assert np.array_equal(q, oracle.quantize_e5m2(xs, s, axis=1))
    assert f32_equal(capi.dequantize_e5m2(to_dev(q, dev), to_dev(s, dev), axis=1).cpu().numpy(),
                     oracle.dequantize_e5m2(q, s, axis=1))


def test_binary_eight_dims_and_unaligned_fp32(dev):
    rng = np.random.default_rng(8)
    sa, sb = (2, 1, 3, 1, 2, 1, 2, 3), (1, 2, 1, 2, 1, 3, 1, 1)
    for dtype in (F, E4, E5):
        if dtype == F:
            a = rng.normal(size=sa).astype(np.float32)
            b = rng.normal(size=sb).astype(np.float32)
        else:
            a = rng.integers(0, 256, size=sa, dtype=np.uint8)
            b = rng.integers(0, 256, size=sb, dtype=np.uint8)
        got = capi.binary(capi.BINARY_MUL, to_dev(a, dev), to_dev(b, dev), dtype).cpu().numpy()
        ref = oracle.fp8_binary(capi.BINARY_MUL, dtype, a, b)
        assert (f32_equal(got, ref) if dtype == F else np.array_equal(got, ref)), dtype
    # same-shape fp32 operands at 4-byte (not 16-byte) alignment: element path
    a = rng.normal(size=1031).astype(np.float32)
    b = rng.normal(size=1031).astype(np.float32)
    ad = to_dev(np.concatenate([[0.0], a]).astype(np.float32), dev)[1:]
    bd = to_dev(np.concatenate([[0.0], b]).astype(np.float32), dev)[1:]
    got = capi.binary(capi.BINARY_DIV, ad, bd, F).cpu().numpy()
    assert f32_equal(got, oracle.fp8_binary(capi.BINARY_DIV, F, a, b))
