"""GPU parity of QuantizeLinear / DequantizeLinear / amax / weight packing.

Bar: bit-exact against the oracle (oracle/lcml_oracle.c, which restates the
reference E4M3 codec include/onnx/fp_quantized.h:149-249).  NaN results are
compared as NaN (IEEE leaves the payload of a NaN produced by arithmetic
unspecified); every non-NaN result is compared bit for bit.
"""
import numpy as np
import pytest
import torch

import oracle
from luisaml_amd import capi, synth

pytestmark = pytest.mark.gpu


def assert_bits_equal_nan_aware(got: np.ndarray, ref: np.ndarray):
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    gn, rn = np.isnan(got), np.isnan(ref)
    assert np.array_equal(gn, rn), f"NaN positions differ at {np.flatnonzero(gn != rn)[:8]}"
    m = ~rn
    bad = np.flatnonzero(got[m].view(np.uint32) != ref[m].view(np.uint32))
    assert bad.size == 0, f"{bad.size} mismatches, first at {bad[:8]}: {got[m][bad[:4]]} vs {ref[m][bad[:4]]}"


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_decode_all_256_codes(dev):
    q = torch.arange(256, dtype=torch.uint8, device=dev)
    y = capi.dequantize(q, torch.ones(1, device=dev)).cpu().numpy()
    assert_bits_equal_nan_aware(y, oracle.e4m3_decode_table())


def _int32_bits(first, count, dev):
    b = torch.arange(first, first + count, dtype=torch.int64, device=dev)
    b = torch.where(b >= 2**31, b - 2**32, b)
    return b.to(torch.int32)


def test_quantize_exhaustive_all_fp32_patterns(dev):
    """Every one of the 2^32 fp32 bit patterns through lcml_fp8_quantize with
    scale 1 (x / 1 == x exactly), against the oracle encoder."""
    chunk = 1 << 28
    one = torch.ones(1, device=dev)
    y = torch.empty(chunk, dtype=torch.uint8, device=dev)
    for c in range((1 << 32) // chunk):
        first = c * chunk
        x = _int32_bits(first, chunk, dev).view(torch.float32)
        capi.quantize(x, one, out=y)
        got = y.cpu().numpy()
        ref = oracle.e4m3_encode_bits(first, chunk)
        if not np.array_equal(got, ref):
            i = int(np.flatnonzero(got != ref)[0])
            pytest.fail(f"pattern 0x{first + i:08x}: gpu 0x{got[i]:02x} oracle 0x{ref[i]:02x}")
        del x


@pytest.mark.parametrize("scale", [0.0137, 1.0 / 448.0])
def test_quantize_exhaustive_all_fp32_patterns_scaled(dev, scale):
    """Every fp32 bit pattern through lcml_fp8_quantize with a non-trivial
    per-tensor scale: the kernel's reciprocal division + hardware conversion
    against the oracle's IEEE x / s + encoder."""
    chunk = 1 << 28
    sd = torch.tensor([scale], dtype=torch.float32, device=dev)
    y = torch.empty(chunk, dtype=torch.uint8, device=dev)
    s32 = np.float32(scale)
    base = np.arange(chunk, dtype=np.uint32)
    bits = np.empty(chunk, dtype=np.uint32)
    for c in range((1 << 32) // chunk):
        first = c * chunk
        x = _int32_bits(first, chunk, dev).view(torch.float32)
        capi.quantize(x, sd, out=y)
        got = y.cpu().numpy()
        np.add(base, np.uint32(first), out=bits)
        ref = oracle.quantize(bits.view(np.float32), s32)
        if not np.array_equal(got, ref):
            i = int(np.flatnonzero(got != ref)[0])
            pytest.fail(f"scale {scale}: pattern 0x{first + i:08x}: gpu 0x{got[i]:02x} oracle 0x{ref[i]:02x}")
        del x


@pytest.mark.parametrize("n", [0, 1, 15, 16, 17, 1000, 4096, 65537, 1 << 20])
@pytest.mark.parametrize("offset", [0, 1])
def test_quantize_per_tensor(dev, n, offset):
    x = synth.normal(11 + n, (n + offset,), std=3.0)
    # salt in specials
    if n >= 16:
        x[offset + 3] = np.inf
        x[offset + 5] = -np.inf
        x[offset + 7] = np.nan
        x[offset + 9] = -0.0
        x[offset + 11] = 1e-30
        x[offset + 13] = -1e-30
    s = np.float32(0.0137)
    xv = to_dev(x, dev)[offset:]  # offset 1: a 4-byte-misaligned view takes the scalar path
    y = torch.empty(n, dtype=torch.uint8, device=dev)
    if n:
        rc = capi.lib().lcml_fp8_quantize(xv.data_ptr(), y.data_ptr(), 1, 1, n,
                                          to_dev(np.array([s], np.float32), dev).data_ptr(),
                                          torch.cuda.current_stream().cuda_stream)
        assert rc == 0, capi.last_error()
    got = y.cpu().numpy()
    ref = oracle.quantize(x[offset:], s)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("shape,axis", [((64, 96), 0), ((64, 96), 1), ((3, 40, 7), 1), ((128, 4096), 0),
                                        ((4096, 1024), 1), ((5, 33), 1)])
def test_quantize_dequantize_per_axis(dev, shape, axis):
    x = synth.normal(5, shape, std=0.7)
    scales = oracle.channel_scales(x, axis)
    q = capi.quantize(to_dev(x, dev), to_dev(scales, dev), axis=axis)
    ref_q = oracle.quantize(x, scales, axis=axis)
    assert np.array_equal(q.cpu().numpy(), ref_q)
    y = capi.dequantize(q, to_dev(scales, dev), axis=axis).cpu().numpy()
    assert_bits_equal_nan_aware(y, oracle.dequantize(ref_q, scales, axis=axis))


# 3 << 20 and up: the two-pass path; 9 << 20 + 3108 walks several grid
# strides with a ragged last chunk in the encode pass's reversed order,
# 4096 * 4096 is a transformer linear's input
@pytest.mark.parametrize("n", [1, 100, 4096, 16 * 4096, 65536, 65537, 3 << 20, (9 << 20) + 3108, 4096 * 4096])
def test_quantize_dynamic_matches_oracle(dev, n):
    x = synth.normal(99 + n, (n,), std=2.5)
    q, s = capi.quantize_dynamic(to_dev(x, dev))
    s_ref = oracle.dynamic_scale(x)
    assert s.cpu().numpy().view(np.uint32)[0] == np.float32(s_ref).view(np.uint32)
    assert np.array_equal(q.cpu().numpy(), oracle.quantize(x, s_ref))


@pytest.mark.parametrize("n", [10, 70000])
def test_quantize_dynamic_edge_scales(dev, n):
    # all zeros: amax 0 -> scale 1
    z = torch.zeros(n, device=dev)
    q, s = capi.quantize_dynamic(z)
    assert float(s.item()) == 1.0 and int(q.max()) == 0
    # an inf: amax inf -> scale 1, inf saturates
    x = synth.normal(3, (n,))
    x[n // 2] = np.inf
    x[1] = np.nan
    q, s = capi.quantize_dynamic(to_dev(x, dev))
    assert float(s.item()) == 1.0
    assert np.array_equal(q.cpu().numpy(), oracle.quantize(x, 1.0))
    # NaN ignored by amax
    x = synth.normal(4, (n,))
    x[7] = np.nan
    q, s = capi.quantize_dynamic(to_dev(x, dev))
    s_ref = oracle.dynamic_scale(x)
    assert float(s.item()) == s_ref
    assert np.array_equal(q.cpu().numpy(), oracle.quantize(x, s_ref))


def test_amax(dev):
    x = synth.normal(8, (1 << 20,), std=4.0)
    x[12345] = -77.5
    x[99] = np.nan
    a = capi.amax(to_dev(x, dev)).item()
    assert a == oracle.amax(x) == 77.5


@pytest.mark.parametrize("K,N", [(128, 64), (784, 256), (256, 10), (4096, 11008), (100, 70), (2304, 256)])
@pytest.mark.parametrize("w_is_nk", [False, True])
def test_pack_roundtrip_and_layout(dev, K, N, w_is_nk):
    rng = np.random.default_rng(K * 7 + N)
    w = rng.integers(0, 256, size=(N, K) if w_is_nk else (K, N), dtype=np.uint8)
    wd = to_dev(w, dev)
    p = capi.pack_weight(wd, w_is_nk)
    Kp, Np = -(-K // 128) * 128, -(-N // 64) * 64
    assert p.numel() == Kp * Np
    back = capi.unpack_weight(p, K, N, w_is_nk).cpu().numpy()
    assert np.array_equal(back, w)
    pc = p.cpu().numpy()
    # padding is zero and a sample of bytes sits where the layout says
    wk = w.T if w_is_nk else w  # logical [K, N]
    full = np.zeros((Kp, Np), np.uint8)
    full[:K, :N] = wk
    ks = rng.integers(0, Kp, 2000)
    ns = rng.integers(0, Np, 2000)
    idx = ((ns // 64) * (Kp // 16) + ks // 16) * 1024 + (ns % 64) * 16 + ks % 16
    assert np.array_equal(pc[idx], full[ks, ns])
    assert int(pc.astype(np.int64).sum()) == int(wk.astype(np.int64).sum())
