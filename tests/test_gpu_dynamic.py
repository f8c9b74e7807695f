"""GPU parity of the one-call dynamically quantised linear
(lcml_fp8_gemm_dynamic) and of the reciprocal-division quantiser.

Bars:
  * the dynamic scale and every quantised activation are bit-exact with the
    oracle (DynamicQuantizeLinear = amax/448, then the reference E4M3 encoder
    of include/onnx/fp_quantized.h:149-223 on x / s);
  * the fused kernel's output is bit-identical to the two-call composition
    lcml_fp8_quantize_dynamic + lcml_fp8_gemm (same kernels' arithmetic, same
    summation order), and within the GEMM tolerance of the oracle's
    dequantise-then-Gemm (gemm.cpp:27-325).
"""
import numpy as np
import pytest
import torch

import oracle
from luisaml_amd import capi, synth
from tests.gemm_cases import assert_close

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def weights(K, N, seed, dev, per_channel=True):
    w = synth.normal(seed, (K, N), std=0.02)
    sw = oracle.channel_scales(w, 1) if per_channel else np.array([oracle.dynamic_scale(w)], np.float32)
    qw = oracle.quantize(w, sw, axis=1) if per_channel else oracle.quantize(w, sw)
    return qw, sw, capi.pack_weight(to_dev(qw, dev), False), to_dev(sw, dev)


def two_step(x_d, bp, d_sw, N, K, kernel, **kw):
    q, s = capi.quantize_dynamic(x_d)
    return capi.gemm(q, s, bp, d_sw, N, K, kernel=kernel, **kw), q, s


# every count of activation slots per lane (1, 2, 4, 8) and partly used
# slots (odd M; rows past M in a slot's upper half-wave)
@pytest.mark.parametrize("M", [1, 2, 3, 4, 7, 9, 13, 16])
@pytest.mark.parametrize("N,K", [(11008, 4096), (320, 272), (100, 784), (4096, 5888)])
@pytest.mark.parametrize("kernel", [capi.KERNEL_AUTO, capi.KERNEL_SKINNY, capi.KERNEL_SKINNY_FP8])
def test_fused_matches_two_step_and_oracle(dev, M, N, K, kernel):
    x = synth.normal(1000 + M + K, (M, K), std=1.5)
    qw, sw, bp, d_sw = weights(K, N, 7 + N, dev)
    x_d = to_dev(x, dev)
    s_out = torch.empty(1, dtype=torch.float32, device=dev)
    y = capi.gemm_dynamic(x_d, bp, d_sw, N, K, kernel=kernel, scale_out=s_out)
    ref_kernel = capi.KERNEL_SKINNY if kernel == capi.KERNEL_AUTO else kernel
    y2, q2, s2 = two_step(x_d, bp, d_sw, N, K, ref_kernel)
    torch.cuda.synchronize()
    s_ref = np.float32(oracle.dynamic_scale(x))
    assert s_out.cpu().numpy().view(np.uint32)[0] == s_ref.view(np.uint32)
    assert np.array_equal(q2.cpu().numpy(), oracle.quantize(x, s_ref))
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32)), "fused and two-step outputs differ"
    if kernel != capi.KERNEL_SKINNY_FP8:
        ref, A, B = oracle.qlinear(oracle.quantize(x, s_ref), s_ref, qw, sw)
        assert_close(y.cpu().numpy(), ref, oracle.gemm_abs_bound(A, B))


@pytest.mark.parametrize("act", [capi.ACT_NONE, capi.ACT_RELU, capi.ACT_GELU_ERF, capi.ACT_GELU_TANH])
def test_fused_epilogue_bias_act_bf16(dev, act):
    M, N, K = 4, 1000, 1024
    x = synth.normal(3, (M, K))
    qw, sw, bp, d_sw = weights(K, N, 4, dev)
    bias = synth.normal(5, (N,), std=0.01)
    x_d = to_dev(x, dev)
    for dt in (torch.float32, torch.bfloat16):
        y = capi.gemm_dynamic(x_d, bp, d_sw, N, K, c=to_dev(bias, dev), act=act, out_dtype=dt, alpha=0.75)
        y2, _, _ = two_step(x_d, bp, d_sw, N, K, capi.KERNEL_SKINNY, c=to_dev(bias, dev), act=act, out_dtype=dt,
                            alpha=0.75)
        assert torch.equal(y.view(torch.int16 if dt == torch.bfloat16 else torch.int32),
                           y2.view(torch.int16 if dt == torch.bfloat16 else torch.int32))


def test_fused_row_pitch_and_specials(dev):
    """ldx > K (rows of a wider buffer), NaN / inf / zeros in x."""
    M, N, K, ldx = 5, 256, 512, 640
    big = synth.normal(9, (M, ldx))
    big[1, 7] = np.nan
    big[3, 100] = -0.0
    big[2, 5] = 1e-38
    qw, sw, bp, d_sw = weights(K, N, 10, dev)
    d_big = to_dev(big, dev)
    x_view = d_big[:, :K]
    s_out = torch.empty(1, dtype=torch.float32, device=dev)
    y = capi.gemm_dynamic(x_view, bp, d_sw, N, K, scale_out=s_out)
    y2, _, s2 = two_step(x_view.contiguous(), bp, d_sw, N, K, capi.KERNEL_SKINNY)
    assert float(s_out.item()) == float(s2.item()) == np.float32(oracle.dynamic_scale(big[:, :K]))
    assert torch.equal(y.view(torch.int32)[~torch.isnan(y)], y2.view(torch.int32)[~torch.isnan(y2)])
    assert torch.equal(torch.isnan(y), torch.isnan(y2))
    # an inf: amax inf -> scale 1
    big[4, 9] = np.inf
    d_big = to_dev(big, dev)
    y = capi.gemm_dynamic(d_big[:, :K], bp, d_sw, N, K, scale_out=s_out)
    assert float(s_out.item()) == 1.0
    # all zeros: scale 1, output = bias-free zero
    z = torch.zeros((3, K), device=dev)
    y = capi.gemm_dynamic(z, bp, d_sw, N, K, scale_out=s_out)
    assert float(s_out.item()) == 1.0 and float(y.abs().max()) == 0.0


@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("big", [448.0, 3.0e5, 2.0e13])
def test_fused_finite_input_tiny_and_signed_zero_quotients(dev, M, big):
    """Finite inputs (no NaN, no inf) take the fused kernel's lean encode;
    its results equal the two-launch composition bit for bit, including
    quotients below 2^-100 (subnormal and tiny normal x against a large
    amax, which take the IEEE-division fallback), +-0, the smallest
    subnormals, values at the amax and ties of the E4M3 grid."""
    K, N = 1024, 320
    rng = np.random.default_rng(int(big) % 1000 + M)
    x = (rng.standard_normal((M, K)) * (big / 8.0)).astype(np.float32)
    flat = x.reshape(-1)
    specials = np.array([big, -big, 0.0, -0.0, 1e-40, -1e-40, 2.0 ** -149, -(2.0 ** -149), 1e-30, -1e-30,
                         2.0 ** -100, -(2.0 ** -126), big * (1.0625 / 448.0), -big * (1.1875 / 448.0)], np.float32)
    idx = rng.choice(flat.size, specials.size, replace=False)
    flat[idx] = specials
    qw, sw, bp, d_sw = weights(K, N, 11, dev)
    x_d = to_dev(x, dev)
    s_out = torch.empty(1, dtype=torch.float32, device=dev)
    y = capi.gemm_dynamic(x_d, bp, d_sw, N, K, scale_out=s_out, kernel=capi.KERNEL_SKINNY)
    y2, q2, s2 = two_step(x_d, bp, d_sw, N, K, capi.KERNEL_SKINNY)
    torch.cuda.synchronize()
    s_ref = np.float32(oracle.dynamic_scale(x))
    assert s_out.cpu().numpy().view(np.uint32)[0] == s_ref.view(np.uint32)
    assert np.array_equal(q2.cpu().numpy(), oracle.quantize(x, s_ref))
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))


@pytest.mark.parametrize("M,kernel", [(64, capi.KERNEL_AUTO), (4, capi.KERNEL_MFMA), (300, capi.KERNEL_MFMA_FP8),
                                      (16, capi.KERNEL_VALU)])
def test_workspace_path(dev, M, kernel):
    N, K = 384, 1024
    x = synth.normal(20 + M, (M, K))
    qw, sw, bp, d_sw = weights(K, N, 21, dev)
    x_d = to_dev(x, dev)
    assert capi.lib().lcml_fp8_gemm_dynamic_workspace_bytes(M, K, kernel) > 0
    y = capi.gemm_dynamic(x_d, bp, d_sw, N, K, kernel=kernel)
    y2, _, _ = two_step(x_d, bp, d_sw, N, K, kernel)
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))


def test_fused_limits_and_errors(dev):
    K = 8192
    ws = capi.lib().lcml_fp8_gemm_dynamic_workspace_bytes
    assert ws(4, 4096, capi.KERNEL_AUTO) == 0 and ws(16, 4096, capi.KERNEL_SKINNY) == 0
    assert ws(8, 4096, capi.KERNEL_AUTO) > 0  # AUTO: the separate quantise kernel is cheaper
    assert ws(16, K, capi.KERNEL_SKINNY) > 0  # LDS copy too large
    qw, sw, bp, d_sw = weights(K, 64, 30, dev)
    x = to_dev(synth.normal(31, (16, K)), dev)
    y = capi.gemm_dynamic(x, bp, d_sw, 64, K, kernel=capi.KERNEL_SKINNY)  # falls back to the workspace path
    y2, _, _ = two_step(x, bp, d_sw, 64, K, capi.KERNEL_SKINNY)
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))
    with pytest.raises(capi.LcmlError):  # missing workspace on the two-step path
        rc = capi.lib().lcml_fp8_gemm_dynamic(16, 64, K, x.data_ptr(), K, bp.data_ptr(), d_sw.data_ptr(), 1, 1.0,
                                             None, 0, 0, 0, 1.0, 0, y.data_ptr(), 1, 64, None, None, 0,
                                             capi.KERNEL_SKINNY, torch.cuda.current_stream().cuda_stream)
        capi._check(rc)


@pytest.mark.parametrize("mag", [1e-25, 1e-3, 3e17, 1e30])
def test_fused_scale_outside_fast_range(dev, mag):
    """Activations so small or large that the scale leaves the reciprocal
    fast path's range: the fused kernel's encode takes the exact-division
    form and still matches the two-call composition and the oracle."""
    M, N, K = 6, 192, 400
    x = (synth.normal(40, (M, K)) * np.float32(mag)).astype(np.float32)
    qw, sw, bp, d_sw = weights(K, N, 41, dev)
    x_d = to_dev(x, dev)
    s_out = torch.empty(1, dtype=torch.float32, device=dev)
    y = capi.gemm_dynamic(x_d, bp, d_sw, N, K, kernel=capi.KERNEL_SKINNY, scale_out=s_out)
    y2, q2, s2 = two_step(x_d, bp, d_sw, N, K, capi.KERNEL_SKINNY)
    s_ref = np.float32(oracle.dynamic_scale(x))
    assert s_out.cpu().numpy().view(np.uint32)[0] == s_ref.view(np.uint32)
    assert np.array_equal(q2.cpu().numpy(), oracle.quantize(x, s_ref))
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))


SCALES = [1.0, 0.0137, 1 / 448, 3.3e-3, 0.7, 5.5, 123.25, 2.0 ** -59, 2.0 ** 39, 1e-30, 3e20, 6.1e-5]


@pytest.mark.parametrize("s", SCALES)
def test_quantize_random_bit_patterns_many_scales(dev, s):
    """Per-tensor QuantizeLinear of 2^22 random fp32 bit patterns (every
    exponent, NaN, inf, subnormals) with scales inside and outside the
    reciprocal-division range, against the oracle's IEEE x / s + encoder."""
    rng = np.random.default_rng(int(s * 1e6) % 2**32)
    bits = rng.integers(0, 2**32, size=1 << 22, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    sd = torch.tensor([s], dtype=torch.float32, device=dev)
    got = capi.quantize(to_dev(x, dev), sd).cpu().numpy()
    ref = oracle.quantize(x, np.float32(s))
    bad = np.flatnonzero(got != ref)
    assert bad.size == 0, f"{bad.size} mismatches, first x=0x{bits[bad[0]]:08x}: {got[bad[0]]:#x} vs {ref[bad[0]]:#x}"


@pytest.mark.parametrize("s", [0.0137, 1 / 448, 0.7, 123.25])
def test_quantize_near_rounding_boundaries(dev, s):
    """x chosen so that x / s lands on and next to every E4M3 rounding
    midpoint and code value (where a wrongly rounded quotient would flip the
    code)."""
    codes = oracle.e4m3_decode_table()[:0x7f].astype(np.float64)
    mids = (codes[1:] + codes[:-1]) / 2
    targets = np.concatenate([codes, mids, -codes, -mids])
    xs = []
    for t in targets:
        base = np.float32(t * s)
        u = np.array([base], np.float32).view(np.uint32)[0]
        for d in range(-3, 4):
            xs.append(np.array([np.uint32(int(u) + d if int(u) + d >= 0 else u)], np.uint32).view(np.float32)[0])
    x = np.array(xs, np.float32)
    sd = torch.tensor([s], dtype=torch.float32, device=dev)
    got = capi.quantize(to_dev(x, dev), sd).cpu().numpy()
    assert np.array_equal(got, oracle.quantize(x, np.float32(s)))
