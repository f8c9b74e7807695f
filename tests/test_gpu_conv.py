"""GPU parity of the FP8 convolution path: NHWC quantisation, conv weight
packing, and the implicit-im2col conv kernel, against the oracle's direct
NCHW convolution (reference src/onnx/operators/conv.cpp:115-207: begin pads,
dilation, reduction over kh, kw, channels) applied to the dequantised
operands (the QDQ composition DQ(x), DQ(W) -> Conv).

Bars: codes and packing bit-exact; conv outputs elementwise within
1e-4 * sum |x*w| (+ the activation's Lipschitz slack) and relative Frobenius
1e-5, as for the GEMM."""
import numpy as np
import pytest
import torch

import oracle
from luisaml_amd import capi, synth
from tests.gemm_cases import assert_close

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def conv_case(n, c, h, w, cout, kh, kw, seed, dev, per_channel=True, group=1):
    x = synth.normal(seed, (n, c, h, w))
    wt = synth.normal(seed + 1, (cout, c // group, kh, kw), std=0.03)
    ws = oracle.channel_scales(wt.reshape(cout, -1), 0) if per_channel else \
        np.array([oracle.dynamic_scale(wt)], np.float32)
    qw = oracle.quantize(wt.reshape(cout, -1), ws, axis=0).reshape(wt.shape) if per_channel else \
        oracle.quantize(wt, ws)
    return x, qw, ws


@pytest.mark.parametrize("shape", [(2, 16, 9, 11), (1, 100, 5, 7), (3, 64, 56, 56)])
@pytest.mark.parametrize("dynamic", [True, False])
def test_quantize_nhwc(dev, shape, dynamic):
    x = synth.normal(sum(shape), shape, std=2.0)
    x[0, 1, 2, 3] = np.nan
    x[-1, -1, -1, -1] = -0.0
    xd = to_dev(x, dev)
    if dynamic:
        y, s = capi.quantize_nhwc(xd)
        s_ref = np.float32(oracle.dynamic_scale(x))
        assert s.cpu().numpy().view(np.uint32)[0] == s_ref.view(np.uint32)
    else:
        s_ref = np.float32(0.0113)
        y, s = capi.quantize_nhwc(xd, torch.tensor([s_ref], device=dev))
    ref = oracle.quantize(x, s_ref).transpose(0, 2, 3, 1)
    assert np.array_equal(y.cpu().numpy(), ref)


@pytest.mark.parametrize("cout,cin,kh,kw", [(256, 256, 3, 3), (20, 16, 3, 3), (33, 48, 5, 5), (64, 32, 1, 1)])
def test_pack_conv_weight_layout(dev, cout, cin, kh, kw):
    rng = np.random.default_rng(cout + cin)
    q = rng.integers(0, 256, size=(cout, cin, kh, kw), dtype=np.uint8)
    p = capi.pack_conv_weight(to_dev(q, dev))
    K = kh * kw * cin
    back = capi.unpack_weight(p, K, cout, w_is_nk=True).cpu().numpy()  # [cout, K]
    assert np.array_equal(back, q.transpose(0, 2, 3, 1).reshape(cout, K))
    # grouped: block g is group g's [K_g, cout/group] packed weight
    for group in (2, 4):
        if cout % group or cin % group:
            continue
        qg = np.ascontiguousarray(q[:, : cin // group])
        pg = capi.pack_conv_weight(to_dev(qg, dev), group=group)
        Kg, Mg = kh * kw * (cin // group), cout // group
        gb = capi.packed_weight_bytes(Kg, Mg)
        assert pg.numel() == group * gb
        for gi in range(group):
            back = capi.unpack_weight(pg[gi * gb:(gi + 1) * gb], Kg, Mg, w_is_nk=True).cpu().numpy()
            assert np.array_equal(back, qg[gi * Mg:(gi + 1) * Mg].transpose(0, 2, 3, 1).reshape(Mg, Kg))


CASES = [  # n, c, h, w, cout, kh, kw, stride, pad, dilation
    (2, 16, 9, 11, 20, 3, 3, 1, 1, 1),
    (1, 32, 8, 8, 64, 1, 1, 1, 0, 1),
    (2, 48, 13, 10, 33, 5, 5, 1, 2, 1),
    (1, 32, 15, 15, 40, 3, 3, 2, 1, 1),
    (1, 16, 17, 17, 24, 3, 3, 1, 2, 2),
    (2, 64, 14, 14, 256, 3, 3, 1, 1, 1),
    (1, 256, 12, 12, 256, 3, 3, 1, 1, 1),
]


def reference(x, qw, ws, bias, stride, pad, dil, act, per_channel=True, group=1):
    s = np.float32(oracle.dynamic_scale(x))
    xq = oracle.quantize(x, s)
    A = oracle.dequantize(xq, s)
    cout = qw.shape[0]
    B = oracle.dequantize(qw.reshape(cout, -1), ws, axis=0).reshape(qw.shape) if ws.size > 1 else \
        oracle.dequantize(qw, ws)
    st, pd, dl = (stride, stride), (pad, pad), (dil, dil)
    Y = oracle.conv2d(A, B, bias, strides=st, pads=pd, dilations=dl, group=group, act=act)
    bound = oracle.conv2d(np.abs(A), np.abs(B), None if bias is None else np.abs(bias), strides=st, pads=pd,
                          dilations=dl, group=group)
    return Y, bound


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("act", [capi.ACT_NONE, capi.ACT_RELU])
@pytest.mark.parametrize("kernel", [capi.KERNEL_AUTO, capi.KERNEL_MFMA, capi.KERNEL_MFMA_128])
def test_conv_matches_oracle(dev, case, act, kernel):
    n, c, h, w, cout, kh, kw, stride, pad, dil = case
    x, qw, ws = conv_case(n, c, h, w, cout, kh, kw, seed=n * 7 + c + cout, dev=dev)
    bias = synth.normal(77, (cout,), std=0.01)
    xq, sx = capi.quantize_nhwc(to_dev(x, dev))
    y = capi.conv2d(xq, sx, capi.pack_conv_weight(to_dev(qw, dev)), to_dev(ws, dev), cout, (kh, kw),
                    (stride, stride), (pad, pad), (dil, dil), bias=to_dev(bias, dev), act=act, kernel=kernel)
    ref, bound = reference(x, qw, ws, bias, stride, pad, dil, act)
    assert y.shape == ref.shape
    assert_close(y.cpu().numpy(), ref, bound, act=act)


@pytest.mark.parametrize("case", [(2, 32, 9, 11, 24, 3, 3, 1, 1, 1, 2), (1, 64, 10, 10, 64, 3, 3, 2, 1, 1, 4),
                                  (1, 48, 8, 8, 30, 1, 1, 1, 0, 1, 3), (2, 128, 7, 7, 256, 3, 3, 1, 2, 2, 8)])
@pytest.mark.parametrize("kernel", [capi.KERNEL_MFMA, capi.KERNEL_MFMA_FP8, capi.KERNEL_MFMA_128,
                                    capi.KERNEL_MFMA_128_FP8])
def test_grouped_conv_matches_oracle(dev, case, kernel):
    """Grouped FP8 conv: each group's GEMM reads its channel slice and writes
    its output-channel slice (conv.cpp:139,158)."""
    n, c, h, w, cout, kh, kw, stride, pad, dil, group = case
    x, qw, ws = conv_case(n, c, h, w, cout, kh, kw, seed=c + cout + group, dev=dev, group=group)
    bias = synth.normal(78, (cout,), std=0.01)
    xq, sx = capi.quantize_nhwc(to_dev(x, dev))
    y = capi.conv2d(xq, sx, capi.pack_conv_weight(to_dev(qw, dev), group=group), to_dev(ws, dev), cout, (kh, kw),
                    (stride, stride), (pad, pad), (dil, dil), bias=to_dev(bias, dev), act=capi.ACT_RELU,
                    kernel=kernel, group=group)
    ref, bound = reference(x, qw, ws, bias, stride, pad, dil, capi.ACT_RELU, group=group)
    if kernel in (capi.KERNEL_MFMA, capi.KERNEL_MFMA_128):
        assert_close(y.cpu().numpy(), ref, bound, act=capi.ACT_RELU)
    else:
        rel = np.linalg.norm(y.cpu().numpy() - ref) / np.linalg.norm(ref)
        assert rel < 3e-5


def test_conv_bf16_out_and_per_tensor_weight_scale(dev):
    n, c, h, w, cout, k = 2, 32, 10, 10, 48, 3
    x, qw, ws = conv_case(n, c, h, w, cout, k, k, seed=5, dev=dev, per_channel=False)
    xq, sx = capi.quantize_nhwc(to_dev(x, dev))
    bp = capi.pack_conv_weight(to_dev(qw, dev))
    y32 = capi.conv2d(xq, sx, bp, to_dev(ws, dev), cout, (k, k), pads=(1, 1))
    y16 = capi.conv2d(xq, sx, bp, to_dev(ws, dev), cout, (k, k), pads=(1, 1), out_dtype=torch.bfloat16)
    ref, bound = reference(x, qw, ws, None, 1, 1, 1, capi.ACT_NONE)
    assert_close(y32.cpu().numpy(), ref, bound)
    assert np.array_equal(y16.view(torch.int16).cpu().numpy().view(np.uint16), oracle.bf16_rne(y32.cpu().numpy()))


@pytest.mark.parametrize("act", [capi.ACT_GELU_ERF, capi.ACT_GELU_TANH])
@pytest.mark.parametrize("with_bias", [True, False])
def test_conv_gelu_epilogue(dev, act, with_bias):
    """The NCHW epilogue specialised per activation, bias and output type:
    GELU with and without bias against the oracle, bf16 = bf16_rne of fp32."""
    n, c, h, w, cout, k = 2, 32, 11, 9, 40, 3
    x, qw, ws = conv_case(n, c, h, w, cout, k, k, seed=act * 5 + with_bias, dev=dev)
    bias = synth.normal(79, (cout,), std=0.01) if with_bias else None
    xq, sx = capi.quantize_nhwc(to_dev(x, dev))
    bp = capi.pack_conv_weight(to_dev(qw, dev))
    d_bias = None if bias is None else to_dev(bias, dev)
    y32 = capi.conv2d(xq, sx, bp, to_dev(ws, dev), cout, (k, k), pads=(1, 1), bias=d_bias, act=act)
    y16 = capi.conv2d(xq, sx, bp, to_dev(ws, dev), cout, (k, k), pads=(1, 1), bias=d_bias, act=act,
                      out_dtype=torch.bfloat16)
    ref, bound = reference(x, qw, ws, bias, 1, 1, 1, act)
    assert_close(y32.cpu().numpy(), ref, bound, act=act)
    assert np.array_equal(y16.view(torch.int16).cpu().numpy().view(np.uint16), oracle.bf16_rne(y32.cpu().numpy()))


def test_conv_native_fp8_close(dev):
    n, c, h, w, cout, k = 1, 64, 14, 14, 64, 3
    x, qw, ws = conv_case(n, c, h, w, cout, k, k, seed=9, dev=dev)
    xq, sx = capi.quantize_nhwc(to_dev(x, dev))
    bp = capi.pack_conv_weight(to_dev(qw, dev))
    y = capi.conv2d(xq, sx, bp, to_dev(ws, dev), cout, (k, k), pads=(1, 1), kernel=capi.KERNEL_MFMA_FP8)
    ref, _ = reference(x, qw, ws, None, 1, 1, 1, capi.ACT_NONE)
    rel = np.linalg.norm(y.cpu().numpy() - ref) / np.linalg.norm(ref)
    assert rel < 3e-5


def test_conv_errors(dev):
    xq = torch.zeros((1, 4, 4, 8), dtype=torch.uint8, device=dev)  # c = 8: not a multiple of 16
    s = torch.ones(1, device=dev)
    bp = capi.pack_conv_weight(torch.zeros((4, 8, 3, 3), dtype=torch.uint8, device=dev))
    with pytest.raises(capi.LcmlError):
        capi.conv2d(xq, s, bp, s, 4, (3, 3), pads=(1, 1))
    xq = torch.zeros((1, 4, 4, 32), dtype=torch.uint8, device=dev)  # 32 channels in 4 groups: 8 per group
    bp = capi.pack_conv_weight(torch.zeros((8, 8, 3, 3), dtype=torch.uint8, device=dev), group=4)
    with pytest.raises(capi.LcmlError):
        capi.conv2d(xq, s, bp, s, 8, (3, 3), pads=(1, 1), group=4)
    with pytest.raises(capi.LcmlError):  # group must divide cout
        capi.conv2d(xq, s, bp, s, 6, (3, 3), pads=(1, 1), group=4)


@pytest.mark.parametrize("case", [(2, 6, 9, 11, 8, 3, 3, 1, 1, 1, 1), (1, 8, 12, 12, 12, 3, 3, 2, 1, 1, 2),
                                  (1, 4, 10, 10, 6, 5, 5, 1, 2, 2, 1), (2, 16, 7, 7, 16, 1, 1, 1, 0, 1, 4)])
@pytest.mark.parametrize("act", [capi.ACT_NONE, capi.ACT_RELU])
def test_conv_f32_matches_oracle(dev, case, act):
    """The plain fp32 Conv (groups, strides, dilation) against the oracle."""
    n, c, h, w, cout, kh, kw, stride, pad, dil, group = case
    x = synth.normal(c + h, (n, c, h, w))
    wt = synth.normal(cout + kh, (cout, c // group, kh, kw), std=0.2)
    b = synth.normal(3, (cout,), std=0.1)
    st, pd, dl = (stride, stride), (pad, pad), (dil, dil)
    y = capi.conv2d_f32(to_dev(x, dev), to_dev(wt, dev), to_dev(b, dev), st, pd, dl, group, act=act)
    ref = oracle.conv2d(x, wt, b, strides=st, pads=pd, dilations=dl, group=group, act=act)
    bound = oracle.conv2d(np.abs(x), np.abs(wt), np.abs(b), strides=st, pads=pd, dilations=dl, group=group)
    assert_close(y.cpu().numpy(), ref, bound, act=act)
