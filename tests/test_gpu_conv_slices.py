"""Row slices of the conv kernel's 256x256-tile layout.  On a grid of one
tile column the last round of whole tiles runs as slices of h rows (h the
rows left over 256 CUs, rounded up to 32, at least 64), each wavefront
multiplying only its own 32-row blocks.  A slice sums every output's
products in the same order as the 128x128-tile kernel, which has no slices,
so the two agree bit for bit; the batch sizes below put slices of every
height from 64 to 224 rows behind whole tiles or alone (M = batch * 56 * 56
output pixels).  The conv's semantics are those of the reference's Conv
(conv.cpp:115-207), checked against the oracle in test_gpu_conv.py and at
full size in test_gpu_fullsize.py; here one sliced batch is also checked
against the oracle on its last image, which lies in the slices."""
import numpy as np
import pytest
import torch

import oracle
from luisaml_amd import capi, synth
from tests.gemm_cases import assert_close

pytestmark = pytest.mark.gpu

# batch -> (rows of the last round per CU, rounded: the slice height on 256 CUs)
BATCHES = [1,    # 3136 rows: 49 slices of 64, no whole tiles
           7,    # 21952: 229 slices of 96 (3 blocks: 2 + 1 per wave row)
           10,   # 31360: 245 of 128
           12,   # 37632: 236 of 160 (3 + 2)
           14,   # 43904: 229 of 192
           18,   # 56448: 252 of 224 (4 + 3)
           21,   # 65856: 256 whole tiles, then 5 slices of 64
           32]   # 100352: 256 whole tiles, then 218 slices of 160


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def operands(n, c, hw, cout, dev, seed):
    x = synth.normal(seed, (n, c, hw, hw))
    wt = synth.normal(seed + 1, (cout, c, 3, 3), std=0.05)
    ws = oracle.channel_scales(wt.reshape(cout, -1), 0)
    qw = oracle.quantize(wt.reshape(cout, -1), ws, axis=0).reshape(wt.shape)
    bias = synth.normal(seed + 2, (cout,), std=0.1)
    xq, sx = capi.quantize_nhwc(to_dev(x, dev))
    return x, qw, ws, bias, xq, sx


@pytest.mark.parametrize("n", BATCHES)
@pytest.mark.parametrize("kernels", [(capi.KERNEL_MFMA, capi.KERNEL_MFMA_128),
                                     (capi.KERNEL_MFMA_FP8, capi.KERNEL_MFMA_128_FP8)])
def test_sliced_conv_matches_unsliced_bit_for_bit(dev, n, kernels):
    _, qw, ws, bias, xq, sx = operands(n, 16, 56, 256, dev, seed=900 + n)
    bp = capi.pack_conv_weight(to_dev(qw, dev))
    ys = [capi.conv2d(xq, sx, bp, to_dev(ws, dev), 256, (3, 3), pads=(1, 1), bias=to_dev(bias, dev),
                      act=capi.ACT_RELU, kernel=k) for k in kernels]
    torch.cuda.synchronize()
    assert torch.equal(ys[0].view(torch.int32), ys[1].view(torch.int32))


@pytest.mark.parametrize("out_dtype,act", [(torch.bfloat16, capi.ACT_GELU_ERF), (torch.float32, capi.ACT_NONE)])
def test_sliced_conv_ragged_columns_and_stride(dev, out_dtype, act):
    """200 output channels (a partial last 64-column panel), stride 2 on
    57x57 images: 20 * 29 * 29 = 16820 rows, 176 slices of 96."""
    _, qw, ws, bias, xq, sx = operands(20, 32, 57, 200, dev, seed=950)
    bp = capi.pack_conv_weight(to_dev(qw, dev))
    ys = [capi.conv2d(xq, sx, bp, to_dev(ws, dev), 200, (3, 3), strides=(2, 2), pads=(1, 1),
                      bias=to_dev(bias, dev), act=act, out_dtype=out_dtype, kernel=k)
          for k in (capi.KERNEL_MFMA, capi.KERNEL_MFMA_128)]
    torch.cuda.synchronize()
    assert ys[0].shape == (20, 200, 29, 29)
    assert torch.equal(ys[0].view(torch.int16 if out_dtype == torch.bfloat16 else torch.int32),
                       ys[1].view(torch.int16 if out_dtype == torch.bfloat16 else torch.int32))


def test_sliced_conv_last_image_matches_oracle(dev):
    """Batch 12 (every row in a slice of 160): the last image against the
    oracle's direct conv of the dequantised operands."""
    x, qw, ws, bias, xq, sx = operands(12, 16, 56, 256, dev, seed=960)
    y = capi.conv2d(xq, sx, capi.pack_conv_weight(to_dev(qw, dev)), to_dev(ws, dev), 256, (3, 3), pads=(1, 1),
                    bias=to_dev(bias, dev), act=capi.ACT_RELU, kernel=capi.KERNEL_MFMA)
    s = np.float32(oracle.dynamic_scale(x))
    A = oracle.dequantize(oracle.quantize(x[-1:], s), s)
    B = oracle.dequantize(qw.reshape(256, -1), ws, axis=0).reshape(qw.shape)
    ref = oracle.conv2d(A, B, bias, pads=(1, 1), act=oracle.ACT_RELU)
    bound = oracle.conv2d(np.abs(A), np.abs(B), np.abs(bias), pads=(1, 1))
    assert_close(y[-1:].cpu().numpy(), ref, bound, act=capi.ACT_RELU)
