"""Chained dynamically quantised linears (lcml_fp8_gemm_dynamic_ex): the
partial maxima of y that a call writes cover y exactly (their maximum is
max |y| over the output, bit for bit, with the padded rows and columns of
the edge tiles left out), and a following call that takes them as its
input's partials gives the same output and scale, bit for bit, as the plain
dynamic linear that reduces its input itself (the reference composition
Abs -> ReduceMax -> Div -> Cast -> Gemm, gemm.cpp:27-325)."""
import numpy as np
import pytest
import torch

import oracle
from luisaml_amd import capi, synth

pytestmark = pytest.mark.gpu


def weight(seed, K, N, dev):
    w = torch.from_numpy(synth.normal(seed, (K, N), std=0.02)).to(dev)
    sw = torch.from_numpy(oracle.channel_scales(w.cpu().numpy(), 1)).to(dev)
    return capi.pack_weight(capi.quantize(w, sw, axis=1), w_is_nk=False), sw


def max_of_parts(part, n):
    return part[:n].cpu().numpy().view(np.float32).max()


@pytest.mark.parametrize("M,N,K,kernel", [
    (600, 1000, 512, capi.KERNEL_MFMA), (600, 1000, 512, capi.KERNEL_MFMA_FP8),
    (600, 999, 512, capi.KERNEL_MFMA),        # odd N: the general epilogue loop
    (300, 1000, 256, capi.KERNEL_MFMA_128), (300, 1000, 256, capi.KERNEL_MFMA_128_FP8),
    (2048, 4096, 1024, capi.KERNEL_AUTO),      # AUTO's 128x128 tiles
    (16, 1000, 512, capi.KERNEL_AUTO),         # skinny kernel, then an amax pass over y
    (4, 1000, 512, capi.KERNEL_AUTO)])         # fused small-M kernel, then an amax pass
@pytest.mark.parametrize("act", [capi.ACT_NONE, capi.ACT_GELU_ERF])
def test_y_amax_partials_cover_y(dev, M, N, K, kernel, act):
    x = torch.from_numpy(synth.normal(M + N, (M, K))).to(dev)
    bp, sw = weight(M + K, K, N, dev)
    bias = torch.from_numpy(synth.normal(7, (N,), std=0.5)).to(dev)  # padded rows would read GELU(bias) != 0
    ref = capi.gemm_dynamic(x, bp, sw, N, K, c=bias, alpha=0.75, act=act, kernel=kernel)
    part = capi.amax_parts_buffer(M, N, dev)
    part.fill_(-1)
    y, n = capi.gemm_dynamic_ex(x, bp, sw, N, K, c=bias, alpha=0.75, act=act, kernel=kernel, y_amax_part=part)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), ref.view(torch.int32))
    assert 0 < n <= part.numel()
    assert int((part[:n] == -1).sum()) == 0  # every reported partial was written
    assert max_of_parts(part, n) == y.abs().max().item()


@pytest.mark.parametrize("M,K1,N1,N2,kernel", [(1024, 512, 2048, 768, capi.KERNEL_AUTO),
                                               (1024, 512, 2048, 768, capi.KERNEL_AUTO_FP8),
                                               (512, 256, 1008, 320, capi.KERNEL_MFMA),
                                               (4, 512, 1008, 256, capi.KERNEL_AUTO)])
def test_chain_uses_partials_bit_for_bit(dev, M, K1, N1, N2, kernel):
    """up (fp32 + GELU, partials of its output) -> down (quantised with those
    partials): the same down output and scale as the plain call."""
    x = torch.from_numpy(synth.normal(M, (M, K1))).to(dev)
    bp1, sw1 = weight(11, K1, N1, dev)
    bp2, sw2 = weight(12, N1, N2, dev)
    b1 = torch.from_numpy(synth.normal(13, (N1,), std=0.01)).to(dev)
    part = capi.amax_parts_buffer(M, N1, dev)
    h, n = capi.gemm_dynamic_ex(x, bp1, sw1, N1, K1, c=b1, act=capi.ACT_GELU_ERF, kernel=kernel, y_amax_part=part)
    s_ref, s_got = torch.empty(1, device=dev), torch.empty(1, device=dev)
    ref = capi.gemm_dynamic(h, bp2, sw2, N2, N1, out_dtype=torch.bfloat16, kernel=kernel, scale_out=s_ref)
    got, _ = capi.gemm_dynamic_ex(h, bp2, sw2, N2, N1, out_dtype=torch.bfloat16, kernel=kernel, scale_out=s_got,
                                  x_amax=(part, n))
    torch.cuda.synchronize()
    assert torch.equal(s_got.view(torch.int32), s_ref.view(torch.int32))
    assert np.float32(s_ref.item()) == np.float32(oracle.dynamic_scale(h.cpu().numpy()))
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
