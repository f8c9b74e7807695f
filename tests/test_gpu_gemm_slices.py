"""Row slices of the 256x256-tile GEMM's 2x4 layout (fp32 outputs, grids of
one tile column, amax partials).  When the last round of tiles would leave
CUs idle, the whole tiles of the first tile columns run first and the other
columns are cut into slices of h rows, one per CU; on a grid of one tile
column the rows below the whole tiles are.  A slice sums every output's
products in the same order as the 128x128-tile kernel, which has no slices,
so the two agree bit for bit (with GELU and a bias, fp32 and bf16 out),
and the partial maxima of a sliced launch still cover y exactly.  The
shapes give the slice plans noted on 256 CUs (whole tiles, slice rows,
whole columns, workgroups); the GEMM's semantics are the reference's Gemm
(gemm.cpp:27-325), checked against the oracle in test_gpu_gemm.py."""
import numpy as np
import pytest
import torch

import oracle
from luisaml_amd import capi, synth
from tests.gemm_cases import assert_close, make_case

pytestmark = pytest.mark.gpu

SHAPES = [(4096, 11008, 256),  # 512 whole tiles (32 columns), 11 x 22 slices of 192 rows
          (3000, 11008, 128),  # 504 whole tiles (42 columns), 47 slices of 64 rows
          (5000, 4096, 128),   # 240 whole tiles (12 columns), 4 x 53 slices of 96 rows
          (1000, 256, 384),    # one tile column: 16 slices of 64 rows
          (4096, 200, 128)]    # one tile column, ragged N: 64 slices of 64 rows


def bias(N):
    return torch.from_numpy(synth.normal(5, (N,), std=0.5))


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("kernels", [(capi.KERNEL_MFMA, capi.KERNEL_MFMA_128),
                                     (capi.KERNEL_MFMA_FP8, capi.KERNEL_MFMA_128_FP8)])
@pytest.mark.parametrize("out_dtype,act", [(torch.float32, capi.ACT_GELU_ERF), (torch.bfloat16, capi.ACT_RELU)])
def test_sliced_gemm_matches_unsliced_bit_for_bit(dev, M, N, K, kernels, out_dtype, act):
    c = make_case(M, N, K, seed=M + N + K, dev=dev)
    b = bias(N).to(dev)
    ys = [capi.gemm(c.d_qa, c.d_sa, c.d_bp, c.d_sb, N, K, c=b, act=act, out_dtype=out_dtype, kernel=k)
          for k in kernels]
    torch.cuda.synchronize()
    view = torch.int16 if out_dtype == torch.bfloat16 else torch.int32
    assert torch.equal(ys[0].view(view), ys[1].view(view))


def test_sliced_gemm_matches_oracle(dev):
    """The up-projection's shape with a short K: against the oracle, rows of
    every slice height's region sampled (whole-tile columns and sliced ones)."""
    M, N, K = 4096, 11008, 256
    c = make_case(M, N, K, seed=77, dev=dev)
    y = capi.gemm(c.d_qa, c.d_sa, c.d_bp, c.d_sb, N, K, kernel=capi.KERNEL_MFMA).cpu().numpy()
    rows = np.array([0, 191, 192, 1000, 2047, 2048, 3839, 4032, 4095])
    A = oracle.dequantize(c.qa[rows], c.sa)
    B = oracle.dequantize(c.qb, c.sb, axis=1)
    assert_close(y[rows], oracle.gemm(A, B), oracle.gemm_abs_bound(A, B))


@pytest.mark.parametrize("M,N,K,kernel", [(4096, 11008, 256, capi.KERNEL_MFMA), (5000, 4096, 128, capi.KERNEL_MFMA_FP8),
                                          (1000, 256, 384, capi.KERNEL_MFMA)])
def test_sliced_gemm_amax_partials_cover_y(dev, M, N, K, kernel):
    x = torch.from_numpy(synth.normal(M + 3, (M, K))).to(dev)
    w = torch.from_numpy(synth.normal(N + 5, (K, N), std=0.02)).to(dev)
    sw = torch.from_numpy(oracle.channel_scales(w.cpu().numpy(), 1)).to(dev)
    bp = capi.pack_weight(capi.quantize(w, sw, axis=1), w_is_nk=False)
    b = bias(N).to(dev)
    part = capi.amax_parts_buffer(M, N, dev)
    part.fill_(-1)
    ref = capi.gemm_dynamic(x, bp, sw, N, K, c=b, act=capi.ACT_GELU_ERF, kernel=kernel)
    y, n = capi.gemm_dynamic_ex(x, bp, sw, N, K, c=b, act=capi.ACT_GELU_ERF, kernel=kernel, y_amax_part=part)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), ref.view(torch.int32))
    assert 0 < n <= part.numel() and int((part[:n] == -1).sum()) == 0
    assert part[:n].cpu().numpy().view(np.float32).max() == y.abs().max().item()
