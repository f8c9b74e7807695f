"""The quantize + GEMM pipeline captured in a HIP graph: every replay, with
eager work and synchronisation between replays, reproduces the eager result
bit for bit (the library records no memset nodes; small dynamic quantisation
is a single kernel with no workspace)."""
import numpy as np
import pytest
import torch

from luisaml_amd import capi
from tests.gemm_cases import make_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,kernel", [(1, capi.KERNEL_SKINNY), (16, capi.KERNEL_SKINNY), (300, capi.KERNEL_MFMA)])
def test_graph_replays_match_eager(dev, M, kernel):
    N, K = 1024, 2048
    c = make_case(M, N, K, seed=M, dev=dev)
    x = torch.randn(M, K, device=dev)
    q = torch.empty((M, K), dtype=torch.uint8, device=dev)
    s = torch.empty(1, device=dev)
    ws = torch.empty(capi.DYNAMIC_WORKSPACE_BYTES, dtype=torch.uint8, device=dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

    def pipeline():
        capi.quantize_dynamic(x, out=q, scale_out=s, workspace=ws)
        capi.gemm(q, s, c.d_bp, c.d_sb, N, K, out=y, act=capi.ACT_GELU_ERF, kernel=kernel)

    pipeline()
    torch.cuda.synchronize()
    eager = y.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        pipeline()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        pipeline()
    for r in range(4):
        y.zero_()
        q.zero_()
        # unrelated eager work between replays
        other = capi.gemm(c.d_qa, c.d_sa, c.d_bp, c.d_sb, N, K, kernel=kernel)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), eager.view(torch.int16)), f"replay {r}"
        del other
