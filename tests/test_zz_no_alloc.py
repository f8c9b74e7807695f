"""lcml_fp8_gemm_dynamic_noalloc against lcml_fp8_gemm_dynamic through the C
ABI: bit-identical outputs and scales on consecutive calls that share the
library's scratch array (the largest accepted M*K first, then a smaller
two-step call, then a fused small-M call), no change in the device's free
memory across a call, and the same bits from calls captured into a HIP
graph and replayed."""
import numpy as np
import pytest
import torch

from luisaml_amd import capi, synth

pytestmark = pytest.mark.gpu


def _ptr(t):
    return None if t is None else t.data_ptr()


def noalloc(x, bp, sw, N, K, c=None, act=capi.ACT_NONE, out_dtype=torch.float32, scale_out=None, out=None,
            stream=None):
    M = x.shape[0]
    y = out if out is not None else torch.empty((M, N), dtype=out_dtype, device=x.device)
    ydt = capi.DTYPE_BFLOAT16 if out_dtype == torch.bfloat16 else capi.DTYPE_FLOAT
    rc = capi.lib().lcml_fp8_gemm_dynamic_noalloc(M, N, K, _ptr(x), x.stride(0), _ptr(bp), _ptr(sw),
                                                  int(sw.numel() > 1), 1.0, _ptr(c), 1 if c is not None else 0,
                                                  N if c is not None else 0, 0, 1.0, act, _ptr(y), ydt, N,
                                                  _ptr(scale_out), capi.KERNEL_AUTO, stream)
    assert rc == capi.OK, capi.last_error()
    return y


def case(seed, M, K, N, dev):
    x = torch.from_numpy(synth.normal(seed, (M, K))).to(dev)
    w = torch.from_numpy(synth.normal(seed + 1, (K, N), std=0.02)).to(dev)
    sw = torch.full((N,), 1.0 / 448, device=dev) * w.abs().amax(dim=0).clamp_min(1e-30)
    bp = capi.pack_weight(capi.quantize(w, sw, axis=1), w_is_nk=False)
    bias = torch.from_numpy(synth.normal(seed + 2, (N,), std=0.01)).to(dev)
    return x, bp, sw, bias


@pytest.mark.parametrize("M,K,N,act,dt", [(4096, 4096, 256, capi.ACT_GELU_ERF, torch.float32),
                                          (64, 1024, 512, capi.ACT_NONE, torch.bfloat16),
                                          (4, 1024, 320, capi.ACT_RELU, torch.float32)])
def test_noalloc_matches_workspace_entry_point(dev, M, K, N, act, dt):
    x, bp, sw, bias = case(10 * M + K, M, K, N, dev)
    s_ref, s_got = torch.empty(1, device=dev), torch.empty(1, device=dev)
    ref = capi.gemm_dynamic(x, bp, sw, N, K, c=bias, act=act, out_dtype=dt, scale_out=s_ref)
    got = noalloc(x, bp, sw, N, K, c=bias, act=act, out_dtype=dt, scale_out=s_got)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16 if dt == torch.bfloat16 else torch.int32),
                       ref.view(torch.int16 if dt == torch.bfloat16 else torch.int32))
    assert torch.equal(s_got.view(torch.int32), s_ref.view(torch.int32))


def test_noalloc_two_calls_in_a_row_second_smaller(dev):
    """The scratch array keeps the first call's bytes; the second, smaller
    call must not depend on them.  Free device memory does not change."""
    big = case(7, 2048, 4096, 1024, dev)
    small = case(8, 96, 2048, 704, dev)
    refs = [capi.gemm_dynamic(x, bp, sw, bp_n, k, c=b) for (x, bp, sw, b), bp_n, k in
            ((big, 1024, 4096), (small, 704, 2048))]
    torch.cuda.synchronize()
    y1, y2 = torch.empty_like(refs[0]), torch.empty_like(refs[1])
    noalloc(big[0], big[1], big[2], 1024, 4096, c=big[3], out=y1)  # warm: resolves the scratch address
    y1.zero_()
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    noalloc(big[0], big[1], big[2], 1024, 4096, c=big[3], out=y1)
    noalloc(small[0], small[1], small[2], 704, 2048, c=small[3], out=y2)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    assert torch.equal(y1.view(torch.int32), refs[0].view(torch.int32))
    assert torch.equal(y2.view(torch.int32), refs[1].view(torch.int32))


def test_noalloc_captured_in_a_graph(dev):
    """The callers it is for: calls captured into a HIP graph (a two-step
    call, whose quantised activations and scale live in the scratch array,
    then a fused small-M call), replayed four times with unrelated eager
    work between replays; every replay gives the outputs and scales of
    lcml_fp8_gemm_dynamic bit for bit, and the replays leave the device's
    free memory unchanged."""
    two = case(21, 96, 2048, 704, dev)   # M*K > 16384: quantise into the scratch, then the GEMM
    fused = case(22, 4, 1024, 320, dev)  # the fused skinny kernel
    s_ref = [torch.empty(1, device=dev) for _ in range(2)]
    refs = [capi.gemm_dynamic(two[0], two[1], two[2], 704, 2048, c=two[3], out_dtype=torch.bfloat16,
                              scale_out=s_ref[0]),
            capi.gemm_dynamic(fused[0], fused[1], fused[2], 320, 1024, c=fused[3], act=capi.ACT_GELU_ERF,
                              scale_out=s_ref[1])]
    ys = [torch.empty_like(refs[0]), torch.empty_like(refs[1])]
    ss = [torch.empty(1, device=dev) for _ in range(2)]

    def calls(stream):
        noalloc(two[0], two[1], two[2], 704, 2048, c=two[3], out_dtype=torch.bfloat16, scale_out=ss[0], out=ys[0],
                stream=stream)
        noalloc(fused[0], fused[1], fused[2], 320, 1024, c=fused[3], act=capi.ACT_GELU_ERF, scale_out=ss[1],
                out=ys[1], stream=stream)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        calls(side.cuda_stream)  # warm, outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        calls(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for r in range(4):
        for t in ys + ss:
            t.zero_()
        other = capi.gemm_dynamic(two[0], two[1], two[2], 704, 2048)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(ys[0].view(torch.int16), refs[0].view(torch.int16)), f"replay {r}"
        assert torch.equal(ys[1].view(torch.int32), refs[1].view(torch.int32)), f"replay {r}"
        for i in range(2):
            assert torch.equal(ss[i].view(torch.int32), s_ref[i].view(torch.int32)), f"replay {r} scale {i}"
        del other
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
