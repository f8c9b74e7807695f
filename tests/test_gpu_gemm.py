"""GPU parity of the FP8 GEMM kernels (MFMA tiles, skinny small-M, VALU
small-M, W8A32) against the oracle's dequantise-then-Gemm composition
(reference src/onnx/operators/gemm.cpp:27-325)."""
import numpy as np
import pytest
import torch

import oracle
from luisaml_amd import capi, synth
from tests.gemm_cases import assert_close, make_case, reference

pytestmark = pytest.mark.gpu

KERNELS = {"mfma": capi.KERNEL_MFMA, "skinny": capi.KERNEL_SKINNY, "valu": capi.KERNEL_VALU,
           "mfma_fp8": capi.KERNEL_MFMA_FP8, "skinny_fp8": capi.KERNEL_SKINNY_FP8,
           "mfma_128": capi.KERNEL_MFMA_128, "mfma_128_fp8": capi.KERNEL_MFMA_128_FP8}


def run(c, kernel, bias=None, alpha=1.0, beta=1.0, act=capi.ACT_NONE, out_dtype=torch.float32, dev=None):
    d_bias = None if bias is None else torch.from_numpy(np.ascontiguousarray(bias, np.float32)).to(dev)
    y = capi.gemm(c.d_qa, c.d_sa, c.d_bp, c.d_sb, c.N, c.K, c=d_bias, alpha=alpha, beta=beta, act=act,
                  out_dtype=out_dtype, kernel=kernel)
    return y


@pytest.mark.parametrize("M,N,K", [(256, 256, 128), (512, 768, 1024), (300, 500, 784), (1, 64, 128),
                                   (257, 100, 2304), (64, 10, 128), (1024, 1024, 4096)])
@pytest.mark.parametrize("per_channel", [True, False])
@pytest.mark.parametrize("kernel", ["mfma", "mfma_128"])
def test_mfma_shapes(dev, M, N, K, per_channel, kernel):
    c = make_case(M, N, K, seed=M + N + K, per_channel=per_channel, dev=dev)
    y = run(c, KERNELS[kernel], dev=dev).cpu().numpy()
    ref, bound = reference(c)
    assert_close(y, ref, bound)


@pytest.mark.parametrize("M", [1, 2, 4, 7, 16])
@pytest.mark.parametrize("N,K", [(64, 128), (11008, 4096), (100, 784), (4096, 11008)])
@pytest.mark.parametrize("kernel", ["skinny", "valu"])
def test_small_m_shapes(dev, M, N, K, kernel):
    c = make_case(M, N, K, seed=M * 31 + N, dev=dev)
    y = run(c, KERNELS[kernel], dev=dev).cpu().numpy()
    ref, bound = reference(c)
    assert_close(y, ref, bound)


@pytest.mark.parametrize("M", [17, 31, 32, 33, 48, 64, 65, 100, 128, 129, 200])
@pytest.mark.parametrize("N,K", [(1024, 2304), (300, 784), (64, 128), (70, 4096)])
def test_medium_m_shapes(dev, M, N, K):
    """Skinny kernel with 2 or 4 row blocks per workgroup and row groups of 64
    (ragged M, N and K; row groups over several XCD ranges)."""
    c = make_case(M, N, K, seed=M * 7 + N + K, dev=dev)
    y = run(c, capi.KERNEL_SKINNY, dev=dev).cpu().numpy()
    ref, bound = reference(c)
    assert_close(y, ref, bound)


@pytest.mark.parametrize("M,N,K", [(48, 11008, 256), (100, 16384, 128), (128, 16384, 128), (65, 11008, 256),
                                   (200, 11008, 128)])
def test_medium_m_row_block_choices(dev, M, N, K):
    """Wide outputs, where the kernel's cost model takes 4 row blocks per
    workgroup (M=48 on 172 panels; M=100 and 128 on 256 panels, two row
    groups) or 2 with several row groups (M=65, M=200)."""
    c = make_case(M, N, K, seed=M + 3, dev=dev)
    y = run(c, capi.KERNEL_SKINNY, dev=dev).cpu().numpy()
    ref, bound = reference(c)
    assert_close(y, ref, bound)


@pytest.mark.parametrize("M", [24, 64, 150])
def test_medium_m_epilogue(dev, M):
    """Row-dependent bias [M, N] and an activation through the row groups."""
    N = 320
    c = make_case(M, N, 1024, seed=M, dev=dev)
    bias = make_bias("MN", M, N, seed=M)
    y = run(c, capi.KERNEL_SKINNY, bias=bias, alpha=0.5, beta=2.0, act=capi.ACT_GELU_ERF, dev=dev).cpu().numpy()
    ref, bound = reference(c, bias=bias, alpha=0.5, beta=2.0, act=capi.ACT_GELU_ERF)
    assert_close(y, ref, bound, act=capi.ACT_GELU_ERF)


@pytest.mark.parametrize("kernel", ["mfma", "skinny", "valu"])
@pytest.mark.parametrize("w_is_nk", [False, True])
def test_weight_layouts(dev, kernel, w_is_nk):
    M = 16 if not kernel.startswith("mfma") else 200
    c = make_case(M, 320, 512, seed=5, w_is_nk=w_is_nk, dev=dev)
    y = run(c, KERNELS[kernel], dev=dev).cpu().numpy()
    ref, bound = reference(c)
    assert_close(y, ref, bound)


BIAS_SHAPES = ["N", "1", "scalar", "M1", "MN", "1N", "M"]


def make_bias(kind, M, N, seed=1):
    rng = np.random.default_rng(seed)
    shape = {"N": (N,), "1": (1,), "scalar": (), "M1": (M, 1), "MN": (M, N), "1N": (1, N), "M": (M,)}[kind]
    return (rng.standard_normal(shape) * 0.01).astype(np.float32)


@pytest.mark.parametrize("kernel", ["mfma", "skinny", "valu", "mfma_128"])
@pytest.mark.parametrize("bias_kind", BIAS_SHAPES)
def test_epilogue_bias_broadcast(dev, kernel, bias_kind):
    M = 12 if not kernel.startswith("mfma") else 130
    N = 192
    c = make_case(M, N, 256, seed=7, dev=dev)
    bias = make_bias(bias_kind, M, N)
    y = run(c, KERNELS[kernel], bias=bias, alpha=0.75, beta=1.5, dev=dev).cpu().numpy()
    ref, bound = reference(c, bias=bias, alpha=0.75, beta=1.5)
    assert_close(y, ref, bound)


@pytest.mark.parametrize("kernel", ["mfma", "skinny", "valu", "mfma_128"])
@pytest.mark.parametrize("act", [capi.ACT_RELU, capi.ACT_GELU_ERF, capi.ACT_GELU_TANH])
def test_epilogue_activation(dev, kernel, act):
    M = 16 if not kernel.startswith("mfma") else 256
    c = make_case(M, 256, 512, seed=9, dev=dev)
    bias = make_bias("N", M, 256, seed=3)
    y = run(c, KERNELS[kernel], bias=bias, act=act, dev=dev).cpu().numpy()
    ref, bound = reference(c, bias=bias, act=act)
    assert_close(y, ref, bound, act=act)


@pytest.mark.parametrize("kernel", ["mfma", "skinny", "valu", "mfma_128"])
@pytest.mark.parametrize("act", [capi.ACT_NONE, capi.ACT_GELU_ERF])
def test_bf16_output_is_rne_of_fp32(dev, kernel, act):
    """bf16 output is bit-exactly bf16_rne of the same kernel's fp32 output.
    For the 256x256 tile kernel (N = 448) the two outputs come from different
    layouts -- bf16 from 2x2 wavefronts of 128x128, fp32 from 2x4 of 128x64
    -- so this also checks that both layouts sum in the same order."""
    M = 16 if not kernel.startswith("mfma") else 384
    c = make_case(M, 448, 1024, seed=13, dev=dev)
    bias = make_bias("N", M, 448, seed=4)
    y32 = run(c, KERNELS[kernel], bias=bias, act=act, dev=dev).cpu().numpy()
    y16 = run(c, KERNELS[kernel], bias=bias, act=act, out_dtype=torch.bfloat16, dev=dev)
    got = y16.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, oracle.bf16_rne(y32))


OUT_LAYOUTS = ["dense", "pitch_even", "pitch_odd", "misaligned", "rows_past_m"]


def out_view(layout, M, N, dtype, dev, fill):
    """An output [M, N] view in a larger buffer filled with `fill`: a padded
    even or odd row pitch, a start one element past an aligned address, or
    64 rows of buffer beyond row M."""
    if layout == "dense":
        buf = torch.full((M, N), fill, dtype=dtype, device=dev)
        return buf, buf
    if layout in ("pitch_even", "pitch_odd"):
        ld = N + (16 if layout == "pitch_even" else 17)
        buf = torch.full((M, ld), fill, dtype=dtype, device=dev)
        return buf, buf[:, :N]
    if layout == "misaligned":
        buf = torch.full((M * N + 1,), fill, dtype=dtype, device=dev)
        return buf, buf[1:].view(M, N)
    buf = torch.full((M + 64, N), fill, dtype=dtype, device=dev)
    return buf, buf[:M]


@pytest.mark.parametrize("kernel", ["mfma", "mfma_128", "mfma_fp8"])
@pytest.mark.parametrize("layout", OUT_LAYOUTS)
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N", [320, 257])
def test_mfma_epilogue_layouts(dev, kernel, layout, out_dtype, N):
    """The tile kernels' row-major epilogue has a path specialised for the
    activation, C and output type (taken when N and the row pitch are even,
    the output is aligned and C does not vary over rows) and a general one;
    both give the same bits, write nothing outside the [M, N] view, and
    match the oracle.  The reference is the same kernel into a dense fp32
    output (bf16: its bf16_rne); for the 256x256 kernels with N > 256 a bf16
    output takes the one-wavefront-per-SIMD layout and fp32 the 2x4 one, so
    the bf16 cases also compare the two layouts bit for bit."""
    M = 300
    c = make_case(M, N, 512, seed=N + 11, dev=dev)
    bias = make_bias("N", M, N, seed=5)
    kw = dict(bias=bias, alpha=0.75, act=capi.ACT_GELU_TANH)
    y32 = run(c, KERNELS[kernel], dev=dev, **kw).cpu().numpy()
    if kernel != "mfma_fp8":
        ref, bound = reference(c, bias=bias, alpha=0.75, act=capi.ACT_GELU_TANH)
        assert_close(y32, ref, bound, act=capi.ACT_GELU_TANH)
    fill = -12345.0
    buf, view = out_view(layout, M, N, out_dtype, dev, fill)
    d_bias = torch.from_numpy(bias).to(dev)
    capi.gemm(c.d_qa, c.d_sa, c.d_bp, c.d_sb, c.N, c.K, c=d_bias, alpha=0.75, act=capi.ACT_GELU_TANH,
              out=view, kernel=KERNELS[kernel])
    torch.cuda.synchronize()
    got = view.cpu()
    if out_dtype == torch.bfloat16:
        assert np.array_equal(got.view(torch.int16).numpy().view(np.uint16), oracle.bf16_rne(y32))
    else:
        assert np.array_equal(got.numpy().view(np.uint32), y32.view(np.uint32))
    # everything outside the view keeps the fill value
    mask = torch.ones_like(buf, dtype=torch.bool)
    if layout == "misaligned":
        mask[1:] = False
    elif layout in ("pitch_even", "pitch_odd"):
        mask[:, :N] = False
    elif layout == "rows_past_m":
        mask[:M] = False
    else:
        mask[:] = False
    assert bool((buf.cpu()[mask.cpu()] == fill).all())


@pytest.mark.parametrize("kernel", ["mfma", "mfma_128", "mfma_fp8"])
@pytest.mark.parametrize("out_dtype,ldy", [(torch.bfloat16, 9_000_000), (torch.float32, 4_500_000)])
@pytest.mark.parametrize("M", [1, 17])
def test_mfma_epilogue_huge_row_pitch(dev, kernel, out_dtype, ldy, M):
    """A few rows with a ~18 MB row pitch: (M + 64) rows of pitch stay below
    2^31 bytes, so the specialised row-major epilogue runs, while the tile's
    256 staged rows reach ~4.6e9 bytes.  A pass of staged rows past M must
    store nothing (its 32-bit offsets would otherwise wrap into row 0's
    pitch padding); the view gets the same bits as a dense output and every
    other element of the buffer keeps its fill."""
    N = 320
    c = make_case(M, N, 512, seed=M + 101, dev=dev)
    ref = run(c, KERNELS[kernel], out_dtype=out_dtype, dev=dev)
    fill = -12288.0  # exact in bf16
    buf = torch.full((M * ldy,), fill, dtype=out_dtype, device=dev)
    view = buf.as_strided((M, N), (ldy, 1))
    capi.gemm(c.d_qa, c.d_sa, c.d_bp, c.d_sb, c.N, c.K, out=view, kernel=KERNELS[kernel])
    torch.cuda.synchronize()
    assert torch.equal(view.view(torch.int16 if out_dtype == torch.bfloat16 else torch.int32),
                       ref.view(torch.int16 if out_dtype == torch.bfloat16 else torch.int32))
    view.fill_(fill)
    assert int((buf != fill).sum().item()) == 0


@pytest.mark.parametrize("kernel", ["mfma", "mfma_fp8"])
@pytest.mark.parametrize("M,N,K", [(4100, 4104, 1008), (4352, 4352, 160), (300, 1000, 320), (8200, 2056, 2048)])
@pytest.mark.parametrize("epi", ["plain", "bias_relu", "scalar_c_alpha"])
def test_mfma_persistent_direct_store(dev, kernel, M, N, K, epi):
    """bf16 outputs with N and the row pitch multiples of 8 take the
    persistent one-wavefront-per-SIMD kernel, whose workgroups walk several
    tiles (more tiles than CUs here: 289, 289 and 297 tiles; a grid of 12
    at 300 x 1000), with ragged last tile rows and columns, K of 4, 5 and 16
    steps, and an epilogue that stores straight from the accumulators.  Its
    output must be, bit for bit, the bf16 rounding of the same kernel
    family's fp32 output (the 2x4 layout with the staged epilogue), write
    nothing outside its [M, N] view of a pitched buffer, and match the
    oracle on sampled rows."""
    per_channel = epi != "scalar_c_alpha"
    c = make_case(M, N, K, seed=M + N + K, per_channel=per_channel, dev=dev)
    if epi == "plain":
        kw, bias = dict(), None
    elif epi == "bias_relu":
        bias = make_bias("N", M, N, seed=17)
        kw = dict(bias=bias, act=capi.ACT_RELU)
    else:
        bias = make_bias("1", M, N, seed=19)
        kw = dict(bias=bias, alpha=0.75, beta=-1.25)
    y32 = run(c, KERNELS[kernel], dev=dev, **kw)
    ld = N + 24
    fill = -12288.0
    buf = torch.full((M, ld), fill, dtype=torch.bfloat16, device=dev)
    view = buf[:, :N]
    d_bias = None if bias is None else torch.from_numpy(np.ascontiguousarray(bias, np.float32)).to(dev)
    capi.gemm(c.d_qa, c.d_sa, c.d_bp, c.d_sb, c.N, c.K, c=d_bias, alpha=kw.get("alpha", 1.0),
              beta=kw.get("beta", 1.0), act=kw.get("act", capi.ACT_NONE), out=view, kernel=KERNELS[kernel])
    torch.cuda.synchronize()
    assert torch.equal(view.view(torch.int16), y32.to(torch.bfloat16).view(torch.int16))
    assert bool((buf[:, N:] == fill).all())
    if kernel == "mfma":
        rows = np.unique(np.array([0, 1, 255, 256, M // 2, M - 2, M - 1]))
        sub = c.__class__()
        sub.__dict__.update(c.__dict__)
        sub.qa = c.qa[rows]
        ref, bound = reference(sub, bias=None if bias is None else (bias if bias.ndim < 2 else bias[rows]),
                               alpha=kw.get("alpha", 1.0), beta=kw.get("beta", 1.0), act=kw.get("act", capi.ACT_NONE))
        assert_close(y32[torch.from_numpy(rows).to(dev)].cpu().numpy(), ref, bound, act=kw.get("act", capi.ACT_NONE))


def test_kernels_agree_small_m(dev):
    """All three kernels on one decode-shaped case agree within the bound."""
    c = make_case(16, 2048, 4096, seed=21, dev=dev)
    ref, bound = reference(c)
    for k in ("mfma", "skinny", "valu"):
        assert_close(run(c, KERNELS[k], dev=dev).cpu().numpy(), ref, bound)


@pytest.mark.parametrize("M,N,K", [(64, 256, 784), (64, 128, 256), (64, 10, 128), (1, 11008, 4096), (33, 70, 100)])
def test_w8a32(dev, M, N, K):
    from luisaml_amd import synth
    a = synth.uniform(M * 5 + 1, (M, K))
    w = synth.normal(M * 5 + 2, (N, K), std=0.05)
    sw = np.array([oracle.dynamic_scale(w)], np.float32)
    qw = oracle.quantize(w, sw)
    bias = synth.normal(M * 5 + 3, (N,), std=0.01)
    bp = capi.pack_weight(torch.from_numpy(qw).to(dev), True)
    y = capi.gemm_w8a32(torch.from_numpy(a).to(dev), bp, torch.from_numpy(sw).to(dev), N, K,
                        c=torch.from_numpy(bias).to(dev), act=capi.ACT_RELU).cpu().numpy()
    B = oracle.dequantize(qw, sw)
    ref = oracle.gemm(a, B, bias, transB=1, act=oracle.ACT_RELU)
    bound = oracle.gemm_abs_bound(a, B, bias, transB=1)
    assert_close(y, ref, bound)


def test_nan_propagates(dev):
    """A NaN code (0x7f) in A makes its output row NaN, in B its column."""
    c = make_case(16, 128, 256, seed=2, dev=dev)
    qa = c.qa.copy()
    qa[3, 17] = 0x7F
    qb = c.qb.copy()
    qb[40, 77] = 0xFF  # [K, N]: column 77
    c.d_qa = torch.from_numpy(qa).to(dev)
    c.d_bp = capi.pack_weight(torch.from_numpy(qb).to(dev), False)
    for k in ("mfma", "skinny", "valu", "mfma_128"):
        y = run(c, KERNELS[k], dev=dev).cpu().numpy()
        assert np.isnan(y[3]).all(), k
        assert np.isnan(y[:, 77]).all(), k
        mask = np.ones_like(y, bool)
        mask[3] = False
        mask[:, 77] = False
        assert not np.isnan(y[mask]).any(), k


def test_errors_are_reported(dev):
    c = make_case(8, 64, 128, seed=1, dev=dev)
    with pytest.raises(capi.LcmlError) as e:
        capi.gemm(c.d_qa, c.d_sa, c.d_bp, c.d_sb, c.N, c.K, out_dtype=torch.float16)
    assert e.value.code == capi.ERR_UNSUPPORTED


@pytest.mark.parametrize("kernel", ["mfma", "skinny", "valu", "mfma_fp8", "skinny_fp8", "mfma_128", "mfma_128_fp8"])
def test_identity_reproduces_every_code(dev, kernel):
    """One-hot A rows (1.0 = 0x38) pick single weights: y[m, n] = to_float(B[m, n])
    exactly, for all 254 non-NaN E4M3 codes, through each kernel's operand
    conversion.  (NaN codes are left out: 0 * NaN from the other rows would
    poison the column; NaN propagation has its own test.)  Zeros compare by
    value: -0.0 + 0 * b sums to +0.0."""
    M = {"skinny": 100, "skinny_fp8": 48, "valu": 16}.get(kernel, 128)
    K, N = 128, 256
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    qa = np.zeros((M, K), np.uint8)
    qa[np.arange(M), np.arange(M)] = 0x38
    rng = np.random.default_rng(0)
    qb = np.zeros((K, N), np.uint8)
    for k in range(M):
        qb[k, :254] = rng.permutation(codes)
    one = torch.ones(1, device=dev)
    bp = capi.pack_weight(torch.from_numpy(qb).to(dev), False)
    y = capi.gemm(torch.from_numpy(qa).to(dev), one, bp, one, N, K, kernel=KERNELS[kernel]).cpu().numpy()
    ref = oracle.e4m3_to_float(qb[:M])
    assert np.array_equal(y, ref)
    nz = ref != 0
    assert np.array_equal(y[nz].view(np.uint32), ref[nz].view(np.uint32))


@pytest.mark.parametrize("kernel", ["mfma_fp8", "skinny_fp8", "mfma_128_fp8"])
def test_native_fp8_mfma_precision_is_documented(dev, kernel):
    """The opt-in native-FP8-MFMA kernels stay inside the elementwise bound and
    within 3e-5 relative Frobenius (gfx950 FP8 MFMA block truncation)."""
    M = 40 if "skinny" in kernel else 512
    c = make_case(M, 1024, 4096, seed=17, dev=dev)
    y = run(c, KERNELS[kernel], dev=dev).cpu().numpy().astype(np.float64)
    ref, bound = reference(c)
    assert np.all(np.abs(y - ref) <= 1e-4 * bound)
    rel = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert rel < 3e-5


def test_concurrent_streams_match_serial(dev):
    """The entry points keep no shared mutable state between calls: the same
    GEMMs (tile, 128-tile, skinny, fused dynamic) issued on two streams at
    once give the bits they give one after another on one stream."""
    cases = [make_case(M, N, K, seed=50 + M, dev=dev) for M, N, K in ((300, 500, 784), (24, 1100, 512),
                                                                      (1024, 640, 256), (4, 2048, 1024))]
    kernels = [capi.KERNEL_MFMA, capi.KERNEL_SKINNY, capi.KERNEL_MFMA_128, capi.KERNEL_SKINNY]
    x4 = torch.from_numpy(synth.normal(59, (4, 1024))).to(dev)
    serial = [run(c, k, dev=dev) for c, k in zip(cases, kernels)]
    serial.append(capi.gemm_dynamic(x4, cases[3].d_bp, cases[3].d_sb, cases[3].N, cases[3].K))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outs = [None] * 5
    for rep in range(3):
        for i, (c, k) in enumerate(zip(cases, kernels)):
            with torch.cuda.stream(streams[i % 2]):
                outs[i] = capi.gemm(c.d_qa, c.d_sa, c.d_bp, c.d_sb, c.N, c.K, kernel=k)
        with torch.cuda.stream(streams[1]):
            outs[4] = capi.gemm_dynamic(x4, cases[3].d_bp, cases[3].d_sb, cases[3].N, cases[3].K)
        torch.cuda.synchronize()
        for i in range(5):
            assert torch.equal(outs[i].view(torch.int32), serial[i].view(torch.int32)), (rep, i)


EXACT_TO_FP8 = {capi.KERNEL_MFMA: capi.KERNEL_MFMA_FP8, capi.KERNEL_MFMA_128: capi.KERNEL_MFMA_128_FP8,
                capi.KERNEL_SKINNY: capi.KERNEL_SKINNY_FP8}


@pytest.mark.parametrize("M,N,K", [(4, 2048, 1024), (40, 1024, 1024), (512, 1024, 1024), (2048, 4096, 512)])
def test_auto_fp8_runs_the_fp8_twin_of_autos_choice(dev, M, N, K):
    """LCML_KERNEL_AUTO_FP8 takes AUTO's tiling with the native FP8 MFMAs:
    its bits are those of the FP8 twin of the exact kernel whose bits AUTO
    reproduces (the skinny kernel at small M, 128x128 or 256x256 tiles
    above), and it stays within the FP8-MFMA bounds of the oracle."""
    c = make_case(M, N, K, seed=M + 3 * N + K, dev=dev)
    auto = run(c, capi.KERNEL_AUTO, dev=dev)
    picked = [k for k in EXACT_TO_FP8 if torch.equal(run(c, k, dev=dev).view(torch.int32), auto.view(torch.int32))]
    assert picked, "AUTO matches none of the exact kernels"
    fast = run(c, capi.KERNEL_AUTO_FP8, dev=dev)
    assert any(torch.equal(fast.view(torch.int32), run(c, EXACT_TO_FP8[k], dev=dev).view(torch.int32))
               for k in picked)
    y = fast.cpu().numpy().astype(np.float64)
    ref, bound = reference(c)
    assert np.all(np.abs(y - ref) <= 1e-4 * bound)
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 3e-5


@pytest.mark.parametrize("M", [1, 4, 64])
def test_auto_fp8_dynamic(dev, M):
    """gemm_dynamic with AUTO_FP8: the fused skinny FP8 kernel where AUTO
    fuses (M*K <= 16384), else quantise + the AUTO_FP8 GEMM; bit-identical
    to the two launches written out."""
    N, K = 2048, 4096
    c = make_case(M, N, K, seed=70 + M, dev=dev)
    x = torch.from_numpy(synth.normal(71 + M, (M, K))).to(dev)
    got = capi.gemm_dynamic(x, c.d_bp, c.d_sb, N, K, kernel=capi.KERNEL_AUTO_FP8)
    qx, sx = capi.quantize_dynamic(x)
    want = capi.gemm(qx, sx, c.d_bp, c.d_sb, N, K, kernel=capi.KERNEL_SKINNY_FP8 if M * K <= 16384
                     else capi.KERNEL_AUTO_FP8)
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


def test_auto_fp8_conv(dev):
    """conv2d with AUTO_FP8 gives the bits of the native-FP8 tile kernel of
    AUTO's tile size."""
    n, cin, h, w, cout = 4, 64, 28, 28, 128
    x = torch.from_numpy(synth.normal(81, (n, cin, h, w))).to(dev)
    wt = synth.normal(82, (cout, cin, 3, 3), std=0.05)
    sw = oracle.channel_scales(wt, axis=0)
    d_sw = torch.from_numpy(sw).to(dev)
    qw = torch.from_numpy(oracle.quantize(wt, sw, axis=0)).to(dev)
    bp = capi.pack_conv_weight(qw)
    xq, sx = capi.quantize_nhwc(x)
    args = dict(kernel_shape=(3, 3), pads=(1, 1))
    auto = capi.conv2d(xq, sx, bp, d_sw, cout, kernel=capi.KERNEL_AUTO, **args)
    fast = capi.conv2d(xq, sx, bp, d_sw, cout, kernel=capi.KERNEL_AUTO_FP8, **args)
    for exact, fp8 in ((capi.KERNEL_MFMA, capi.KERNEL_MFMA_FP8), (capi.KERNEL_MFMA_128, capi.KERNEL_MFMA_128_FP8)):
        if torch.equal(capi.conv2d(xq, sx, bp, d_sw, cout, kernel=exact, **args).view(torch.int32),
                       auto.view(torch.int32)):
            assert torch.equal(capi.conv2d(xq, sx, bp, d_sw, cout, kernel=fp8, **args).view(torch.int32),
                               fast.view(torch.int32))
            break
    else:
        pytest.fail("AUTO matches neither tile kernel")
    assert not torch.equal(fast.view(torch.int32), auto.view(torch.int32))
