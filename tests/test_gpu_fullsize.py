"""Parity at the benchmarked sizes (the configurations bench.py measures).

Same bars as the smaller parity tests: quantisation bit-exact, GEMM outputs
elementwise within 1e-4 * sum|a*b| and relative Frobenius 1e-5 against the
oracle's dequantise-then-Gemm / direct conv (reference gemm.cpp:27-325,
conv.cpp:115-207).  Where the full oracle product would take minutes on the
host, a fixed sample of output rows (or one image of the conv batch) is
checked against the oracle; the GPU computes the full problem.
"""
import numpy as np
import pytest
import torch

import oracle
from luisaml_amd import capi, synth
from tests.gemm_cases import assert_close, gelu_tol

pytestmark = pytest.mark.gpu


def full_matrix_check(y, qa, sa, qb_kn, sb, bias=None, frob=None):
    """Every element of y against a float32 GEMM of the dequantised operands
    computed on the GPU by torch (A = to_float(qa) * sa, B = to_float(qb) *
    sb, as DequantizeLinear does): |y - ref| <= 1e-4 * (|A| @ |B| + |bias|).
    The sampled rows are checked against the oracle; this covers every tile
    of the grid.  With frob, also the relative Frobenius error."""
    torch.backends.cuda.matmul.allow_tf32 = False
    A = qa.view(torch.float8_e4m3fn).float() * sa
    B = qb_kn.view(torch.float8_e4m3fn).float() * sb
    ref = A @ B
    bound = A.abs() @ B.abs()
    del A, B
    if bias is not None:
        ref += bias
        bound += bias.abs()
    err = (y.float() - ref).abs()
    bad = int((~(err <= 1e-4 * bound)).sum())
    assert bad == 0, f"{bad} elements outside 1e-4 * sum|ab|"
    if frob is not None:
        rel = float(torch.linalg.vector_norm(y.float() - ref) / torch.linalg.vector_norm(ref))
        assert rel < frob, rel


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def per_channel_weight(w, dev):
    """W [K, N] -> per-output-channel E4M3 (codes checked bit-exact)."""
    sw = oracle.channel_scales(w, 1)
    qw = oracle.quantize(w, sw, axis=1)
    d_sw = to_dev(sw, dev)
    q_dev = capi.quantize(to_dev(w, dev), d_sw, axis=1)
    assert np.array_equal(q_dev.cpu().numpy(), qw)
    return qw, sw, capi.pack_weight(q_dev, w_is_nk=False), d_sw


@pytest.fixture(scope="module")
def decode_weight(dev):
    w = synth.normal(101, (4096, 11008), std=0.02)
    return per_channel_weight(w, dev)


@pytest.mark.parametrize("M", [1, 4, 16])
def test_small_m_decode_linear_full(dev, decode_weight, M):
    """x[M,4096] fp32 N(0,1) -> dynamic E4M3 -> x W[4096,11008] (per-channel) -> bf16."""
    qw, sw, bp, d_sw = decode_weight
    x = synth.normal(200 + M, (M, 4096))
    s_out = torch.empty(1, device=dev)
    y = capi.gemm_dynamic(to_dev(x, dev), bp, d_sw, 11008, 4096, out_dtype=torch.float32, scale_out=s_out)
    s_ref = np.float32(oracle.dynamic_scale(x))
    assert s_out.cpu().numpy().view(np.uint32)[0] == s_ref.view(np.uint32)
    ref, A, B = oracle.qlinear(oracle.quantize(x, s_ref), s_ref, qw, sw)
    assert_close(y.cpu().numpy(), ref, oracle.gemm_abs_bound(A, B))
    y16 = capi.gemm_dynamic(to_dev(x, dev), bp, d_sw, 11008, 4096, out_dtype=torch.bfloat16)
    assert np.array_equal(y16.view(torch.int16).cpu().numpy().view(np.uint16), oracle.bf16_rne(y.cpu().numpy()))


ROWS = np.array([0, 1, 255, 256, 1023, 2048, 4095, 4096, 5000, 6143, 7777, 8191])


@pytest.fixture(scope="module")
def cube_8192(dev):
    """8192^3 operands: A and B from N(0,1), per-tensor scales amax/448
    (checked bit-exact), B packed; the oracle's sampled-row reference."""
    n = 8192
    a = synth.normal(301, (n, n))
    b = synth.normal(302, (n, n))
    qa, sa = capi.quantize_dynamic(to_dev(a, dev))
    qb, sb = capi.quantize_dynamic(to_dev(b, dev))
    sa_ref, sb_ref = np.float32(oracle.dynamic_scale(a)), np.float32(oracle.dynamic_scale(b))
    assert float(sa.item()) == sa_ref and float(sb.item()) == sb_ref
    bp = capi.pack_weight(qb, w_is_nk=False)
    qa_rows = qa[torch.from_numpy(ROWS).to(dev)].cpu().numpy()
    assert np.array_equal(qa_rows, oracle.quantize(a[ROWS], sa_ref))
    ref, A, B = oracle.qlinear(qa_rows, sa_ref, qb.cpu().numpy(), sb_ref)
    del a, b, qb
    return qa, sa, bp, sb, ref, oracle.gemm_abs_bound(A, B)


def test_gemm_8192_cubed_sampled_rows(dev, cube_8192):
    """8192^3 with the default (exact) tile kernel: 12 rows (tile edges
    included) against the oracle over all 8192 columns; the bf16 output is
    the round-to-nearest-even of the fp32 one everywhere."""
    qa, sa, bp, sb, ref, bound = cube_8192
    n = 8192
    y = capi.gemm(qa, sa, bp, sb, n, n, out_dtype=torch.float32, kernel=capi.KERNEL_MFMA)
    assert_close(y[torch.from_numpy(ROWS).to(dev)].cpu().numpy(), ref, bound)
    full_matrix_check(y, qa, sa, capi.unpack_weight(bp, n, n, w_is_nk=False), sb)
    # the bf16 output comes from the other 256x256 layout (2x2 wavefronts of
    # 128x128): bit for bit the rounding of the fp32 one on every element
    y16 = capi.gemm(qa, sa, bp, sb, n, n, out_dtype=torch.bfloat16, kernel=capi.KERNEL_MFMA)
    assert torch.equal(y16.view(torch.int16), y.to(torch.bfloat16).view(torch.int16))


def test_gemm_8192_cubed_native_fp8_sampled_rows(dev, cube_8192):
    """The native-FP8-MFMA tile kernel (the opt-in fast kernel) at 8192^3:
    inside the elementwise bound 1e-4 * sum|a*b| and below its documented
    relative Frobenius error of 3e-5 (gfx950 FP8 MFMA block truncation)."""
    qa, sa, bp, sb, ref, bound = cube_8192
    y = capi.gemm(qa, sa, bp, sb, 8192, 8192, out_dtype=torch.float32, kernel=capi.KERNEL_MFMA_FP8)
    ys = y[torch.from_numpy(ROWS).to(dev)].cpu().numpy().astype(np.float64)
    assert np.all(np.abs(ys - ref) <= 1e-4 * bound)
    rel = np.linalg.norm(ys - ref) / np.linalg.norm(ref)
    assert rel < 3e-5, rel
    full_matrix_check(y, qa, sa, capi.unpack_weight(bp, 8192, 8192, w_is_nk=False), sb, frob=3e-5)
    y16 = capi.gemm(qa, sa, bp, sb, 8192, 8192, out_dtype=torch.bfloat16, kernel=capi.KERNEL_MFMA_FP8)
    assert torch.equal(y16.view(torch.int16), y.to(torch.bfloat16).view(torch.int16))


def test_transformer_up_projection_gelu_sampled_rows(dev):
    """M=4096 x 4096 -> 11008 with bias and GELU, dynamic activation scale,
    per-channel weights (the up-projection of the transformer block)."""
    x = synth.normal(420, (4096, 4096))
    w = synth.normal(402, (4096, 11008), std=0.02)
    bias = synth.normal(412, (11008,), std=0.01)
    qw, sw, bp, d_sw = per_channel_weight(w, dev)
    y = capi.gemm_dynamic(to_dev(x, dev), bp, d_sw, 11008, 4096, c=to_dev(bias, dev), act=capi.ACT_GELU_ERF,
                          kernel=capi.KERNEL_MFMA)
    s_ref = np.float32(oracle.dynamic_scale(x))
    rows = ROWS[ROWS < 4096]
    ref, A, B = oracle.qlinear(oracle.quantize(x[rows], s_ref), s_ref, qw, sw, bias=bias, act=oracle.ACT_GELU_ERF)
    assert_close(y[torch.from_numpy(rows).to(dev)].cpu().numpy(), ref, oracle.gemm_abs_bound(A, B, bias),
                 act=oracle.ACT_GELU_ERF)
    # every element: GELU (exact erf, torch) of a GPU fp32 GEMM of the
    # dequantised operands, at the GELU tolerance of the oracle checks
    qx, sx = capi.quantize_dynamic(to_dev(x, dev))
    Ad = qx.view(torch.float8_e4m3fn).float() * sx
    Bd = capi.unpack_weight(bp, 4096, 11008, w_is_nk=False).view(torch.float8_e4m3fn).float() * d_sw
    d_b = to_dev(bias, dev)
    torch.backends.cuda.matmul.allow_tf32 = False
    pre = Ad @ Bd + d_b
    bound_all = Ad.abs() @ Bd.abs() + d_b.abs()
    del Ad, Bd
    bad = int((~((y - torch.nn.functional.gelu(pre)).abs() <= gelu_tol(oracle.ACT_GELU_ERF) * bound_all)).sum())
    assert bad == 0, f"{bad} elements outside the GELU tolerance"


@pytest.fixture(scope="module")
def block_input(dev):
    """The transformer block's activation x [4096, 4096] fp32 N(0,1), its
    dynamic scale (bit-exact against the oracle) and sampled rows."""
    x = synth.normal(420, (4096, 4096))
    return x, np.float32(oracle.dynamic_scale(x)), ROWS[ROWS < 4096]


def block_weight(i, K, N, dev):
    w = synth.normal(400 + i, (K, N), std=0.02)
    return per_channel_weight(w, dev) + (synth.normal(410 + i, (N,), std=0.01),)


@pytest.mark.parametrize("name,i,N", [("qkv", 0, 12288), ("o", 1, 4096)])
def test_transformer_qkv_and_o_projection_sampled_rows(dev, block_input, name, i, N):
    """QKV 4096 -> 12288 and O 4096 -> 4096 at M = 4096 (dynamic activation
    scale, per-channel weights, fp32 bias): the fp32 output on 12 sampled rows
    against the oracle; the bf16 output the block uses is the
    round-to-nearest-even of the fp32 output on every element."""
    x, s_ref, rows = block_input
    qw, sw, bp, d_sw, bias = block_weight(i, 4096, N, dev)
    d_x, d_b = to_dev(x, dev), to_dev(bias, dev)
    s_out = torch.empty(1, device=dev)
    y = capi.gemm_dynamic(d_x, bp, d_sw, N, 4096, c=d_b, out_dtype=torch.float32, scale_out=s_out)
    assert s_out.cpu().numpy().view(np.uint32)[0] == s_ref.view(np.uint32)
    ref, A, B = oracle.qlinear(oracle.quantize(x[rows], s_ref), s_ref, qw, sw, bias=bias)
    assert_close(y[torch.from_numpy(rows).to(dev)].cpu().numpy(), ref, oracle.gemm_abs_bound(A, B, bias))
    y16 = capi.gemm_dynamic(d_x, bp, d_sw, N, 4096, c=d_b, out_dtype=torch.bfloat16)
    assert torch.equal(y16.view(torch.int16), y.to(torch.bfloat16).view(torch.int16))
    qx, sx = capi.quantize_dynamic(d_x)
    full_matrix_check(y, qx.view(4096, 4096), sx, capi.unpack_weight(bp, 4096, N, w_is_nk=False), d_sw, bias=d_b)


def test_transformer_down_projection_from_gelu_output(dev, block_input):
    """Up 4096 -> 11008 + GELU (fp32 out), then down 11008 -> 4096 on that
    output: the down projection re-quantises the GELU output per tensor
    through the two-launch workspace path (amax partials + encode, then the
    tile kernel over K = 11008).  The scale is bit-exact against the oracle's
    amax/448 over the whole GPU up-projection output, the sampled rows' codes
    feed the oracle's Gemm."""
    x, s_ref, rows = block_input
    _, _, bp_up, d_sw_up, b_up = block_weight(2, 4096, 11008, dev)
    qw, sw, bp, d_sw, bias = block_weight(3, 11008, 4096, dev)
    h = capi.gemm_dynamic(to_dev(x, dev), bp_up, d_sw_up, 11008, 4096, c=to_dev(b_up, dev), act=capi.ACT_GELU_ERF)
    assert capi.lib().lcml_fp8_gemm_dynamic_workspace_bytes(4096, 11008, capi.KERNEL_AUTO) > 0  # two-step path
    s_out = torch.empty(1, device=dev)
    y = capi.gemm_dynamic(h, bp, d_sw, 4096, 11008, c=to_dev(bias, dev), out_dtype=torch.float32, scale_out=s_out)
    h_host = h.cpu().numpy()
    sh_ref = np.float32(oracle.dynamic_scale(h_host))
    assert s_out.cpu().numpy().view(np.uint32)[0] == sh_ref.view(np.uint32)
    ref, A, B = oracle.qlinear(oracle.quantize(h_host[rows], sh_ref), sh_ref, qw, sw, bias=bias)
    assert_close(y[torch.from_numpy(rows).to(dev)].cpu().numpy(), ref, oracle.gemm_abs_bound(A, B, bias))
    qh, shd = capi.quantize_dynamic(h)
    full_matrix_check(y, qh.view(4096, 11008), shd, capi.unpack_weight(bp, 11008, 4096, w_is_nk=False), d_sw,
                      bias=to_dev(bias, dev))
    # the chained form the benchmark runs: the up-projection's epilogue writes
    # the partial maxima of its output, and the down-projection quantises
    # from them without an amax pass -- the same scale and output, bit for bit
    part = capi.amax_parts_buffer(4096, 11008, dev)
    h2, n = capi.gemm_dynamic_ex(to_dev(x, dev), bp_up, d_sw_up, 11008, 4096, c=to_dev(b_up, dev),
                                 act=capi.ACT_GELU_ERF, y_amax_part=part)
    assert torch.equal(h2.view(torch.int32), h.view(torch.int32))
    assert part[:n].cpu().numpy().view(np.float32).max() == np.abs(h_host).max()
    s2 = torch.empty(1, device=dev)
    y2, _ = capi.gemm_dynamic_ex(h2, bp, d_sw, 4096, 11008, c=to_dev(bias, dev), out_dtype=torch.float32,
                                 scale_out=s2, x_amax=(part, n))
    assert s2.cpu().numpy().view(np.uint32)[0] == sh_ref.view(np.uint32)
    assert torch.equal(y2.view(torch.int32), y.view(torch.int32))


NATIVE_FROB = 3e-5  # documented relative Frobenius error of the native FP8 MFMA kernels (block truncation)


def check_native(y_rows, ref, bound, act=oracle.ACT_NONE):
    """Sampled outputs of a native-FP8-MFMA kernel against the oracle: the
    elementwise bar (with GELU's tolerance where it applies) and relative
    Frobenius below NATIVE_FROB."""
    y_rows = np.asarray(y_rows, np.float64)
    assert_close(y_rows, ref, bound, act=act, frob=False)
    rel = np.linalg.norm(y_rows - ref) / np.linalg.norm(ref)
    assert rel < NATIVE_FROB, rel


@pytest.mark.parametrize("name,i,K,N", [("qkv", 0, 4096, 12288), ("o", 1, 4096, 4096), ("up", 2, 4096, 11008),
                                        ("down", 3, 11008, 4096)])
def test_transformer_linears_native_fp8_full(dev, block_input, name, i, K, N):
    """The four M = 4096 transformer linears on the native-FP8-MFMA tile
    kernel (KERNEL_MFMA_FP8, as the benchmark's native line runs them):
    dynamic activation scale (bit-exact), per-channel weights, fp32 bias,
    GELU on the up-projection, the down-projection fed by the up-projection's
    GELU output of the same kernel.  Sampled rows against the oracle and
    every element against a GPU fp32 GEMM of the dequantised operands, both
    at the elementwise bar and below the documented relative Frobenius
    error; the bf16 output is the rounding of the fp32 one."""
    x, s_ref, rows = block_input
    qw, sw, bp, d_sw, bias = block_weight(i, K, N, dev)
    d_b = to_dev(bias, dev)
    act = oracle.ACT_GELU_ERF if name == "up" else oracle.ACT_NONE
    if name == "down":
        _, _, bp_up, d_sw_up, b_up = block_weight(2, 4096, 11008, dev)
        d_x = capi.gemm_dynamic(to_dev(x, dev), bp_up, d_sw_up, 11008, 4096, c=to_dev(b_up, dev),
                                act=capi.ACT_GELU_ERF, kernel=capi.KERNEL_MFMA_FP8)
        x = d_x.cpu().numpy()
        s_ref = np.float32(oracle.dynamic_scale(x))
    else:
        d_x = to_dev(x, dev)
    s_out = torch.empty(1, device=dev)
    y = capi.gemm_dynamic(d_x, bp, d_sw, N, K, c=d_b, act=act, out_dtype=torch.float32, scale_out=s_out,
                          kernel=capi.KERNEL_MFMA_FP8)
    assert s_out.cpu().numpy().view(np.uint32)[0] == s_ref.view(np.uint32)
    ref, A, B = oracle.qlinear(oracle.quantize(x[rows], s_ref), s_ref, qw, sw, bias=bias, act=act)
    check_native(y[torch.from_numpy(rows).to(dev)].cpu().numpy(), ref, oracle.gemm_abs_bound(A, B, bias), act=act)
    if name != "up":
        y16 = capi.gemm_dynamic(d_x, bp, d_sw, N, K, c=d_b, out_dtype=torch.bfloat16, kernel=capi.KERNEL_MFMA_FP8)
        assert torch.equal(y16.view(torch.int16), y.to(torch.bfloat16).view(torch.int16))
    qx, sx = capi.quantize_dynamic(d_x)
    Ad = qx.view(torch.float8_e4m3fn).float() * sx
    Bd = capi.unpack_weight(bp, K, N, w_is_nk=False).view(torch.float8_e4m3fn).float() * d_sw
    torch.backends.cuda.matmul.allow_tf32 = False
    pre = Ad @ Bd + d_b
    bound_all = Ad.abs() @ Bd.abs() + d_b.abs()
    del Ad, Bd
    ref_all = torch.nn.functional.gelu(pre) if name == "up" else pre
    bad = int((~((y - ref_all).abs() <= gelu_tol(act) * bound_all)).sum())
    assert bad == 0, f"{bad} elements outside the elementwise bar"
    rel = float(torch.linalg.vector_norm(y - ref_all) / torch.linalg.vector_norm(ref_all))
    assert rel < NATIVE_FROB, rel


@pytest.mark.parametrize("kernel", [capi.KERNEL_AUTO, capi.KERNEL_MFMA_FP8], ids=["auto", "native_fp8"])
def test_conv3x3_resnet_one_image(dev, kernel):
    """x[32,256,56,56] -> NHWC E4M3 (dynamic) -> 3x3 conv pad 1, 256 out,
    per-channel weights, bias + ReLU; image 5 of the batch against the
    oracle's direct conv, all 32 images against a GPU fp32 direct conv.
    AUTO takes the exact tile kernel (relative Frobenius 1e-5); the native
    FP8 MFMA kernel (the benchmark's native line) is held to its documented
    3e-5."""
    x = synth.normal(600, (32, 256, 56, 56))
    w = synth.normal(601, (256, 256, 3, 3), std=0.03)
    bias = synth.normal(602, (256,), std=0.01)
    ws = oracle.channel_scales(w.reshape(256, -1), 0)
    qw = oracle.quantize(w.reshape(256, -1), ws, axis=0).reshape(w.shape)
    xq, sx = capi.quantize_nhwc(to_dev(x, dev))
    s_ref = np.float32(oracle.dynamic_scale(x))
    assert float(sx.item()) == s_ref
    y = capi.conv2d(xq, sx, capi.pack_conv_weight(to_dev(qw, dev)), to_dev(ws, dev), 256, (3, 3), pads=(1, 1),
                    bias=to_dev(bias, dev), act=capi.ACT_RELU, kernel=kernel)
    img = 5
    xi = x[img:img + 1]
    assert np.array_equal(xq[img].cpu().numpy(), oracle.quantize(xi, s_ref)[0].transpose(1, 2, 0))
    A = oracle.dequantize(oracle.quantize(xi, s_ref), s_ref)
    B = oracle.dequantize(qw.reshape(256, -1), ws, axis=0).reshape(qw.shape)
    ref = oracle.conv2d(A, B, bias, pads=(1, 1), act=oracle.ACT_RELU)
    bound = oracle.conv2d(np.abs(A), np.abs(B), np.abs(bias), pads=(1, 1))
    if kernel == capi.KERNEL_MFMA_FP8:
        check_native(y[img:img + 1].cpu().numpy(), ref, bound, act=oracle.ACT_RELU)
    else:
        assert_close(y[img:img + 1].cpu().numpy(), ref, bound, act=oracle.ACT_RELU)
    # all 32 images against torch's fp32 direct conv of the dequantised
    # operands on the GPU (MIOpen off: no Winograd transform in the reference)
    xd = xq.view(torch.float8_e4m3fn).float().permute(0, 3, 1, 2).contiguous() * sx
    wd = torch.from_numpy(B).to(dev)
    d_b = to_dev(bias, dev)
    cudnn = torch.backends.cudnn.enabled
    torch.backends.cudnn.enabled = False
    try:
        ref_all = torch.relu(torch.nn.functional.conv2d(xd, wd, d_b, padding=1))
        bound_all = torch.nn.functional.conv2d(xd.abs(), wd.abs(), d_b.abs(), padding=1)
    finally:
        torch.backends.cudnn.enabled = cudnn
    bad = int((~((y - ref_all).abs() <= 1e-4 * bound_all)).sum())
    assert bad == 0, f"{bad} conv outputs outside 1e-4 * sum|xw|"
    rel = float(torch.linalg.vector_norm(y - ref_all) / torch.linalg.vector_norm(ref_all))
    assert rel < (NATIVE_FROB if kernel == capi.KERNEL_MFMA_FP8 else 1e-5), rel


@pytest.mark.parametrize("M", [64, 256, 512])
def test_decode_linear_medium_m_auto(dev, decode_weight, M):
    """The same 4096x11008 linear past decode sizes, through AUTO (skinny
    kernel with row groups at M=64, 128x128 tiles at M=256 and 512), fp32
    out; 12 sampled rows against the oracle."""
    qw, sw, bp, d_sw = decode_weight
    x = synth.normal(700 + M, (M, 4096))
    y = capi.gemm_dynamic(to_dev(x, dev), bp, d_sw, 11008, 4096, out_dtype=torch.float32)
    s_ref = np.float32(oracle.dynamic_scale(x))
    rows = np.unique(np.array([0, 1, 15, 16, 31, 32, 63, M // 2, M - 17, M - 2, M - 1]) % M)
    ref, A, B = oracle.qlinear(oracle.quantize(x[rows], s_ref), s_ref, qw, sw)
    assert_close(y[torch.from_numpy(rows).to(dev)].cpu().numpy(), ref, oracle.gemm_abs_bound(A, B))


def test_mid_size_gemm_128_tiles_sampled_rows(dev):
    """M=2048 x 4096 -> 4096, where AUTO takes the 128x128 tiles; the 256x256
    kernel's output on the same operands agrees within the bound too."""
    x = synth.normal(710, (2048, 4096))
    w = synth.normal(711, (4096, 4096), std=0.02)
    qw, sw, bp, d_sw = per_channel_weight(w, dev)
    qa, sa = capi.quantize_dynamic(to_dev(x, dev))
    s_ref = np.float32(oracle.dynamic_scale(x))
    rows = np.array([0, 127, 128, 1000, 2047])
    ref, A, B = oracle.qlinear(oracle.quantize(x[rows], s_ref), s_ref, qw, sw)
    bound = oracle.gemm_abs_bound(A, B)
    for kernel in (capi.KERNEL_AUTO, capi.KERNEL_MFMA_128, capi.KERNEL_MFMA):
        y = capi.gemm(qa, sa, bp, d_sw, 4096, 4096, out_dtype=torch.float32, kernel=kernel)
        assert_close(y[torch.from_numpy(rows).to(dev)].cpu().numpy(), ref, bound)
