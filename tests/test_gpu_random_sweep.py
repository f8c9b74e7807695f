"""Seeded random sweep over the FP8 GEMM entry points: each case draws the
kernel, shape, weight layout and scale kind, activation, C broadcast, alpha,
beta, output type and output layout at once, so that feature combinations
the one-feature tests do not pair up are still checked against the oracle's
dequantise-then-Gemm (reference src/onnx/operators/gemm.cpp:27-325).

Bars (per case):
  * exact kernels (mfma, mfma_128, skinny, valu): |y - y_ref| <= tol * bound
    elementwise, tol the summation-order bar (GELU: its Lipschitz factor and
    evaluation allowance), and relative Frobenius <= 1e-5 for fp32 output;
  * native FP8-MFMA kernels: the same elementwise bar and relative Frobenius
    <= 3e-5 (their documented in-instruction truncation);
  * bf16 output: the elementwise bar plus the bf16 rounding of the result,
    2^-8 * |y_ref|;
  * nothing outside the [M, N] output view is written;
  * lcml_fp8_gemm_dynamic: the returned scale is bit-exact with the oracle's
    amax/448, and the output meets the bars above.
"""
import numpy as np
import pytest
import torch

import oracle
from luisaml_amd import capi, synth
from tests.gemm_cases import TOL_FROB, gelu_tol

pytestmark = pytest.mark.gpu

EXACT = {"mfma": capi.KERNEL_MFMA, "mfma_128": capi.KERNEL_MFMA_128, "skinny": capi.KERNEL_SKINNY,
         "valu": capi.KERNEL_VALU, "auto": capi.KERNEL_AUTO}
NATIVE = {"mfma_fp8": capi.KERNEL_MFMA_FP8, "mfma_128_fp8": capi.KERNEL_MFMA_128_FP8,
          "skinny_fp8": capi.KERNEL_SKINNY_FP8}
# the opt-in AUTO_FP8 (AUTO's tiling on the native FP8 kernels): drawn in
# cases of its own, so the draws of the cases above stay as they were
OPT_IN = {"auto_fp8": capi.KERNEL_AUTO_FP8}
FP8_FROB = 3e-5
ACTS = [capi.ACT_NONE, capi.ACT_RELU, capi.ACT_GELU_ERF, capi.ACT_GELU_TANH]
C_KINDS = [None, "N", "1", "scalar", "M1", "MN", "1N", "M"]
FILL = -7777.0


def draw_case(i):
    rng = np.random.default_rng(20_000 + i)
    names = list(EXACT) + list(NATIVE)
    kname = names[rng.integers(len(names))]
    small = kname in ("skinny", "skinny_fp8", "valu") or rng.random() < 0.3
    M = int(rng.integers(1, 17)) if small and rng.random() < 0.6 else int(rng.integers(1, 300))
    N = int(rng.integers(1, 700))
    K = 16 * int(rng.integers(1, 80 if rng.random() < 0.8 else 300))
    return dict(
        kname=kname, M=M, N=N, K=K,
        w_is_nk=bool(rng.random() < 0.5),
        per_channel=bool(rng.random() < 0.7),
        act=ACTS[rng.integers(len(ACTS))],
        c_kind=C_KINDS[rng.integers(len(C_KINDS))],
        alpha=float(rng.choice([1.0, 0.75, -2.0])),
        beta=float(rng.choice([1.0, 0.5, 0.0])),
        bf16=bool(rng.random() < 0.5),
        layout=["dense", "pitch", "misaligned"][rng.integers(3)],
        pitch_pad=int(rng.integers(1, 18)),
        a_std=float(rng.choice([1.0, 30.0, 1e-3])),
        seed=int(rng.integers(1 << 30)),
    )


def make_c(kind, M, N, seed):
    if kind is None:
        return None
    if kind == "M" and M == N:  # a 1-D C of length N broadcasts over rows; keep the case unambiguous
        kind = "N"
    shape = {"N": (N,), "1": (1,), "scalar": (), "M1": (M, 1), "MN": (M, N), "1N": (1, N), "M": (M,)}[kind]
    return np.array(np.random.default_rng(seed).standard_normal(shape) * 0.05, dtype=np.float32)


SPARE_ROWS = 256  # buffer rows past M: the stores of a tile's rows past M must be dropped


def out_buffer(layout, M, N, pad, dtype, dev):
    """The output view in a larger buffer filled with FILL (256 spare rows
    past M in every layout), and the mask of the elements outside the view."""
    if layout == "dense":
        buf = torch.full((M + SPARE_ROWS, N), FILL, dtype=dtype, device=dev)
        mask = torch.ones_like(buf, dtype=torch.bool)
        mask[:M] = False
        return buf, buf[:M], mask
    if layout == "pitch":
        buf = torch.full((M + SPARE_ROWS, N + pad), FILL, dtype=dtype, device=dev)
        mask = torch.ones_like(buf, dtype=torch.bool)
        mask[:M, :N] = False
        return buf, buf[:M, :N], mask
    buf = torch.full(((M + SPARE_ROWS) * N + 1,), FILL, dtype=dtype, device=dev)
    mask = torch.ones_like(buf, dtype=torch.bool)
    mask[1:1 + M * N] = False
    return buf, buf[1:1 + M * N].view(M, N), mask


def check(y, ref, bound, p):
    y = y.float().cpu().numpy().astype(np.float64) if p["bf16"] else y.cpu().numpy().astype(np.float64)
    ref = np.asarray(ref, np.float64)
    tol = gelu_tol(p["act"]) * bound
    if p["bf16"]:
        tol = tol * (1 + 2.0 ** -8) + 2.0 ** -8 * np.abs(ref)
    d = np.abs(y - ref)
    bad = np.argwhere(~(d <= tol))
    assert bad.size == 0, (f"{p}: {len(bad)} elements outside tolerance; first {bad[:3].tolist()}: "
                           f"got {y[tuple(bad[0])]} ref {ref[tuple(bad[0])]} tol {tol[tuple(bad[0])]}")
    if not p["bf16"]:
        nr = np.linalg.norm(ref)
        rel = np.linalg.norm(y - ref) / nr if nr > 0 else np.linalg.norm(y)
        lim = FP8_FROB if p["kname"] in NATIVE or p["kname"] in OPT_IN else TOL_FROB
        assert rel <= lim, f"{p}: relative Frobenius error {rel:.3e} > {lim}"


def weights(p, dev):
    K, N = p["K"], p["N"]
    w = synth.normal(p["seed"] + 2, (N, K) if p["w_is_nk"] else (K, N), std=0.02)
    axis = 0 if p["w_is_nk"] else 1
    sw = oracle.channel_scales(w, axis) if p["per_channel"] else np.array([oracle.dynamic_scale(w)], np.float32)
    qw = oracle.quantize(w, sw, axis=axis) if p["per_channel"] else oracle.quantize(w, sw)
    bp = capi.pack_weight(torch.from_numpy(qw).to(dev), p["w_is_nk"])
    return qw, sw, bp, torch.from_numpy(sw).to(dev)


def oracle_out(qa, sa, qw, sw, C, p):
    A = oracle.dequantize(qa, sa)
    B = oracle.dequantize(qw, sw, axis=0 if p["w_is_nk"] else 1) if sw.size > 1 else oracle.dequantize(qw, sw)
    tb = int(p["w_is_nk"])
    Y = oracle.gemm(A, B, C, alpha=p["alpha"], beta=p["beta"], transB=tb, act=p["act"])
    bound = oracle.gemm_abs_bound(A, B, C, alpha=p["alpha"], beta=p["beta"], transB=tb)
    return Y, bound


def run_case(p, dev, dynamic):
    M, N, K = p["M"], p["N"], p["K"]
    kernel = {**EXACT, **NATIVE, **OPT_IN}[p["kname"]]
    print(f"case {p}", flush=True)
    x = synth.normal(p["seed"] + 1, (M, K), std=p["a_std"])
    sa = np.float32(oracle.dynamic_scale(x))
    qa = oracle.quantize(x, sa)
    qw, sw, bp, d_sw = weights(p, dev)
    C = make_c(p["c_kind"], M, N, p["seed"] + 3)
    d_c = None if C is None else torch.from_numpy(C).to(dev)
    buf, view, mask = out_buffer(p["layout"], M, N, p["pitch_pad"],
                                 torch.bfloat16 if p["bf16"] else torch.float32, dev)
    kw = dict(c=d_c, alpha=p["alpha"], beta=p["beta"], act=p["act"], kernel=kernel, out=view)
    if dynamic:
        s_out = torch.empty(1, dtype=torch.float32, device=dev)
        capi.gemm_dynamic(torch.from_numpy(x).to(dev), bp, d_sw, N, K, scale_out=s_out, **kw)
        torch.cuda.synchronize()
        assert s_out.cpu().numpy().view(np.uint32)[0] == sa.view(np.uint32), f"{p}: dynamic scale"
    else:
        capi.gemm(torch.from_numpy(qa).to(dev), torch.from_numpy(np.array([sa], np.float32)).to(dev), bp, d_sw,
                  N, K, **kw)
        torch.cuda.synchronize()
    ref, bound = oracle_out(qa, sa, qw, sw, C, p)
    check(view, ref, bound, p)
    if mask is not None:
        assert bool((buf.cpu()[mask.cpu()] == FILL).all()), f"{p}: write outside the output view"


@pytest.mark.parametrize("i", range(256))
def test_random_gemm(dev, i):
    run_case(draw_case(i), dev, dynamic=False)


@pytest.mark.parametrize("i", range(64))
def test_random_gemm_dynamic(dev, i):
    run_case(draw_case(1000 + i), dev, dynamic=True)


CONV_KERNELS = {"auto": capi.KERNEL_AUTO, "mfma": capi.KERNEL_MFMA, "mfma_128": capi.KERNEL_MFMA_128,
                "mfma_fp8": capi.KERNEL_MFMA_FP8, "mfma_128_fp8": capi.KERNEL_MFMA_128_FP8}


def draw_conv(i):
    rng = np.random.default_rng(30_000 + i)
    group = int(rng.choice([1, 1, 1, 2, 4]))
    c = 16 * group * int(rng.integers(1, 5))
    cout = group * int(rng.integers(1, 300 // group))
    kh, kw = int(rng.choice([1, 2, 3, 5])), int(rng.choice([1, 3, 5]))
    dil = int(rng.choice([1, 1, 2]))
    pad = int(rng.integers(0, 3))
    h = int(rng.integers(max(1, dil * (kh - 1) + 1 - 2 * pad), 20))
    w = int(rng.integers(max(1, dil * (kw - 1) + 1 - 2 * pad), 20))
    return dict(
        kname=list(CONV_KERNELS)[rng.integers(len(CONV_KERNELS))],
        n=int(rng.integers(1, 4)), c=c, h=h, w=w, cout=cout, kh=kh, kw=kw,
        stride=int(rng.integers(1, 4)), pad=pad, dil=dil, group=group,
        per_channel=bool(rng.random() < 0.7),
        act=ACTS[rng.integers(len(ACTS))],
        bias=bool(rng.random() < 0.7),
        bf16=bool(rng.random() < 0.5),
        offset=int(rng.integers(0, 2)),
        seed=int(rng.integers(1 << 30)),
    )


@pytest.mark.parametrize("i", range(96))
def test_random_conv(dev, i):
    """Implicit-im2col FP8 conv (NHWC E4M3 in, NCHW out) against the oracle's
    direct conv of the dequantised operands (conv.cpp:115-207)."""
    run_conv(draw_conv(i), dev)


@pytest.mark.parametrize("i", range(48))
def test_random_gemm_auto_fp8(dev, i):
    """LCML_KERNEL_AUTO_FP8 through lcml_fp8_gemm (two cases in three) and
    lcml_fp8_gemm_dynamic, at the native-FP8 bars."""
    p = draw_case(5000 + i)
    p["kname"] = "auto_fp8"
    run_case(p, dev, dynamic=i % 3 == 0)


@pytest.mark.parametrize("i", range(24))
def test_random_conv_auto_fp8(dev, i):
    p = draw_conv(6000 + i)
    p["kname"] = "auto_fp8"
    run_conv(p, dev)


def run_conv(p, dev):
    print(f"case {p}", flush=True)
    n, c, h, w, cout, kh, kw, g = p["n"], p["c"], p["h"], p["w"], p["cout"], p["kh"], p["kw"], p["group"]
    st, pd, dl = (p["stride"],) * 2, (p["pad"],) * 2, (p["dil"],) * 2
    x = synth.normal(p["seed"], (n, c, h, w))
    wt = synth.normal(p["seed"] + 1, (cout, c // g, kh, kw), std=0.03)
    if p["per_channel"]:
        ws = oracle.channel_scales(wt.reshape(cout, -1), 0)
        qw = oracle.quantize(wt.reshape(cout, -1), ws, axis=0).reshape(wt.shape)
        B = oracle.dequantize(qw.reshape(cout, -1), ws, axis=0).reshape(qw.shape)
    else:
        ws = np.array([oracle.dynamic_scale(wt)], np.float32)
        qw = oracle.quantize(wt, ws)
        B = oracle.dequantize(qw, ws)
    bias = synth.normal(p["seed"] + 2, (cout,), std=0.05) if p["bias"] else None
    sx = np.float32(oracle.dynamic_scale(x))
    A = oracle.dequantize(oracle.quantize(x, sx), sx)
    ref = oracle.conv2d(A, B, bias, strides=st, pads=pd, dilations=dl, group=g, act=p["act"])
    bound = oracle.conv2d(np.abs(A), np.abs(B), None if bias is None else np.abs(bias), strides=st, pads=pd,
                          dilations=dl, group=g)
    dtype = torch.bfloat16 if p["bf16"] else torch.float32
    total = ref.size
    buf = torch.full((total + 2,), FILL, dtype=dtype, device=dev)
    out = buf[p["offset"]:p["offset"] + total].view(ref.shape)
    xq, d_sx = capi.quantize_nhwc(torch.from_numpy(x).to(dev))
    capi.conv2d(xq, d_sx, capi.pack_conv_weight(torch.from_numpy(qw).to(dev), group=g),
                torch.from_numpy(ws).to(dev), cout, (kh, kw), st, pd, dl,
                bias=None if bias is None else torch.from_numpy(bias).to(dev), act=p["act"],
                kernel={**CONV_KERNELS, **OPT_IN}[p["kname"]], out=out, group=g)
    torch.cuda.synchronize()
    assert d_sx.cpu().numpy().view(np.uint32)[0] == sx.view(np.uint32)
    check(out, ref, bound, p)
    outside = torch.ones_like(buf, dtype=torch.bool)
    outside[p["offset"]:p["offset"] + total] = False
    assert bool((buf.cpu()[outside.cpu()] == FILL).all()), f"{p}: write outside the output"
