"""CPU checks that pin the oracle's Gemm / activations / Conv.

  * the reference's own golden vectors: the fp32 MLP fixture of
    tests/onnx/test_onnx_inference.cpp:115-302 (Gemm transB=1 + bias + Relu,
    784->256->256->10), compared with the 1e-3 tolerance the reference uses
    (test_onnx_inference.cpp:232-241);
  * brute force in float64 on small shapes; alpha/beta/bias broadcast rules of
    gemm.cpp:81-110 against numpy broadcasting; linearity and one-hot
    invariants of the dequantise-then-Gemm composition;
  * GELU against an exact erf (the A&S erf is accurate to 1.5e-7);
  * Conv against im2col times Gemm and a float64 direct sum.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle
from luisaml_amd import synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_reference_mlp():
    j = json.load(open(os.path.join(GOLDEN, "simple_mlp.onnx.json")))
    blob = open(os.path.join(GOLDEN, "simple_mlp.safetensors"), "rb").read()
    inits = {}
    for ini in j["graph"]["initializer"]:
        a, b = ini["data_offsets"]
        shape = tuple(int(d) for d in ini["dims"])
        inits[ini["name"]] = np.frombuffer(blob[a:b], np.float32).reshape(shape)
    x = np.fromfile(os.path.join(GOLDEN, "input_ref.bin"), np.float32).reshape(1, 784)
    y = np.fromfile(os.path.join(GOLDEN, "output_ref.bin"), np.float32).reshape(1, 10)
    return j["graph"], inits, x, y


def test_reference_mlp_fixture_fp32():
    graph, w, x, y_ref = load_reference_mlp()
    act = x
    vals = {"input": x}
    for node in graph["node"]:
        ins = [vals.get(n, w.get(n)) for n in node["input"]]
        if node["op_type"] == "Gemm":
            at = {a["name"]: a for a in node.get("attribute", [])}
            out = oracle.gemm(ins[0], ins[1], ins[2], alpha=at["alpha"]["f"], beta=at["beta"]["f"],
                              transA=int(at["transA"]["i"]), transB=int(at["transB"]["i"]))
        elif node["op_type"] == "Relu":
            out = oracle.activation(ins[0], oracle.ACT_RELU)
        else:
            raise AssertionError(node["op_type"])
        vals[node["output"][0]] = out
    got = vals["output"]
    assert np.all(np.abs(got - y_ref) <= 1e-3), (got, y_ref)


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (3, 5, 7), (16, 9, 33), (40, 70, 300)])
@pytest.mark.parametrize("tA,tB", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_vs_float64(M, N, K, tA, tB):
    rng = np.random.default_rng(M * 100 + N + K)
    A = rng.standard_normal((K, M) if tA else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if tB else (K, N)).astype(np.float32)
    got = oracle.gemm(A, B, transA=tA, transB=tB)
    Ad = A.T.astype(np.float64) if tA else A.astype(np.float64)
    Bd = B.T.astype(np.float64) if tB else B.astype(np.float64)
    exact = Ad @ Bd
    bound = np.abs(Ad) @ np.abs(Bd)
    assert np.all(np.abs(got - exact) <= K * 2.0 ** -24 * bound + 1e-30)


@pytest.mark.parametrize("kind", ["scalar", "1", "N", "M", "1N", "M1", "MN"])
def test_gemm_bias_broadcast_and_alpha_beta(kind):
    M, N, K = 6, 5, 4
    rng = np.random.default_rng(1)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    shape = {"scalar": (), "1": (1,), "N": (N,), "M": (M,), "1N": (1, N), "M1": (M, 1), "MN": (M, N)}[kind]
    C = rng.standard_normal(shape).astype(np.float32)
    alpha, beta = np.float32(0.5), np.float32(-2.0)
    got = oracle.gemm(A, B, C, alpha=alpha, beta=beta)
    # numpy broadcasting, except the reference's 1-D length-M (!= N) rule:
    # a 1-D C whose length is not N is indexed by row (gemm.cpp:87-91).
    Cb = C.reshape(M, 1) if kind == "M" else C
    want = (oracle.gemm(A, B) * alpha) + beta * np.broadcast_to(Cb, (M, N)).astype(np.float32)
    assert np.array_equal(got, want.astype(np.float32))


def test_gemm_sequential_fma_order():
    """Each output is one fma chain over k from 0: sum_k fma(a_k, b_k, s)."""
    rng = np.random.default_rng(5)
    a = (rng.standard_normal(257) * 1e3).astype(np.float32)
    b = rng.standard_normal(257).astype(np.float32)
    s = np.float32(0)
    for k in range(257):
        s = np.float32(math.fma(float(a[k]), float(b[k]), float(s))) if hasattr(math, "fma") else \
            np.float32(np.float64(a[k]) * np.float64(b[k]) + np.float64(s))
    got = oracle.gemm(a.reshape(1, -1), b.reshape(-1, 1))[0, 0]
    assert got == s


def test_qlinear_linearity_and_one_hot():
    rng = np.random.default_rng(2)
    K, N = 64, 48
    qb = oracle.quantize(rng.standard_normal((K, N)).astype(np.float32), 0.01)
    sb = oracle.channel_scales(rng.standard_normal((K, N)).astype(np.float32), axis=1)
    # one-hot rows select rows of DQ(B)
    qa = np.zeros((K, K), np.uint8)
    qa[np.arange(K), np.arange(K)] = 0x38  # 1.0
    Y, _, B = oracle.qlinear(qa, 1.0, qb, sb)
    assert np.array_equal(Y, B)
    # scaling the activation scale by 2 scales the output by 2 exactly
    qa2 = oracle.quantize(rng.standard_normal((8, K)).astype(np.float32), 0.05)
    Y1, _, _ = oracle.qlinear(qa2, 0.5, qb, sb)
    Y2, _, _ = oracle.qlinear(qa2, 1.0, qb, sb)
    assert np.array_equal(2 * Y1, Y2)


def test_gelu_against_exact_erf():
    x = np.linspace(-8, 8, 20001, dtype=np.float32)
    got = oracle.activation(x, oracle.ACT_GELU_ERF).astype(np.float64)
    xd = x.astype(np.float64)
    exact = 0.5 * xd * (1 + np.vectorize(math.erf)(xd / math.sqrt(2)))
    assert np.max(np.abs(got - exact)) < 2e-6 * 8
    tanh = oracle.activation(x, oracle.ACT_GELU_TANH).astype(np.float64)
    exact_t = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd ** 3)))
    assert np.max(np.abs(tanh - exact_t)) < 1e-5
    relu = oracle.activation(x, oracle.ACT_RELU)
    assert np.array_equal(relu, np.maximum(x, 0))


def _im2col_conv(X, W, bias, stride, pad, dil, group=1):
    """Conv as one GEMM over im2col columns in float64.  With groups the
    weight matrix is block diagonal: output channel m (group m // (M/group))
    sees only its group's Cg input channels (conv.cpp:139,158), zeros
    elsewhere -- an arithmetic independent of the oracle's group loop."""
    N, C, H, Wd = X.shape
    M, Cg, kH, kW = W.shape
    assert Cg * group == C and M % group == 0
    Wfull = np.zeros((M, C, kH, kW), np.float64)
    Mg = M // group
    for m in range(M):
        g = m // Mg
        Wfull[m, g * Cg:(g + 1) * Cg] = W[m]
    W = Wfull
    oH = (H + 2 * pad - dil * (kH - 1) - 1) // stride + 1
    oW = (Wd + 2 * pad - dil * (kW - 1) - 1) // stride + 1
    Xp = np.zeros((N, C, H + 2 * pad, Wd + 2 * pad), np.float64)
    Xp[:, :, pad:pad + H, pad:pad + Wd] = X
    cols = np.zeros((N, oH, oW, C, kH, kW))
    for kh in range(kH):
        for kw in range(kW):
            cols[:, :, :, :, kh, kw] = Xp[:, :, kh * dil: kh * dil + stride * oH: stride,
                                           kw * dil: kw * dil + stride * oW: stride].transpose(0, 2, 3, 1)
    Y = cols.reshape(N * oH * oW, -1) @ W.reshape(M, -1).T.astype(np.float64)
    Y = Y.reshape(N, oH, oW, M).transpose(0, 3, 1, 2)
    if bias is not None:
        Y += bias.reshape(1, M, 1, 1)
    return Y


@pytest.mark.parametrize("stride,pad,dil", [(1, 1, 1), (2, 0, 1), (1, 2, 2)])
def test_conv_against_im2col(stride, pad, dil):
    X = synth.normal(1, (2, 8, 9, 11))
    W = synth.normal(2, (6, 8, 3, 3), std=0.2)
    b = synth.normal(3, (6,), std=0.1)
    got = oracle.conv2d(X, W, b, strides=(stride, stride), pads=(pad, pad), dilations=(dil, dil))
    want = _im2col_conv(X, W, b, stride, pad, dil)
    assert got.shape == want.shape
    assert np.max(np.abs(got - want)) < 1e-4


@pytest.mark.parametrize("group,stride,pad,dil", [(2, 1, 1, 1), (4, 2, 1, 1), (8, 1, 2, 2), (3, 1, 0, 1)])
def test_grouped_conv_against_block_diagonal_im2col(group, stride, pad, dil):
    """The oracle's grouped conv (group g reads input channels g*Cg.. and
    writes output channels g*M/group.., conv.cpp:139,158) against im2col with
    a block-diagonal weight; depthwise (group = C = M) included."""
    C = 24 if group == 3 else 8
    M = 12 if group == 3 else 8
    X = synth.normal(11 + group, (2, C, 9, 11))
    W = synth.normal(12 + group, (M, C // group, 3, 3), std=0.2)
    b = synth.normal(13 + group, (M,), std=0.1)
    got = oracle.conv2d(X, W, b, strides=(stride, stride), pads=(pad, pad), dilations=(dil, dil), group=group)
    want = _im2col_conv(X, W, b, stride, pad, dil, group=group)
    assert got.shape == want.shape
    assert np.max(np.abs(got - want)) < 1e-4
    # a plausible slip (every group reading group 0's channels) is caught
    if group > 1:
        wrong = _im2col_conv(X[:, :C // group].repeat(group, axis=1), W, b, stride, pad, dil, group=group)
        assert np.max(np.abs(got - wrong)) > 1e-2
