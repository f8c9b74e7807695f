"""Device activations against the oracle's fp32 evaluation of the reference's
formulas: ReLU (src/onnx/operators/unary.cpp:85) and GELU, exact
(x*0.5*(1+erf(x/sqrt2)) with the A&S erf, src/onnx/operators/gelu.cpp:122-126,
include/onnx/operators/common.h:176-195) and tanh (gelu.cpp:84-91).

The device evaluates the A&S erf with the hardware reciprocal and exponential
(the GEMM epilogues and the standalone activation kernel share the code).
This test pins how far that evaluation may drift from the oracle's:
    |gelu_device(x) - gelu_oracle(x)| <= GELU_EVAL_C * 2^-24 * |x|
on a dense grid over [-12, 12] and on every 4099th positive fp32 bit pattern
(and its negative).  The bound is in units of |x| rather than of the result
because 1 + erf(x/sqrt2) cancels for negative x: there both evaluations are
exact to a few units of 2^-24 in erf, i.e. in |x|, while the result itself is
tiny.  The GEMM tests use it: a pre-activation is at most the bound
sum|a*b| + |bias| in magnitude, so the epilogue's evaluation adds at most
GELU_EVAL_C * 2^-24 times that bound on top of GELU's Lipschitz constant
(1.13) times the pre-activation's summation-order error.
"""
import numpy as np
import pytest
import torch

import oracle
from luisaml_amd import capi
from tests.gemm_cases import GELU_EVAL_C

pytestmark = pytest.mark.gpu


def _inputs():
    grid = np.linspace(-12.0, 12.0, 1 << 22, dtype=np.float32)
    pos = np.arange(1, 0x7F800000, 4099, dtype=np.uint32).view(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3e38, -3e38], np.float32)
    return np.concatenate([grid, pos, -pos, special]).astype(np.float32)


@pytest.mark.parametrize("act", [capi.ACT_GELU_ERF, capi.ACT_GELU_TANH])
def test_gelu_evaluation_within_bound(dev, act):
    x = _inputs()
    y = capi.activation(torch.from_numpy(x).to(dev), act).cpu().numpy()
    ref = oracle.activation(x, act)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(y), nan), "NaN positions differ"
    inf = np.isinf(ref)
    assert np.array_equal(y[inf], ref[inf]), "infinite results differ"
    ok = ~nan & ~inf
    err = np.abs(y[ok].astype(np.float64) - ref[ok].astype(np.float64))
    unit = np.abs(x[ok].astype(np.float64)) * 2.0 ** -24
    ratio = np.where(unit > 0, err / np.where(unit > 0, unit, 1.0), np.where(err > 0, np.inf, 0.0))
    worst = int(np.argmax(ratio))
    print(f"act {act}: max |dev - oracle| / (2^-24 |x|) = {ratio[worst]:.3f} at x = {x[ok][worst]!r}")
    assert ratio[worst] <= GELU_EVAL_C, (ratio[worst], x[ok][worst], y[ok][worst], ref[ok][worst])


def test_relu_bit_exact(dev):
    x = _inputs()
    y = capi.activation(torch.from_numpy(x).to(dev), capi.ACT_RELU).cpu().numpy()
    ref = oracle.activation(x, capi.ACT_RELU)
    assert np.array_equal(y.view(np.uint32)[~np.isnan(ref)], ref.view(np.uint32)[~np.isnan(ref)])
