"""Shared builders for the GEMM parity tests.

A case is generated on the host with the seeded generator, quantised by the
oracle (dynamic per-tensor activation scale, per-tensor or per-output-channel
weight scales, amax/448), and checked against the oracle's
dequantise-then-Gemm composition (gemm.cpp:27-325 arithmetic) with the
tolerance the path is held to:
    |y - y_ref| <= 1e-4 * sum_k |a_k b_k|  (+|beta C|)   elementwise
    ||y - y_ref||_F / ||y_ref||_F <= 1e-5                (fp32 output)
"""
from __future__ import annotations

import numpy as np
import torch

import oracle
from luisaml_amd import capi, synth

TOL_ELEM = 1e-4
TOL_FROB = 1e-5
# The device GELU's evaluation differs from the oracle's fp32 evaluation of
# the same formula by at most GELU_EVAL_C * 2^-24 * |x| (measured 6.2 for the
# erf form, 3.4 for tanh; pinned by tests/test_gpu_activation.py).
GELU_EVAL_C = 8.0


def gelu_tol(act) -> float:
    """Elementwise tolerance factor on the bound sum|a*b| + |beta*C| of an output.

    Without an activation (or with ReLU, 1-Lipschitz and exact) it is the
    summation-order bar TOL_ELEM.  GELU is 1.13-Lipschitz, so a pre-activation
    error of TOL_ELEM * bound becomes at most 1.13 times that; the device's
    evaluation of GELU adds GELU_EVAL_C * 2^-24 * |pre-activation| <=
    GELU_EVAL_C * 2^-24 * bound, and the oracle's own fp32 evaluation at the
    slightly different pre-activation as much again.
    """
    if act in (oracle.ACT_NONE, oracle.ACT_RELU):
        return TOL_ELEM
    return 1.13 * TOL_ELEM + 2.0 * GELU_EVAL_C * 2.0 ** -24


class Case:
    pass


def make_case(M, N, K, seed=0, per_channel=True, w_is_nk=False, a_std=1.0, w_std=0.02,
              bias=None, dev=None):
    c = Case()
    c.M, c.N, c.K = M, N, K
    a = synth.normal(seed * 3 + 1, (M, K), std=a_std)
    w = synth.normal(seed * 3 + 2, (N, K) if w_is_nk else (K, N), std=w_std)
    c.sa = np.float32(oracle.dynamic_scale(a))
    c.qa = oracle.quantize(a, c.sa)
    ch_axis = 0 if w_is_nk else 1
    c.sb = oracle.channel_scales(w, ch_axis) if per_channel else np.array([oracle.dynamic_scale(w)], np.float32)
    c.qb = oracle.quantize(w, c.sb, axis=ch_axis) if per_channel else oracle.quantize(w, c.sb)
    c.w_is_nk = w_is_nk
    c.bias = bias
    if dev is not None:
        c.d_qa = torch.from_numpy(c.qa).to(dev)
        c.d_sa = torch.from_numpy(np.array([c.sa], np.float32)).to(dev)
        c.d_sb = torch.from_numpy(c.sb).to(dev)
        c.d_bp = capi.pack_weight(torch.from_numpy(c.qb).to(dev), w_is_nk)
    return c


def reference(c, bias=None, alpha=1.0, beta=1.0, act=oracle.ACT_NONE):
    """Oracle output and the per-element tolerance scale."""
    A = oracle.dequantize(c.qa, c.sa)
    if c.sb.size == 1:
        B = oracle.dequantize(c.qb, c.sb)
    else:
        B = oracle.dequantize(c.qb, c.sb, axis=0 if c.w_is_nk else 1)
    tb = int(c.w_is_nk)
    Y = oracle.gemm(A, B, bias, alpha=alpha, beta=beta, transB=tb, act=act)
    bound = oracle.gemm_abs_bound(A, B, bias, alpha=alpha, beta=beta, transB=tb)
    return Y, bound


def assert_close(y, ref, bound, act=oracle.ACT_NONE, frob=True):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    tol = gelu_tol(act) * bound
    d = np.abs(y - ref)
    bad = np.argwhere(~(d <= tol))
    assert bad.size == 0, (f"{len(bad)} elements outside tolerance; first {bad[:4].tolist()}: "
                           f"got {y[tuple(bad[0])]} ref {ref[tuple(bad[0])]} tol {tol[tuple(bad[0])]}")
    if frob:
        nr = np.linalg.norm(ref)
        rel = np.linalg.norm(y - ref) / nr if nr > 0 else np.linalg.norm(y)
        assert rel <= TOL_FROB, f"relative Frobenius error {rel:.3e} > {TOL_FROB}"
