"""CPU checks that pin the oracle's test helpers: the tolerance scale
orc_gemm_abs_bound (|alpha| * sum_k |a_k b_k| + |beta * C|, which every GEMM
and conv parity bar multiplies) and the maxima behind the dynamic and
per-channel scales (orc_amax, orc_amax_axis).  Neither restates reference
arithmetic; both are checked against independent float64 numpy forms on
mixed-sign data, where a dropped absolute value, a wrong transpose or a
wrong broadcast changes the result.
"""
import numpy as np
import pytest

import oracle

RNG = np.random.default_rng(1234)


def c_broadcast(kind, M, N, rng):
    """A bias of the given broadcast kind and its [M, N] numpy expansion
    (Gemm's C rules, reference gemm.cpp:81-103: scalar / [1], [N], [M]
    (length M != N), and 2-D with size-1 dimensions)."""
    shape = {"N": (N,), "1": (1,), "scalar": (), "M1": (M, 1), "MN": (M, N), "1N": (1, N), "M": (M,)}[kind]
    C = rng.standard_normal(shape).astype(np.float32)
    if kind == "M":
        full = np.broadcast_to(C[:, None], (M, N))
    else:
        full = np.broadcast_to(C, (M, N))
    return C, full.astype(np.float64)


@pytest.mark.parametrize("tA", [0, 1])
@pytest.mark.parametrize("tB", [0, 1])
@pytest.mark.parametrize("kind", [None, "N", "1", "scalar", "M1", "MN", "1N", "M"])
@pytest.mark.parametrize("alpha,beta", [(1.0, 1.0), (-0.75, 1.5), (2.0, -0.5), (1.0, 0.0)])
def test_gemm_abs_bound_against_float64(tA, tB, kind, alpha, beta):
    M, N, K = 7, 5, 33  # M != N so the length-M bias rule is distinct
    A = RNG.standard_normal((K, M) if tA else (M, K)).astype(np.float32)
    B = RNG.standard_normal((N, K) if tB else (K, N)).astype(np.float32)
    Am = (A.T if tA else A).astype(np.float64)
    Bm = (B.T if tB else B).astype(np.float64)
    want = abs(alpha) * (np.abs(Am) @ np.abs(Bm))
    C = None
    if kind is not None:
        C, full = c_broadcast(kind, M, N, RNG)
        if beta != 0.0:
            want = want + np.abs(beta * full)
    got = oracle.gemm_abs_bound(A, B, C, alpha=alpha, beta=beta, transA=tA, transB=tB)
    assert got.shape == (M, N)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=0)
    # the bound dominates the magnitude of the exact result
    exact = alpha * (Am @ Bm) + (beta * full if kind is not None else 0.0)
    assert np.all(np.abs(exact) <= got * (1 + 1e-12))


def test_gemm_abs_bound_is_not_the_abs_of_the_product():
    """Cancelling products: sum|ab| is 2 where |sum ab| is 0."""
    A = np.array([[1.0, 1.0]], np.float32)
    B = np.array([[1.0], [-1.0]], np.float32)
    assert oracle.gemm_abs_bound(A, B)[0, 0] == 2.0
    assert oracle.gemm(A, B)[0, 0] == 0.0


@pytest.mark.parametrize("shape,axis", [((6, 9), 0), ((6, 9), 1), ((3, 4, 5), 1), ((3, 4, 5), 2), ((3, 4, 5), 0),
                                        ((2, 3, 4, 5), 1), ((1, 7), 1), ((7, 1), 0)])
def test_amax_axis_against_numpy(shape, axis):
    x = RNG.standard_normal(shape).astype(np.float32) * 3.0
    other = tuple(i for i in range(len(shape)) if i != axis)
    want = np.abs(x).max(axis=other) if other else np.abs(x)
    got = oracle.amax_axis(x, axis)
    assert got.shape == (shape[axis],)
    assert np.array_equal(got, want.astype(np.float32))
    # the per-channel scales follow: amax / 448 with the non-finite / zero rule
    sc = oracle.channel_scales(x, axis)
    assert np.array_equal(sc, np.array([oracle.scale_from_amax(float(v)) for v in want], np.float32))


def test_amax_axis_specials():
    """NaN is skipped (it never compares greater), +-inf counts, an all-zero
    channel gives 0 and with it the scale 1.0, -0 gives +0."""
    x = np.array([[1.0, np.nan, -0.0], [-3.0, np.inf, 0.0], [2.0, 5.0, -0.0]], np.float32)
    got = oracle.amax_axis(x, 1)
    assert got.tolist() == [3.0, np.inf, 0.0]
    assert not np.signbit(got[2])
    assert oracle.channel_scales(x, 1).tolist() == [np.float32(3.0 / 448.0), 1.0, 1.0]
    assert oracle.amax(x) == np.inf
    assert oracle.amax(np.array([np.nan, -2.5], np.float32)) == 2.5


def test_amax_per_tensor_against_numpy():
    x = RNG.standard_normal(100003).astype(np.float32)
    x[777] = -9.5
    assert oracle.amax(x) == 9.5
    assert oracle.dynamic_scale(x) == np.float32(np.float32(9.5) / np.float32(448.0))
