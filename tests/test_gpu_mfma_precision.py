"""Why the default GEMM kernels widen E4M3 to bf16 instead of using gfx950's
FP8 MFMAs: the FP8 matrix-core instructions drop product bits that lie far
below the largest product of their block, while the bf16 MFMAs on the
exactly widened operands keep every product (each E4M3 x E4M3 product is
exact in fp32).

Two-term cases, one output each, all operands in one 64-k block:
  1 * 1 + 2^-7 * 2^-7  = 1 + 2^-14   (a term 14 binades below the largest)
  1 * 1 + 2^-7 * 2^-6  = 1 + 2^-13   (13 binades below)
Every kernel that meets the reference tolerance returns both sums exactly;
the native-FP8 kernels return 1.0 for the first and 1 + 2^-13 for the second.
A random block (N(0,1)-quantised operands, K = 128) then shows the size of
the effect on ordinary data: below 1e-6 relative Frobenius error for the
exact kernels, above 4e-6 (and within the documented 3e-5) for the FP8 ones.
The exact sums are float64 sums of the closed-form decoded operands.
"""
import numpy as np
import pytest
import torch

import oracle
from luisaml_amd import capi, synth

pytestmark = pytest.mark.gpu

EXACT = {"mfma": capi.KERNEL_MFMA, "mfma_128": capi.KERNEL_MFMA_128, "skinny": capi.KERNEL_SKINNY,
         "valu": capi.KERNEL_VALU}
FP8 = {"mfma_fp8": capi.KERNEL_MFMA_FP8, "mfma_128_fp8": capi.KERNEL_MFMA_128_FP8,
       "skinny_fp8": capi.KERNEL_SKINNY_FP8}
M, K, N = 32, 128, 64
ONE, P7, P6 = 0x38, 0x04, 0x08  # E4M3 codes of 1.0, 2^-7 (subnormal 4 * 2^-9), 2^-6


def two_term_operands():
    qa = np.zeros((M, K), np.uint8)
    qb = np.zeros((K, N), np.uint8)
    qa[0, 0], qa[0, 1] = ONE, P7           # row 0: 1, 2^-7
    qb[0, 0], qb[1, 0] = ONE, P7           # column 0: 1, 2^-7  -> 1 + 2^-14
    qb[0, 1], qb[1, 1] = ONE, P6           # column 1: 1, 2^-6  -> 1 + 2^-13
    assert oracle.e4m3_to_float(np.array([ONE, P7, P6], np.uint8)).tolist() == [1.0, 2.0 ** -7, 2.0 ** -6]
    return qa, qb


def run(qa, qb, kernel, dev):
    one = torch.ones(1, device=dev)
    bp = capi.pack_weight(torch.from_numpy(qb).to(dev), False)
    return capi.gemm(torch.from_numpy(qa).to(dev), one, bp, one, N, K, kernel=kernel).cpu().numpy()


@pytest.mark.parametrize("name", list(EXACT))
def test_exact_kernels_keep_a_term_14_binades_down(dev, name):
    y = run(*two_term_operands(), EXACT[name], dev)
    assert y[0, 0] == np.float32(1 + 2.0 ** -14)
    assert y[0, 1] == np.float32(1 + 2.0 ** -13)


@pytest.mark.parametrize("name", list(FP8))
def test_fp8_mfma_drops_a_term_14_binades_down(dev, name):
    y = run(*two_term_operands(), FP8[name], dev)
    assert y[0, 0] == np.float32(1.0), f"{y[0, 0]!r}: the 2^-14 product was kept"
    assert y[0, 1] == np.float32(1 + 2.0 ** -13)


def random_block():
    a = synth.normal(901, (M, K))
    w = synth.normal(902, (K, N))
    sa, sw = oracle.dynamic_scale(a), oracle.dynamic_scale(w)
    qa, qb = oracle.quantize(a, sa), oracle.quantize(w, sw)
    exact = oracle.e4m3_to_float(qa).astype(np.float64) @ oracle.e4m3_to_float(qb).astype(np.float64)
    return qa, qb, exact


@pytest.mark.parametrize("name", list(EXACT) + list(FP8))
def test_random_block_relative_error(dev, name):
    qa, qb, exact = random_block()
    kern = EXACT.get(name, FP8.get(name))
    y = run(qa, qb, kern, dev).astype(np.float64)
    rel = np.linalg.norm(y - exact) / np.linalg.norm(exact)
    if name in EXACT:
        assert rel < 1e-6, rel
    else:
        assert 4e-6 < rel < 3e-5, rel
