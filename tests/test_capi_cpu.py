"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and rejects invalid arguments with the documented status
codes before touching the device."""
import ctypes
import subprocess

import pytest

from luisaml_amd import capi


def test_library_exports_every_declared_symbol():
    lib = capi.lib()
    declared = capi.header_symbols()
    assert len(declared) >= 10
    for name in declared:
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True, text=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    assert set(declared) <= exported
    # nothing but the C ABI is exported
    assert all(s.startswith("lcml_fp8_") for s in exported if not s.startswith("_")), \
        sorted(s for s in exported if not s.startswith("lcml_fp8_"))[:10]


def header_define(name):
    import re
    m = re.search(r"#define\s+" + name + r"\s+(\d+)", open(capi.HEADER).read())
    return int(m.group(1))


def test_abi_version():
    assert capi.lib().lcml_fp8_abi_version() == header_define("LCML_FP8_ABI_VERSION") == 2


def test_python_constants_match_header():
    assert capi.DYNAMIC_WORKSPACE_BYTES == header_define("LCML_FP8_DYNAMIC_WORKSPACE_BYTES")
    for name in ("AUTO", "MFMA", "SKINNY", "VALU", "MFMA_FP8", "SKINNY_FP8", "MFMA_128", "MFMA_128_FP8",
                 "AUTO_FP8"):
        assert getattr(capi, "KERNEL_" + name) == header_define("LCML_KERNEL_" + name), name


def test_packed_weight_bytes():
    f = capi.lib().lcml_fp8_packed_weight_bytes
    assert f(128, 64) == 128 * 64
    assert f(784, 256) == 896 * 256
    assert f(256, 10) == 256 * 64
    assert f(4096, 11008) == 4096 * 11008
    assert f(0, 5) == 0 and f(5, -1) == 0


def _gemm(**kw):
    args = dict(M=4, N=64, K=128, a=0x1000, lda=128, a_scale=0x1000, b=0x1000, b_scale=0x1000, pc=0,
                alpha=1.0, c=None, c_ndim=0, c0=0, c1=0, beta=1.0, act=0, y=0x1000, y_dtype=1, ldy=64,
                kernel=0)
    args.update(kw)
    return capi.lib().lcml_fp8_gemm(args["M"], args["N"], args["K"], args["a"], args["lda"], args["a_scale"],
                                    args["b"], args["b_scale"], args["pc"], args["alpha"], args["c"],
                                    args["c_ndim"], args["c0"], args["c1"], args["beta"], args["act"],
                                    args["y"], args["y_dtype"], args["ldy"], args["kernel"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(N=0), capi.ERR_INVALID_ARG),
    (dict(K=-1), capi.ERR_INVALID_ARG),
    (dict(y_dtype=10), capi.ERR_UNSUPPORTED),
    (dict(act=9), capi.ERR_UNSUPPORTED),
    (dict(ldy=10), capi.ERR_INVALID_ARG),
    (dict(b_scale=None), capi.ERR_INVALID_ARG),
    (dict(K=100, lda=112), capi.ERR_UNSUPPORTED),
    (dict(lda=100), capi.ERR_INVALID_ARG),
    (dict(a=0x1001), capi.ERR_INVALID_ARG),
    (dict(kernel=99), capi.ERR_INVALID_ARG),
    (dict(M=1 << 20, K=4096, lda=4096, kernel=capi.KERNEL_SKINNY), capi.ERR_UNSUPPORTED),  # > 2 GiB of A
    (dict(c=0x1000, c_ndim=1, c0=7), capi.ERR_INVALID_ARG),
    (dict(c=0x1000, c_ndim=2, c0=3, c1=64), capi.ERR_INVALID_ARG),
])
def test_gemm_argument_validation(kw, code):
    rc = _gemm(**kw)
    assert rc == code, capi.last_error()
    assert capi.last_error()


def test_other_entry_point_validation():
    L = capi.lib()
    assert L.lcml_fp8_quantize(0x1000, 0x1000, 1, 0, 4, 0x1000, None) == capi.ERR_INVALID_ARG
    assert L.lcml_fp8_quantize(None, None, 1, 1, 0, None, None) == capi.OK  # empty tensor: no-op
    assert L.lcml_fp8_dequantize(0x1000, None, 1, 1, 4, 0x1000, None) == capi.ERR_INVALID_ARG
    assert L.lcml_fp8_quantize_dynamic(0x1000, 0x1000, 70000, 0x1000, None, None) == capi.ERR_INVALID_ARG
    assert "workspace" in capi.last_error()
    assert L.lcml_fp8_pack_weight(0x1000, 0, 64, 0, 0x1000, None) == capi.ERR_INVALID_ARG
    assert L.lcml_fp8_pack_weight(0x1000, 64, 64, 0, 0x1001, None) == capi.ERR_INVALID_ARG
    assert L.lcml_fp8_gemm_w8a32(4, 64, 128, 0x1000, 100, 0x1000, 0x1000, 0, 1.0, None, 0, 0, 0, 1.0, 0,
                                 0x1000, 1, 64, None) == capi.ERR_INVALID_ARG
    assert L.lcml_fp8_gemm(0, 64, 128, None, 128, None, None, 0x1000, 0, 1.0, None, 0, 0, 0, 1.0, 0,
                           0x1000, 1, 64, 0, None) == capi.OK  # M == 0: nothing to do


def test_fp8_data_type_entry_point_validation():
    L = capi.lib()
    sh = lambda t: (ctypes.c_int64 * max(1, len(t)))(*t)
    F, E4, E5 = capi.DTYPE_FLOAT, capi.DTYPE_FLOAT8E4M3FN, capi.DTYPE_FLOAT8E5M2
    assert L.lcml_fp8_cast(0x1000, 16, 0x1000, F, 4, None) == capi.ERR_UNSUPPORTED  # bf16 is not an fp8 type
    assert L.lcml_fp8_cast(0x1000, E4, 0x1000, 99, 4, None) == capi.ERR_UNSUPPORTED
    assert L.lcml_fp8_cast(None, E4, None, E5, 0, None) == capi.OK  # empty: no-op
    assert L.lcml_fp8_cast(0x1000, E4, None, E5, 4, None) == capi.ERR_INVALID_ARG
    assert L.lcml_fp8_quantize_e5m2(0x1000, 0x1000, 1, 1, 4, 0x1000, 2, None) == capi.ERR_INVALID_ARG
    assert L.lcml_fp8_quantize_e5m2(0x1000, 0x1000, 1, 0, 4, 0x1000, 1, None) == capi.ERR_INVALID_ARG
    assert L.lcml_fp8_dequantize_e5m2(0x1000, None, 1, 1, 4, 0x1000, None) == capi.ERR_INVALID_ARG
    # broadcasting: (2,3) with (4,) does not broadcast; y must be the broadcast shape
    assert L.lcml_fp8_binary(0, F, 0x1000, sh((2, 3)), 2, 0x1000, sh((4,)), 1, 0x1000, sh((2, 3)), 2,
                             None) == capi.ERR_INVALID_ARG
    assert L.lcml_fp8_binary(0, E4, 0x1000, sh((2, 3)), 2, 0x1000, sh((3,)), 1, 0x1000, sh((2, 4)), 2,
                             None) == capi.ERR_INVALID_ARG
    assert L.lcml_fp8_binary(7, E4, 0x1000, sh((3,)), 1, 0x1000, sh((3,)), 1, 0x1000, sh((3,)), 1,
                             None) == capi.ERR_INVALID_ARG
    assert L.lcml_fp8_binary(0, 16, 0x1000, sh((3,)), 1, 0x1000, sh((3,)), 1, 0x1000, sh((3,)), 1,
                             None) == capi.ERR_UNSUPPORTED
    nine = sh((1,) * 9)
    assert L.lcml_fp8_binary(0, E5, 0x1000, nine, 9, 0x1000, nine, 9, 0x1000, nine, 9,
                             None) == capi.ERR_INVALID_ARG  # at most 8 dimensions
    assert L.lcml_fp8_binary(0, E5, None, sh((0, 3)), 2, None, sh((3,)), 1, None, sh((0, 3)), 2,
                             None) == capi.OK  # empty output: no-op


def _gemm_dynamic(M, K, x, ldx, ws, ws_bytes, kernel=0, N=64):
    return capi.lib().lcml_fp8_gemm_dynamic(M, N, K, x, ldx, 0x1000, 0x1000, 0, 1.0, None, 0, 0, 0, 1.0, 0,
                                            0x1000, 1, N, None, ws, ws_bytes, kernel, None)


@pytest.mark.parametrize("kernel", [capi.KERNEL_AUTO, capi.KERNEL_SKINNY, capi.KERNEL_AUTO_FP8])
def test_dynamic_gemm_misaligned_x_needs_the_two_step_workspace(kernel):
    """A 4-byte-aligned x cannot take the fused kernel, so the call quantises
    into the workspace: the size query (which assumes an aligned x) says 0
    here, and the call must reject a workspace smaller than the two-step path
    writes, before any launch."""
    L = capi.lib()
    M, K = 4, 1024
    assert L.lcml_fp8_gemm_dynamic_workspace_bytes(M, K, kernel) == 0  # aligned x would fuse
    two_step = L.lcml_fp8_gemm_dynamic_workspace_bytes(M, K, capi.KERNEL_MFMA)
    assert two_step == (M * K + 255) // 256 * 256 + capi.DYNAMIC_WORKSPACE_BYTES + 256
    x = 0x100004  # 4-byte aligned only
    for ws, nbytes in ((None, 0), (0x200000, 256), (0x200000, two_step - 1)):
        assert _gemm_dynamic(M, K, x, K, ws, nbytes, kernel) == capi.ERR_INVALID_ARG
        assert "workspace" in capi.last_error()
    # a misaligned workspace is rejected too
    assert _gemm_dynamic(M, K, x, K, 0x200010, two_step, kernel) == capi.ERR_INVALID_ARG


def test_noalloc_dynamic_gemm_rejects_oversize_before_any_launch():
    """The no-allocation entry point refuses M*K above its scratch limit with
    LCML_ERR_UNSUPPORTED (no device is touched: this runs without a GPU)."""
    L = capi.lib()
    limit = header_define("LCML_FP8_NOALLOC_MAX_ELEMS")
    assert limit == 16 << 20
    K = 4096
    M = limit // K + 1
    rc = L.lcml_fp8_gemm_dynamic_noalloc(M, 64, K, 0x1000, K, 0x1000, 0x1000, 0, 1.0, None, 0, 0, 0, 1.0, 0,
                                         0x1000, 1, 64, None, 0, None)
    assert rc == capi.ERR_UNSUPPORTED
    assert "no-allocation limit" in capi.last_error()
    # M == 0: nothing to do, no scratch needed
    assert L.lcml_fp8_gemm_dynamic_noalloc(0, 64, K, None, K, None, 0x1000, 0, 1.0, None, 0, 0, 0, 1.0, 0,
                                           0x1000, 1, 64, None, 0, None) == capi.OK


def test_auto_fp8_is_accepted_where_auto_is():
    """LCML_KERNEL_AUTO_FP8 sizes the dynamic workspace as AUTO does (fused
    at small M*K, two-step otherwise), and the conv entry point takes it as
    a tile-kernel choice: with a batch of 0 images the call validates
    everything and returns before any launch."""
    L = capi.lib()
    for M, K in ((1, 4096), (4, 4096), (16, 4096), (64, 4096)):
        assert (L.lcml_fp8_gemm_dynamic_workspace_bytes(M, K, capi.KERNEL_AUTO_FP8)
                == L.lcml_fp8_gemm_dynamic_workspace_bytes(M, K, capi.KERNEL_AUTO)), (M, K)

    def conv(kernel):
        return L.lcml_fp8_conv2d(0x1000, 0x1000, 0, 32, 8, 8, 0x1000, 0x1000, 0, 16, 3, 3, 1, 1, 1, 1, 1, 1, 1,
                                 8, 8, None, 0, 0x1000, 1, kernel, None)

    assert conv(capi.KERNEL_AUTO) == capi.OK
    assert conv(capi.KERNEL_AUTO_FP8) == capi.OK
    assert conv(capi.KERNEL_SKINNY) == capi.ERR_UNSUPPORTED and "AUTO_FP8" in capi.last_error()


def test_dynamic_gemm_ex_validates_amax_partials_before_any_launch():
    """lcml_fp8_gemm_dynamic_ex: partials of y need a dense fp32 y and a
    buffer of lcml_fp8_amax_parts_max words, partials of x a positive count;
    everything is rejected before a launch (this runs without a GPU)."""
    import ctypes as C
    L = capi.lib()
    M, N, K = 512, 1000, 256
    cap = L.lcml_fp8_amax_parts_max(M, N)
    assert cap >= 4 * 8 and cap >= (M + 127) // 128 * ((N + 127) // 128)
    assert L.lcml_fp8_amax_parts_max(0, N) == 0
    n = C.c_int(-5)

    def call(y_dtype=1, ldy=N, ypart=0x3000, capv=cap, npart=C.byref(n), xpart=None, xn=0, m=M):
        return L.lcml_fp8_gemm_dynamic_ex(m, N, K, 0x1000, K, 0x1000, 0x1000, 0, 1.0, None, 0, 0, 0, 1.0, 0,
                                          0x2000, y_dtype, ldy, None, xpart, xn, ypart, capv, npart, None, 0, 0, None)

    assert call(y_dtype=16) == capi.ERR_UNSUPPORTED and "fp32" in capi.last_error()
    assert call(ldy=N + 8) == capi.ERR_UNSUPPORTED
    assert call(capv=cap - 1) == capi.ERR_INVALID_ARG and "capacity" in capi.last_error()
    assert call(npart=None) == capi.ERR_INVALID_ARG
    assert call(ypart=None, xpart=0x4000, xn=0) == capi.ERR_INVALID_ARG
    assert call(m=0) == capi.OK and n.value == 0  # nothing to do: no partials
