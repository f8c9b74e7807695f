"""ctypes bindings for the CPU oracle (oracle/lcml_oracle.c).

TEST INFRASTRUCTURE ONLY: the oracle is what parity is judged against and the timed CPU
baseline.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
import this package; the product library (luisaml_amd) never does.

Every function here is a thin numpy wrapper over a C function whose comment
names the reference file:line it restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liblcml_oracle.so")
_lib = None

ACT_NONE, ACT_RELU, ACT_GELU_ERF, ACT_GELU_TANH = 0, 1, 2, 3


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc); returns the .so path."""
    if force and os.path.exists(_LIB_PATH):
        os.remove(_LIB_PATH)
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        f32p, u8p, u16p, f64p = (C.POINTER(C.c_float), C.POINTER(C.c_uint8),
                                 C.POINTER(C.c_uint16), C.POINTER(C.c_double))
        i64 = C.c_int64
        sig = {
            "orc_set_threads": (None, [C.c_int]),
            "orc_get_threads": (C.c_int, []),
            "orc_e4m3_from_float": (C.c_uint8, [C.c_float]),
            "orc_e4m3_to_float": (C.c_float, [C.c_uint8]),
            "orc_e4m3_spec_encode": (C.c_uint8, [C.c_float]),
            "orc_e4m3_encode_bits": (None, [C.c_uint32, C.c_uint64, u8p]),
            "orc_e4m3_sweep_vs_spec": (C.c_uint64, [C.c_uint32, C.c_uint64, C.POINTER(C.c_uint32)]),
            "orc_e4m3_decode_table": (None, [f32p]),
            "orc_bf16_rne": (C.c_uint16, [C.c_float]),
            "orc_bf16_rne_array": (None, [f32p, u16p, i64]),
            "orc_quantize": (None, [f32p, u8p, i64, i64, i64, f32p]),
            "orc_dequantize": (None, [u8p, f32p, i64, i64, i64, f32p]),
            "orc_amax": (C.c_float, [f32p, i64]),
            "orc_scale_from_amax": (C.c_float, [C.c_float]),
            "orc_amax_axis": (None, [f32p, i64, i64, i64, f32p]),
            "orc_relu": (C.c_float, [C.c_float]),
            "orc_gelu_erf": (C.c_float, [C.c_float]),
            "orc_gelu_tanh": (C.c_float, [C.c_float]),
            "orc_activation": (None, [f32p, f32p, i64, C.c_int]),
            "orc_gemm": (None, [i64, i64, i64, f32p, C.c_int, f32p, C.c_int, C.c_float,
                                C.c_float, f32p, C.c_int, i64, i64, C.c_int, f32p]),
            "orc_gemm_abs_bound": (None, [i64, i64, i64, f32p, C.c_int, f32p, C.c_int,
                                          C.c_float, C.c_float, f32p, C.c_int, i64, i64, f64p]),
            "orc_gemm_f64": (None, [i64, i64, i64, f32p, f32p, f64p]),
            "orc_conv2d": (None, [f32p, f32p, f32p, f32p] + [i64] * 16 + [C.c_int]),
            "orc_e5m2_from_float": (C.c_uint8, [C.c_float]),
            "orc_e5m2_to_float": (C.c_float, [C.c_uint8]),
            "orc_e5m2_spec_encode": (C.c_uint8, [C.c_float]),
            "orc_e5m2_encode_bits": (None, [C.c_uint32, C.c_uint64, u8p]),
            "orc_e5m2_sweep_vs_spec": (C.c_uint64, [C.c_uint32, C.c_uint64, C.POINTER(C.c_uint32)]),
            "orc_e5m2_decode_table": (None, [f32p]),
            "orc_half_round": (C.c_float, [C.c_double]),
            "orc_half_round_array": (None, [f32p, f32p, i64]),
            "orc_fp8_binary": (None, [C.c_int, C.c_int, C.c_void_p, C.POINTER(C.c_int64), C.c_int, C.c_void_p,
                                      C.POINTER(C.c_int64), C.c_int, C.c_void_p, C.POINTER(C.c_int64), C.c_int]),
            "orc_quantize_e5m2": (None, [f32p, u8p, i64, i64, i64, f32p, C.c_int]),
            "orc_dequantize_e5m2": (None, [u8p, f32p, i64, i64, i64, f32p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray | None, ctype):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.POINTER(ctype))


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def threads() -> int:
    return int(lib().orc_get_threads())


# ---------------------------------------------------------------- codec ----

def e4m3_from_float(x) -> np.ndarray:
    """Vectorised FP8E4M3FN::from_float (fp_quantized.h:149-223)."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    out = np.empty(x.shape, np.uint8)
    one = np.ones(1, np.float32)
    lib().orc_quantize(_p(x.reshape(-1), C.c_float), _p(out.reshape(-1), C.c_uint8),
                       1, 1, x.size, _p(one, C.c_float))
    return out


def e4m3_spec_encode(x: float) -> int:
    return int(lib().orc_e4m3_spec_encode(float(x)))


def e4m3_encode_bits(first: int, count: int) -> np.ndarray:
    out = np.empty(count, np.uint8)
    lib().orc_e4m3_encode_bits(first, count, _p(out, C.c_uint8))
    return out


def e4m3_sweep_vs_spec(first: int, count: int) -> tuple[int, int | None]:
    bad_at = C.c_uint32(0)
    n = lib().orc_e4m3_sweep_vs_spec(first, count, C.byref(bad_at))
    return int(n), (int(bad_at.value) if n else None)


def e4m3_decode_table() -> np.ndarray:
    """FP8E4M3FN::to_float (fp_quantized.h:226-249) for all 256 codes."""
    out = np.empty(256, np.float32)
    lib().orc_e4m3_decode_table(_p(out, C.c_float))
    return out


def e4m3_to_float(q) -> np.ndarray:
    return e4m3_decode_table()[np.asarray(q, dtype=np.uint8)]


def bf16_rne(x) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    out = np.empty(x.shape, np.uint16)
    lib().orc_bf16_rne_array(_p(x.reshape(-1), C.c_float), _p(out.reshape(-1), C.c_uint16), x.size)
    return out


# ------------------------------------------------------------- Q / DQ -------

def _axis_view(shape, axis, nscale):
    shape = tuple(int(s) for s in shape)
    if nscale == 1:
        n = int(np.prod(shape)) if shape else 1
        return 1, 1, n
    axis = axis % len(shape)
    assert shape[axis] == nscale, "per-axis scale length must equal shape[axis]"
    outer = int(np.prod(shape[:axis])) if axis else 1
    inner = int(np.prod(shape[axis + 1:])) if axis + 1 < len(shape) else 1
    return outer, shape[axis], inner


def quantize(x, scale, axis: int = 1) -> np.ndarray:
    """QuantizeLinear to E4M3: from_float(x / scale), scale per tensor or per axis."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    s = np.ascontiguousarray(np.atleast_1d(np.asarray(scale, dtype=np.float32)))
    o, a, i = _axis_view(x.shape, axis, s.size)
    out = np.empty(x.shape, np.uint8)
    lib().orc_quantize(_p(x.reshape(-1), C.c_float), _p(out.reshape(-1), C.c_uint8), o, a, i,
                       _p(s, C.c_float))
    return out


def dequantize(q, scale, axis: int = 1) -> np.ndarray:
    """DequantizeLinear from E4M3: to_float(q) * scale (one fp32 multiply)."""
    q = np.ascontiguousarray(np.asarray(q, dtype=np.uint8))
    s = np.ascontiguousarray(np.atleast_1d(np.asarray(scale, dtype=np.float32)))
    o, a, i = _axis_view(q.shape, axis, s.size)
    out = np.empty(q.shape, np.float32)
    lib().orc_dequantize(_p(q.reshape(-1), C.c_uint8), _p(out.reshape(-1), C.c_float), o, a, i,
                         _p(s, C.c_float))
    return out


def amax(x) -> float:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).reshape(-1)
    return float(lib().orc_amax(_p(x, C.c_float), x.size))


def scale_from_amax(a: float) -> float:
    return float(lib().orc_scale_from_amax(float(a)))


def dynamic_scale(x) -> float:
    """Per-tensor dynamic scale: amax/448 (1.0 when that is not a positive finite number)."""
    return scale_from_amax(amax(x))


def amax_axis(x, axis: int) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    axis = axis % x.ndim
    o, a, i = _axis_view(x.shape, axis, x.shape[axis])
    out = np.empty(a, np.float32)
    lib().orc_amax_axis(_p(x.reshape(-1), C.c_float), o, a, i, _p(out, C.c_float))
    return out


def channel_scales(x, axis: int) -> np.ndarray:
    return np.array([scale_from_amax(float(v)) for v in amax_axis(x, axis)], np.float32)


# ---------------------------------------------------------- activations ----

def activation(x, act: int) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    out = np.empty_like(x)
    lib().orc_activation(_p(x.reshape(-1), C.c_float), _p(out.reshape(-1), C.c_float), x.size, act)
    return out


# ----------------------------------------------------------------- Gemm ----

def _c_args(Cb):
    if Cb is None:
        return None, -1, 0, 0
    Cb = np.ascontiguousarray(np.asarray(Cb, dtype=np.float32))
    nd = Cb.ndim
    c0 = Cb.shape[0] if nd >= 1 else 0
    c1 = Cb.shape[1] if nd >= 2 else 0
    return Cb, nd, c0, c1


def gemm(A, B, C_=None, alpha=1.0, beta=1.0, transA=0, transB=0, act=ACT_NONE) -> np.ndarray:
    """ONNX Gemm in the reference's arithmetic (gemm.cpp:27-325), fp32 in and out."""
    A = np.ascontiguousarray(np.asarray(A, dtype=np.float32))
    B = np.ascontiguousarray(np.asarray(B, dtype=np.float32))
    M, K = (A.shape[1], A.shape[0]) if transA else A.shape
    K2, N = (B.shape[1], B.shape[0]) if transB else B.shape
    assert K == K2, "Gemm: inner dimensions mismatch"
    Cb, nd, c0, c1 = _c_args(C_)
    Y = np.empty((M, N), np.float32)
    lib().orc_gemm(M, N, K, _p(A, C.c_float), int(transA), _p(B, C.c_float), int(transB),
                   float(alpha), float(beta), _p(Cb, C.c_float), nd, c0, c1, int(act),
                   _p(Y, C.c_float))
    return Y


def gemm_abs_bound(A, B, C_=None, alpha=1.0, beta=1.0, transA=0, transB=0) -> np.ndarray:
    """sum_k |a b| (+|beta C|) per output, in double: the tolerance scale."""
    A = np.ascontiguousarray(np.asarray(A, dtype=np.float32))
    B = np.ascontiguousarray(np.asarray(B, dtype=np.float32))
    M, K = (A.shape[1], A.shape[0]) if transA else A.shape
    N = B.shape[0] if transB else B.shape[1]
    Cb, nd, c0, c1 = _c_args(C_)
    out = np.empty((M, N), np.float64)
    lib().orc_gemm_abs_bound(M, N, K, _p(A, C.c_float), int(transA), _p(B, C.c_float),
                             int(transB), float(alpha), float(beta), _p(Cb, C.c_float), nd, c0,
                             c1, _p(out, C.c_double))
    return out


def gemm_f64(A, B) -> np.ndarray:
    A = np.ascontiguousarray(np.asarray(A, dtype=np.float32))
    B = np.ascontiguousarray(np.asarray(B, dtype=np.float32))
    M, K = A.shape
    N = B.shape[1]
    out = np.empty((M, N), np.float64)
    lib().orc_gemm_f64(M, N, K, _p(A, C.c_float), _p(B, C.c_float), _p(out, C.c_double))
    return out


def qlinear(qa, sa, qb, sb, bias=None, transB=0, act=ACT_NONE, alpha=1.0):
    """Dequantize-then-Gemm composition: Gemm(DQ(qa, sa), DQ(qb, sb), bias).

    qa [M,K] E4M3 with per-tensor scale sa; qb [K,N] (transB=0) or [N,K]
    (transB=1) E4M3 with per-tensor or per-output-channel (length N) scale sb.
    Returns (Y, A_f32, B_f32) so callers can form the tolerance bound.
    """
    A = dequantize(qa, sa)
    sb = np.atleast_1d(np.asarray(sb, np.float32))
    if sb.size == 1:
        B = dequantize(qb, sb)
    else:
        B = dequantize(qb, sb, axis=0 if transB else 1)
    Y = gemm(A, B, bias, alpha=alpha, beta=1.0, transB=transB, act=act)
    return Y, A, B


# ----------------------------------------------------------------- Conv ----

def conv2d(X, W, bias=None, strides=(1, 1), pads=(0, 0), dilations=(1, 1), group=1,
           act=ACT_NONE) -> np.ndarray:
    """Direct NCHW Conv (conv.cpp:115-207 semantics: begin pads), fp32 accumulate."""
    X = np.ascontiguousarray(np.asarray(X, dtype=np.float32))
    W = np.ascontiguousarray(np.asarray(W, dtype=np.float32))
    N, Cc, H, Wd = X.shape
    M, Cg, kH, kW = W.shape
    assert Cg * group == Cc
    sH, sW = strides
    pH, pW = pads
    dH, dW = dilations
    oH = (H + 2 * pH - dH * (kH - 1) - 1) // sH + 1
    oW = (Wd + 2 * pW - dW * (kW - 1) - 1) // sW + 1
    b = None if bias is None else np.ascontiguousarray(np.asarray(bias, np.float32))
    Y = np.empty((N, M, oH, oW), np.float32)
    lib().orc_conv2d(_p(X, C.c_float), _p(W, C.c_float), _p(b, C.c_float), _p(Y, C.c_float),
                     N, Cc, H, Wd, M, kH, kW, sH, sW, pH, pW, dH, dW, group, oH, oW, int(act))
    return Y


# --------------------------------------------------------------- E5M2 -------

DTYPE_FLOAT, DTYPE_E4M3, DTYPE_E5M2 = 1, 17, 19
OP_ADD, OP_SUB, OP_MUL, OP_DIV = 0, 1, 2, 3


def e5m2_from_float(x) -> np.ndarray:
    """Vectorised FP8E5M2::from_float (fp_quantized.h:272-346): no saturation."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    out = np.empty(x.shape, np.uint8)
    one = np.ones(1, np.float32)
    lib().orc_quantize_e5m2(_p(x.reshape(-1), C.c_float), _p(out.reshape(-1), C.c_uint8), 1, 1, x.size,
                            _p(one, C.c_float), 0)
    return out


def e5m2_spec_encode(x: float) -> int:
    return int(lib().orc_e5m2_spec_encode(float(x)))


def e5m2_encode_bits(first: int, count: int) -> np.ndarray:
    out = np.empty(count, np.uint8)
    lib().orc_e5m2_encode_bits(first, count, _p(out, C.c_uint8))
    return out


def e5m2_sweep_vs_spec(first: int, count: int) -> tuple[int, int | None]:
    bad_at = C.c_uint32(0)
    n = lib().orc_e5m2_sweep_vs_spec(first, count, C.byref(bad_at))
    return int(n), (int(bad_at.value) if n else None)


def e5m2_decode_table() -> np.ndarray:
    """FP8E5M2::to_float (fp_quantized.h:350-377) for all 256 codes."""
    out = np.empty(256, np.float32)
    lib().orc_e5m2_decode_table(_p(out, C.c_float))
    return out


def e5m2_to_float(q) -> np.ndarray:
    return e5m2_decode_table()[np.asarray(q, dtype=np.uint8)]


def half_round(x) -> np.ndarray:
    """IEEE binary16 round-to-nearest-even of fp32 values, as fp32."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    out = np.empty(x.shape, np.float32)
    lib().orc_half_round_array(_p(x.reshape(-1), C.c_float), _p(out.reshape(-1), C.c_float), x.size)
    return out


def quantize_e5m2(x, scale, axis: int = 1, saturate: int = 1) -> np.ndarray:
    """QuantizeLinear to E5M2: from_float(x / scale), saturate=1 clamps to +-57344."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    s = np.ascontiguousarray(np.atleast_1d(np.asarray(scale, dtype=np.float32)))
    o, a, i = _axis_view(x.shape, axis, s.size)
    out = np.empty(x.shape, np.uint8)
    lib().orc_quantize_e5m2(_p(x.reshape(-1), C.c_float), _p(out.reshape(-1), C.c_uint8), o, a, i,
                            _p(s, C.c_float), int(saturate))
    return out


def dequantize_e5m2(q, scale, axis: int = 1) -> np.ndarray:
    q = np.ascontiguousarray(np.asarray(q, dtype=np.uint8))
    s = np.ascontiguousarray(np.atleast_1d(np.asarray(scale, dtype=np.float32)))
    o, a, i = _axis_view(q.shape, axis, s.size)
    out = np.empty(q.shape, np.float32)
    lib().orc_dequantize_e5m2(_p(q.reshape(-1), C.c_uint8), _p(out.reshape(-1), C.c_float), o, a, i,
                              _p(s, C.c_float))
    return out


def broadcast_shape(sa, sb):
    return tuple(np.broadcast_shapes(tuple(sa), tuple(sb)))


def fp8_binary(op: int, dtype: int, a, b) -> np.ndarray:
    """Add/Sub/Mul/Div with numpy broadcasting: fp32 arithmetic for FLOAT,
    decode -> op in half -> encode for E4M3 / E5M2 (binary.cpp:184-285)."""
    npdt = np.float32 if dtype == DTYPE_FLOAT else np.uint8
    a = np.ascontiguousarray(np.asarray(a, dtype=npdt))
    b = np.ascontiguousarray(np.asarray(b, dtype=npdt))
    ys = broadcast_shape(a.shape, b.shape)
    y = np.empty(ys, npdt)
    sh = lambda t: (C.c_int64 * max(1, len(t)))(*t)
    lib().orc_fp8_binary(op, dtype, a.ctypes.data, sh(a.shape), a.ndim, b.ctypes.data, sh(b.shape), b.ndim,
                         y.ctypes.data, sh(ys), len(ys))
    return y
