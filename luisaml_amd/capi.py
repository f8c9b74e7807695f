"""ctypes binding of the C ABI in include/lcml_fp8.h (liblcml_fp8.so).

torch supplies device memory and the current HIP stream; every call goes
straight to the gfx950 kernels of liblcml_fp8.so.  There is no fallback:
if the library is missing or a call fails, an exception is raised.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblcml_fp8.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "lcml_fp8.h")

OK, ERR_INVALID_ARG, ERR_UNSUPPORTED, ERR_HIP = 0, -1, -2, -3
DTYPE_FLOAT, DTYPE_BFLOAT16, DTYPE_FLOAT8E4M3FN, DTYPE_FLOAT8E5M2 = 1, 16, 17, 19
BINARY_ADD, BINARY_SUB, BINARY_MUL, BINARY_DIV = 0, 1, 2, 3
ACT_NONE, ACT_RELU, ACT_GELU_ERF, ACT_GELU_TANH = 0, 1, 2, 3
KERNEL_AUTO, KERNEL_MFMA, KERNEL_SKINNY, KERNEL_VALU, KERNEL_MFMA_FP8, KERNEL_SKINNY_FP8 = 0, 1, 2, 3, 4, 5
KERNEL_MFMA_128, KERNEL_MFMA_128_FP8 = 6, 7
KERNEL_AUTO_FP8 = 8  # AUTO's tiling with the native FP8 MFMA kernels (opt-in)
DYNAMIC_WORKSPACE_BYTES = 4096
DYNAMIC_SMALL_MAX = 65536
PACK_K, PANEL_COLS = 128, 64


class LcmlError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


_lib = None

_vp, _i64, _int, _f32 = C.c_void_p, C.c_int64, C.c_int, C.c_float
_SIGS = {
    "lcml_fp8_last_error": (C.c_char_p, []),
    "lcml_fp8_kernel_trace": (C.c_char_p, []),
    "lcml_fp8_abi_version": (_int, []),
    "lcml_fp8_quantize": (_int, [_vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    "lcml_fp8_dequantize": (_int, [_vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    "lcml_fp8_quantize_dynamic": (_int, [_vp, _vp, _i64, _vp, _vp, _vp]),
    "lcml_fp8_amax": (_int, [_vp, _i64, _vp, _vp]),
    "lcml_fp8_packed_weight_bytes": (_i64, [_i64, _i64]),
    "lcml_fp8_pack_weight": (_int, [_vp, _i64, _i64, _int, _vp, _vp]),
    "lcml_fp8_unpack_weight": (_int, [_vp, _i64, _i64, _int, _vp, _vp]),
    "lcml_fp8_gemm": (_int, [_i64, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _int, _f32, _vp, _int,
                             _i64, _i64, _f32, _int, _vp, _int, _i64, _int, _vp]),
    "lcml_fp8_gemm_dynamic_workspace_bytes": (_i64, [_i64, _i64, _int]),
    "lcml_fp8_gemm_dynamic": (_int, [_i64, _i64, _i64, _vp, _i64, _vp, _vp, _int, _f32, _vp, _int, _i64, _i64,
                                     _f32, _int, _vp, _int, _i64, _vp, _vp, _i64, _int, _vp]),
    "lcml_fp8_amax_parts_max": (_i64, [_i64, _i64]),
    "lcml_fp8_gemm_dynamic_ex": (_int, [_i64, _i64, _i64, _vp, _i64, _vp, _vp, _int, _f32, _vp, _int, _i64, _i64,
                                        _f32, _int, _vp, _int, _i64, _vp, _vp, _int, _vp, _i64,
                                        C.POINTER(C.c_int), _vp, _i64, _int, _vp]),
    "lcml_fp8_gemm_dynamic_noalloc": (_int, [_i64, _i64, _i64, _vp, _i64, _vp, _vp, _int, _f32, _vp, _int, _i64,
                                             _i64, _f32, _int, _vp, _int, _i64, _vp, _int, _vp]),
    "lcml_fp8_quantize_nhwc": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "lcml_fp8_cast": (_int, [_vp, _int, _vp, _int, _i64, _vp]),
    "lcml_fp8_quantize_e5m2": (_int, [_vp, _vp, _i64, _i64, _i64, _vp, _int, _vp]),
    "lcml_fp8_dequantize_e5m2": (_int, [_vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    "lcml_fp8_binary": (_int, [_int, _int, _vp, C.POINTER(C.c_int64), _int, _vp, C.POINTER(C.c_int64), _int,
                               _vp, C.POINTER(C.c_int64), _int, _vp]),
    "lcml_fp8_packed_conv_weight_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "lcml_fp8_pack_conv_weight": (_int, [_vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp]),
    "lcml_fp8_conv2d": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _int, _i64, _i64, _i64, _i64, _i64,
                               _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _int, _vp, _int, _int, _vp]),
    "lcml_fp8_conv2d_f32": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                   _i64, _i64, _i64, _i64, _i64, _i64, _int, _vp]),
    "lcml_fp8_gemm_w8a32": (_int, [_i64, _i64, _i64, _vp, _i64, _vp, _vp, _int, _f32, _vp, _int,
                                   _i64, _i64, _f32, _int, _vp, _int, _i64, _vp]),
    "lcml_fp8_sgemm": (_int, [_i64, _i64, _i64, _vp, _i64, _int, _vp, _i64, _int, _f32, _vp, _int, _i64,
                              _i64, _f32, _int, _vp, _int, _i64, _vp]),
    "lcml_fp8_activation": (_int, [_vp, _vp, _i64, _int, _vp]),
    "lcml_fp8_stream_read": (_int, [_vp, _i64, _int, _vp, _vp]),
}


def header_symbols() -> list[str]:
    """Every lcml_fp8_* function declared in include/lcml_fp8.h."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(lcml_fp8_\w+)\s*\(", text)))


def lib():
    """Load liblcml_fp8.so (built by luisaml_amd.build); raise if it is absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m luisaml_amd.build`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return lib().lcml_fp8_last_error().decode()


def kernel_trace() -> list[str]:
    """Kernels launched on this thread since the previous call, in order."""
    t = lib().lcml_fp8_kernel_trace().decode()
    return t.split(", ") if t else []


def _check(rc: int) -> None:
    if rc != OK:
        raise LcmlError(rc, last_error())


def _ptr(t: torch.Tensor | None):
    if t is None:
        return None
    assert t.is_cuda, "device tensor expected"
    return t.data_ptr()


def _stream(stream=None):
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else stream


# ----------------------------------------------------------- Q / DQ ---------

def _axis_view(shape, axis, nscale):
    n = 1
    for s in shape:
        n *= int(s)
    if nscale == 1:
        return 1, 1, n
    axis = axis % len(shape)
    outer = 1
    for s in shape[:axis]:
        outer *= int(s)
    inner = 1
    for s in shape[axis + 1:]:
        inner *= int(s)
    assert shape[axis] == nscale, "per-axis scale length must equal shape[axis]"
    return outer, int(shape[axis]), inner


def quantize(x: torch.Tensor, scale: torch.Tensor, axis: int = 1, out: torch.Tensor | None = None,
             stream=None) -> torch.Tensor:
    """QuantizeLinear fp32 -> E4M3 (uint8 tensor)."""
    assert x.dtype == torch.float32 and x.is_contiguous()
    scale = scale.reshape(-1)
    y = out if out is not None else torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    o, a, i = _axis_view(tuple(x.shape), axis, scale.numel())
    _check(lib().lcml_fp8_quantize(_ptr(x), _ptr(y), o, a, i, _ptr(scale), _stream(stream)))
    return y


def dequantize(q: torch.Tensor, scale: torch.Tensor, axis: int = 1, out: torch.Tensor | None = None,
               stream=None) -> torch.Tensor:
    """DequantizeLinear E4M3 (uint8) -> fp32."""
    assert q.dtype == torch.uint8 and q.is_contiguous()
    scale = scale.reshape(-1)
    y = out if out is not None else torch.empty(q.shape, dtype=torch.float32, device=q.device)
    o, a, i = _axis_view(tuple(q.shape), axis, scale.numel())
    _check(lib().lcml_fp8_dequantize(_ptr(q), _ptr(y), o, a, i, _ptr(scale), _stream(stream)))
    return y


def quantize_dynamic(x: torch.Tensor, out: torch.Tensor | None = None,
                     scale_out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                     stream=None):
    """Dynamic per-tensor quantisation; returns (codes, scale[1])."""
    assert x.dtype == torch.float32 and x.is_contiguous()
    y = out if out is not None else torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    s = scale_out if scale_out is not None else torch.empty(1, dtype=torch.float32, device=x.device)
    if workspace is None and x.numel() > DYNAMIC_SMALL_MAX:
        workspace = torch.empty(DYNAMIC_WORKSPACE_BYTES, dtype=torch.uint8, device=x.device)
    _check(lib().lcml_fp8_quantize_dynamic(_ptr(x), _ptr(y), x.numel(), _ptr(s), _ptr(workspace),
                                           _stream(stream)))
    return y, s


def amax(x: torch.Tensor, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    assert x.dtype == torch.float32 and x.is_contiguous()
    o = out if out is not None else torch.empty(1, dtype=torch.float32, device=x.device)
    _check(lib().lcml_fp8_amax(_ptr(x), x.numel(), _ptr(o), _stream(stream)))
    return o


# ------------------------------------------------------------ packing -------

def packed_weight_bytes(K: int, N: int) -> int:
    return int(lib().lcml_fp8_packed_weight_bytes(K, N))


def pack_weight(w: torch.Tensor, w_is_nk: bool, stream=None) -> torch.Tensor:
    """Pack an E4M3 weight ([K,N], or [N,K] when w_is_nk) into MFMA panels."""
    assert w.dtype == torch.uint8 and w.is_contiguous() and w.dim() == 2
    N, K = (w.shape[0], w.shape[1]) if w_is_nk else (w.shape[1], w.shape[0])
    p = torch.empty(packed_weight_bytes(K, N), dtype=torch.uint8, device=w.device)
    _check(lib().lcml_fp8_pack_weight(_ptr(w), K, N, int(w_is_nk), _ptr(p), _stream(stream)))
    return p


def unpack_weight(p: torch.Tensor, K: int, N: int, w_is_nk: bool, stream=None) -> torch.Tensor:
    shape = (N, K) if w_is_nk else (K, N)
    w = torch.empty(shape, dtype=torch.uint8, device=p.device)
    _check(lib().lcml_fp8_unpack_weight(_ptr(p), K, N, int(w_is_nk), _ptr(w), _stream(stream)))
    return w


# --------------------------------------------------------------- GEMM -------

_DTYPE_CODE = {torch.float32: DTYPE_FLOAT, torch.bfloat16: DTYPE_BFLOAT16, torch.float16: 10}


def _c_args(c):
    if c is None:
        return None, 0, 0, 0
    nd = c.dim()
    return c, nd, (c.shape[0] if nd >= 1 else 0), (c.shape[1] if nd >= 2 else 0)


def gemm(a: torch.Tensor, a_scale: torch.Tensor, b_packed: torch.Tensor, b_scale: torch.Tensor,
         N: int, K: int, c: torch.Tensor | None = None, alpha: float = 1.0, beta: float = 1.0,
         act: int = ACT_NONE, out_dtype=torch.float32, kernel: int = KERNEL_AUTO,
         out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """W8A8 GEMM: a [M,K] E4M3 (uint8) x packed E4M3 weight -> [M,N] fp32/bf16."""
    assert a.dtype == torch.uint8 and a.dim() == 2 and a.stride(1) == 1
    M = a.shape[0]
    y = out if out is not None else torch.empty((M, N), dtype=out_dtype, device=a.device)
    ydt = _DTYPE_CODE.get(y.dtype, 0)
    cc, nd, c0, c1 = _c_args(c)
    per_ch = int(b_scale.numel() > 1)
    _check(lib().lcml_fp8_gemm(M, N, K, _ptr(a), a.stride(0), _ptr(a_scale), _ptr(b_packed),
                               _ptr(b_scale), per_ch, float(alpha), _ptr(cc), nd, c0, c1,
                               float(beta), int(act), _ptr(y), ydt, y.stride(0), int(kernel),
                               _stream(stream)))
    return y


def gemm_dynamic(x: torch.Tensor, b_packed: torch.Tensor, b_scale: torch.Tensor, N: int, K: int,
                 c: torch.Tensor | None = None, alpha: float = 1.0, beta: float = 1.0, act: int = ACT_NONE,
                 out_dtype=torch.float32, kernel: int = KERNEL_AUTO, out: torch.Tensor | None = None,
                 scale_out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                 stream=None) -> torch.Tensor:
    """DynamicQuantizeLinear(x) -> FP8 linear in one call: x [M,K] fp32 -> [M,N].
    The workspace (uint8, allocated here when needed and not given) is only
    used when the fused small-M kernel does not apply."""
    assert x.dtype == torch.float32 and x.dim() == 2 and x.stride(1) == 1
    M = x.shape[0]
    y = out if out is not None else torch.empty((M, N), dtype=out_dtype, device=x.device)
    ydt = _DTYPE_CODE.get(y.dtype, 0)
    cc, nd, c0, c1 = _c_args(c)
    per_ch = int(b_scale.numel() > 1)
    # the size query assumes a 16-byte aligned x; a misaligned x takes the
    # two-step path, whose size the (never fusing) MFMA kernel's query gives
    need = lib().lcml_fp8_gemm_dynamic_workspace_bytes(M, K, int(kernel) if x.data_ptr() % 16 == 0 else KERNEL_MFMA)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    ws_bytes = workspace.numel() if workspace is not None else 0
    _check(lib().lcml_fp8_gemm_dynamic(M, N, K, _ptr(x), x.stride(0), _ptr(b_packed), _ptr(b_scale), per_ch,
                                       float(alpha), _ptr(cc), nd, c0, c1, float(beta), int(act), _ptr(y), ydt,
                                       y.stride(0), _ptr(scale_out), _ptr(workspace), ws_bytes, int(kernel),
                                       _stream(stream)))
    return y


def amax_parts_buffer(M: int, N: int, device) -> torch.Tensor:
    """A device buffer for the partial maxima of an M x N output."""
    return torch.empty(int(lib().lcml_fp8_amax_parts_max(M, N)), dtype=torch.int32, device=device)


def gemm_dynamic_ex(x: torch.Tensor, b_packed: torch.Tensor, b_scale: torch.Tensor, N: int, K: int,
                    c: torch.Tensor | None = None, alpha: float = 1.0, beta: float = 1.0, act: int = ACT_NONE,
                    out_dtype=torch.float32, kernel: int = KERNEL_AUTO, out: torch.Tensor | None = None,
                    scale_out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                    x_amax: tuple | None = None, y_amax_part: torch.Tensor | None = None, stream=None):
    """gemm_dynamic for chains of dynamically quantised linears: x_amax =
    (partials, count) of x from an earlier call skips the amax pass over x;
    y_amax_part (from amax_parts_buffer) receives partials of y.  Returns
    (y, count of y partials written, or 0)."""
    assert x.dtype == torch.float32 and x.dim() == 2 and x.stride(1) == 1
    M = x.shape[0]
    y = out if out is not None else torch.empty((M, N), dtype=out_dtype, device=x.device)
    ydt = _DTYPE_CODE.get(y.dtype, 0)
    cc, nd, c0, c1 = _c_args(c)
    per_ch = int(b_scale.numel() > 1)
    need = lib().lcml_fp8_gemm_dynamic_workspace_bytes(M, K, int(kernel) if x.data_ptr() % 16 == 0 else KERNEL_MFMA)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    ws_bytes = workspace.numel() if workspace is not None else 0
    xp, xn = (x_amax[0], int(x_amax[1])) if x_amax is not None else (None, 0)
    npart = C.c_int(0)
    _check(lib().lcml_fp8_gemm_dynamic_ex(M, N, K, _ptr(x), x.stride(0), _ptr(b_packed), _ptr(b_scale), per_ch,
                                          float(alpha), _ptr(cc), nd, c0, c1, float(beta), int(act), _ptr(y), ydt,
                                          y.stride(0), _ptr(scale_out), _ptr(xp), xn, _ptr(y_amax_part),
                                          y_amax_part.numel() if y_amax_part is not None else 0, C.byref(npart),
                                          _ptr(workspace), ws_bytes, int(kernel), _stream(stream)))
    return y, npart.value


# --------------------------------------------------------------- Conv -------

def quantize_nhwc(x: torch.Tensor, scale: torch.Tensor | None = None, out: torch.Tensor | None = None,
                  scale_out: torch.Tensor | None = None, workspace: torch.Tensor | None = None, stream=None):
    """QuantizeLinear of NCHW fp32 x into NHWC E4M3; scale None = dynamic.
    Returns (codes [n, h, w, c], scale[1])."""
    assert x.dtype == torch.float32 and x.is_contiguous() and x.dim() == 4
    n, c, h, w = x.shape
    y = out if out is not None else torch.empty((n, h, w, c), dtype=torch.uint8, device=x.device)
    if scale is None:
        s = scale_out if scale_out is not None else torch.empty(1, dtype=torch.float32, device=x.device)
        ws = workspace if workspace is not None else torch.empty(DYNAMIC_WORKSPACE_BYTES, dtype=torch.uint8,
                                                                 device=x.device)
        _check(lib().lcml_fp8_quantize_nhwc(_ptr(x), _ptr(y), n, c, h, w, None, _ptr(s), _ptr(ws), _stream(stream)))
        return y, s
    _check(lib().lcml_fp8_quantize_nhwc(_ptr(x), _ptr(y), n, c, h, w, _ptr(scale), None, None, _stream(stream)))
    return y, scale


def pack_conv_weight(w: torch.Tensor, group: int = 1, stream=None) -> torch.Tensor:
    """Pack E4M3 conv weights [cout, cin/group, kh, kw] for conv2d."""
    assert w.dtype == torch.uint8 and w.is_contiguous() and w.dim() == 4
    cout, cin_g, kh, kw = w.shape
    p = torch.empty(lib().lcml_fp8_packed_conv_weight_bytes(cout, cin_g, kh, kw, group), dtype=torch.uint8,
                    device=w.device)
    _check(lib().lcml_fp8_pack_conv_weight(_ptr(w), cout, cin_g, kh, kw, group, _ptr(p), _stream(stream)))
    return p


def conv2d(x_nhwc: torch.Tensor, x_scale: torch.Tensor, w_packed: torch.Tensor, w_scale: torch.Tensor,
           cout: int, kernel_shape, strides=(1, 1), pads=(0, 0), dilations=(1, 1), out_hw=None,
           bias: torch.Tensor | None = None, act: int = ACT_NONE, out_dtype=torch.float32,
           kernel: int = KERNEL_AUTO, out: torch.Tensor | None = None, group: int = 1,
           stream=None) -> torch.Tensor:
    """FP8 conv (implicit im2col on the matrix cores): NHWC E4M3 in, NCHW out.
    pads are begin pads; out_hw defaults to symmetric padding."""
    n, h, w, c = x_nhwc.shape
    kh, kw = kernel_shape
    if out_hw is None:
        out_hw = ((h + 2 * pads[0] - dilations[0] * (kh - 1) - 1) // strides[0] + 1,
                  (w + 2 * pads[1] - dilations[1] * (kw - 1) - 1) // strides[1] + 1)
    oh, ow = out_hw
    y = out if out is not None else torch.empty((n, cout, oh, ow), dtype=out_dtype, device=x_nhwc.device)
    per_ch = int(w_scale.numel() > 1)
    _check(lib().lcml_fp8_conv2d(_ptr(x_nhwc), _ptr(x_scale), n, c, h, w, _ptr(w_packed), _ptr(w_scale), per_ch,
                                 cout, kh, kw, strides[0], strides[1], pads[0], pads[1], dilations[0], dilations[1],
                                 group, oh, ow, _ptr(bias), int(act), _ptr(y), _DTYPE_CODE.get(y.dtype, 0), int(kernel),
                                 _stream(stream)))
    return y


def conv2d_f32(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None, strides=(1, 1), pads=(0, 0),
               dilations=(1, 1), group: int = 1, out_hw=None, act: int = ACT_NONE, stream=None) -> torch.Tensor:
    """Plain fp32 NCHW Conv (begin pads; out_hw defaults to symmetric padding)."""
    assert x.dtype == torch.float32 and w.dtype == torch.float32 and x.is_contiguous() and w.is_contiguous()
    n, c, h, wd = x.shape
    cout, _, kh, kw = w.shape
    if out_hw is None:
        out_hw = ((h + 2 * pads[0] - dilations[0] * (kh - 1) - 1) // strides[0] + 1,
                  (wd + 2 * pads[1] - dilations[1] * (kw - 1) - 1) // strides[1] + 1)
    y = torch.empty((n, cout, *out_hw), dtype=torch.float32, device=x.device)
    _check(lib().lcml_fp8_conv2d_f32(_ptr(x), _ptr(w), _ptr(bias), _ptr(y), n, c, h, wd, cout, kh, kw, strides[0],
                                     strides[1], pads[0], pads[1], dilations[0], dilations[1], group, out_hw[0],
                                     out_hw[1], int(act), _stream(stream)))
    return y


def gemm_w8a32(a: torch.Tensor, b_packed: torch.Tensor, b_scale: torch.Tensor, N: int, K: int,
               c: torch.Tensor | None = None, alpha: float = 1.0, beta: float = 1.0,
               act: int = ACT_NONE, out_dtype=torch.float32, out: torch.Tensor | None = None,
               stream=None) -> torch.Tensor:
    """W8A32 linear: a [M,K] fp32 x packed E4M3 weight -> [M,N]."""
    assert a.dtype == torch.float32 and a.dim() == 2 and a.stride(1) == 1
    M = a.shape[0]
    y = out if out is not None else torch.empty((M, N), dtype=out_dtype, device=a.device)
    ydt = _DTYPE_CODE.get(y.dtype, 0)
    cc, nd, c0, c1 = _c_args(c)
    per_ch = int(b_scale.numel() > 1)
    _check(lib().lcml_fp8_gemm_w8a32(M, N, K, _ptr(a), a.stride(0), _ptr(b_packed), _ptr(b_scale),
                                     per_ch, float(alpha), _ptr(cc), nd, c0, c1, float(beta),
                                     int(act), _ptr(y), ydt, y.stride(0), _stream(stream)))
    return y


def sgemm(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor | None = None, alpha: float = 1.0, beta: float = 1.0,
          trans_a: bool = False, trans_b: bool = False, act: int = ACT_NONE, stream=None) -> torch.Tensor:
    """Plain fp32 Gemm in the reference's per-output fma-chain order."""
    assert a.dtype == torch.float32 and b.dtype == torch.float32 and a.is_contiguous() and b.is_contiguous()
    M, K = (a.shape[1], a.shape[0]) if trans_a else (a.shape[0], a.shape[1])
    N = b.shape[0] if trans_b else b.shape[1]
    y = torch.empty((M, N), dtype=torch.float32, device=a.device)
    cc, nd, c0, c1 = _c_args(c)
    _check(lib().lcml_fp8_sgemm(M, N, K, _ptr(a), a.shape[1], int(trans_a), _ptr(b), b.shape[1], int(trans_b),
                                float(alpha), _ptr(cc), nd, c0, c1, float(beta), int(act), _ptr(y), DTYPE_FLOAT,
                                N, _stream(stream)))
    return y


def activation(x: torch.Tensor, act: int, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    assert x.dtype == torch.float32 and x.is_contiguous()
    y = out if out is not None else torch.empty_like(x)
    _check(lib().lcml_fp8_activation(_ptr(x), _ptr(y), x.numel(), int(act), _stream(stream)))
    return y


def stream_read(buf: torch.Tensor, sink: torch.Tensor, workgroups: int = 1024, stream=None) -> None:
    """Read every byte of buf (contiguous, 16-byte multiple) and nothing else:
    the HBM read floor for the same bytes.  sink: one int32/uint32 device word."""
    assert buf.is_contiguous() and (buf.numel() * buf.element_size()) % 16 == 0
    _check(lib().lcml_fp8_stream_read(_ptr(buf), buf.numel() * buf.element_size(), int(workgroups), _ptr(sink),
                                      _stream(stream)))


# ---------------------------------------------------- fp8 data-type ops ----

def cast(x: torch.Tensor, x_dtype: int, y_dtype: int, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Cast between DTYPE_FLOAT (float32 tensor) and DTYPE_FLOAT8E4M3FN /
    DTYPE_FLOAT8E5M2 (uint8 code tensors)."""
    assert x.is_contiguous()
    tdt = torch.float32 if y_dtype == DTYPE_FLOAT else torch.uint8
    y = out if out is not None else torch.empty(x.shape, dtype=tdt, device=x.device)
    _check(lib().lcml_fp8_cast(_ptr(x), int(x_dtype), _ptr(y), int(y_dtype), x.numel(), _stream(stream)))
    return y


def quantize_e5m2(x: torch.Tensor, scale: torch.Tensor, axis: int = 1, saturate: int = 1,
                  out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """QuantizeLinear fp32 -> E5M2 codes (uint8)."""
    assert x.dtype == torch.float32 and x.is_contiguous()
    scale = scale.reshape(-1)
    y = out if out is not None else torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    o, a, i = _axis_view(tuple(x.shape), axis, scale.numel())
    _check(lib().lcml_fp8_quantize_e5m2(_ptr(x), _ptr(y), o, a, i, _ptr(scale), int(saturate), _stream(stream)))
    return y


def dequantize_e5m2(q: torch.Tensor, scale: torch.Tensor, axis: int = 1, out: torch.Tensor | None = None,
                    stream=None) -> torch.Tensor:
    assert q.dtype == torch.uint8 and q.is_contiguous()
    scale = scale.reshape(-1)
    y = out if out is not None else torch.empty(q.shape, dtype=torch.float32, device=q.device)
    o, a, i = _axis_view(tuple(q.shape), axis, scale.numel())
    _check(lib().lcml_fp8_dequantize_e5m2(_ptr(q), _ptr(y), o, a, i, _ptr(scale), _stream(stream)))
    return y


def binary(op: int, a: torch.Tensor, b: torch.Tensor, dtype: int, out: torch.Tensor | None = None,
           stream=None) -> torch.Tensor:
    """y = a OP b with numpy broadcasting; dtype DTYPE_FLOAT (float32 tensors)
    or DTYPE_FLOAT8E4M3FN / DTYPE_FLOAT8E5M2 (uint8 code tensors)."""
    assert a.is_contiguous() and b.is_contiguous()
    ys = tuple(torch.broadcast_shapes(a.shape, b.shape))
    y = out if out is not None else torch.empty(ys, dtype=a.dtype, device=a.device)
    sh = lambda t: (C.c_int64 * max(1, len(t)))(*t)
    _check(lib().lcml_fp8_binary(int(op), int(dtype), _ptr(a), sh(tuple(a.shape)), a.dim(), _ptr(b),
                                 sh(tuple(b.shape)), b.dim(), _ptr(y), sh(tuple(y.shape)), y.dim(), _stream(stream)))
    return y
