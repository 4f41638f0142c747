"""ctypes front end of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker. The product path
(breeze_tts_cpp_amd) never imports it.

All arrays are numpy; 16-bit floats travel as uint16 bit patterns.
Reference citations for each function are in qlinear_oracle.c.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

BF16, F32, I32, FP8, I8, F16 = 0, 1, 2, 3, 4, 5

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build(force: bool = False) -> str:
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-C", _HERE, "-B" if force else "all"], check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i = ctypes.c_int
        L.orc_bf16_to_f32.restype = ctypes.c_float
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_fp8_decode.restype = ctypes.c_float
        L.orc_fp8_decode.argtypes = [ctypes.c_uint8]
        L.orc_fp8_encode.restype = ctypes.c_uint8
        L.orc_fp8_encode.argtypes = [ctypes.c_float]
        L.orc_i8_round.restype = i
        L.orc_i8_round.argtypes = [ctypes.c_float]
        L.orc_scale.restype = ctypes.c_float
        L.orc_scale.argtypes = [ctypes.c_float, i]
        L.orc_rotation_sign.restype = ctypes.c_float
        L.orc_rotation_sign.argtypes = [i]
        L.orc_rotate128.restype = None
        L.orc_rotate128.argtypes = [P, i]
        L.orc_quantize_rows.restype = i
        L.orc_quantize_rows.argtypes = [P, i, i, i, i, i, i, i, P, P]
        L.orc_gemm_i8_acc.restype = None
        L.orc_gemm_i8_acc.argtypes = [P, P, i, i, i, P]
        L.orc_epilogue_i8.restype = None
        L.orc_epilogue_i8.argtypes = [P, P, P, i, i, i, i, P]
        L.orc_gemm_fp8_ideal.restype = None
        L.orc_gemm_fp8_ideal.argtypes = [P, P, P, P, i, i, i, P]
        L.orc_gemm_grouped.restype = i
        L.orc_gemm_grouped.argtypes = [P, P, P, P, i, i, i, i, i, i, i, i, i, i, P, P]
        L.orc_gemm_grouped_ideal.restype = None
        L.orc_gemm_grouped_ideal.argtypes = [P, P, P, P, i, i, i, i, i, i, P]
        L.orc_rsqrt_rn.restype = ctypes.c_float
        L.orc_rsqrt_rn.argtypes = [ctypes.c_float]
        L.orc_norm_sumsq.restype = ctypes.c_float
        L.orc_norm_sumsq.argtypes = [P, i]
        L.orc_quantized_norm.restype = i
        L.orc_quantized_norm.argtypes = [P, P, P, P, i, i, i, ctypes.c_float, i, i, i, i, P, P, P]
        L.orc_activate.restype = ctypes.c_float
        L.orc_activate.argtypes = [ctypes.c_float, i]
        L.orc_quantized_gated.restype = i
        L.orc_quantized_gated.argtypes = [P, i, i, i, i, i, i, i, P, P, P]
        L.orc_finish.restype = None
        L.orc_finish.argtypes = [P, P, i, i, i, i]
        L.orc_cub_sum256.restype = ctypes.c_float
        L.orc_cub_sum256.argtypes = [P]
        L.orc_norm_linear.restype = i
        L.orc_norm_linear.argtypes = [P, P, P, P, i, i, i, ctypes.c_float, P, P, i, i, P, i, P,
                                      P, P, P]
        L.orc_norm_rows.restype = i
        L.orc_norm_rows.argtypes = [P, i, i, i, i, P, P, ctypes.c_float, P, P]
        L.orc_layer_norm_quantize.restype = i
        L.orc_layer_norm_quantize.argtypes = [P, i, i, P, P, ctypes.c_float, P, P, i, i, P, P, i,
                                              i, i]
        L.orc_qexp.restype = ctypes.c_float
        L.orc_qexp.argtypes = [ctypes.c_float]
        L.orc_qtanh.restype = ctypes.c_float
        L.orc_qtanh.argtypes = [ctypes.c_float]
        L.orc_act.restype = ctypes.c_float
        L.orc_act.argtypes = [ctypes.c_float, i, ctypes.c_float]
        L.orc_gelu_tanh_contracted.restype = ctypes.c_float
        L.orc_gelu_tanh_contracted.argtypes = [ctypes.c_float]
        L.orc_pointwise_quantize.restype = i
        L.orc_pointwise_quantize.argtypes = [P, i, i, P, P, i, i, P, P, i, i, i]
        L.orc_pack_weights.restype = i
        L.orc_pack_weights.argtypes = [P, i, i, P]
        L.orc_cpu_qlinear.restype = i
        L.orc_cpu_qlinear.argtypes = [P, i, i, i, i, P, P, i, i, i, i, P, P, P, i]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- scalar codecs
def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    f = lib().orc_f32_to_bf16
    flat = np.asarray(x, np.float32).ravel()
    return np.fromiter((f(float(v)) for v in flat), np.uint16, flat.size).reshape(np.shape(x))


def fp8_decode_table() -> np.ndarray:
    f = lib().orc_fp8_decode
    return np.array([f(c) for c in range(256)], np.float32)


def fp8_encode(x) -> np.ndarray:
    f = lib().orc_fp8_encode
    flat = np.asarray(x, np.float32).ravel()
    return np.fromiter((f(float(v)) for v in flat), np.uint8, flat.size).reshape(np.shape(x))


def i8_round(x) -> np.ndarray:
    f = lib().orc_i8_round
    flat = np.asarray(x, np.float32).ravel()
    return np.fromiter((f(float(v)) for v in flat), np.int32, flat.size).reshape(np.shape(x))


def quant_scale(amax: float, fmt: int) -> float:
    return lib().orc_scale(float(amax), fmt)


def rotation_signs(columns: int) -> np.ndarray:
    f = lib().orc_rotation_sign
    return np.array([f(c) for c in range(columns)], np.float32)


def rotate128(v: np.ndarray, c0: int) -> np.ndarray:
    out = np.ascontiguousarray(v, np.float32).copy()
    assert out.size == 128
    lib().orc_rotate128(_p(out), c0)
    return out


# ---------------------------------------------------------------- quantizer / GEMMs
def quantize_rows(src_bits: np.ndarray, fmt: int, group: int = 0, rotation: int = 0,
                  src_type: int = BF16, ld: int | None = None, cols: int | None = None):
    """Returns (values uint8 [rows, cols], scales f32 [rows] or [G, rows])."""
    src_bits = np.ascontiguousarray(src_bits, np.uint16)
    rows = src_bits.shape[0]
    ld = src_bits.shape[1] if ld is None else ld
    cols = src_bits.shape[1] if cols is None else cols
    q = np.zeros((rows, cols), np.uint8)
    groups = (cols + group - 1) // group if group else 1
    scales = np.zeros((groups, rows) if group else (rows,), np.float32)
    rc = lib().orc_quantize_rows(_p(src_bits), src_type, ld, rows, cols, fmt, group, rotation,
                                 _p(q), _p(scales))
    if rc:
        raise ValueError("oracle: unsupported quantization layout")
    return q, scales


def gemm_i8_acc(xq: np.ndarray, wq: np.ndarray) -> np.ndarray:
    xq = np.ascontiguousarray(xq).view(np.int8)
    wq = np.ascontiguousarray(wq).view(np.int8)
    M, K = xq.shape
    N = wq.shape[0]
    acc = np.zeros((M, N), np.int32)
    lib().orc_gemm_i8_acc(_p(xq), _p(wq), M, N, K, _p(acc))
    return acc


def epilogue_i8(acc, sx, sw, order: int = 0, out_type: int = BF16) -> np.ndarray:
    acc = np.ascontiguousarray(acc, np.int32)
    sx = np.ascontiguousarray(sx, np.float32)
    sw = np.ascontiguousarray(sw, np.float32)
    M, N = acc.shape
    y = np.zeros((M, N), np.uint16)
    lib().orc_epilogue_i8(_p(acc), _p(sx), _p(sw), M, N, order, out_type, _p(y))
    return y


def gemm_fp8_ideal(xq, sx, wq, sw) -> np.ndarray:
    xq = np.ascontiguousarray(xq, np.uint8)
    wq = np.ascontiguousarray(wq, np.uint8)
    sx = np.ascontiguousarray(sx, np.float32)
    sw = np.ascontiguousarray(sw, np.float32)
    M, K = xq.shape
    N = wq.shape[0]
    y = np.zeros((M, N), np.float32)
    lib().orc_gemm_fp8_ideal(_p(xq), _p(sx), _p(wq), _p(sw), M, N, K, _p(y))
    return y


def gemm_grouped(xq, sx, wq, sw, fmt: int, input_group: int, weight_group: int,
                 splits: int = 1, waves: int = 1, span: int | None = None,
                 out_type: int = BF16):
    """Returns (y 16-bit bits [M,N], y fp32 before the final rounding)."""
    xq = np.ascontiguousarray(xq, np.uint8)
    wq = np.ascontiguousarray(wq, np.uint8)
    sx = np.ascontiguousarray(sx, np.float32)
    sw = np.ascontiguousarray(sw, np.float32)
    M, K = xq.shape
    N = wq.shape[0]
    if span is None:
        span = -(-K // (splits * waves))
    y = np.zeros((M, N), np.uint16)
    yf = np.zeros((M, N), np.float32)
    rc = lib().orc_gemm_grouped(_p(xq), _p(sx), _p(wq), _p(sw), M, N, K, fmt, input_group,
                                weight_group, splits, waves, span, out_type, _p(y), _p(yf))
    if rc:
        raise ValueError("oracle: unsupported grouped GEMM layout")
    return y, yf


def gemm_grouped_ideal(xq, sx, wq, sw, fmt: int, input_group: int, weight_group: int):
    xq = np.ascontiguousarray(xq, np.uint8)
    wq = np.ascontiguousarray(wq, np.uint8)
    sx = np.ascontiguousarray(sx, np.float32)
    sw = np.ascontiguousarray(sw, np.float32)
    M, K = xq.shape
    N = wq.shape[0]
    y = np.zeros((M, N), np.float32)
    lib().orc_gemm_grouped_ideal(_p(xq), _p(sx), _p(wq), _p(sw), M, N, K, fmt, input_group,
                                 weight_group, _p(y))
    return y


_cpu_lib = None


def host_has_avx512() -> bool:
    """The x86-64-v4 feature set (AVX-512 F/BW/CD/DQ/VL) on this host."""
    try:
        flags = next(l for l in open("/proc/cpuinfo") if l.startswith("flags")).split()
    except (OSError, StopIteration):
        return False
    return all(f in flags for f in ("avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"))


def cpu_lib():
    """The library the CPU baseline times: liboracle_v4.so (the same source
    built for x86-64-v4) on an AVX-512 host, else liboracle.so."""
    global _cpu_lib
    if _cpu_lib is None:
        v4 = os.path.join(_HERE, "liboracle_v4.so")
        if host_has_avx512() and os.path.exists(v4):
            L = ctypes.CDLL(v4)
            P, i = ctypes.c_void_p, ctypes.c_int
            L.orc_cpu_qlinear.restype = i
            L.orc_cpu_qlinear.argtypes = [P, i, i, i, i, P, P, i, i, i, i, P, P, P, i]
            _cpu_lib = (L, "x86-64-v4")
        else:
            _cpu_lib = (lib(), "x86-64-v3")
    return _cpu_lib


def cpu_qlinear(x_bits, wq, sw, fmt: int, group: int = 0, rotation: int = 0,
                threads: int = 1, out_type: int = BF16, fast: bool = False):
    """The whole per-call path on the CPU (quantize X, GEMM, dequant). fast:
    the build for this host's widest vector ISA (cpu_lib), same results."""
    x_bits = np.ascontiguousarray(x_bits, np.uint16)
    wq = np.ascontiguousarray(wq, np.uint8)
    sw = np.ascontiguousarray(sw, np.float32)
    M, K = x_bits.shape
    N = wq.shape[0]
    y = np.zeros((M, N), np.uint16)
    xq = np.zeros((M, K), np.uint8)
    groups = (K + group - 1) // group if group else 1
    sx = np.zeros((groups * M,), np.float32)
    L = cpu_lib()[0] if fast else lib()
    L.orc_cpu_qlinear(_p(x_bits), BF16, M, N, K, _p(wq), _p(sw), fmt, group, rotation,
                      out_type, _p(y), _p(xq), _p(sx), threads)
    return y


# ---------------------------------------------------------------- fused producers
def rsqrt_rn(a: float) -> float:
    return lib().orc_rsqrt_rn(float(a))


def norm_sumsq(v: np.ndarray) -> float:
    v = np.ascontiguousarray(v, np.float32)
    return lib().orc_norm_sumsq(_p(v), v.size)


def activate(x: float, kind: int) -> float:
    return lib().orc_activate(float(x), kind)


def quantized_norm(residual_bits, weight_bits, fmt: int, update_bits=None, scale_bits=None,
                   eps: float = 1e-6, gemma: bool = False, group: int = 0, rotation: int = 0,
                   src_type: int = BF16):
    """Returns (updated residual bits, values uint8 [rows, cols], scales,
    normalized 16-bit rows)."""
    res = np.ascontiguousarray(residual_bits, np.uint16).copy()
    rows, cols = res.shape
    w = np.ascontiguousarray(weight_bits, np.uint16)
    u = None if update_bits is None else np.ascontiguousarray(update_bits, np.uint16)
    s = None if scale_bits is None else np.ascontiguousarray(scale_bits, np.uint16)
    q = np.zeros((rows, cols), np.uint8)
    n = np.zeros((rows, cols), np.uint16)
    groups = (cols + group - 1) // group if group else 1
    scales = np.zeros((groups, rows) if group else (rows,), np.float32)
    rc = lib().orc_quantized_norm(_p(res), None if u is None else _p(u),
                                  None if s is None else _p(s), _p(w), src_type, rows, cols,
                                  float(eps), int(gemma), fmt, group, rotation, _p(q), _p(scales),
                                  _p(n))
    if rc:
        raise ValueError("oracle: unsupported quantized norm layout")
    return res, q, scales, n


def quantized_gated(input_bits, kind: int, fmt: int, group: int = 0, rotation: int = 0,
                    src_type: int = BF16):
    """input [rows, 2*width] (gate | up). Returns (values [rows, width], scales,
    activated 16-bit rows)."""
    x = np.ascontiguousarray(input_bits, np.uint16)
    rows, width = x.shape[0], x.shape[1] // 2
    q = np.zeros((rows, width), np.uint8)
    a = np.zeros((rows, width), np.uint16)
    groups = (width + group - 1) // group if group else 1
    scales = np.zeros((groups, rows) if group else (rows,), np.float32)
    rc = lib().orc_quantized_gated(_p(x), src_type, rows, width, kind, fmt, group, rotation,
                                   _p(q), _p(scales), _p(a))
    if rc:
        raise ValueError("oracle: unsupported quantized gated layout")
    return q, scales, a


def pack_weights(wq: np.ndarray) -> np.ndarray:
    """Packed fragment-tile layout of uint8 weights [N, K] (N % 16 == 0)."""
    wq = np.ascontiguousarray(wq, np.uint8)
    N, K = wq.shape
    out = np.zeros(N * ((K + 63) // 64) * 64, np.uint8)
    if lib().orc_pack_weights(_p(wq), N, K, _p(out)):
        raise ValueError("oracle: packed weights need N % 16 == 0")
    return out


def finish(y_bits: np.ndarray, bias_bits=None, act: int = 0, out_type: int = BF16) -> np.ndarray:
    """s16(act(s16(y + bias))) on a stored 16-bit GEMM result [M, N]."""
    y = np.ascontiguousarray(y_bits, np.uint16).copy()
    M, N = y.shape
    b = None if bias_bits is None else np.ascontiguousarray(bias_bits, np.uint16)
    lib().orc_finish(_p(y), None if b is None else _p(b), M, N, act, out_type)
    return y


def cub_sum256(v: np.ndarray) -> float:
    v = np.ascontiguousarray(v, np.float32)
    assert v.size == 256
    return lib().orc_cub_sum256(_p(v))


class NormFusion(ctypes.Structure):
    """orc_norm_fusion (the library's qlin_norm_fusion layout)."""
    _fields_ = [("residual", ctypes.c_void_p), ("projection_bias", ctypes.c_void_p),
                ("gate", ctypes.c_void_p), ("shift", ctypes.c_void_p), ("scale", ctypes.c_void_p),
                ("gate_rows", ctypes.c_int), ("shift_rows", ctypes.c_int),
                ("scale_rows", ctypes.c_int), ("raw", ctypes.c_void_p),
                ("rows_per_sequence", ctypes.c_int), ("source_rows", ctypes.c_void_p)]


class Epilogue(ctypes.Structure):
    """orc_epilogue (the library's qlin_epilogue layout)."""
    _fields_ = [("bias", ctypes.c_void_p), ("residual", ctypes.c_void_p),
                ("residual_rows", ctypes.c_int), ("residual_index", ctypes.c_void_p),
                ("value_scale", ctypes.c_float), ("output_scale", ctypes.c_float),
                ("residual_scale", ctypes.c_float), ("activation", ctypes.c_int),
                ("alpha", ctypes.c_float), ("raw", ctypes.c_void_p), ("gate", ctypes.c_void_p),
                ("gate_rows", ctypes.c_int), ("condition", ctypes.c_void_p),
                ("condition_rows", ctypes.c_int), ("rows_per_sequence", ctypes.c_int),
                ("valid_rows_per_sequence", ctypes.c_int), ("input_repeat", ctypes.c_int)]


def _u16(a):
    return None if a is None else np.ascontiguousarray(a, np.uint16)


def _opt(a):
    return None if a is None else _p(a)


def _fusion(keep, rows, cols, residual=None, projection_bias=None, gate=None, shift=None,
            scale=None, rows_per_sequence=1, source_rows=None, raw=False):
    """A NormFusion over numpy arrays (kept alive in `keep`); returns
    (fusion, raw array or None)."""
    f = NormFusion()
    f.rows_per_sequence = rows_per_sequence
    for name, a in (("residual", residual), ("projection_bias", projection_bias), ("gate", gate),
                    ("shift", shift), ("scale", scale)):
        a = _u16(a)
        if a is not None:
            keep.append(a)
            setattr(f, name, _p(a).value)
            if name in ("gate", "shift", "scale"):
                setattr(f, name + "_rows", a.shape[0] if a.ndim == 2 else 1)
    if source_rows is not None:
        sr = np.ascontiguousarray(source_rows, np.int32)
        keep.append(sr)
        f.source_rows = _p(sr).value
    raw_out = None
    if raw:
        raw_out = np.zeros((rows, cols), np.uint16)
        keep.append(raw_out)
        f.raw = _p(raw_out).value
    return f, raw_out


def norm_linear(x_bits, wq, sw, fmt: int, norm_weight=None, norm_bias=None, bias=None,
                act: int = 0, eps: float = 1e-5, src_type: int = BF16, raw: bool = False,
                **fusion):
    """LayerNorm (NormFusion keywords: residual, projection_bias, gate, shift,
    scale, rows_per_sequence) -> quant -> GEMV. Returns (y bits [rows, n],
    normalized bits [rows, k], codes [rows, k], scales [rows], raw or None)."""
    x = np.ascontiguousarray(x_bits, np.uint16)
    rows, k = x.shape
    wq = np.ascontiguousarray(wq, np.uint8)
    sw = np.ascontiguousarray(sw, np.float32)
    n = wq.shape[0]
    keep = []
    f, raw_out = _fusion(keep, rows, k, raw=raw, **fusion)
    nw, nb, b = _u16(norm_weight), _u16(norm_bias), _u16(bias)
    y = np.zeros((rows, n), np.uint16)
    nrm = np.zeros((rows, k), np.uint16)
    enc = np.zeros((rows, k), np.uint8)
    esc = np.zeros(rows, np.float32)
    rc = lib().orc_norm_linear(_p(x), ctypes.byref(f), _opt(nw), _opt(nb), src_type, rows, k,
                               float(eps), _p(wq), _p(sw), fmt, n, _opt(b), act, _p(y), _p(nrm),
                               _p(enc), _p(esc))
    if rc:
        raise ValueError("oracle: unsupported normalized linear shape")
    return y, nrm, enc, esc, raw_out


def norm_rows(x_bits, norm_weight=None, norm_bias=None, eps: float = 1e-5, rows=None,
              src_type: int = BF16, **fusion):
    """The LayerNorm rows alone (16-bit bits [rows, cols])."""
    x = np.ascontiguousarray(x_bits, np.uint16)
    x_rows, cols = x.shape
    rows = x_rows if rows is None else rows
    keep = []
    f, _ = _fusion(keep, rows, cols, **fusion)
    nw, nb = _u16(norm_weight), _u16(norm_bias)
    u = np.zeros((rows, cols), np.uint16)
    lib().orc_norm_rows(_p(x), x_rows, src_type, rows, cols, _opt(nw), _opt(nb), float(eps),
                        ctypes.byref(f), _p(u))
    return u


def layer_norm_quantize(x_bits, fmt: int, norm_weight=None, norm_bias=None, eps: float = 1e-5,
                        rows=None, group: int = 0, rotation: int = 0, src_type: int = BF16,
                        raw: bool = False, **fusion):
    """Returns (codes [rows, cols], scales, retained bits [rows, cols], raw or None)."""
    x = np.ascontiguousarray(x_bits, np.uint16)
    x_rows, cols = x.shape
    rows = x_rows if rows is None else rows
    keep = []
    f, raw_out = _fusion(keep, rows, cols, raw=raw, **fusion)
    nw, nb = _u16(norm_weight), _u16(norm_bias)
    q = np.zeros((rows, cols), np.uint8)
    groups = (cols + group - 1) // group if group else 1
    sc = np.zeros((groups, rows) if group else (rows,), np.float32)
    ret = np.zeros((rows, cols), np.uint16)
    rc = lib().orc_layer_norm_quantize(_p(x), x_rows, src_type, _opt(nw), _opt(nb), float(eps),
                                       ctypes.byref(f), _p(ret), rows, cols, _p(q), _p(sc), fmt,
                                       group, rotation)
    if rc:
        raise ValueError("oracle: unsupported layer norm quantize layout")
    return q, sc, ret, raw_out


def qexp(x: float) -> float:
    return lib().orc_qexp(float(x))


def qtanh(x: float) -> float:
    return lib().orc_qtanh(float(x))


def act(x: float, kind: int, alpha: float = 0.1) -> float:
    """ops::activate (numbering of ops::Activation)."""
    return lib().orc_act(float(x), kind, float(alpha))


def pointwise_quantize(x_bits, fmt: int, rows=None, group: int = 0, rotation: int = 0,
                       src_type: int = BF16, raw: bool = False, bias=None, residual=None,
                       residual_index=None, gate=None, condition=None, value_scale=1.0,
                       output_scale=1.0, residual_scale=1.0, activation=0, alpha=0.1,
                       rows_per_sequence=1, valid_rows_per_sequence=0, input_repeat=1):
    """Returns (codes [rows, cols], scales, retained bits [rows, cols], raw or None)."""
    x = np.ascontiguousarray(x_bits, np.uint16)
    x_rows, cols = x.shape
    rows = x_rows * input_repeat if rows is None else rows
    keep = []
    e = Epilogue(value_scale=value_scale, output_scale=output_scale,
                 residual_scale=residual_scale, activation=activation, alpha=alpha,
                 rows_per_sequence=rows_per_sequence,
                 valid_rows_per_sequence=valid_rows_per_sequence, input_repeat=input_repeat)
    for name, a in (("bias", bias), ("residual", residual), ("gate", gate),
                    ("condition", condition)):
        a = _u16(a)
        if a is not None:
            keep.append(a)
            setattr(e, name, _p(a).value)
            if name != "bias":
                setattr(e, name + "_rows", a.shape[0] if a.ndim == 2 else 1)
    if residual_index is not None:
        ri = np.ascontiguousarray(residual_index, np.int32)
        keep.append(ri)
        e.residual_index = _p(ri).value
    raw_out = None
    if raw:
        raw_out = np.zeros((rows, cols), np.uint16)
        e.raw = _p(raw_out).value
    q = np.zeros((rows, cols), np.uint8)
    groups = (cols + group - 1) // group if group else 1
    sc = np.zeros((groups, rows) if group else (rows,), np.float32)
    ret = np.zeros((rows, cols), np.uint16)
    rc = lib().orc_pointwise_quantize(_p(x), x_rows, src_type, ctypes.byref(e), _p(ret), rows,
                                      cols, _p(q), _p(sc), fmt, group, rotation)
    if rc:
        raise ValueError("oracle: unsupported pointwise quantize layout")
    return q, sc, ret, raw_out
