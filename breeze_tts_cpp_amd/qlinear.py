"""Python host binding of libqlinear.so (ctypes over the C ABI in
include/qlinear.h). Device memory and streams come from PyTorch; all compute
is the HIP library. There is no fallback: if the library is missing or a
call fails, this raises.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import torch

BF16, F32, I32, FP8, I8, F16 = 0, 1, 2, 3, 4, 5
KIND_AUTO, KIND_SKINNY, KIND_TILED = 0, 1, 2
STATUS = {0: "ok", -1: "invalid", -2: "alignment", -3: "workspace", -4: "unsupported", -5: "hip"}

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("QLINEAR_LIB") or os.path.join(_HERE, "libqlinear.so")
_lib = None


class QLinearError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"qlinear error {status} ({STATUS.get(status, '?')}): {message}")
        self.status = status


class qlin_path(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("tokens", ctypes.c_int), ("channels", ctypes.c_int),
                ("splits", ctypes.c_int), ("waves", ctypes.c_int), ("staged", ctypes.c_int)]


@dataclass
class Path:
    kind: int = KIND_AUTO
    tokens: int = 0
    channels: int = 0
    splits: int = 1
    waves: int = 1
    staged: int = 0

    def to_c(self) -> qlin_path:
        return qlin_path(self.kind, self.tokens, self.channels, self.splits, self.waves,
                         self.staged)


def grouped_partition(path: Path, K: int, fmt: int = I8, input_group: int = 128,
                      weight_group: int = 128, packed: bool = False) -> tuple[int, int, int]:
    """(splits, waves, span) of the K ranges a planned path sums separately
    (the K-group oracle takes the same partition).

    A tiled launch sums all of K in one range (given as K rounded up to 128,
    a whole number of groups), and so does an INT8 skinny launch with K
    groups of 128 on a staged slab of at most 6 (blocks x token tiles) and no
    split: it runs the reference's single chain over every group of K
    (quant_grouped.cu:112-146). Any other skinny launch splits K into
    splits*8 wave ranges of ceil(ceil(K/256) / (splits*8)) 256-byte blocks
    (trailing ranges may be empty), each summed on its own."""
    if path.kind == KIND_SKINNY:
        blocks = -(-K // 256)
        ranges = path.splits * path.waves
        span_blocks = -(-blocks // ranges)
        groups = [g for g in (input_group, weight_group) if g]
        if (fmt == I8 and groups and min(groups) == 128 and not packed and path.splits == 1
                and path.staged in (1, 2) and span_blocks * (path.tokens // 16) <= 6):
            return 1, 1, -(-K // 128) * 128
        return path.splits, path.waves, span_blocks * 256
    return 1, 1, -(-K // 128) * 128


EXPORTS = ("qlin_version", "qlin_last_error", "qlin_row_quantize", "qlin_plan",
           "qlin_workspace_bytes", "qlin_gemm", "qlin_linear", "qlin_quantized_norm",
           "qlin_quantized_gated", "qlin_packed_weight_bytes", "qlin_pack_weights",
           "qlin_gemm_packed", "qlin_linear_packed", "qlin_gemm_finish", "qlin_norm_linear",
           "qlin_norm_fusion_init", "qlin_epilogue_init", "qlin_layer_norm_quantize",
           "qlin_pointwise_quantize", "qlin_pointwise", "qlin_linear_noalloc", "qlin_noalloc_scratch_bytes")


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() "
                           "(make -C breeze_tts_cpp_amd)")
    L = ctypes.CDLL(LIB_PATH)
    P, i, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    L.qlin_version.restype = i
    L.qlin_version.argtypes = []
    L.qlin_last_error.restype = ctypes.c_char_p
    L.qlin_last_error.argtypes = []
    L.qlin_row_quantize.restype = i
    L.qlin_row_quantize.argtypes = [P, i, i, i, i, P, P, i, i, i, P]
    L.qlin_plan.restype = i
    L.qlin_plan.argtypes = [i, i, i, i, i, i, ctypes.POINTER(qlin_path)]
    L.qlin_workspace_bytes.restype = sz
    L.qlin_workspace_bytes.argtypes = [ctypes.POINTER(qlin_path), i, i, i, i, i, i]
    L.qlin_gemm.restype = i
    L.qlin_gemm.argtypes = [ctypes.POINTER(qlin_path), P, P, P, P, P, i, i, i, i, i, i, i, P, sz, P]
    L.qlin_linear.restype = i
    L.qlin_linear_noalloc.restype = i
    L.qlin_linear_noalloc.argtypes = [ctypes.POINTER(qlin_path), P, i, i, P, P, P, i, i, i, i, i,
                                      i, i, i, P]
    L.qlin_noalloc_scratch_bytes.restype = sz
    L.qlin_noalloc_scratch_bytes.argtypes = []
    L.qlin_linear.argtypes = [ctypes.POINTER(qlin_path), P, i, i, P, P, P, P, P, i, i, i, i, i,
                              i, i, i, P, sz, P]
    L.qlin_quantized_norm.restype = i
    L.qlin_quantized_norm.argtypes = [P, P, P, P, i, i, i, ctypes.c_float, i, P, P, i, i, i, P]
    L.qlin_packed_weight_bytes.restype = sz
    L.qlin_packed_weight_bytes.argtypes = [i, i]
    L.qlin_pack_weights.restype = i
    L.qlin_pack_weights.argtypes = [P, i, i, P, P]
    L.qlin_gemm_packed.restype = i
    L.qlin_gemm_packed.argtypes = L.qlin_gemm.argtypes
    L.qlin_linear_packed.restype = i
    L.qlin_linear_packed.argtypes = L.qlin_linear.argtypes
    L.qlin_gemm_finish.restype = i
    L.qlin_gemm_finish.argtypes = [ctypes.POINTER(qlin_path), P, P, P, P, P, i, P, i, i, i, i, i,
                                   i, i, i, P, sz, P]
    L.qlin_norm_linear.restype = i
    L.qlin_norm_linear.argtypes = [P, P, P, P, i, i, i, ctypes.c_float, P, P, i, i, P, i, P, P,
                                   P, P, P]
    L.qlin_norm_fusion_init.restype = None
    L.qlin_norm_fusion_init.argtypes = [P]
    L.qlin_epilogue_init.restype = None
    L.qlin_epilogue_init.argtypes = [P]
    L.qlin_layer_norm_quantize.restype = i
    L.qlin_layer_norm_quantize.argtypes = [P, i, i, P, P, ctypes.c_float, P, P, i, i, P, P, i, i,
                                           i, P]
    L.qlin_pointwise_quantize.restype = i
    L.qlin_pointwise_quantize.argtypes = [P, i, i, P, P, i, i, P, P, i, i, i, P]
    L.qlin_pointwise.restype = i
    L.qlin_pointwise.argtypes = [P, i, i, P, P, i, i, P]
    L.qlin_quantized_gated.restype = i
    L.qlin_quantized_gated.argtypes = [P, i, i, i, i, P, P, i, i, i, P]
    _lib = L
    return L


def _check(status: int):
    if status:
        raise QLinearError(status, load().qlin_last_error().decode())


def _stream(stream) -> int:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


_TYPES = {torch.bfloat16: BF16, torch.float16: F16}


def row_quantize(x: torch.Tensor, fmt: int, group: int = 0, rotation: int = 0,
                 values: torch.Tensor | None = None, scales: torch.Tensor | None = None,
                 stream=None):
    """Quantize rows of a 2-D bf16/f16 tensor (row stride allowed).
    Returns (values uint8 [rows, cols], scales f32 [rows] or [groups, rows])."""
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("row_quantize expects a 2-D tensor with unit column stride")
    if x.dtype not in _TYPES:
        raise ValueError("quantization source must be BF16 or F16")
    rows, cols = x.shape
    if values is None:
        values = torch.empty((rows, cols), dtype=torch.uint8, device=x.device)
    if scales is None:
        shape = ((cols + group - 1) // group, rows) if group else (rows,)
        scales = torch.empty(shape, dtype=torch.float32, device=x.device)
    _check(load().qlin_row_quantize(x.data_ptr(), x.stride(0), rows, cols, _TYPES[x.dtype],
                                    values.data_ptr(), scales.data_ptr(), fmt, group, rotation,
                                    _stream(stream)))
    return values, scales


def _outputs(rows, cols, group, device, values, scales):
    if values is None:
        values = torch.empty((rows, cols), dtype=torch.uint8, device=device)
    if scales is None:
        shape = ((cols + group - 1) // group, rows) if group else (rows,)
        scales = torch.empty(shape, dtype=torch.float32, device=device)
    return values, scales


def quantized_norm(residual: torch.Tensor, weight: torch.Tensor, fmt: int,
                   update: torch.Tensor | None = None, update_scale: torch.Tensor | None = None,
                   eps: float = 1e-6, gemma: bool = False, group: int = 0, rotation: int = 0,
                   values: torch.Tensor | None = None, scales: torch.Tensor | None = None,
                   stream=None):
    """Residual update (in place, when `update` is given) + RMSNorm + row
    quantization of a dense [rows, cols] bf16/f16 tensor (cols <= 2048).
    Returns (values, scales)."""
    if residual.dim() != 2 or not residual.is_contiguous() or residual.dtype not in _TYPES:
        raise ValueError("quantized_norm expects a dense 2-D bf16/f16 residual")
    for t in (weight, update, update_scale):
        if t is not None and (t.dtype != residual.dtype or not t.is_contiguous()):
            raise ValueError("quantized_norm tensors must share the residual dtype and be dense")
    rows, cols = residual.shape
    values, scales = _outputs(rows, cols, group, residual.device, values, scales)
    _check(load().qlin_quantized_norm(
        residual.data_ptr(), None if update is None else update.data_ptr(),
        None if update_scale is None else update_scale.data_ptr(), weight.data_ptr(),
        _TYPES[residual.dtype], rows, cols, float(eps), int(gemma), values.data_ptr(),
        scales.data_ptr(), fmt, group, rotation, _stream(stream)))
    return values, scales


def quantized_gated(x: torch.Tensor, fmt: int, kind: int = 0, group: int = 0, rotation: int = 0,
                    values: torch.Tensor | None = None, scales: torch.Tensor | None = None,
                    stream=None):
    """act(gate) * up of a dense [rows, 2*width] gate|up tensor (kind 0 =
    SiLU, 1 = tanh-GeLU), then row quantization. Returns (values, scales)."""
    if x.dim() != 2 or not x.is_contiguous() or x.dtype not in _TYPES or x.shape[1] % 2:
        raise ValueError("quantized_gated expects a dense [rows, 2*width] bf16/f16 tensor")
    rows, width = x.shape[0], x.shape[1] // 2
    values, scales = _outputs(rows, width, group, x.device, values, scales)
    _check(load().qlin_quantized_gated(x.data_ptr(), _TYPES[x.dtype], rows, width, kind,
                                       values.data_ptr(), scales.data_ptr(), fmt, group,
                                       rotation, _stream(stream)))
    return values, scales


class qlin_norm_fusion(ctypes.Structure):
    """NormFusion of the LayerNorm producers (include/qlinear.h)."""
    _fields_ = [("residual", ctypes.c_void_p), ("projection_bias", ctypes.c_void_p),
                ("gate", ctypes.c_void_p), ("shift", ctypes.c_void_p), ("scale", ctypes.c_void_p),
                ("gate_rows", ctypes.c_int), ("shift_rows", ctypes.c_int),
                ("scale_rows", ctypes.c_int), ("raw", ctypes.c_void_p),
                ("rows_per_sequence", ctypes.c_int), ("source_rows", ctypes.c_void_p)]


class qlin_epilogue(ctypes.Structure):
    """Dense pointwise epilogue of qlin_pointwise_quantize (include/qlinear.h)."""
    _fields_ = [("bias", ctypes.c_void_p), ("residual", ctypes.c_void_p),
                ("residual_rows", ctypes.c_int), ("residual_index", ctypes.c_void_p),
                ("value_scale", ctypes.c_float), ("output_scale", ctypes.c_float),
                ("residual_scale", ctypes.c_float), ("activation", ctypes.c_int),
                ("alpha", ctypes.c_float), ("raw", ctypes.c_void_p), ("gate", ctypes.c_void_p),
                ("gate_rows", ctypes.c_int), ("condition", ctypes.c_void_p),
                ("condition_rows", ctypes.c_int), ("rows_per_sequence", ctypes.c_int),
                ("valid_rows_per_sequence", ctypes.c_int), ("input_repeat", ctypes.c_int)]


# ops::Activation numbering (QLIN_ACT_*).
(ACT_IDENTITY, ACT_RELU, ACT_LEAKY_RELU, ACT_SILU, ACT_GELU, ACT_GELU_TANH, ACT_MISH, ACT_TANH,
 ACT_SIGMOID) = range(9)


def _ptr(t):
    return None if t is None else t.data_ptr()


def _rows(t):
    return 0 if t is None else (t.shape[0] if t.dim() == 2 else 1)


def norm_fusion(residual=None, projection_bias=None, gate=None, shift=None, scale=None,
                raw=None, rows_per_sequence: int = 1, source_rows=None) -> qlin_norm_fusion:
    """A qlin_norm_fusion over device tensors (the caller keeps them alive)."""
    f = qlin_norm_fusion()
    load().qlin_norm_fusion_init(ctypes.byref(f))
    f.residual, f.projection_bias = _ptr(residual), _ptr(projection_bias)
    f.gate, f.shift, f.scale, f.raw = _ptr(gate), _ptr(shift), _ptr(scale), _ptr(raw)
    f.gate_rows, f.shift_rows, f.scale_rows = _rows(gate), _rows(shift), _rows(scale)
    f.rows_per_sequence = rows_per_sequence
    f.source_rows = _ptr(source_rows)
    return f


def epilogue(bias=None, residual=None, residual_index=None, gate=None, condition=None, raw=None,
             value_scale: float = 1.0, output_scale: float = 1.0, residual_scale: float = 1.0,
             activation: int = ACT_IDENTITY, alpha: float = 0.1, rows_per_sequence: int = 1,
             valid_rows_per_sequence: int = 0, input_repeat: int = 1) -> qlin_epilogue:
    """A qlin_epilogue over device tensors (the caller keeps them alive)."""
    e = qlin_epilogue()
    load().qlin_epilogue_init(ctypes.byref(e))
    e.bias, e.residual, e.residual_index = _ptr(bias), _ptr(residual), _ptr(residual_index)
    e.residual_rows = _rows(residual)
    e.gate, e.gate_rows = _ptr(gate), _rows(gate)
    e.condition, e.condition_rows = _ptr(condition), _rows(condition)
    e.raw = _ptr(raw)
    e.value_scale, e.output_scale, e.residual_scale = value_scale, output_scale, residual_scale
    e.activation, e.alpha = activation, alpha
    e.rows_per_sequence, e.valid_rows_per_sequence = rows_per_sequence, valid_rows_per_sequence
    e.input_repeat = input_repeat
    return e


def _quantized_out(rows, cols, group, device, values, scales):
    if values is None:
        values = torch.empty((rows, cols), dtype=torch.uint8, device=device)
    if scales is None:
        groups = (cols + group - 1) // group if group else 1
        shape = (groups, rows) if group else (rows,)
        scales = torch.empty(shape, dtype=torch.float32, device=device)
    return values, scales


def norm_linear(x: torch.Tensor, wq: torch.Tensor, sw: torch.Tensor, fmt: int,
                norm_weight: torch.Tensor | None = None, norm_bias: torch.Tensor | None = None,
                fusion: qlin_norm_fusion | None = None, bias: torch.Tensor | None = None,
                activation: int = 0, eps: float = 1e-5, normalized: torch.Tensor | None = None,
                encoded: tuple | None = None, out: torch.Tensor | None = None,
                stream=None) -> torch.Tensor:
    """LayerNorm -> per-token quantization -> quantized GEMV (qlin_norm_linear),
    hidden k <= 512. `fusion` from norm_fusion(); `encoded` = (codes uint8
    [rows, k], scales f32 [rows])."""
    if x.dim() != 2 or not x.is_contiguous() or x.dtype not in _TYPES:
        raise ValueError("norm_linear expects a dense 2-D bf16/f16 input")
    rows, k = x.shape
    n = wq.shape[0]
    if out is None:
        out = torch.empty((rows, n), dtype=x.dtype, device=x.device)
    codes, scales = encoded if encoded is not None else (None, None)
    _check(load().qlin_norm_linear(x.data_ptr(), None if fusion is None else ctypes.byref(fusion),
                                   _ptr(norm_weight), _ptr(norm_bias), _TYPES[x.dtype], rows, k,
                                   float(eps), wq.data_ptr(), sw.data_ptr(), fmt, n, _ptr(bias),
                                   activation, out.data_ptr(), _ptr(normalized), _ptr(codes),
                                   _ptr(scales), _stream(stream)))
    return out


def layer_norm_quantize(x: torch.Tensor, fmt: int, norm_weight: torch.Tensor | None = None,
                        norm_bias: torch.Tensor | None = None, eps: float = 1e-5,
                        fusion: qlin_norm_fusion | None = None, rows: int | None = None,
                        retained: torch.Tensor | None = None, group: int = 0, rotation: int = 0,
                        values=None, scales=None, stream=None):
    """LayerNorm -> row quantization (qlin_layer_norm_quantize). Returns
    (codes uint8 [rows, cols], scales)."""
    if x.dim() != 2 or not x.is_contiguous() or x.dtype not in _TYPES:
        raise ValueError("layer_norm_quantize expects a dense 2-D bf16/f16 input")
    x_rows, cols = x.shape
    rows = x_rows if rows is None else rows
    values, scales = _quantized_out(rows, cols, group, x.device, values, scales)
    _check(load().qlin_layer_norm_quantize(
        x.data_ptr(), x_rows, _TYPES[x.dtype], _ptr(norm_weight), _ptr(norm_bias), float(eps),
        None if fusion is None else ctypes.byref(fusion), _ptr(retained), rows, cols,
        values.data_ptr(), scales.data_ptr(), fmt, group, rotation, _stream(stream)))
    return values, scales


def pointwise_quantize(x: torch.Tensor, fmt: int, epilogue: qlin_epilogue | None = None,
                       rows: int | None = None, retained: torch.Tensor | None = None,
                       group: int = 0, rotation: int = 0, values=None, scales=None, stream=None):
    """Pointwise epilogue -> row quantization (qlin_pointwise_quantize). Returns
    (codes uint8 [rows, cols], scales)."""
    if x.dim() != 2 or not x.is_contiguous() or x.dtype not in _TYPES:
        raise ValueError("pointwise_quantize expects a dense 2-D bf16/f16 input")
    x_rows, cols = x.shape
    if rows is None:
        rows = x_rows * (epilogue.input_repeat if epilogue is not None else 1)
    values, scales = _quantized_out(rows, cols, group, x.device, values, scales)
    _check(load().qlin_pointwise_quantize(
        x.data_ptr(), x_rows, _TYPES[x.dtype], None if epilogue is None else ctypes.byref(epilogue),
        _ptr(retained), rows, cols, values.data_ptr(), scales.data_ptr(), fmt, group, rotation,
        _stream(stream)))
    return values, scales


def pointwise(x: torch.Tensor, epilogue: qlin_epilogue | None = None,
              out: torch.Tensor | None = None, rows: int | None = None, stream=None):
    """Dense pointwise epilogue (qlin_pointwise): out = epilogue(x) in x's
    16-bit type; out may be x. Returns out."""
    if x.dim() != 2 or not x.is_contiguous() or x.dtype not in _TYPES:
        raise ValueError("pointwise expects a dense 2-D bf16/f16 input")
    x_rows, cols = x.shape
    if rows is None:
        rows = x_rows * (epilogue.input_repeat if epilogue is not None else 1)
    if out is None:
        out = torch.empty((rows, cols), dtype=x.dtype, device=x.device)
    if out.shape != (rows, cols) or out.dtype != x.dtype or not out.is_contiguous():
        raise ValueError("pointwise output must be dense [rows, cols] in the input type")
    _check(load().qlin_pointwise(
        x.data_ptr(), x_rows, _TYPES[x.dtype], None if epilogue is None else ctypes.byref(epilogue),
        out.data_ptr(), rows, cols, _stream(stream)))
    return out


def plan(rows: int, N: int, K: int, fmt: int, input_group: int = 0, weight_group: int = 0) -> Path:
    p = qlin_path()
    _check(load().qlin_plan(rows, N, K, fmt, input_group, weight_group, ctypes.byref(p)))
    return Path(p.kind, p.tokens, p.channels, p.splits, p.waves, p.staged)


def workspace_bytes(path: Path | None, rows: int, N: int, K: int, fmt: int,
                    input_group: int = 0, weight_group: int = 0) -> int:
    p = (path or Path()).to_c()
    return int(load().qlin_workspace_bytes(ctypes.byref(p), rows, N, K, fmt, input_group,
                                           weight_group))


@dataclass
class PackedWeights:
    """Weights [N, K] in the packed fragment-tile layout (qlin_pack_weights)."""
    data: torch.Tensor  # uint8 [qlin_packed_weight_bytes(N, K)]
    N: int
    K: int

    @property
    def shape(self):
        return (self.N, self.K)

    def data_ptr(self):
        return self.data.data_ptr()


def pack_weights(wq: torch.Tensor, stream=None) -> PackedWeights:
    """Repack row-major quantized weights [N, K] (once, at load time)."""
    if wq.dim() != 2 or not wq.is_contiguous() or wq.dtype != torch.uint8:
        raise ValueError("pack_weights expects dense uint8 [N, K] weights")
    N, K = wq.shape
    nbytes = int(load().qlin_packed_weight_bytes(N, K))
    if nbytes == 0:
        raise ValueError("packed weights need N % 16 == 0")
    out = torch.empty(nbytes, dtype=torch.uint8, device=wq.device)
    _check(load().qlin_pack_weights(wq.data_ptr(), N, K, out.data_ptr(), _stream(stream)))
    return PackedWeights(out, N, K)


def gemm(xq: torch.Tensor, sx: torch.Tensor, wq: torch.Tensor, sw: torch.Tensor, fmt: int,
         out_dtype=torch.bfloat16, input_group: int = 0, weight_group: int = 0,
         path: Path | None = None, workspace: torch.Tensor | None = None,
         out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    M, K = xq.shape
    N = wq.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=xq.device)
    need = workspace_bytes(path, M, N, K, fmt, input_group, weight_group)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=xq.device)
    p = (path or Path()).to_c()
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    fn = load().qlin_gemm_packed if isinstance(wq, PackedWeights) else load().qlin_gemm
    _check(fn(ctypes.byref(p), xq.data_ptr(), sx.data_ptr(), wq.data_ptr(),
                            sw.data_ptr(), out.data_ptr(), M, N, K, fmt,
                            F16 if out.dtype == torch.float16 else BF16, input_group,
                            weight_group, ws_ptr, ws_bytes, _stream(stream)))
    return out


FINISH_NONE, FINISH_RELU, FINISH_GELU_TANH = 0, 1, 2


def gemm_finish(xq: torch.Tensor, sx: torch.Tensor, wq, sw: torch.Tensor, fmt: int,
                bias: torch.Tensor | None = None, activation: int = FINISH_NONE,
                out_dtype=torch.bfloat16, input_group: int = 0, weight_group: int = 0,
                path: Path | None = None, workspace: torch.Tensor | None = None,
                out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """GEMM + the reference's finish, y = s16(act(s16(s16(d) + bias))), in one
    epilogue (qlin_gemm_finish). `wq` may be PackedWeights."""
    M, K = xq.shape
    N = wq.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=xq.device)
    if bias is not None and (bias.dtype != out.dtype or bias.numel() != N or not bias.is_contiguous()):
        raise ValueError("finish bias must be a dense [N] tensor of the output dtype")
    need = workspace_bytes(path, M, N, K, fmt, input_group, weight_group)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=xq.device)
    p = (path or Path()).to_c()
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check(load().qlin_gemm_finish(ctypes.byref(p), xq.data_ptr(), sx.data_ptr(), wq.data_ptr(),
                                   sw.data_ptr(), None if bias is None else bias.data_ptr(),
                                   activation, out.data_ptr(), M, N, K, fmt,
                                   F16 if out.dtype == torch.float16 else BF16, input_group,
                                   weight_group, int(isinstance(wq, PackedWeights)), ws_ptr,
                                   ws_bytes, _stream(stream)))
    return out


def linear(x: torch.Tensor, wq: torch.Tensor, sw: torch.Tensor, fmt: int, group: int = 0,
           rotation: int = 0, out_dtype=torch.bfloat16, path: Path | None = None,
           scratch: tuple[torch.Tensor, torch.Tensor] | None = None,
           out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
           stream=None) -> torch.Tensor:
    """Quantize the 16-bit activations into the scratch activation (xq, sx) and
    run the GEMM: the quantized branch of the reference ops::linear
    (ops/linear.cpp:51-71) through qlin_linear. `scratch` is allocated when
    not given."""
    if x.dim() != 2 or x.stride(1) != 1 or x.dtype not in _TYPES:
        raise ValueError("linear expects a 2-D bf16/f16 tensor with unit column stride")
    rows, K = x.shape
    N = wq.shape[0]
    if out is None:
        out = torch.empty((rows, N), dtype=out_dtype, device=x.device)
    if scratch is None:
        shape = ((K + group - 1) // group, rows) if group else (rows,)
        scratch = (torch.empty((rows, K), dtype=torch.uint8, device=x.device),
                   torch.empty(shape, dtype=torch.float32, device=x.device))
    need = workspace_bytes(path, rows, N, K, fmt, group, group)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    p = (path or Path()).to_c()
    fn = load().qlin_linear_packed if isinstance(wq, PackedWeights) else load().qlin_linear
    _check(fn(ctypes.byref(p), x.data_ptr(), x.stride(0), _TYPES[x.dtype],
                              scratch[0].data_ptr(), scratch[1].data_ptr(), wq.data_ptr(),
                              sw.data_ptr(), out.data_ptr(), rows, N, K, fmt, _TYPES[out.dtype],
                              group, group, rotation, ws_ptr, ws_bytes, _stream(stream)))
    return out


def linear_noalloc(x: torch.Tensor, wq: torch.Tensor, sw: torch.Tensor, fmt: int, group: int = 0,
                   rotation: int = 0, out_dtype=torch.bfloat16, path: Path | None = None,
                   out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """qlin_linear_noalloc: the same quantize + GEMM as `linear`, with the
    scratch activation and split-K partials in the library's fixed device
    array (nothing is allocated by the call itself)."""
    if x.dim() != 2 or x.stride(1) != 1 or x.dtype not in _TYPES:
        raise ValueError("linear_noalloc expects a 2-D bf16/f16 tensor with unit column stride")
    rows, K = x.shape
    N = wq.shape[0]
    if out is None:
        out = torch.empty((rows, N), dtype=out_dtype, device=x.device)
    p = (path or Path()).to_c()
    _check(load().qlin_linear_noalloc(ctypes.byref(p), x.data_ptr(), x.stride(0), _TYPES[x.dtype],
                                      wq.data_ptr(), sw.data_ptr(), out.data_ptr(), rows, N, K,
                                      fmt, _TYPES[out.dtype], group, group, rotation,
                                      _stream(stream)))
    return out
