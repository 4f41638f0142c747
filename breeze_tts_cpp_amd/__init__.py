"""MI355X (gfx950) quantized linear path of TTS.cpp: per-token / K-group
INT8 and OCP-FP8 activation quantization (optional H128 rotation) and the
quantized GEMM with fused dequant epilogue, as hand-written HIP kernels in
libqlinear.so behind a C ABI (include/qlinear.h)."""
from . import synthetic  # noqa: F401

__all__ = ["synthetic"]
