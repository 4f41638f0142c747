"""ctypes binding of libqlin_measure.so (include/qlin_measure.h): the
streaming-read ceiling kernel that bench.py times the decode GEMMs against.
It is a measurement helper, outside the quantized linear ABI."""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqlin_measure.so")
_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (make -C breeze_tts_cpp_amd)")
        L = ctypes.CDLL(LIB_PATH)
        L.qlm_stream_read.restype = ctypes.c_int
        L.qlm_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                      ctypes.c_void_p]
        _lib = L
    return _lib


def stream_read(buf: torch.Tensor, stream=None) -> None:
    """Reads every byte of the contiguous device tensor `buf` (its size a
    multiple of 16) once."""
    assert buf.is_contiguous()
    if stream is None:
        stream = torch.cuda.current_stream()
    rc = load().qlm_stream_read(buf.data_ptr(), buf.numel() * buf.element_size(), None,
                                ctypes.c_void_p(stream.cuda_stream))
    if rc:
        raise RuntimeError(f"qlm_stream_read failed ({rc})")
