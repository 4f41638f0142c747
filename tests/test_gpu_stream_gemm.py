"""The 512x128 register-streamed INT8 prefill GEMM (explicit path channels
512 x tokens 128, four waves; disabled, see below), on row-major and packed weights:
bf16 output bit-exact against D((acc*sx)*sw) with exact int32 acc (the
CUTLASS EVT order, quant_gemm_sm80.cu:24-29), against the other tiled paths,
through the fused finish epilogue and with f16 output. Ragged M and N edges,
K from one 64-byte stage up, grids of several rounds."""
import numpy as np
import pytest
import torch

from tests.test_gpu_gemm import (BF16, F16, I8, PROJ, check_i8, dev_f32, dev_u8, gpu_gemm,
                                 operands, out_bits)

# The path is disabled: a run that replayed CUDA graphs of this kernel
# alternately with the planned tiled kernels (gate_up, M = 4096) faulted the
# GPU twice, its cause not found, while every case below passed when run
# eagerly. The library now rejects the path (QLIN_ERR_UNSUPPORTED) and does not
# build the kernel.
pytestmark = [pytest.mark.gpu,
              pytest.mark.skip(reason="512x128 register-streamed path disabled: GPU fault "
                                      "under graph replay, cause not found")]


def stream_path():
    from breeze_tts_cpp_amd.qlinear import Path, KIND_TILED
    return Path(KIND_TILED, 128, 512, 1, 4)


def packed_gemm(dev, xq, sx, wq, sw, path, out_dtype=torch.bfloat16):
    from breeze_tts_cpp_amd import qlinear
    pw = qlinear.pack_weights(dev_u8(wq, dev))
    y = qlinear.gemm(dev_u8(xq, dev), dev_f32(sx, dev), pw, dev_f32(sw, dev), I8,
                     out_dtype=out_dtype, path=path)
    torch.cuda.synchronize()
    return out_bits(y)


@pytest.mark.parametrize("M,N,K", [(1, 512, 64), (77, 528, 64), (130, 560, 128),
                                   (200, 144, 320), (300, 1040, 1024), (129, 2064, 6144)])
def test_stream_ragged(dev, orc, M, N, K):
    """Whole output against the oracle, row-major and packed weights."""
    print(f"stream gemm ragged M={M} N={N} K={K}", flush=True)
    xq, sx, wq, sw = operands(orc, M, N, K, I8, seed=M + N + K)
    y = gpu_gemm(dev, xq, sx, wq, sw, I8, path=stream_path())
    check_i8(orc, y, xq, sx, wq, sw)
    yp = packed_gemm(dev, xq, sx, wq, sw, stream_path())
    assert np.array_equal(yp, y)


@pytest.mark.parametrize("M", [1024, 4096])
@pytest.mark.parametrize("N,K", PROJ)
def test_stream_projections(dev, orc, M, N, K):
    """Full prefill shapes: the whole output against the planned path, sampled
    token rows against the oracle; packed weights give the same bits."""
    print(f"stream gemm M={M} N={N} K={K}", flush=True)
    xq, sx, wq, sw = operands(orc, M, N, K, I8, seed=M + N)
    y = gpu_gemm(dev, xq, sx, wq, sw, I8, path=stream_path())
    assert np.array_equal(y, gpu_gemm(dev, xq, sx, wq, sw, I8))
    assert np.array_equal(packed_gemm(dev, xq, sx, wq, sw, stream_path()), y)
    rng = np.random.default_rng(M + N + K)
    rows = np.unique(np.concatenate([[0, 127, 128, M - 1], rng.choice(M, 28, replace=False)]))
    check_i8(orc, y[rows], xq[rows], sx[rows], wq, sw)


def test_stream_f16_and_finish(dev, orc):
    """f16 output, and the bias + tanh-GeLU finish, equal to the planned
    tiled kernel's (same epilogue arithmetic)."""
    from breeze_tts_cpp_amd import qlinear
    M, N, K = 384, 1536, 512
    print(f"stream gemm f16 / finish M={M} N={N} K={K}", flush=True)
    xq, sx, wq, sw = operands(orc, M, N, K, I8, seed=7)
    y16 = gpu_gemm(dev, xq, sx, wq, sw, I8, path=stream_path(), out_dtype=torch.float16)
    check_i8(orc, y16, xq, sx, wq, sw, out_type=F16)
    bias = torch.from_numpy(np.random.default_rng(3).standard_normal(N).astype(np.float32)).to(
        torch.bfloat16).to(dev)
    args = (dev_u8(xq, dev), dev_f32(sx, dev), dev_u8(wq, dev), dev_f32(sw, dev), I8)
    for act in (qlinear.FINISH_RELU, qlinear.FINISH_GELU_TANH):
        a = qlinear.gemm_finish(*args, bias=bias, activation=act, path=stream_path())
        b = qlinear.gemm_finish(*args, bias=bias, activation=act)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"activation {act}"
