"""Packed weight layout on the GPU, through the C ABI: qlin_pack_weights
against the oracle's packing, and qlin_gemm_packed / qlin_linear_packed
against the oracle (INT8 bit-exact, FP8 bit-identical to the row-major GEMM)
in the decode (register-streamed packed tiles) and prefill (LDS-staged)
regimes, per-channel and K-group, with ragged K (K % 64 != 0)."""
import numpy as np
import pytest
import torch

from breeze_tts_cpp_amd import synthetic
from tests.test_gpu_gemm import (FP8_REL_L2, PROJ, bits_to_f32, check_i8, dev_f32, dev_u8,
                                 operands, out_bits, rel_l2)

pytestmark = pytest.mark.gpu
I8, FP8 = 4, 3


def packed_gemm(dev, xq, sx, wq, sw, fmt, group=0, path=None, out_dtype=torch.bfloat16):
    from breeze_tts_cpp_amd import qlinear
    pw = qlinear.pack_weights(dev_u8(wq, dev))
    y = qlinear.gemm(dev_u8(xq, dev), dev_f32(sx, dev), pw, dev_f32(sw, dev), fmt,
                     out_dtype=out_dtype, input_group=group, weight_group=group, path=path)
    torch.cuda.synchronize()
    return out_bits(y), pw


@pytest.mark.parametrize("N,K", [(64, 2048), (48, 80), (4096, 2048), (2048, 6144), (32, 1040)])
def test_pack_matches_oracle(dev, orc, N, K):
    from breeze_tts_cpp_amd import qlinear
    print(f"pack N={N} K={K}", flush=True)
    wq = np.random.default_rng(N + K).integers(0, 256, (N, K), dtype=np.uint8)
    pw = qlinear.pack_weights(dev_u8(wq, dev))
    torch.cuda.synchronize()
    assert np.array_equal(pw.data.cpu().numpy(), orc.pack_weights(wq))


@pytest.mark.parametrize("M", [1, 8, 32, 64])
@pytest.mark.parametrize("N,K", PROJ)
def test_packed_decode_projections(dev, orc, M, N, K):
    print(f"packed decode M={M} N={N} K={K}", flush=True)
    xq, sx, wq, sw = operands(orc, M, N, K, I8, seed=M + N)
    y, _ = packed_gemm(dev, xq, sx, wq, sw, I8)
    check_i8(orc, y, xq, sx, wq, sw)


@pytest.mark.parametrize("M,N,K", [(16, 48, 80), (32, 112, 1040), (5, 64, 4160), (64, 256, 336)])
def test_packed_ragged_k(dev, orc, M, N, K):
    """K not a multiple of 64 (zero-padded tiles) and few K blocks per wave."""
    print(f"packed ragged M={M} N={N} K={K}", flush=True)
    for fmt in (I8, FP8):
        xq, sx, wq, sw = operands(orc, M, N, K, fmt, seed=K)
        y, _ = packed_gemm(dev, xq, sx, wq, sw, fmt)
        if fmt == I8:
            check_i8(orc, y, xq, sx, wq, sw)
        else:
            from tests.test_gpu_gemm import gpu_gemm
            assert np.array_equal(y, gpu_gemm(dev, xq, sx, wq, sw, fmt))


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("M", [32, 4096])
def test_packed_grouped(dev, orc, fmt, M):
    """group_int8 / group_fp8 (H128 rotation + K128 groups) on packed weights.
    Prefill: identical to the row-major GEMM. Decode: the packed kernel sums
    its wave ranges separately, so INT8 is bit-exact against the oracle's
    grouped GEMM over that partition, and FP8 within rel-L2 1e-2."""
    from breeze_tts_cpp_amd import qlinear
    from tests.test_gpu_gemm import gpu_gemm, bits_to_f32, rel_l2
    N, K = 2048, 2048
    print(f"packed grouped fmt={fmt} M={M}", flush=True)
    xq, sx, wq, sw = operands(orc, M, N, K, fmt, group=128, rotation=128, seed=M + 5)
    y, _ = packed_gemm(dev, xq, sx, wq, sw, fmt, group=128)
    if M > 64:
        assert np.array_equal(y, gpu_gemm(dev, xq, sx, wq, sw, fmt, group=128))
    elif fmt == I8:
        p = qlinear.plan(M, N, K, fmt, 128, 128)
        part = qlinear.grouped_partition(p, K, fmt, 128, 128, packed=True)
        ref, _ = orc.gemm_grouped(xq, sx, wq, sw, fmt, 128, 128, *part)
        assert np.array_equal(y, ref), f"{np.count_nonzero(y != ref)} mismatches"
    else:
        ideal = orc.gemm_grouped_ideal(xq, sx, wq, sw, fmt, 128, 128)
        assert rel_l2(bits_to_f32(y), ideal) <= 1e-2


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("N,K", PROJ)
def test_packed_prefill(dev, orc, fmt, N, K):
    """M=4096 through every tiled macro-tile shape on packed weights; sampled
    rows against the oracle, whole output against the row-major GEMM."""
    from breeze_tts_cpp_amd.qlinear import Path, KIND_TILED
    from tests.test_gpu_gemm import gpu_gemm
    M = 4096
    xq, sx, wq, sw = operands(orc, M, N, K, fmt, seed=N + K)
    rows = np.unique(np.concatenate([[0, 255, 256, M - 1],
                                     np.random.default_rng(N).choice(M, 28, replace=False)]))
    shapes = [(256, 256, 4), (256, 128, 2), (256, 128, 1), (256, 128, 8), (128, 128, 1), (128, 128, 8)]
    if fmt == I8:
        shapes += [(256, 256, 8)]
    for channels, tokens, waves, *staged in shapes:
        p = Path(KIND_TILED, tokens, channels, 1, waves, *staged)
        print(f"packed prefill fmt={fmt} N={N} K={K} path={p}", flush=True)
        y, _ = packed_gemm(dev, xq, sx, wq, sw, fmt, path=p)
        assert np.array_equal(y, gpu_gemm(dev, xq, sx, wq, sw, fmt, path=p))
        if fmt == I8:
            check_i8(orc, y[rows], xq[rows], sx[rows], wq, sw)
        else:
            ideal = orc.gemm_fp8_ideal(xq[rows], sx[rows], wq, sw)
            assert rel_l2(bits_to_f32(y[rows]), ideal) <= FP8_REL_L2


def test_packed_linear(dev, orc):
    """qlin_linear_packed: quantize into the scratch activation, then the
    packed GEMM (the bench's decode step)."""
    from breeze_tts_cpp_amd import qlinear
    M, N, K = 32, 12288, 2048
    xb = synthetic.activations(M, K, seed=3)
    wb = synthetic.weights(N, K, seed=3)
    wq, sw = orc.quantize_rows(wb, I8)
    pw = qlinear.pack_weights(dev_u8(wq, dev))
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev)
    y = qlinear.linear(x, pw, dev_f32(sw, dev), I8)
    torch.cuda.synchronize()
    xq, sx = orc.quantize_rows(xb, I8)
    check_i8(orc, out_bits(y), xq, sx, wq, sw)


def test_packed_rejects_split_and_staged(dev, orc):
    from breeze_tts_cpp_amd import qlinear
    from breeze_tts_cpp_amd.qlinear import Path, KIND_SKINNY
    xq, sx, wq, sw = operands(orc, 32, 256, 2048, I8, seed=1)
    pw = qlinear.pack_weights(dev_u8(wq, dev))
    for p in (Path(KIND_SKINNY, 32, 16, 2, 8), Path(KIND_SKINNY, 32, 16, 1, 8, 1)):
        with pytest.raises(qlinear.QLinearError):
            qlinear.gemm(dev_u8(xq, dev), dev_f32(sx, dev), pw, dev_f32(sw, dev), I8, path=p)
