"""Parity of qlin_linear, the quantized branch of the reference ops::linear
(ops/linear.cpp:51-71: quantize_rows into the scratch activation, then
QuantizedGemm::linear), on the GPU through the C ABI: the scratch activation
equals the oracle's quantizer output, and the output equals the oracle's
INT8 GEMM + epilogue D((acc*sx)*sw) bit for bit (FP8: rel-L2 <= 1e-2 of the
fp64 product of the quantized operands, the task's FP8 contract)."""
import numpy as np
import pytest
import torch

from breeze_tts_cpp_amd import synthetic

BF16, F32, I32, FP8, I8, F16 = 0, 1, 2, 3, 4, 5
pytestmark = pytest.mark.gpu


def bits(y):
    return y.cpu().view(torch.int16).numpy().view(np.uint16)


def to_dev16(xb, dtype, dev):
    """bf16 bit patterns -> device tensor of `dtype` (f16 via float32)."""
    t = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16)
    return (t if dtype == torch.bfloat16 else t.float().to(dtype)).to(dev)


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("M,N,K", [(16, 2048, 2048), (32, 4096, 2048), (5, 96, 2048),
                                   (17, 48, 4096), (40, 144, 2048), (64, 32, 2048),
                                   (3, 64, 6144), (300, 272, 1024)])
def test_linear_against_oracle(dev, orc, fmt, M, N, K):
    from breeze_tts_cpp_amd import qlinear
    print(f"linear fmt={fmt} M={M} N={N} K={K}", flush=True)
    xb = synthetic.activations(M, K, seed=M * 7 + K)
    wq, sw = orc.quantize_rows(synthetic.weights(N, K, seed=N), fmt)
    xq_d = torch.empty((M, K), dtype=torch.uint8, device=dev)
    sx_d = torch.empty((M,), dtype=torch.float32, device=dev)
    y = qlinear.linear(to_dev16(xb, torch.bfloat16, dev), torch.from_numpy(wq).to(dev),
                       torch.from_numpy(sw).to(dev), fmt, scratch=(xq_d, sx_d))
    torch.cuda.synchronize()
    xq, sx = orc.quantize_rows(xb, fmt)
    assert np.array_equal(xq_d.cpu().numpy(), xq)
    assert np.array_equal(sx_d.cpu().numpy(), sx)
    if fmt == I8:
        assert np.array_equal(bits(y), orc.epilogue_i8(orc.gemm_i8_acc(xq, wq), sx, sw))
    else:
        ideal = orc.gemm_fp8_ideal(xq, sx, wq, sw)
        got = synthetic.bf16_bits_to_f32(bits(y)).astype(np.float64)
        assert np.linalg.norm(got - ideal) / np.linalg.norm(ideal) <= 1e-2


def test_linear_f16_strided_special_rows(dev, orc):
    """f16 activations and output, row stride > K, an all-zero row (scale 1,
    codes 0), a row with one huge value and a row of tiny values."""
    from breeze_tts_cpp_amd import qlinear
    M, N, K, ld = 24, 256, 2048, 2048 + 64
    xb = synthetic.activations(M, K, seed=5)
    xb[3] = 0
    xb[7, 100] = synthetic.f32_to_bf16_bits(np.float32(3.0e4)).item()
    xb[11] = synthetic.f32_to_bf16_bits(np.full(K, 1e-3, np.float32))
    wide = np.zeros((M, ld), np.uint16)
    wide[:, :K] = xb
    x = to_dev16(wide, torch.float16, dev)[:, :K]
    assert x.stride(0) == ld
    wq, sw = orc.quantize_rows(synthetic.weights(N, K, seed=9), I8)
    xq_d = torch.empty((M, K), dtype=torch.uint8, device=dev)
    sx_d = torch.empty((M,), dtype=torch.float32, device=dev)
    y = qlinear.linear(x, torch.from_numpy(wq).to(dev), torch.from_numpy(sw).to(dev), I8,
                       out_dtype=torch.float16, scratch=(xq_d, sx_d))
    torch.cuda.synchronize()
    xh = x.cpu().view(torch.int16).numpy().view(np.uint16)
    xq, sx = orc.quantize_rows(xh, I8, src_type=F16)
    assert np.array_equal(xq_d.cpu().numpy(), xq) and np.array_equal(sx_d.cpu().numpy(), sx)
    assert sx[3] == 1.0 and not xq[3].any()
    ref = orc.epilogue_i8(orc.gemm_i8_acc(xq, wq), sx, sw, out_type=F16)
    assert np.array_equal(bits(y), ref)


def test_linear_group_rotation(dev, orc):
    """group_int8 (H128 rotation + K128 groups, config 3) at M=32: the scratch
    activation and the output equal row_quantize followed by gemm."""
    from breeze_tts_cpp_amd import qlinear
    M, N, K = 32, 4096, 2048
    xb = synthetic.activations(M, K, seed=4)
    wq, sw = orc.quantize_rows(synthetic.weights(N, K, seed=4), I8, group=128, rotation=128)
    wq_d, sw_d = torch.from_numpy(wq).to(dev), torch.from_numpy(sw).to(dev)
    x = to_dev16(xb, torch.bfloat16, dev)
    y = qlinear.linear(x, wq_d, sw_d, I8, group=128, rotation=128)
    xq, sx = qlinear.row_quantize(x, I8, group=128, rotation=128)
    y_ref = qlinear.gemm(xq, sx, wq_d, sw_d, I8, input_group=128, weight_group=128)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)


def test_stream_read_ceiling_kernel(dev):
    """The streaming-read measurement kernel reads a buffer without writing:
    the sink stays untouched and the buffer unchanged, for sizes that are not
    a multiple of its 512-workgroup split (a tail workgroup with fewer
    16-byte rows) and for the decode weight sizes."""
    from breeze_tts_cpp_amd import measure
    L = measure.load()
    for nbytes in (16, 16 * 1000 + 16, 2048 * 2048, 12288 * 2048):
        print(f"stream_read bytes={nbytes}", flush=True)
        buf = torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device=dev)
        ref = buf.clone()
        sink = torch.full((1024,), 7, dtype=torch.int32, device=dev)
        assert L.qlm_stream_read(buf.data_ptr(), nbytes, sink.data_ptr(), None) == 0
        torch.cuda.synchronize()
        assert torch.equal(buf, ref)
        assert bool((sink == 7).all())
