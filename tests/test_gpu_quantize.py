"""Parity of the HIP row quantizer (qlin_row_quantize through the C ABI)
against the oracle: values and scales bit-exact for INT8 and FP8, every
layout of the reference dispatch (row_quantize.cu:167-193)."""
import numpy as np
import pytest
import torch

from breeze_tts_cpp_amd import synthetic

BF16, F32, I32, FP8, I8, F16 = 0, 1, 2, 3, 4, 5
pytestmark = pytest.mark.gpu


def to_dev(bits: np.ndarray, dev, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(dtype).to(dev)


def run(dev, bits, fmt, group=0, rotation=0, dtype=torch.bfloat16, ld=None):
    from breeze_tts_cpp_amd import qlinear
    rows, cols = bits.shape
    if ld is not None and ld != cols:
        wide = np.zeros((rows, ld), np.uint16)
        wide[:, :cols] = bits
        x = to_dev(wide, dev, dtype)[:, :cols]
    else:
        x = to_dev(bits, dev, dtype)
    q, s = qlinear.row_quantize(x, fmt, group, rotation)
    torch.cuda.synchronize()
    return q.cpu().numpy(), s.cpu().numpy()


CASES = [
    # rows, cols
    (16, 2048),   # config 0 activations
    (32, 6144),   # down-projection input (K=6144, three cached chunks)
    (3, 128),
    (5, 4096),
    (64, 2048),
    # one 8-column piece per lane over 512..1024 threads (decode-sized rows)
    (7, 2056), (9, 8192), (3, 7000),
    (600, 6144),  # many rows: 256 threads of three pieces
]


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("rows,cols", CASES)
def test_token_quant(dev, orc, fmt, rows, cols):
    print(f"token_quant fmt={fmt} rows={rows} cols={cols}", flush=True)
    bits = synthetic.activations(rows, cols, seed=rows * 7 + cols)
    q, s = run(dev, bits, fmt)
    q_ref, s_ref = orc.quantize_rows(bits, fmt)
    assert np.array_equal(s, s_ref)
    assert np.array_equal(q, q_ref)


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("rows,cols", [(4, 2048), (8, 6144), (2, 128), (3, 20480), (5, 8192)])
def test_rotated_token_quant(dev, orc, fmt, rows, cols):
    print(f"rotated_token_quant fmt={fmt} rows={rows} cols={cols}", flush=True)
    bits = synthetic.activations(rows, cols, seed=cols + 1)
    q, s = run(dev, bits, fmt, rotation=128)
    q_ref, s_ref = orc.quantize_rows(bits, fmt, rotation=128)
    assert np.array_equal(s, s_ref)
    assert np.array_equal(q, q_ref)


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("rotation", [0, 128])
@pytest.mark.parametrize("rows,cols", [(32, 2048), (7, 6144), (3, 384)])
def test_group_quant(dev, orc, fmt, group, rotation, rows, cols):
    print(f"group_quant fmt={fmt} g={group} rot={rotation} rows={rows} cols={cols}", flush=True)
    bits = synthetic.activations(rows, cols, seed=group + rotation + cols)
    q, s = run(dev, bits, fmt, group=group, rotation=rotation)
    q_ref, s_ref = orc.quantize_rows(bits, fmt, group=group, rotation=rotation)
    assert np.array_equal(s, s_ref)
    assert np.array_equal(q, q_ref)


@pytest.mark.parametrize("fmt", [I8, FP8])
def test_long_rows_stream_twice(dev, orc, fmt):
    """cols > 16384 leaves the register-cached kernel for the two-pass one."""
    bits = synthetic.activations(3, 20000, seed=3)
    q, s = run(dev, bits, fmt)
    q_ref, s_ref = orc.quantize_rows(bits, fmt)
    assert np.array_equal(s, s_ref) and np.array_equal(q, q_ref)


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("group", [0, 64])
def test_ragged_and_strided(dev, orc, fmt, group):
    """Columns not a multiple of 8 and a padded row stride take the
    element-wise variant; results must not change."""
    for rows, cols, ld in ((5, 1000, 1000), (4, 2051, 2051), (6, 512, 600), (2, 96, 104)):
        bits = synthetic.activations(rows, cols, seed=cols)
        q, s = run(dev, bits, fmt, group=group, ld=ld)
        q_ref, s_ref = orc.quantize_rows(bits, fmt, group=group)
        assert np.array_equal(s, s_ref), (rows, cols, ld)
        assert np.array_equal(q, q_ref), (rows, cols, ld)


@pytest.mark.parametrize("fmt", [I8, FP8])
def test_f16_source(dev, orc, fmt):
    xf = synthetic.bf16_bits_to_f32(synthetic.activations(8, 2048, seed=8))
    h = xf.astype(np.float16).view(np.uint16)
    q, s = run(dev, h, fmt, dtype=torch.float16)
    q_ref, s_ref = orc.quantize_rows(h, fmt, src_type=F16)
    assert np.array_equal(s, s_ref) and np.array_equal(q, q_ref)
    q, s = run(dev, h, fmt, group=128, rotation=128, dtype=torch.float16)
    q_ref, s_ref = orc.quantize_rows(h, fmt, group=128, rotation=128, src_type=F16)
    assert np.array_equal(s, s_ref) and np.array_equal(q, q_ref)


def test_fp8_encoder_every_bf16_value(dev, orc):
    """A row whose amax is exactly 448 has scale 1 and inverse 1, so the
    codes are the e4m3fn encoding of every other element: sweep all finite
    bf16 values of magnitude <= 448 through the GPU encoder."""
    vals = np.arange(0, 0x7F80, dtype=np.uint32).astype(np.uint16)
    f = synthetic.bf16_bits_to_f32(vals)
    vals = vals[np.abs(f) <= 448]
    vals = np.concatenate([vals, vals | np.uint16(0x8000)])
    cols = 2048
    pad = (-len(vals)) % (cols - 1)
    vals = np.concatenate([vals, np.zeros(pad, np.uint16)]).reshape(-1, cols - 1)
    head = np.full((vals.shape[0], 1), synthetic.f32_to_bf16_bits(np.float32(448.0)), np.uint16)
    bits = np.concatenate([head, vals], axis=1)
    q, s = run(dev, bits, FP8)
    assert np.all(s == 1.0)
    ref = orc.fp8_encode(synthetic.bf16_bits_to_f32(bits))
    assert np.array_equal(q, ref)


def test_zero_rows_and_extremes(dev, orc):
    bits = synthetic.activations(6, 2048, seed=9)
    bits[0] = 0
    bits[1, :] = synthetic.f32_to_bf16_bits(np.float32(1e-30))  # amax/127 below FLT_MIN? no: > tiny
    bits[2, 5] = synthetic.f32_to_bf16_bits(np.float32(3.0e38)).item()
    for fmt in (I8, FP8):
        for group, rotation in ((0, 0), (0, 128), (128, 0), (128, 128)):
            q, s = run(dev, bits, fmt, group=group, rotation=rotation)
            q_ref, s_ref = orc.quantize_rows(bits, fmt, group=group, rotation=rotation)
            assert np.array_equal(s, s_ref), (fmt, group, rotation)
            assert np.array_equal(q, q_ref), (fmt, group, rotation)
