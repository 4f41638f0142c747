"""CPU pin of the identity behind the fused decode GEMM's INT8 encoder
(encode_i8x4 in csrc/qlin_device.hpp): after the clamp to [-127, 127], the
fp32 sum x + 1.5 * 2^23 (round-to-nearest-even, as numpy's float32 add)
holds rint(x) -- ties to even -- in two's complement in its low byte, so the
byte equals the quantizer's encode_i8 code int(rintf(clamp(x))) & 0xff
(reference quant_format.cuh:37-47). Checked on every tie n + 0.5 and its
float neighbours, a dense grid, random values and out-of-range values."""
import numpy as np

MAGIC = np.float32(12582912.0)  # 1.5 * 2^23


def magic_codes(x):
    c = np.minimum(np.float32(127), np.maximum(np.float32(-127), x.astype(np.float32)))
    return ((c + MAGIC).view(np.uint32) & 0xFF).astype(np.uint8)


def rint_codes(x):
    c = np.minimum(np.float32(127), np.maximum(np.float32(-127), x.astype(np.float32)))
    return (np.rint(c).astype(np.int32) & 0xFF).astype(np.uint8)


def test_ties_and_neighbours():
    ties = (np.arange(-128, 128, dtype=np.float32) + np.float32(0.5))
    up = np.nextafter(ties, np.float32(np.inf))
    down = np.nextafter(ties, np.float32(-np.inf))
    for x in (ties, up, down, np.arange(-127, 128, dtype=np.float32)):
        assert np.array_equal(magic_codes(x), rint_codes(x))
    # ties go to even: 0.5 -> 0, 1.5 -> 2, -2.5 -> -2
    assert list(magic_codes(np.float32([0.5, 1.5, -2.5, -0.5]))) == [0, 2, 254, 0]


def test_dense_grid_and_random():
    grid = np.arange(-130 * 4096, 130 * 4096 + 1, dtype=np.int64).astype(np.float32) / np.float32(4096)
    assert np.array_equal(magic_codes(grid), rint_codes(grid))
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(2_000_000) * 60).astype(np.float32)
    assert np.array_equal(magic_codes(x), rint_codes(x))
    tiny = (rng.standard_normal(100_000) * 1e-30).astype(np.float32)  # incl. -0 results
    assert np.array_equal(magic_codes(tiny), rint_codes(tiny))


def test_out_of_range_clamps():
    x = np.float32([127.4, 127.5, 128, 1e30, np.inf, -127.6, -1e30, -np.inf])
    assert list(magic_codes(x)) == [127, 127, 127, 127, 127, 129, 129, 129]
    assert np.array_equal(magic_codes(x), rint_codes(x))
