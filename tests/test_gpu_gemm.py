"""Parity of the HIP quantized GEMM (qlin_gemm through the C ABI) against the
oracle.

INT8 per-channel: bf16 output bit-exact against D((acc*sx)*sw) with exact
int32 acc (the CUTLASS EVT order, quant_gemm_sm80.cu:24-29), hence within one
bf16 ulp of the GEMV order (acc*sw)*sx (quant_dispatch.cu:125).
INT8 K-group: bit-exact against the oracle's grouped accumulation with the
same K partition (quant_grouped.cu:112-166).
FP8: rel-L2 <= 1e-2 against the fp64 product of the quantized operands
(tolerance of the task contract; the reference's fp32 accumulation order is
hardware-defined)."""
import numpy as np
import pytest
import torch

from breeze_tts_cpp_amd import synthetic

BF16, F32, I32, FP8, I8, F16 = 0, 1, 2, 3, 4, 5
pytestmark = pytest.mark.gpu
FP8_REL_L2 = 1e-2


def dev_u8(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint8)).to(dev)


def dev_f32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def out_bits(y: torch.Tensor) -> np.ndarray:
    return y.cpu().view(torch.int16).numpy().view(np.uint16)


def bits_to_f32(bits, out_type=BF16):
    if out_type == F16:
        return bits.view(np.float16).astype(np.float32)
    return synthetic.bf16_bits_to_f32(bits)


def rel_l2(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / np.linalg.norm(b))


_cache = {}


def operands(orc, M, N, K, fmt, group=0, rotation=0, seed=0):
    key = (M, N, K, fmt, group, rotation, seed)
    if key not in _cache:
        xb = synthetic.activations(M, K, seed=seed)
        wb = synthetic.weights(N, K, seed=seed)
        xq, sx = orc.quantize_rows(xb, fmt, group=group, rotation=rotation)
        wq, sw = orc.quantize_rows(wb, fmt, group=group, rotation=rotation)
        _cache.clear()
        _cache[key] = (xq, sx, wq, sw)
    return _cache[key]


def gpu_gemm(dev, xq, sx, wq, sw, fmt, group=0, path=None, out_dtype=torch.bfloat16):
    from breeze_tts_cpp_amd import qlinear
    y = qlinear.gemm(dev_u8(xq, dev), dev_f32(sx, dev), dev_u8(wq, dev), dev_f32(sw, dev), fmt,
                     out_dtype=out_dtype, input_group=group, weight_group=group, path=path)
    torch.cuda.synchronize()
    return out_bits(y)


def check_i8(orc, y, xq, sx, wq, sw, out_type=BF16):
    acc = orc.gemm_i8_acc(xq, wq)
    ref = orc.epilogue_i8(acc, sx, sw, order=0, out_type=out_type)
    alt = orc.epilogue_i8(acc, sx, sw, order=1, out_type=out_type)
    assert np.array_equal(y, ref), f"{np.count_nonzero(y != ref)} mismatches of {y.size}"
    assert np.abs(y.astype(np.int32) - alt.astype(np.int32)).max() <= 1


PROJ = [(4096, 2048), (2048, 2048), (12288, 2048), (2048, 6144)]


@pytest.mark.parametrize("M", [1, 8, 16, 32, 64])
@pytest.mark.parametrize("N,K", PROJ)
def test_i8_decode_projections(dev, orc, M, N, K):
    print(f"i8 decode M={M} N={N} K={K}", flush=True)
    xq, sx, wq, sw = operands(orc, M, N, K, I8, seed=M + N)
    y = gpu_gemm(dev, xq, sx, wq, sw, I8)
    check_i8(orc, y, xq, sx, wq, sw)


def test_i8_config0(dev, orc):
    """M=16, N=K=2048, seed 0."""
    xq, sx, wq, sw = operands(orc, 16, 2048, 2048, I8, seed=0)
    y = gpu_gemm(dev, xq, sx, wq, sw, I8)
    check_i8(orc, y, xq, sx, wq, sw)


def _skinny_paths(K):
    """Every skinny variant: token tile, channel tile, grid K splits (eight
    waves per workgroup; with 6 blocks of K some wave ranges are empty)."""
    from breeze_tts_cpp_amd.qlinear import Path, KIND_SKINNY
    for tokens in (16, 32, 64):
        for channels in (16, 32, 48):
            for splits in (1, 2, 3):
                yield Path(KIND_SKINNY, tokens, channels, splits, 8)


@pytest.mark.parametrize("fmt", [I8, FP8])
def test_skinny_path_variants(dev, orc, fmt):
    """Every skinny variant (token tile, channel tile, in-workgroup and grid
    K splits) gives the same bits for INT8 and agrees within tolerance for FP8."""
    M, N, K = 40, 96, 1536
    xq, sx, wq, sw = operands(orc, M, N, K, fmt, seed=21)
    for p in _skinny_paths(K):
        print(f"skinny path {p}", flush=True)
        y = gpu_gemm(dev, xq, sx, wq, sw, fmt, path=p)
        if fmt == I8:
            check_i8(orc, y, xq, sx, wq, sw)
        else:
            ideal = orc.gemm_fp8_ideal(xq, sx, wq, sw)
            assert rel_l2(bits_to_f32(y), ideal) <= FP8_REL_L2


@pytest.mark.parametrize("M", [1, 32, 64])
@pytest.mark.parametrize("N,K", PROJ)
def test_fp8_decode_projections(dev, orc, M, N, K):
    print(f"fp8 decode M={M} N={N} K={K}", flush=True)
    xq, sx, wq, sw = operands(orc, M, N, K, FP8, seed=M + 3)
    y = gpu_gemm(dev, xq, sx, wq, sw, FP8)
    ideal = orc.gemm_fp8_ideal(xq, sx, wq, sw)
    err = rel_l2(bits_to_f32(y), ideal)
    print(f"  rel_l2={err:.3e}")
    assert err <= FP8_REL_L2
    # much tighter in practice: bf16 output rounding dominates
    assert err <= 4e-3


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("M", [1, 32, 64])
@pytest.mark.parametrize("N,K", PROJ)
def test_grouped_decode(dev, orc, fmt, M, N, K):
    """group_int8 / group_fp8 (BASELINE configs 3 and 4) at decode sizes on
    all four projections through the planned path. INT8: bit-exact against
    the oracle's grouped accumulation in the reference's order -- one chain
    r = fmaf(p_g, sx_g*sw_g, r) over every K group ascending, as the
    reference's unsplit grouped_gemm (quant_grouped.cu:112-146) -- which is
    also the partition the planner reports. FP8: rel-L2 <= 1e-2 of the fp64
    product."""
    from breeze_tts_cpp_amd import qlinear
    print(f"grouped decode fmt={fmt} M={M} N={N} K={K}", flush=True)
    xq, sx, wq, sw = operands(orc, M, N, K, fmt, group=128, rotation=128, seed=M + 5)
    p = qlinear.plan(M, N, K, fmt, 128, 128)
    y = gpu_gemm(dev, xq, sx, wq, sw, fmt, group=128, path=p)
    if fmt == I8:
        assert qlinear.grouped_partition(p, K, fmt) == (1, 1, K)
        ref, _ = orc.gemm_grouped(xq, sx, wq, sw, fmt, 128, 128, 1, 1, K)
        diff = np.abs(y.astype(np.int32) - ref.astype(np.int32))
        print(f"  max bf16 ulp vs the single-chain order: {int(diff.max())}")
        assert np.array_equal(y, ref), f"{np.count_nonzero(y != ref)} mismatches"
    else:
        ideal = orc.gemm_grouped_ideal(xq, sx, wq, sw, fmt, 128, 128)
        assert rel_l2(bits_to_f32(y), ideal) <= FP8_REL_L2


def test_grouped_path_variants(dev, orc):
    M, N, K = 24, 64, 1536
    xq, sx, wq, sw = operands(orc, M, N, K, I8, group=128, rotation=128, seed=31)
    from breeze_tts_cpp_amd import qlinear
    for p in _skinny_paths(K):
        y = gpu_gemm(dev, xq, sx, wq, sw, I8, group=128, path=p)
        splits, waves, span = qlinear.grouped_partition(p, K)
        ref, _ = orc.gemm_grouped(xq, sx, wq, sw, I8, 128, 128, splits, waves, span)
        assert np.array_equal(y, ref), p


@pytest.mark.parametrize("fmt", [I8, FP8])
def test_f16_output(dev, orc, fmt):
    M, N, K = 32, 256, 2048
    xq, sx, wq, sw = operands(orc, M, N, K, fmt, seed=41)
    y = gpu_gemm(dev, xq, sx, wq, sw, fmt, out_dtype=torch.float16)
    if fmt == I8:
        check_i8(orc, y, xq, sx, wq, sw, out_type=F16)
    else:
        ideal = orc.gemm_fp8_ideal(xq, sx, wq, sw)
        assert rel_l2(bits_to_f32(y, F16), ideal) <= FP8_REL_L2


@pytest.mark.parametrize("M", [16, 300])
@pytest.mark.parametrize("exp_x,exp_w", [(-110, -30), (95, 20)])
def test_i8_extreme_scales(dev, orc, M, exp_x, exp_w):
    """Scales that push the epilogue into fp32/bf16 subnormals (products down
    to 2^-150) or past the bf16 range (to inf): the output rounding keeps
    subnormals and overflows like the oracle, on the skinny and tiled paths."""
    N, K = 272, 512
    xq, sx, wq, sw = operands(orc, M, N, K, I8, seed=M + abs(exp_x))
    rng = np.random.default_rng(abs(exp_w) + M)
    sx = (np.ldexp(1.0, exp_x) * rng.uniform(0.5, 2.0, M)).astype(np.float32)
    sw = (np.ldexp(1.0, exp_w) * rng.uniform(0.5, 2.0, N)).astype(np.float32)
    y = gpu_gemm(dev, xq, sx, wq, sw, I8)
    ref = orc.epilogue_i8(orc.gemm_i8_acc(xq, wq), sx, sw, order=0, out_type=BF16)
    if exp_x < 0:
        assert np.count_nonzero((ref & 0x7f80) == 0) > 0  # subnormal outputs occur
    else:
        assert np.count_nonzero((ref & 0x7fff) == 0x7f80) > 0  # infinities occur
    check_i8(orc, y, xq, sx, wq, sw)


def test_ragged_k(dev, orc):
    """K a multiple of 16 but not of 64/256 (masked tail pieces)."""
    for K in (16, 80, 272, 2064):
        xq, sx, wq, sw = operands(orc, 9, 48, K, I8, seed=K)
        y = gpu_gemm(dev, xq, sx, wq, sw, I8)
        check_i8(orc, y, xq, sx, wq, sw)


def test_end_to_end_linear(dev, orc):
    """quantize -> GEMM -> bf16 through the library equals the CPU pipeline."""
    from breeze_tts_cpp_amd import qlinear
    M, N, K = 16, 2048, 2048
    xb = synthetic.activations(M, K, seed=0)
    wb = synthetic.weights(N, K, seed=0)
    for fmt, group, rot in ((I8, 0, 0), (I8, 128, 128)):
        wq, sw = orc.quantize_rows(wb, fmt, group=group, rotation=rot)
        x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev)
        p = qlinear.plan(M, N, K, fmt, group, group)
        y = qlinear.linear(x, dev_u8(wq, dev), dev_f32(sw, dev), fmt, group, rot, path=p)
        torch.cuda.synchronize()
        xq, sx = orc.quantize_rows(xb, fmt, group=group, rotation=rot)
        if group:
            splits, waves, span = qlinear.grouped_partition(p, K)
            ref, _ = orc.gemm_grouped(xq, sx, wq, sw, fmt, 128, 128, splits, waves, span)
        else:
            ref = orc.epilogue_i8(orc.gemm_i8_acc(xq, wq), sx, sw)
        assert np.array_equal(out_bits(y), ref)


# ---------------------------------------------------------------- prefill (tiled) GEMM
def _tiled_paths(grouped=False, fmt=I8):
    """Every instantiated macro tile (channels x tokens, waves) for the mode."""
    from breeze_tts_cpp_amd.qlinear import Path, KIND_TILED
    shapes = [(128, 128, 1), (256, 128, 8), (128, 128, 8), (128, 64, 4), (128, 64, 8)]
    if not grouped:
        shapes = [(256, 128, 1)] + shapes
        # 32x32-MFMA kernels: four waves of 128x128, two waves of 128x128
        shapes = [(256, 256, 8), (256, 256, 4), (256, 128, 2)] + shapes
    for channels, tokens, waves in shapes:
        yield Path(KIND_TILED, tokens, channels, 1, waves)


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("M,N,K", [(200, 144, 336), (300, 272, 1024), (130, 512, 2048),
                                   (150, 208, 2112)])
def test_tiled_variants_ragged(dev, orc, fmt, M, N, K):
    """Every macro-tile shape on ragged M/N edges and K not a multiple of 128
    (K above 2048 takes the FP8 128x128 tile's four-stage form)."""
    xq, sx, wq, sw = operands(orc, M, N, K, fmt, seed=M + N + K)
    ideal = None if fmt == I8 else orc.gemm_fp8_ideal(xq, sx, wq, sw)
    for p in _tiled_paths(fmt=fmt):
        print(f"tiled path {p} M={M} N={N} K={K}", flush=True)
        y = gpu_gemm(dev, xq, sx, wq, sw, fmt, path=p)
        if fmt == I8:
            check_i8(orc, y, xq, sx, wq, sw)
        else:
            assert rel_l2(bits_to_f32(y), ideal) <= FP8_REL_L2


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("M,N,K", [(2100, 4112, 320), (4096, 6144, 256)])
def test_tiled_many_tiles(dev, orc, fmt, M, N, K):
    """More tiles than CUs, ragged last tiles, every tile shape: sampled rows
    against the oracle (tile order and per-tile scale staging)."""
    xq, sx, wq, sw = operands(orc, M, N, K, fmt, seed=M + K)
    rng = np.random.default_rng(M)
    rows = np.unique(np.concatenate([[0, 127, 128, M - 1], rng.choice(M, 60, replace=False)]))
    for p in _tiled_paths(fmt=fmt):
        print(f"tiled path {p} M={M} N={N} K={K}", flush=True)
        y = gpu_gemm(dev, xq, sx, wq, sw, fmt, path=p)
        if fmt == I8:
            check_i8(orc, y[rows], xq[rows], sx[rows], wq, sw)
        else:
            ideal = orc.gemm_fp8_ideal(xq[rows], sx[rows], wq, sw)
            assert rel_l2(bits_to_f32(y[rows]), ideal) <= FP8_REL_L2


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("M", [1024, 4096])
@pytest.mark.parametrize("N,K", PROJ)
def test_prefill_projections(dev, orc, fmt, M, N, K):
    """Full prefill shapes (BASELINE configs 2 and 4) through the planned path.
    Rows are independent, so the oracle checks a sample of 48 token rows
    (including the first and last tile) against the full GPU output."""
    print(f"prefill fmt={fmt} M={M} N={N} K={K}", flush=True)
    xq, sx, wq, sw = operands(orc, M, N, K, fmt, seed=M + N)
    y = gpu_gemm(dev, xq, sx, wq, sw, fmt)
    rng = np.random.default_rng(M + N + K)
    rows = np.unique(np.concatenate([[0, 1, 255, 256, M - 1], rng.choice(M, 43, replace=False)]))
    xs, sxs = xq[rows], sx[rows]
    if fmt == I8:
        check_i8(orc, y[rows], xs, sxs, wq, sw)
    else:
        ideal = orc.gemm_fp8_ideal(xs, sxs, wq, sw)
        assert rel_l2(bits_to_f32(y[rows]), ideal) <= FP8_REL_L2


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("M,N,K", [(256, 256, 1024), (320, 400, 2048)] +
                         [(4096, N, K) for N, K in PROJ] + [(1024, 12288, 2048)])
def test_tiled_grouped(dev, orc, fmt, M, N, K):
    """group_int8 / group_fp8 on the tiled kernel: every tile shape on small
    ragged problems, and the BASELINE projections at M = 4096 (and gate_up at
    1024) through the planned path on sampled rows."""
    from breeze_tts_cpp_amd.qlinear import Path, KIND_TILED
    print(f"tiled grouped fmt={fmt} M={M} N={N} K={K}", flush=True)
    xq, sx, wq, sw = operands(orc, M, N, K, fmt, group=128, rotation=128, seed=M + 9)
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M).choice(M, 30)]))
    paths = list(_tiled_paths(grouped=True, fmt=fmt)) if M * N <= 320 * 400 else [None]
    for p in paths:
        y = gpu_gemm(dev, xq, sx, wq, sw, fmt, group=128, path=p)
        xs = xq[rows]
        sxs = np.ascontiguousarray(sx[:, rows])
        if fmt == I8:
            ref, _ = orc.gemm_grouped(xs, sxs, wq, sw, fmt, 128, 128)
            assert np.array_equal(y[rows], ref), p
        else:
            ideal = orc.gemm_grouped_ideal(xs, sxs, wq, sw, fmt, 128, 128)
            assert rel_l2(bits_to_f32(y[rows]), ideal) <= FP8_REL_L2


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("grouped", [False, True])
def test_staged_skinny_variants(dev, orc, fmt, grouped):
    """Weight slabs staged through LDS (staged 1), and activation tiles with
    them (staged 2, where both fit in LDS): same results as the oracle, on
    partial token tiles, ragged K and K ranges of 1-3 blocks."""
    from breeze_tts_cpp_amd.qlinear import Path, KIND_SKINNY
    g = 128 if grouped else 0
    for M, N, K in ((32, 96, 2048), (5, 48, 4096), (64, 64, 6144), (17, 32, 2064), (40, 48, 4000)):
        rot = g if K % 128 == 0 else 0
        xq, sx, wq, sw = operands(orc, M, N, K, fmt, group=g, rotation=rot, seed=N + K)
        nb = -(-(-(-K // 256)) // 8)
        tokens = 64 if M > 32 else -(-M // 16) * 16
        for channels, staged in ((16, 1), (32, 1), (48, 1), (16, 2), (32, 2), (48, 2)):
            lds = 8 * 256 * nb * (channels + (tokens if staged == 2 else 0))
            if nb > 3 or lds > 160 * 1024:
                continue
            p = Path(KIND_SKINNY, tokens, channels, 1, 8, staged)
            print(f"staged {p} M={M} N={N} K={K}", flush=True)
            y = gpu_gemm(dev, xq, sx, wq, sw, fmt, group=g, path=p)
            if grouped and fmt == I8:
                from breeze_tts_cpp_amd import qlinear
                ref, _ = orc.gemm_grouped(xq, sx, wq, sw, fmt, 128, 128,
                                          *qlinear.grouped_partition(p, K))
                assert np.array_equal(y, ref)
            elif grouped:
                ideal = orc.gemm_grouped_ideal(xq, sx, wq, sw, fmt, 128, 128)
                assert rel_l2(bits_to_f32(y), ideal) <= FP8_REL_L2
            elif fmt == I8:
                check_i8(orc, y, xq, sx, wq, sw)
            else:
                ideal = orc.gemm_fp8_ideal(xq, sx, wq, sw)
                assert rel_l2(bits_to_f32(y), ideal) <= FP8_REL_L2


@pytest.mark.parametrize("fmt", [I8, FP8])
def test_prefill_graph_replay(dev, orc, fmt):
    """The planned prefill GEMMs (256x256 and 256x128 double-buffered tiles)
    captured in a HIP graph: every one of several replays, with eager work
    and synchronizations between them, reproduces the eager output bit for
    bit."""
    from breeze_tts_cpp_amd import qlinear
    M = 1024
    stream = torch.cuda.Stream()
    for N, K in ((12288, 2048), (2048, 6144)):
        print(f"prefill graph replay fmt={fmt} M={M} N={N} K={K}", flush=True)
        xq, sx, wq, sw = operands(orc, M, N, K, fmt, seed=N + 3)
        args = (dev_u8(xq, dev), dev_f32(sx, dev), dev_u8(wq, dev), dev_f32(sw, dev), fmt)
        ref = qlinear.gemm(*args)
        y = torch.empty_like(ref)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            qlinear.gemm(*args, out=y, stream=stream)
        for r in range(3):
            y.fill_(0)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"replay {r}"
            qlinear.gemm(*args)  # eager work between replays
        del g
