"""K groups of 32 and 64 in the quantized GEMM, as the reference's
grouped_gemm dispatch accepts them (quant_grouped.cu:185-202): partials per
the smaller of the two group sizes, each scaled by its own activation and
weight scales (a 32-column partial of a 128-column activation group takes
that group's scale) and fma-accumulated in ascending K order
(quant_grouped.cu:85-146). INT8 bit-exact against the oracle's grouped
GEMM with the planned wave split; FP8 within rel-L2 1e-2 of the exact
product. Up to 64 rows run on the skinny (decode) kernel; more rows on the
tiled kernel's small-group variant (both eight-wave tiles)."""
import numpy as np
import pytest
import torch

from breeze_tts_cpp_amd import synthetic

BF16, F32, I32, FP8, I8, F16 = 0, 1, 2, 3, 4, 5
pytestmark = pytest.mark.gpu


def bits(y):
    return y.cpu().view(torch.int16).numpy().view(np.uint16)


def quantize(orc, b, fmt, group):
    return orc.quantize_rows(b, fmt, group=group) if group else orc.quantize_rows(b, fmt)


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("ig,wg", [(32, 32), (64, 64), (128, 32), (32, 128), (64, 128),
                                   (128, 64), (0, 64), (32, 0)])
@pytest.mark.parametrize("M,N,K", [(8, 256, 2048), (32, 4096, 2048), (100, 272, 1536),
                                   (3, 48, 4000), (200, 528, 1008), (300, 256, 2048)])
def test_small_groups(dev, orc, fmt, ig, wg, M, N, K):
    from breeze_tts_cpp_amd import qlinear
    print(f"small groups fmt={fmt} ig={ig} wg={wg} M={M} N={N} K={K}", flush=True)
    xq, sx = quantize(orc, synthetic.activations(M, K, seed=M + ig), fmt, ig)
    wq, sw = quantize(orc, synthetic.weights(N, K, seed=N + wg), fmt, wg)
    planned = qlinear.plan(M, N, K, fmt, ig, wg)
    assert planned.kind == (qlinear.KIND_SKINNY if M <= 64 else qlinear.KIND_TILED)
    assert planned.splits == 1
    paths = [planned]
    if M > 64:  # the eight-wave tiles of the small-group variant
        paths = [qlinear.Path(qlinear.KIND_TILED, 128, 128, 1, 8, 0)]
        if fmt == I8:
            paths.append(qlinear.Path(qlinear.KIND_TILED, 128, 256, 1, 8, 0))
    for p in paths:
        y = qlinear.gemm(torch.from_numpy(xq).to(dev), torch.from_numpy(sx).to(dev),
                         torch.from_numpy(wq).to(dev), torch.from_numpy(sw).to(dev), fmt,
                         input_group=ig, weight_group=wg, path=p)
        torch.cuda.synchronize()
        got = bits(y)
        if fmt == I8:
            splits, waves, span = qlinear.grouped_partition(p, K, fmt, ig, wg)
            ref, _ = orc.gemm_grouped(xq, sx, wq, sw, fmt, ig, wg, splits, waves, span)
            assert np.array_equal(got, ref), f"{p}: {np.count_nonzero(got != ref)} mismatches"
        else:
            ideal = orc.gemm_grouped_ideal(xq, sx, wq, sw, fmt, ig, wg)
            f = synthetic.bf16_bits_to_f32(got).astype(np.float64)
            assert np.linalg.norm(f - ideal) / np.linalg.norm(ideal) <= 1e-2, p


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("ig,wg", [(32, 32), (64, 128)])
def test_small_groups_prefill_projection(dev, orc, fmt, ig, wg):
    """A BASELINE-sized prefill projection (qkv 4096x2048 at M = 1024) with
    32/64 groups through the planned tiled path, checked on sampled rows."""
    from breeze_tts_cpp_amd import qlinear
    M, N, K = 1024, 4096, 2048
    print(f"small groups prefill fmt={fmt} ig={ig} wg={wg}", flush=True)
    xq, sx = quantize(orc, synthetic.activations(M, K, seed=5), fmt, ig)
    wq, sw = quantize(orc, synthetic.weights(N, K, seed=6), fmt, wg)
    p = qlinear.plan(M, N, K, fmt, ig, wg)
    assert p.kind == qlinear.KIND_TILED
    y = qlinear.gemm(torch.from_numpy(xq).to(dev), torch.from_numpy(sx).to(dev),
                     torch.from_numpy(wq).to(dev), torch.from_numpy(sw).to(dev), fmt,
                     input_group=ig, weight_group=wg, path=p)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(3).choice(M, 24)]))
    got = bits(y)[rows]
    xs = xq[rows]
    sxs = np.ascontiguousarray(sx[:, rows]) if ig else sx[rows]
    if fmt == I8:
        ref, _ = orc.gemm_grouped(xs, sxs, wq, sw, fmt, ig, wg)
        assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} mismatches"
    else:
        ideal = orc.gemm_grouped_ideal(xs, sxs, wq, sw, fmt, ig, wg)
        f = synthetic.bf16_bits_to_f32(got).astype(np.float64)
        assert np.linalg.norm(f - ideal) / np.linalg.norm(ideal) <= 1e-2


def test_small_groups_unsupported_forms(dev, orc):
    """Four-wave tiled paths decline 32/64 groups (split-K skinny paths take
    them, test_small_groups_split_and_packed)."""
    from breeze_tts_cpp_amd import qlinear
    M, N, K = 8, 64, 1024
    xq, sx = orc.quantize_rows(synthetic.activations(M, K, seed=1), I8, group=32)
    wq, sw = orc.quantize_rows(synthetic.weights(N, K, seed=1), I8, group=32)
    args = [torch.from_numpy(a).to(dev) for a in (xq, sx, wq, sw)]
    for path in (qlinear.Path(2, 128, 128, 1, 1, 0),):
        with pytest.raises(qlinear.QLinearError):
            qlinear.gemm(*args, I8, input_group=32, weight_group=32, path=path,
                         workspace=torch.empty(1 << 20, dtype=torch.uint8, device=dev))


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("group", [0, 128, 64, 32])
@pytest.mark.parametrize("M,K", [(3, 3968), (8, 4000), (20, 2000), (33, 1808), (40, 6000)])
def test_staged_ragged_k(dev, orc, fmt, group, M, K):
    """Staged (LDS slab) decode paths with K not a multiple of 256: the last
    wave's range ends inside a 256-K block, so some of its activation pieces
    lie past K. Regression test for a slab wait that counted the activation
    loads issued behind the slab DMA: a wave that skipped out-of-range loads
    came up short and read weight rows 14-15 of each tile before the last DMA
    instruction landed. The kernel now waits for every load before it reads
    the slab."""
    from breeze_tts_cpp_amd import qlinear
    N = 48
    print(f"staged ragged fmt={fmt} group={group} M={M} K={K}", flush=True)
    xq, sx = quantize(orc, synthetic.activations(M, K, seed=K), fmt, group)
    wq, sw = quantize(orc, synthetic.weights(N, K, seed=K + 1), fmt, group)
    p = qlinear.plan(M, N, K, fmt, group, group)
    y = qlinear.gemm(torch.from_numpy(xq).to(dev), torch.from_numpy(sx).to(dev),
                     torch.from_numpy(wq).to(dev), torch.from_numpy(sw).to(dev), fmt,
                     input_group=group, weight_group=group, path=p)
    torch.cuda.synchronize()
    got = bits(y)
    if fmt == I8 and group:
        splits, waves, span = qlinear.grouped_partition(p, K, fmt, group, group)
        ref, _ = orc.gemm_grouped(xq, sx, wq, sw, fmt, group, group, splits, waves, span)
        assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} mismatches, {p}"
    elif fmt == I8:
        ref = orc.epilogue_i8(orc.gemm_i8_acc(xq, wq), sx, sw)
        assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} mismatches, {p}"
    else:
        ideal = (orc.gemm_grouped_ideal(xq, sx, wq, sw, fmt, group, group) if group
                 else orc.gemm_fp8_ideal(xq, sx, wq, sw))
        f = synthetic.bf16_bits_to_f32(got).astype(np.float64)
        assert np.linalg.norm(f - ideal) / np.linalg.norm(ideal) <= 1e-2


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("ig,wg", [(32, 32), (64, 128), (0, 64), (32, 0)])
@pytest.mark.parametrize("M,N,K", [(8, 256, 2048), (32, 512, 6144), (5, 48, 1536)])
def test_small_groups_split_and_packed(dev, orc, fmt, ig, wg, M, N, K):
    """K groups of 32 / 64 on the decode kernel's grid split-K (2 and 3
    splits: wave ranges of each split summed in order, then fp32 partials
    carrying their outer scales summed in split order, as the reference's
    split grouped GEMM and quant_split_reduce_scale do, quant_grouped.cu:
    171-239, quant_reduce.cuh:9-19) and on packed weights: INT8 bit-exact
    against the oracle over the same partition, FP8 within rel-L2 1e-2."""
    from breeze_tts_cpp_amd import qlinear
    print(f"small groups split/packed fmt={fmt} ig={ig} wg={wg} M={M} N={N} K={K}", flush=True)
    xq, sx = quantize(orc, synthetic.activations(M, K, seed=M + ig + 3), fmt, ig)
    wq, sw = quantize(orc, synthetic.weights(N, K, seed=N + wg + 3), fmt, wg)
    xd, sxd = torch.from_numpy(xq).to(dev), torch.from_numpy(sx).to(dev)
    wd, swd = torch.from_numpy(wq).to(dev), torch.from_numpy(sw).to(dev)
    runs = []
    for splits in (2, 3):
        p = qlinear.Path(qlinear.KIND_SKINNY, 16 * -(-min(M, 32) // 16), 16, splits, 8, 0)
        runs.append((p, False))
    runs.append((qlinear.plan(M, N, K, fmt, ig, wg), True))
    for p, packed in runs:
        if packed:
            w_in = qlinear.pack_weights(wd)
            path = qlinear.Path(p.kind, p.tokens, p.channels, p.splits, p.waves, 0)
        else:
            w_in, path = wd, p
        print(f"  path {path} packed={packed}", flush=True)
        y = qlinear.gemm(xd, sxd, w_in, swd, fmt, input_group=ig, weight_group=wg, path=path)
        torch.cuda.synchronize()
        got = bits(y)
        if fmt == I8:
            part = qlinear.grouped_partition(path, K, fmt, ig, wg, packed=packed)
            ref, _ = orc.gemm_grouped(xq, sx, wq, sw, fmt, ig, wg, *part)
            assert np.array_equal(got, ref), f"{path}: {np.count_nonzero(got != ref)} mismatches"
        else:
            ideal = orc.gemm_grouped_ideal(xq, sx, wq, sw, fmt, ig, wg)
            f = synthetic.bf16_bits_to_f32(got).astype(np.float64)
            assert np.linalg.norm(f - ideal) / np.linalg.norm(ideal) <= 1e-2, path


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("ig,wg", [(32, 32), (64, 64), (128, 32)])
def test_small_groups_packed_prefill(dev, orc, fmt, ig, wg):
    """The prefill kernel's small-group tiles on packed weights: identical to
    the row-major weights (both sum all of K in one range)."""
    from breeze_tts_cpp_amd import qlinear
    M, N, K = 300, 256, 2048
    print(f"small groups packed prefill fmt={fmt} ig={ig} wg={wg}", flush=True)
    xq, sx = quantize(orc, synthetic.activations(M, K, seed=ig + wg), fmt, ig)
    wq, sw = quantize(orc, synthetic.weights(N, K, seed=ig * wg), fmt, wg)
    xd, sxd = torch.from_numpy(xq).to(dev), torch.from_numpy(sx).to(dev)
    wd, swd = torch.from_numpy(wq).to(dev), torch.from_numpy(sw).to(dev)
    packed = qlinear.pack_weights(wd)
    paths = [qlinear.Path(qlinear.KIND_TILED, 128, 128, 1, 8, 0)]
    if fmt == I8:
        paths.append(qlinear.Path(qlinear.KIND_TILED, 128, 256, 1, 8, 0))
    for p in paths:
        y_row = qlinear.gemm(xd, sxd, wd, swd, fmt, input_group=ig, weight_group=wg, path=p)
        y_pk = qlinear.gemm(xd, sxd, packed, swd, fmt, input_group=ig, weight_group=wg, path=p)
        torch.cuda.synchronize()
        assert np.array_equal(bits(y_pk), bits(y_row)), p
