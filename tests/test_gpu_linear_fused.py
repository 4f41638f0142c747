"""qlin_linear's one-launch decode form: for per-token INT8 or FP8 scales on
a decode path with 16-token tiles, per-wave weight slabs and one 256-column
block of K per wave (K <= 2048), the GEMM quantizes its own token rows (the
arithmetic of the per-token quantizer, reference row_quantize.cu:24-87)
instead of a separate quantizer launch. Checked against the two-launch form
on the same inputs (qlin_row_quantize + qlin_gemm with the same path):
output bits identical, and the scratch activation (codes and scales) equal
to the oracle's quantizer; paths outside the form take the two launches and
are checked the same way."""
import numpy as np
import pytest
import torch

from breeze_tts_cpp_amd import synthetic

BF16, F32, I32, FP8, I8, F16 = 0, 1, 2, 3, 4, 5
pytestmark = pytest.mark.gpu


def bits(y):
    return y.cpu().view(torch.int16).numpy().view(np.uint16)


def dev16(xb, dtype, dev):
    t = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16)
    return (t if dtype == torch.bfloat16 else t.float().to(dtype)).to(dev)


def lds_bytes(path, K, fused=False):
    """LDS of a staged skinny launch: weight slabs, (staged 2) activation
    tiles (16-bit rows when fused), (fused) the absmax / scale exchange."""
    nb = -(-(-(-K // 256)) // 8)
    act = path.tokens * (2 if fused else 1) if path.staged == 2 else 0
    return 8 * 256 * nb * (path.channels + act) + (9 * path.tokens * 4 if fused else 0)


def fused_eligible(path, M, N, K, fmt=I8):
    """The library's rule for the fused form: per-token scales on a
    planned skinny path with per-wave slabs, eight waves, no split, 16-token
    tiles, one 256-column block of K per wave (the activation tile in LDS for
    staged 2), at most 256 workgroups, within LDS."""
    nb = -(-(-(-K // 256)) // 8)
    if not (path.kind == 1 and path.splits == 1 and path.waves == 8
            and path.staged in (1, 2) and path.tokens == 16 and path.channels in (16, 32, 48)
            and nb == 1):
        return False
    if -(-N // path.channels) * -(-M // 16) > 256:
        return False
    lds = 8 * 256 * path.channels + (8 * 16 * 2 * 256 if path.staged == 2 else 0) + 9 * 16 * 4
    return lds <= 160 * 1024


def run_pair(dev, orc, xb, fmt, N, K, path=None, src=torch.bfloat16, out=torch.bfloat16, ld=None,
             oracle=True):
    from breeze_tts_cpp_amd import qlinear
    M = xb.shape[0]
    wq, sw = orc.quantize_rows(synthetic.weights(N, K, seed=N + K), fmt)
    wq_d, sw_d = torch.from_numpy(wq).to(dev), torch.from_numpy(sw).to(dev)
    x = dev16(xb, src, dev)
    if ld is not None:
        wide = torch.zeros((M, ld), dtype=src, device=dev)
        wide[:, :K] = x
        x = wide[:, :K]
    xq_f = torch.full((M, K), 0x5a, dtype=torch.uint8, device=dev)
    sx_f = torch.full((M,), -1.0, dtype=torch.float32, device=dev)
    y_f = qlinear.linear(x, wq_d, sw_d, fmt, out_dtype=out, path=path, scratch=(xq_f, sx_f))
    xq_s, sx_s = qlinear.row_quantize(x, fmt)
    y_s = qlinear.gemm(xq_s, sx_s, wq_d, sw_d, fmt, out_dtype=out, path=path)
    torch.cuda.synchronize()
    assert np.array_equal(xq_f.cpu().numpy(), xq_s.cpu().numpy()), "scratch codes differ"
    assert np.array_equal(sx_f.cpu().numpy(), sx_s.cpu().numpy()), "scratch scales differ"
    assert np.array_equal(bits(y_f), bits(y_s)), \
        f"{np.count_nonzero(bits(y_f) != bits(y_s))} outputs differ from the two-launch form"
    if oracle and src == torch.bfloat16 and ld is None:
        xq, sx = orc.quantize_rows(xb, fmt)
        assert np.array_equal(xq_f.cpu().numpy(), xq) and np.array_equal(sx_f.cpu().numpy(), sx)
        if fmt == I8 and out == torch.bfloat16:
            assert np.array_equal(bits(y_f), orc.epilogue_i8(orc.gemm_i8_acc(xq, wq), sx, sw))


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("M,N,K", [(1, 4096, 2048), (8, 2048, 2048), (16, 2048, 2048),
                                   (17, 4096, 2048), (32, 4096, 2048), (32, 12288, 2048),
                                   (5, 48, 4096), (32, 2048, 4096), (32, 2048, 6144),
                                   (16, 12288, 2048), (8, 2048, 6144), (64, 12288, 2048)])
def test_fused_linear_planned(dev, orc, fmt, M, N, K):
    from breeze_tts_cpp_amd import qlinear
    path = qlinear.plan(M, N, K, fmt)
    print(f"fused linear fmt={fmt} M={M} N={N} K={K} path={path}", flush=True)
    run_pair(dev, orc, synthetic.activations(M, K, seed=M + N), fmt, N, K)


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("staged", [1, 2])
@pytest.mark.parametrize("tokens,channels,K", [(16, 16, 2048), (16, 32, 2048), (16, 48, 2048),
                                               (16, 32, 4096), (16, 48, 4096), (16, 16, 6144),
                                               (16, 48, 6144), (16, 32, 5120), (32, 16, 2048),
                                               (32, 32, 2048), (32, 48, 2048), (16, 32, 1024),
                                               (32, 32, 4096), (64, 16, 2048)])
def test_fused_linear_tiles(dev, orc, fmt, tokens, channels, K, staged):
    """Every fused channel tile (K 2048 and the short wave ranges of K 1024),
    partial token and channel tiles, weight slabs with and without the
    activation tiles in LDS; the paths the fused form does not cover (wider
    token tiles, several blocks per wave, FP8) take the two-launch form,
    checked the same way."""
    from breeze_tts_cpp_amd import qlinear
    M, N = 29, 16 * 37
    path = qlinear.Path(1, tokens, channels, 1, 8, staged)
    if lds_bytes(path, K) > 160 * 1024:
        pytest.skip("no variant: the staged tiles exceed LDS")
    print(f"fused tile fmt={fmt} {tokens}x{channels} K={K} staged={staged} "
          f"fused={fused_eligible(path, M, N, K, fmt)}", flush=True)
    run_pair(dev, orc, synthetic.activations(M, K, seed=tokens * channels + K), fmt, N, K, path=path)


@pytest.mark.parametrize("fmt", [I8, FP8])
def test_fused_linear_f16_strided_special_rows(dev, orc, fmt):
    """f16 source and output, row stride > K, a zero row (scale 1), a row
    with one huge value and a row of tiny values."""
    M, N, K = 24, 2048, 2048
    xb = synthetic.activations(M, K, seed=9)
    xb[3] = 0
    xb[7, 100] = synthetic.f32_to_bf16_bits(np.float32(3.0e4)).item()
    xb[11] = synthetic.f32_to_bf16_bits(np.full(K, 1e-3, np.float32))
    # absmax 127 / 448: unit INT8 / FP8 scale, so the codes round exact
    # half-integers (ties to even) and every representable magnitude.
    ties = np.resize(np.arange(-127.0, 127.5, 0.5, dtype=np.float32), K)
    ties[0] = 127.0
    xb[13] = synthetic.f32_to_bf16_bits(ties)
    xb[14] = synthetic.f32_to_bf16_bits(np.resize(np.linspace(-448, 448, 97, dtype=np.float32), K))
    print(f"fused f16 strided fmt={fmt}", flush=True)
    run_pair(dev, orc, xb, fmt, N, K, src=torch.float16, out=torch.float16, ld=K + 64)
    run_pair(dev, orc, xb, fmt, N, K, src=torch.bfloat16, out=torch.bfloat16, ld=K + 8)


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("src", [torch.bfloat16, torch.float16])
def test_fused_linear_nan_inf_rows(dev, orc, src, fmt):
    """Rows with a NaN among finite values, +Inf, -Inf and all NaN: the fused
    form's absmax (a packed 16-bit max of the sign-cleared bits, redone with
    fmaxf where a lane holds a NaN pattern) gives the same scratch codes,
    scales and output bits as the standalone quantizer + GEMM. (The
    reference's NaN handling is not pinned by any fixture, so the oracle is
    not consulted for these rows.)"""
    M, N, K = 16, 2048, 2048
    xb = synthetic.activations(M, K, seed=21)
    nan, inf = np.uint16(0x7fc0), np.uint16(0x7f80)
    xb[2, 5] = nan
    xb[4, 9] = inf
    xb[6] = nan
    xb[8, 2000] = inf | np.uint16(0x8000)
    xb[10, 1] = np.uint16(0x7f81)  # a signalling-NaN pattern
    print(f"fused nan/inf rows src={src} fmt={fmt}", flush=True)
    run_pair(dev, orc, xb, fmt, N, K, src=src, out=src, oracle=False)


def test_fused_linear_repeated_calls(dev, orc):
    """Two calls in a row into one scratch, the second with fewer rows: the
    second call's scratch rows and output are its own."""
    from breeze_tts_cpp_amd import qlinear
    N, K = 4096, 2048
    wq, sw = orc.quantize_rows(synthetic.weights(N, K, seed=3), I8)
    wq_d, sw_d = torch.from_numpy(wq).to(dev), torch.from_numpy(sw).to(dev)
    xq = torch.empty((32, K), dtype=torch.uint8, device=dev)
    sx = torch.empty((32,), dtype=torch.float32, device=dev)
    for M, seed in ((32, 1), (9, 2)):
        xb = synthetic.activations(M, K, seed=seed)
        y = qlinear.linear(dev16(xb, torch.bfloat16, dev), wq_d, sw_d, I8,
                           scratch=(xq[:M], sx[:M]))
        torch.cuda.synchronize()
        xr, sr = orc.quantize_rows(xb, I8)
        assert np.array_equal(xq[:M].cpu().numpy(), xr) and np.array_equal(sx[:M].cpu().numpy(), sr)
        assert np.array_equal(bits(y), orc.epilogue_i8(orc.gemm_i8_acc(xr, wq), sr, sw))


def run_group_pair(dev, orc, xb, fmt, N, K, rotation, weight_group=128, path=None,
                   src=torch.bfloat16, oracle=True):
    """qlin_linear with activation groups of 128 (optionally H128-rotated)
    against quantizer + GEMM on the same path: scratch codes, [K/128, M]
    scales and output bits identical; the scratch also equals the oracle's
    group quantizer for bf16 sources."""
    from breeze_tts_cpp_amd import qlinear
    M = xb.shape[0]
    wq, sw = orc.quantize_rows(synthetic.weights(N, K, seed=N + K + 7), fmt, group=weight_group,
                               rotation=rotation)
    wq_d, sw_d = torch.from_numpy(wq).to(dev), torch.from_numpy(sw).to(dev)
    x = dev16(xb, src, dev)
    groups = -(-K // 128)
    xq_f = torch.full((M, K), 0x5a, dtype=torch.uint8, device=dev)
    sx_f = torch.full((groups, M), -1.0, dtype=torch.float32, device=dev)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    qlinear.load().qlin_linear(  # activation groups 128, weight groups weight_group
        __import__("ctypes").byref((path or qlinear.Path()).to_c()), x.data_ptr(), x.stride(0),
        {torch.bfloat16: BF16, torch.float16: F16}[src], xq_f.data_ptr(), sx_f.data_ptr(),
        wq_d.data_ptr(), sw_d.data_ptr(), out.data_ptr(), M, N, K, fmt, BF16, 128, weight_group,
        rotation, None, 0, None)
    xq_s, sx_s = qlinear.row_quantize(x, fmt, group=128, rotation=rotation)
    y_s = qlinear.gemm(xq_s, sx_s, wq_d, sw_d, fmt, input_group=128, weight_group=weight_group,
                       path=path)
    torch.cuda.synchronize()
    assert np.array_equal(xq_f.cpu().numpy(), xq_s.cpu().numpy()), "scratch codes differ"
    assert np.array_equal(sx_f.cpu().numpy().reshape(-1), sx_s.cpu().numpy().reshape(-1)), \
        "scratch scales differ"
    assert np.array_equal(bits(out), bits(y_s)), \
        f"{np.count_nonzero(bits(out) != bits(y_s))} outputs differ from the two-launch form"
    if oracle and src == torch.bfloat16:
        xr, sr = orc.quantize_rows(xb, fmt, group=128, rotation=rotation)
        assert np.array_equal(xq_f.cpu().numpy(), xr)
        assert np.array_equal(sx_f.cpu().numpy().reshape(-1), np.asarray(sr).reshape(-1))


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("rotation", [0, 128])
@pytest.mark.parametrize("M,N,K", [(1, 4096, 2048), (32, 4096, 2048), (32, 2048, 2048),
                                   (17, 2048, 1024), (32, 12288, 2048), (32, 2048, 6144)])
def test_fused_group_linear_planned(dev, orc, fmt, rotation, M, N, K):
    """K-group decode linears on the planned path: one launch for unrotated
    groups where the path has 16-token tiles over one 256-column block per
    wave (qkv, o_proj); two launches otherwise (rotated groups, as group_int8
    / group_fp8 use, and gate_up, down); both checked."""
    print(f"fused group linear fmt={fmt} rot={rotation} M={M} N={N} K={K}", flush=True)
    run_group_pair(dev, orc, synthetic.activations(M, K, seed=M + N + rotation), fmt, N, K, rotation)


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("staged", [1, 2])
@pytest.mark.parametrize("channels", [16, 32, 48])
def test_fused_group_linear_tiles(dev, orc, fmt, staged, channels):
    """Every fused channel tile, activation tile in LDS or in registers,
    partial token and channel tiles; weights with per-channel scales as well
    as 128-groups."""
    from breeze_tts_cpp_amd import qlinear
    M, N, K = 29, 16 * 37, 2048
    path = qlinear.Path(1, 16, channels, 1, 8, staged)
    print(f"fused group tile fmt={fmt} 16x{channels} staged={staged}", flush=True)
    xb = synthetic.activations(M, K, seed=channels + staged)
    run_group_pair(dev, orc, xb, fmt, N, K, 0, path=path)
    run_group_pair(dev, orc, xb, fmt, N, K, 0, weight_group=0, path=path)


@pytest.mark.parametrize("src", [torch.bfloat16, torch.float16])
def test_fused_group_linear_special_rows(dev, orc, src):
    """Zero, NaN, Inf and huge values and an all-zero group through the
    grouped one-launch form against the two-launch form (the oracle is not
    consulted for these rows)."""
    M, N, K = 16, 2048, 2048
    xb = synthetic.activations(M, K, seed=33)
    xb[1] = 0
    xb[2, 5] = np.uint16(0x7fc0)
    xb[3, 300] = np.uint16(0x7f80)
    xb[4, 1000] = synthetic.f32_to_bf16_bits(np.float32(3.0e4)).item()
    xb[5, 128:256] = 0
    for fmt in (I8, FP8):
        for rotation in (0, 128):
            print(f"fused group special rows src={src} fmt={fmt} rot={rotation}", flush=True)
            run_group_pair(dev, orc, xb, fmt, N, K, rotation, src=src, oracle=False)


@pytest.mark.parametrize("case", ["y_aliases_x", "sx_in_x_row_tail", "xq_in_x_allocation"])
def test_fused_linear_aliasing_falls_back(dev, orc, case):
    """A fused-eligible decode linear (M = 16, N = K = 2048) whose output or
    scratch overlaps x's span (rows * ld elements) takes the two-launch form,
    which reads all of x before anything is written: y in place over x; the
    scales in the unused tail of x's first strided row (ld = 2K); the codes
    starting in the unused tail of x's last strided row and running on into
    the rest of x's allocation. Output bits equal quantizer + GEMM on a copy
    of x."""
    from breeze_tts_cpp_amd import qlinear
    M, N, K = 16, 2048, 2048
    assert fused_eligible(qlinear.plan(M, N, K, I8), M, N, K)
    print(f"aliasing {case}", flush=True)
    xb = synthetic.activations(M, K, seed=77)
    wq, sw = orc.quantize_rows(synthetic.weights(N, K, seed=78), I8)
    wq_d, sw_d = torch.from_numpy(wq).to(dev), torch.from_numpy(sw).to(dev)
    x_ref = dev16(xb, torch.bfloat16, dev)
    xq_ref, sx_ref = qlinear.row_quantize(x_ref, I8)
    y_ref = qlinear.gemm(xq_ref, sx_ref, wq_d, sw_d, I8)
    xq = torch.empty((M, K), dtype=torch.uint8, device=dev)
    sx = torch.empty((M,), dtype=torch.float32, device=dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    if case == "y_aliases_x":
        buf = x_ref.clone()
        ld, x_ptr, xq_ptr, sx_ptr, y_ptr = K, buf.data_ptr(), xq.data_ptr(), sx.data_ptr(), buf.data_ptr()
    else:
        # rows of 2K bf16 (ld = 2K): columns [K, 2K) of each row are unused;
        # 4 extra rows hold the rest of a codes block that starts in the
        # last row's tail
        buf = torch.zeros((M + 4, 2 * K), dtype=torch.bfloat16, device=dev)
        buf[:M, :K] = x_ref
        ld, x_ptr, y_ptr = 2 * K, buf.data_ptr(), y.data_ptr()
        row_bytes = 2 * K * 2
        if case == "sx_in_x_row_tail":
            xq_ptr, sx_ptr = xq.data_ptr(), buf.data_ptr() + K * 2
        else:
            xq_ptr, sx_ptr = buf.data_ptr() + (M - 1) * row_bytes + K * 2, sx.data_ptr()
            assert (M - 1) * row_bytes + K * 2 + M * K <= buf.numel() * 2
    L = qlinear.load()
    rc = L.qlin_linear(None, x_ptr, ld, BF16, xq_ptr, sx_ptr, wq_d.data_ptr(), sw_d.data_ptr(),
                       y_ptr, M, N, K, I8, BF16, 0, 0, 0, None, 0, None)
    assert rc == 0, L.qlin_last_error()
    torch.cuda.synchronize()
    assert np.array_equal(bits(buf if case == "y_aliases_x" else y), bits(y_ref))
