"""Pins the CPU oracle (oracle/qlinear_oracle.c) before it is trusted as the
parity checker. The reference ships no tests, golden vectors or fixtures for
this path, so each oracle function is pinned here by an independent route:
closed forms evaluated with numpy/torch, exhaustive enumeration, invariants
(orthogonality, layout equivalences) and brute force."""
import math

import numpy as np
import pytest
import torch

from breeze_tts_cpp_amd import synthetic

BF16, F32, I32, FP8, I8, F16 = 0, 1, 2, 3, 4, 5


# ---------------------------------------------------------------- 16-bit floats
def test_bf16_rounding_matches_torch(orc):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(4000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 1.0, 65504.0, 3.0e38, 1e-40], np.float32)])
    # ties: values exactly halfway between bf16 neighbours
    base = rng.integers(0, 0x7f00, 500).astype(np.uint32) << 16
    ties = (base | 0x8000).view(np.float32)
    x = np.concatenate([x, ties, -ties])
    ours = orc.f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


def test_f16_codec_matches_numpy(orc):
    L = orc.lib()
    codes = np.arange(65536, dtype=np.uint32)
    dec = np.array([L.orc_f16_to_f32(int(c)) for c in codes], np.float32)
    ref = codes.astype(np.uint16).view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(dec[finite], ref[finite])
    assert np.all(np.isnan(dec[np.isnan(ref)]))
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(3000).astype(np.float32) * 1000,
                        rng.standard_normal(1000).astype(np.float32) * 1e-5,
                        np.array([65504, 65519.99, 65520, 1e9, 6.1e-5, 5.96e-8, 2.98e-8],
                                 np.float32)])
    enc = np.array([L.orc_f32_to_f16(float(v)) for v in x], np.uint16)
    with np.errstate(over="ignore"):  # 65520 and 1e9 round to inf on purpose
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(enc, want)


# ---------------------------------------------------------------- FP8 e4m3fn
def test_fp8_decode_exhaustive(orc):
    table = orc.fp8_decode_table()
    codes = torch.arange(256, dtype=torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert nan.sum() == 2 and nan[0x7F] and nan[0xFF]
    assert np.array_equal(table[~nan], ref[~nan])
    assert np.all(np.isnan(table[nan]))
    # closed form for a few codes: bias 7, 3 mantissa bits
    assert table[0x7E] == 448.0 and table[0x08] == 2.0 ** -6 and table[0x01] == 2.0 ** -9
    assert table[0x38] == 1.0 and table[0xB8] == -1.0


def test_fp8_encode_round_trip_and_ties(orc):
    table = orc.fp8_decode_table()
    finite = [c for c in range(256) if not math.isnan(table[c])]
    enc = orc.fp8_encode(table[finite])
    # -0 encodes to 0x80, every other finite code round-trips
    assert np.array_equal(enc, np.array(finite, np.uint8))
    # midpoints between adjacent positive codes go to the even code
    pos = sorted(c for c in finite if c < 0x80)
    for a, b in zip(pos[:-1], pos[1:]):
        mid = (np.float64(table[a]) + np.float64(table[b])) / 2
        got = orc.fp8_encode(np.array([mid], np.float32))[0]
        assert got == (a if a % 2 == 0 else b), (a, b, mid)


def test_fp8_encode_matches_torch_and_saturates(orc):
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 100,
                        rng.uniform(-463.9, 463.9, 20000).astype(np.float32),
                        rng.standard_normal(5000).astype(np.float32) * 1e-3,
                        np.array([448, 449, 463.99, -463.99, 0.0, -0.0], np.float32)])
    ours = orc.fp8_encode(x)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)
    # satfinite: at and beyond the last rounding boundary the code is +-448
    big = np.array([464, 480, 1e6, np.inf, -464, -1e30, -np.inf], np.float32)
    assert list(orc.fp8_encode(big)) == [0x7E] * 4 + [0xFE] * 3


# ---------------------------------------------------------------- INT8 rounding and scale
def test_i8_round_closed_form(orc):
    rng = np.random.default_rng(4)
    x = np.concatenate([rng.uniform(-200, 200, 20000).astype(np.float32),
                        np.arange(-130, 131, dtype=np.float32) + 0.5,
                        np.array([126.5, 127.49, -127.5, 0.5, -0.5, 1.5, 2.5], np.float32)])
    ref = np.rint(np.clip(x, -127, 127)).astype(np.int32)  # numpy rint: half to even
    assert np.array_equal(orc.i8_round(x), ref)


def test_quant_scale_special_cases(orc):
    assert orc.quant_scale(0.0, I8) == 1.0 and orc.quant_scale(0.0, FP8) == 1.0
    assert orc.quant_scale(1e-45, I8) == np.finfo(np.float32).tiny
    assert orc.quant_scale(127.0, I8) == 1.0 and orc.quant_scale(448.0, FP8) == 1.0
    a = np.float32(3.7)
    assert orc.quant_scale(a, I8) == np.float32(a / np.float32(127))


# ---------------------------------------------------------------- per-token quantization
def _np_token_quant_i8(xf):
    amax = np.abs(xf).max(axis=1)
    scale = np.where(amax == 0, np.float32(1), np.maximum(amax / np.float32(127),
                                                         np.finfo(np.float32).tiny)).astype(np.float32)
    inv = (np.float32(1) / scale).astype(np.float32)
    q = np.rint(np.clip((xf * inv[:, None]).astype(np.float32), -127, 127)).astype(np.int8)
    return q, scale


def test_token_quant_i8_closed_form_and_invariants(orc):
    bits = synthetic.activations(16, 2048, seed=0)
    q, s = orc.quantize_rows(bits, I8)
    xf = synthetic.bf16_bits_to_f32(bits)
    q_ref, s_ref = _np_token_quant_i8(xf)
    assert np.array_equal(q.view(np.int8), q_ref)
    assert np.array_equal(s, s_ref)
    qi = q.view(np.int8).astype(np.int32)
    # element with |x| == amax encodes to +-127
    arg = np.abs(xf).argmax(axis=1)
    assert np.all(np.abs(qi[np.arange(16), arg]) == 127)
    # reconstruction within half a step
    assert np.all(np.abs(qi * s[:, None] - xf) <= s[:, None] * 0.5000001)
    # sign symmetry q(-x) = -q(x)
    qn, sn = orc.quantize_rows(bits ^ np.uint16(0x8000), I8)
    assert np.array_equal(qn.view(np.int8), -q.view(np.int8)) and np.array_equal(sn, s)


def test_token_quant_zero_row_and_outliers(orc):
    bits = synthetic.activations(4, 256, seed=5)
    bits[1] = 0
    q, s = orc.quantize_rows(bits, I8)
    assert s[1] == 1.0 and not q[1].any()
    # outlier channels (x20) own the range: ordinary channels use few codes
    ch = synthetic.outlier_channels(2048, 0)
    assert len(ch) == 10


def test_token_quant_fp8_matches_torch_cast(orc):
    bits = synthetic.activations(8, 2048, seed=6)
    q, s = orc.quantize_rows(bits, FP8)
    xf = synthetic.bf16_bits_to_f32(bits)
    amax = np.abs(xf).max(axis=1)
    assert np.array_equal(s, (amax / np.float32(448)).astype(np.float32))
    inv = (np.float32(1) / s).astype(np.float32)
    scaled = (xf * inv[:, None]).astype(np.float32)
    ref = torch.from_numpy(scaled).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(q, ref)


def test_strided_and_f16_sources(orc):
    bits = synthetic.activations(6, 320, seed=7)
    wide = np.zeros((6, 400), np.uint16)
    wide[:, :320] = bits
    q1, s1 = orc.quantize_rows(bits, I8)
    q2, s2 = orc.quantize_rows(wide, I8, ld=400, cols=320)
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)
    xf = synthetic.bf16_bits_to_f32(bits)
    h = xf.astype(np.float16)
    q3, s3 = orc.quantize_rows(h.view(np.uint16), I8, src_type=F16)
    q_ref, s_ref = _np_token_quant_i8(h.astype(np.float32))
    assert np.array_equal(q3.view(np.int8), q_ref) and np.array_equal(s3, s_ref)


# ---------------------------------------------------------------- H128 rotation
def _sylvester(n):
    i = np.arange(n)
    pc = np.vectorize(lambda v: bin(v).count("1"))(i[:, None] & i[None, :])
    return np.where(pc % 2, -1.0, 1.0)


def test_rotation_signs_hash(orc):
    c = np.arange(6144, dtype=np.uint64)
    h = (c * 0x45D9F3B) & 0xFFFFFFFF
    h = ((h ^ (h >> 16)) * 0x45D9F3B) & 0xFFFFFFFF
    ref = np.where((h ^ (h >> 16)) & 1, 1.0, -1.0).astype(np.float32)
    assert np.array_equal(orc.rotation_signs(6144), ref)
    assert 0.4 < (ref > 0).mean() < 0.6


def test_rotation_matches_matrix_and_is_orthogonal(orc):
    H = _sylvester(128)
    assert np.allclose(H @ H.T, 128 * np.eye(128))
    rng = np.random.default_rng(8)
    for c0 in (0, 128, 5888):
        x = rng.standard_normal(128).astype(np.float32)
        y = orc.rotate128(x, c0)
        d = orc.rotation_signs(c0 + 128)[c0:]
        ref = (H @ (d.astype(np.float64) * x)) * (1 / math.sqrt(128))
        assert np.allclose(y, ref, rtol=1e-5, atol=1e-5)
        assert math.isclose(np.linalg.norm(y), np.linalg.norm(x), rel_tol=1e-5)
    # a basis vector maps to +-1/sqrt(128) everywhere
    e = np.zeros(128, np.float32)
    e[5] = 1
    y = orc.rotate128(e, 0)
    assert np.allclose(np.abs(y), np.float32(0.08838834764831845))
    # matched rotations preserve dot products: x.w == Rx.Rw
    a, b = rng.standard_normal(128).astype(np.float32), rng.standard_normal(128).astype(np.float32)
    assert math.isclose(float(orc.rotate128(a, 256) @ orc.rotate128(b, 256)), float(a @ b),
                        rel_tol=1e-4, abs_tol=1e-4)


def test_rotated_token_quant_uses_rotated_amax(orc):
    bits = synthetic.activations(3, 512, seed=9)
    q, s = orc.quantize_rows(bits, I8, rotation=128)
    xf = synthetic.bf16_bits_to_f32(bits)
    rot = np.stack([np.concatenate([orc.rotate128(xf[r, c:c + 128], c) for c in range(0, 512, 128)])
                    for r in range(3)])
    q_ref, s_ref = _np_token_quant_i8(rot)
    assert np.array_equal(s, s_ref) and np.array_equal(q.view(np.int8), q_ref)


# ---------------------------------------------------------------- group quantization
@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_group_quant_equals_per_token_of_slices(orc, fmt, group):
    """Layout invariant: group g of row r is the per-token quantization of the
    slice [r, g*G:(g+1)*G], and its scale sits at scales[g, r]."""
    rows, cols = 5, 4 * group + 16  # ragged last group
    bits = synthetic.activations(rows, cols, seed=10)
    q, s = orc.quantize_rows(bits, fmt, group=group)
    groups = -(-cols // group)
    assert s.shape == (groups, rows)
    for g in range(groups):
        sl = np.ascontiguousarray(bits[:, g * group:(g + 1) * group])
        qg, sg = orc.quantize_rows(sl, fmt)
        assert np.array_equal(q[:, g * group:(g + 1) * group], qg)
        assert np.array_equal(s[g], sg)


def test_rotated_group_quant_equals_group_quant_of_rotated(orc):
    bits = synthetic.activations(4, 256, seed=11)
    q, s = orc.quantize_rows(bits, I8, group=128, rotation=128)
    xf = synthetic.bf16_bits_to_f32(bits)
    for r in range(4):
        for g in range(2):
            v = orc.rotate128(xf[r, g * 128:(g + 1) * 128], g * 128)
            qr, sr = _np_token_quant_i8(v[None, :])
            assert np.array_equal(q[r, g * 128:(g + 1) * 128].view(np.int8), qr[0])
            assert s[g, r] == sr[0]


# ---------------------------------------------------------------- GEMMs
def test_i8_gemm_brute_force_and_epilogue(orc):
    rng = np.random.default_rng(12)
    xq = rng.integers(-127, 128, (7, 160)).astype(np.int8)
    wq = rng.integers(-127, 128, (48, 160)).astype(np.int8)
    acc = orc.gemm_i8_acc(xq, wq)
    assert np.array_equal(acc, xq.astype(np.int64) @ wq.astype(np.int64).T)
    # extreme magnitudes: K=131071 bound keeps int32 exact (127*127*K < 2^31)
    assert 127 * 127 * 131071 < 2 ** 31
    sx = rng.uniform(0.01, 0.1, 7).astype(np.float32)
    sw = rng.uniform(1e-4, 1e-3, 48).astype(np.float32)
    y0 = orc.epilogue_i8(acc, sx, sw, order=0)
    y1 = orc.epilogue_i8(acc, sx, sw, order=1)
    a = acc.astype(np.float32)
    ref0 = torch.from_numpy(((a * sx[:, None]).astype(np.float32) * sw[None, :]).astype(np.float32))
    ref1 = torch.from_numpy(((a * sw[None, :]).astype(np.float32) * sx[:, None]).astype(np.float32))
    assert np.array_equal(y0, ref0.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(y1, ref1.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
    # the two reference orders differ by at most one bf16 ulp
    assert np.abs(y0.astype(np.int32) - y1.astype(np.int32)).max() <= 1


def test_fp8_ideal_matches_float64_matmul(orc):
    rng = np.random.default_rng(13)
    table = orc.fp8_decode_table()
    finite = np.array([c for c in range(256) if not math.isnan(table[c])], np.uint8)
    xq = rng.choice(finite, (5, 256))
    wq = rng.choice(finite, (32, 256))
    sx = rng.uniform(0.01, 0.1, 5).astype(np.float32)
    sw = rng.uniform(1e-4, 1e-3, 32).astype(np.float32)
    y = orc.gemm_fp8_ideal(xq, sx, wq, sw)
    ref = (table[xq].astype(np.float64) @ table[wq].astype(np.float64).T) * sx[:, None] * sw[None, :]
    assert np.allclose(y, ref.astype(np.float32), rtol=1e-6, atol=0)


def test_grouped_single_group_closed_form(orc):
    """One K group: y = fmaf(p, sx*sw, 0), i.e. a single rounding of p*(sx*sw)."""
    rng = np.random.default_rng(14)
    xq = rng.integers(-127, 128, (4, 128)).astype(np.int8)
    wq = rng.integers(-127, 128, (16, 128)).astype(np.int8)
    sx = rng.uniform(0.01, 0.1, (1, 4)).astype(np.float32)
    sw = rng.uniform(1e-4, 1e-3, (1, 16)).astype(np.float32)
    _, yf = orc.gemm_grouped(xq.view(np.uint8), sx, wq.view(np.uint8), sw, I8, 128, 128)
    p = (xq.astype(np.int64) @ wq.astype(np.int64).T).astype(np.float64)
    scale = (sx[0][:, None] * sw[0][None, :]).astype(np.float32).astype(np.float64)
    assert np.array_equal(yf, (p * scale).astype(np.float32))


def test_grouped_matches_ideal_and_splits(orc):
    rng = np.random.default_rng(15)
    M, N, K = 6, 32, 1024
    bits_x = synthetic.activations(M, K, seed=16)
    bits_w = synthetic.weights(N, K, seed=16)
    for fmt in (I8, FP8):
        xq, sx = orc.quantize_rows(bits_x, fmt, group=128, rotation=128)
        wq, sw = orc.quantize_rows(bits_w, fmt, group=128, rotation=128)
        ideal = orc.gemm_grouped_ideal(xq, sx, wq, sw, fmt, 128, 128)
        for splits, waves in ((1, 1), (2, 1), (1, 4), (2, 2)):
            _, yf = orc.gemm_grouped(xq, sx, wq, sw, fmt, 128, 128, splits, waves)
            err = np.abs(yf - ideal).max() / np.abs(ideal).max()
            assert err < 1e-5, (fmt, splits, waves, err)
        # the rotated group GEMM approximates the unquantized product
        xf = synthetic.bf16_bits_to_f32(bits_x).astype(np.float64)
        wf = synthetic.bf16_bits_to_f32(bits_w).astype(np.float64)
        exact = xf @ wf.T
        rel = np.linalg.norm(ideal - exact) / np.linalg.norm(exact)
        assert rel < (0.02 if fmt == I8 else 0.06), rel
    del rng


@pytest.mark.parametrize("fast", [False, True])
@pytest.mark.parametrize("M", [8, 70])
def test_cpu_baseline_equals_oracle_pipeline(orc, M, fast):
    """The timed CPU baseline (both builds; M = 70 spans three 32-row blocks)
    equals the oracle pipeline: INT8, group_int8, FP8 (the per-channel FP8
    dot sums decoded products in K order in fp32, as orc_gemm_grouped does
    for one group spanning K)."""
    N, K = 64, 512
    bits_x = synthetic.activations(M, K, seed=17)
    bits_w = synthetic.weights(N, K, seed=17)
    wq, sw = orc.quantize_rows(bits_w, I8)
    y = orc.cpu_qlinear(bits_x, wq, sw, I8, threads=3, fast=fast)
    xq, sx = orc.quantize_rows(bits_x, I8)
    ref = orc.epilogue_i8(orc.gemm_i8_acc(xq, wq), sx, sw, order=0)
    assert np.array_equal(y, ref)
    wq, sw = orc.quantize_rows(bits_w, I8, group=128, rotation=128)
    y = orc.cpu_qlinear(bits_x, wq, sw, I8, group=128, rotation=128, threads=2, fast=fast)
    xq, sx = orc.quantize_rows(bits_x, I8, group=128, rotation=128)
    ref, _ = orc.gemm_grouped(xq, sx, wq, sw, I8, 128, 128)
    assert np.array_equal(y, ref)
    wq, sw = orc.quantize_rows(bits_w, FP8)
    y = orc.cpu_qlinear(bits_x, wq, sw, FP8, threads=4, fast=fast)
    xq, sx = orc.quantize_rows(bits_x, FP8)
    ideal = orc.gemm_fp8_ideal(xq, sx, wq, sw)
    got = synthetic.bf16_bits_to_f32(y).astype(np.float64)
    assert np.linalg.norm(got - ideal) / np.linalg.norm(ideal) <= 1e-2


# ---------------------------------------------------------------- evaluation orders
def _butterflies_f32(v, strides):
    v = v.astype(np.float32).copy()
    for span in strides:
        for i in range(128):
            if not i & span:
                a, b = v[i], v[i | span]
                v[i], v[i | span] = a + b, a - b
    return v


def test_rotation_stride_order_is_observable_and_ascending(orc):
    """The H128 transform is order-free in exact arithmetic, so the fp32 result
    pins the butterfly order only where the orders round differently. The
    reference runs strides 1, 2, ..., 64 with the sum on the lower index and a
    separate multiply by 1/sqrt(128) afterwards (quant_device.cuh:96-125).
    On random blocks the descending order and a scale folded into the sign
    step differ from that in fp32; the oracle must give the ascending result on
    every block and differ from each alternative on some block."""
    rng = np.random.default_rng(21)
    inv = np.float32(0.08838834764831845)
    differs_desc = differs_folded = 0
    for c0 in range(0, 20 * 128, 128):
        x = (rng.standard_normal(128) * 3).astype(np.float32)
        signed = x * orc.rotation_signs(c0 + 128)[c0:]
        asc = _butterflies_f32(signed, [1, 2, 4, 8, 16, 32, 64]) * inv
        desc = _butterflies_f32(signed, [64, 32, 16, 8, 4, 2, 1]) * inv
        folded = _butterflies_f32(signed * inv, [1, 2, 4, 8, 16, 32, 64])
        y = orc.rotate128(x, c0)
        assert np.array_equal(y, asc), c0
        differs_desc += not np.array_equal(y, desc)
        differs_folded += not np.array_equal(y, folded)
    assert differs_desc > 0 and differs_folded > 0


def _round_f32(q):
    """Correctly rounded (ties to even) float32 of an exact Fraction."""
    from fractions import Fraction
    c = np.float32(float(q))
    best = None
    for cand in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
        d = abs(Fraction(float(cand)) - q)
        key = (d, int(np.array(cand).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, cand)
    return best[1]


def test_grouped_accumulation_is_one_fma_per_group(orc):
    """Group partials accumulate as r = fmaf(p, sa*sb, r): the scale product is
    rounded first and the product-plus-sum is rounded once (quant_grouped.cu:144,
    compiled with nvcc's default contraction). Evaluated exactly with
    fractions, that differs from the uncontracted round(round(p*s) + r) and from
    fmaf(p*sa, sb, r) on many random two-group dot products; the oracle must
    give the contracted value every time."""
    from fractions import Fraction
    rng = np.random.default_rng(22)
    seen_unfused = seen_other_assoc = 0
    for _ in range(200):
        xq = rng.integers(-127, 128, (1, 256)).astype(np.int8)
        wq = rng.integers(-127, 128, (1, 256)).astype(np.int8)
        sx = rng.uniform(0.001, 0.1, (2, 1)).astype(np.float32)
        sw = rng.uniform(1e-4, 1e-2, (2, 1)).astype(np.float32)
        _, yf = orc.gemm_grouped(xq.view(np.uint8), sx, wq.view(np.uint8), sw, I8, 128, 128)
        p = [int(xq[0, g * 128:(g + 1) * 128].astype(np.int64) @ wq[0, g * 128:(g + 1) * 128].astype(np.int64))
             for g in range(2)]
        s = [np.float32(sx[g, 0] * sw[g, 0]) for g in range(2)]
        r0 = _round_f32(Fraction(p[0]) * Fraction(float(s[0])))
        fused = _round_f32(Fraction(p[1]) * Fraction(float(s[1])) + Fraction(float(r0)))
        assert yf[0, 0] == fused
        unfused = np.float32(_round_f32(Fraction(p[1]) * Fraction(float(s[1]))) + r0)
        seen_unfused += unfused != fused
        ps = [_round_f32(Fraction(p[g]) * Fraction(float(sx[g, 0]))) for g in range(2)]
        r0b = _round_f32(Fraction(float(ps[0])) * Fraction(float(sw[0, 0])))
        other = _round_f32(Fraction(float(ps[1])) * Fraction(float(sw[1, 0])) + Fraction(float(r0b)))
        seen_other_assoc += other != fused
    assert seen_unfused > 0 and seen_other_assoc > 0, (seen_unfused, seen_other_assoc)
