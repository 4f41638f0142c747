"""Pins the oracle's fused producers (residual + RMSNorm -> quant and gated
activation -> quant; reference ops/kernels/quant/quant_norm.cu:14-123 and
quant_gated.cu:9-85) by routes independent of its C code: exact decimal
arithmetic for the reciprocal square root, exact sums for the reduction,
torch's bf16/f16 arithmetic and fp64 activations for the element-wise steps,
and the already pinned row quantizer for the encoding step."""
import decimal
import math

import numpy as np
import pytest
import torch

from breeze_tts_cpp_amd import synthetic


def bits_to_torch(bits, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).view(dtype)


def torch_to_bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_rsqrt_rn_is_correctly_rounded(orc):
    """1/sqrt(a) is the fp32 value nearest the exact result (decimal, 60 digits)."""
    decimal.getcontext().prec = 60
    rng = np.random.default_rng(5)
    cases = np.concatenate([rng.uniform(1e-3, 1e3, 400), 2.0 ** rng.integers(-120, 120, 60),
                            [1.0, 2.0, 3.0, 1e-30, 1e30, 1.17549435e-38, 0.5000001]])
    for a in cases.astype(np.float32):
        r = np.float32(orc.rsqrt_rn(float(a)))
        exact = decimal.Decimal(1) / decimal.Decimal(float(a)).sqrt()
        err = abs(decimal.Decimal(float(r)) - exact)
        for nb in (np.nextafter(r, np.float32(0)), np.nextafter(r, np.float32(np.inf))):
            assert err <= abs(decimal.Decimal(float(nb)) - exact), (a, r)


def test_norm_sumsq_exact_cases(orc):
    """Every column enters the squared sum exactly once, for every row length
    up to 2048 (one-hot rows), and small-integer rows sum exactly."""
    for cols in (1, 7, 8, 9, 255, 256, 1000, 2047, 2048):
        for c in sorted({0, cols // 2, cols - 1}):
            v = np.zeros(cols, np.float32)
            v[c] = 3.0
            assert orc.norm_sumsq(v) == 9.0
    rng = np.random.default_rng(1)
    v = rng.integers(-8, 9, 2048).astype(np.float32)
    assert orc.norm_sumsq(v) == float(np.sum(v.astype(np.int64) ** 2))
    w = rng.standard_normal(1536).astype(np.float32)
    ref = float(np.sum(w.astype(np.float64) ** 2))
    assert abs(orc.norm_sumsq(w) - ref) <= 1e-6 * ref


def _torch_norm(x, w, inv, gemma):
    """Element-wise normalization with torch's 16-bit rounding (fp32 compute,
    round to the storage dtype after each reference rounding point)."""
    xf = x.float()
    if gemma:
        return ((xf * inv) * (w.float() + 1.0)).to(x.dtype)
    return ((xf * inv).to(x.dtype).float() * w.float()).to(x.dtype)


@pytest.mark.parametrize("dtype,src_type", [(torch.bfloat16, 0), (torch.float16, 5)])
@pytest.mark.parametrize("gemma", [False, True])
@pytest.mark.parametrize("update", ["none", "add", "scaled"])
def test_quantized_norm_matches_torch(orc, dtype, src_type, gemma, update):
    rows, cols, eps = 6, 2000, 1e-6
    g = torch.Generator().manual_seed(rows + cols + int(gemma))
    x = torch.randn(rows, cols, generator=g).to(dtype)
    w = (1.0 + 0.1 * torch.randn(cols, generator=g)).to(dtype)
    u = torch.randn(rows, cols, generator=g).to(dtype) if update != "none" else None
    s = (0.5 + torch.rand(cols, generator=g)).to(dtype) if update == "scaled" else None
    res, q, scales, n = orc.quantized_norm(
        torch_to_bits(x), torch_to_bits(w), orc.I8,
        update_bits=None if u is None else torch_to_bits(u),
        scale_bits=None if s is None else torch_to_bits(s), eps=eps, gemma=gemma,
        src_type=src_type)
    # residual update: x + u (* s) with 16-bit rounding of each operation
    v = x if u is None else (x.float() + (u if s is None else (u.float() * s.float()).to(dtype)).float()).to(dtype)
    assert np.array_equal(res, torch_to_bits(v))
    nt = bits_to_torch(n, dtype)
    for r in range(rows):
        vr = v[r].double()
        inv64 = 1.0 / math.sqrt(float((vr * vr).sum()) / cols + eps)
        # with the fp64 normalizer: within one 16-bit ulp everywhere
        near = _torch_norm(v[r], w, inv64, gemma).float()
        ulp = (near.abs() * (2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10)).clamp_min(1e-30)
        assert torch.all((nt[r].float() - near).abs() <= ulp + 1e-30)
        # with the oracle's own fp32 normalizer: bit-exact element-wise steps
        inv32 = orc.rsqrt_rn(orc.norm_sumsq(v[r].float().numpy()) / np.float32(cols) + np.float32(eps))
        assert abs(inv32 - inv64) <= 2e-7 * inv64
        assert torch.equal(torch_to_bits_t(nt[r]), torch_to_bits_t(_torch_norm(v[r], w, inv32, gemma)))
    # the normalized rows go through the (separately pinned) row quantizer
    q2, s2 = orc.quantize_rows(n, orc.I8, src_type=src_type)
    assert np.array_equal(q, q2) and np.array_equal(scales, s2)


def torch_to_bits_t(t):
    return t.contiguous().view(torch.int16)


def test_quantized_norm_rms_and_modes(orc):
    """Unit weights: the normalized row has RMS 1 (to bf16 precision); group
    and rotated modes equal the row quantizer applied to the normalized row."""
    x = synthetic.activations(4, 2048, seed=3)
    w = synthetic.f32_to_bf16_bits(np.ones(2048, np.float32))
    _, _, _, n = orc.quantized_norm(x, w, orc.I8)
    nf = synthetic.bf16_bits_to_f32(n).astype(np.float64)
    assert np.allclose(np.sqrt((nf ** 2).mean(axis=1)), 1.0, atol=5e-3)
    for fmt in (orc.I8, orc.FP8):
        for group, rot in ((0, 128), (128, 0), (64, 128), (32, 0)):
            _, q, s, n2 = orc.quantized_norm(x, w, fmt, group=group, rotation=rot)
            q2, s2 = orc.quantize_rows(n2, fmt, group=group, rotation=rot)
            assert np.array_equal(q, q2) and np.array_equal(s, s2)


@pytest.mark.parametrize("kind", [0, 1])
def test_activation_matches_fp64(orc, kind):
    """SiLU / tanh-GeLU against torch's fp64 functions: the fp32 result is
    within 3 ulp of the fp64 value, and special values are exact."""
    xs = np.concatenate([np.linspace(-20, 20, 4001), [-100.0, -88.0, 0.0, 1e-30, 50.0]])
    xs = xs.astype(np.float32)
    t = torch.from_numpy(xs.astype(np.float64))
    ref = (torch.nn.functional.silu(t) if kind == 0
           else torch.nn.functional.gelu(t, approximate="tanh")).numpy()
    got = np.array([orc.activate(float(v), kind) for v in xs], np.float64)
    # three fp32 roundings (exp, 1 + e, the quotient) bound the error to 3 ulp
    tol = 3 * np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64) + 1e-40
    # tanh-GeLU's fp32 form (0.5x)(1 + tanh(.)) cancels for negative x: its
    # absolute error is a few ulp of 1 times |0.5x|, plus the fp32 argument
    if kind == 1:
        tol = tol * 4 + 1e-7 * np.abs(ref) + np.abs(xs.astype(np.float64)) * 2.0 ** -22
    assert np.all(np.abs(got - ref) <= tol)
    assert orc.activate(0.0, kind) == 0.0
    if kind == 0:
        assert orc.activate(-100.0, 0) == 0.0 and math.copysign(1, orc.activate(-100.0, 0)) < 0
        assert orc.activate(50.0, 0) == 50.0


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("fmt", [3, 4])
def test_quantized_gated_matches_torch(orc, kind, fmt):
    """act(gate) rounded to bf16 equals torch's fp64 activation rounded to bf16
    except on rare rounding boundaries (never by more than one ulp); the
    product with `up` is torch's bf16 multiply; the encoding is the row
    quantizer of the activated rows."""
    rows, width = 4, 3000
    g = torch.Generator().manual_seed(11 + kind)
    inp = (2.0 * torch.randn(rows, 2 * width, generator=g)).to(torch.bfloat16)
    q, s, a = orc.quantized_gated(torch_to_bits(inp), kind, fmt)
    gate, up = inp[:, :width], inp[:, width:]
    t64 = gate.double()
    act64 = torch.nn.functional.silu(t64) if kind == 0 else torch.nn.functional.gelu(
        t64, approximate="tanh")
    act_bits = np.array([[orc.f32_to_bf16_bits(np.float32(orc.activate(float(v), kind)))
                          for v in row] for row in gate.float().numpy()], np.uint16)
    ref_bits = torch_to_bits(act64.float().to(torch.bfloat16))
    if kind == 0:
        diff = np.abs(act_bits.astype(np.int32) - ref_bits.astype(np.int32))
        assert diff.max() <= 1 and (diff > 0).mean() < 1e-3
    else:
        # fp32 cancellation of (0.5x)(1 + tanh) for negative x (the reference's form)
        got = bits_to_torch(act_bits).double()
        tol = act64.abs() * 2.0 ** -8 + gate.double().abs() * 2.0 ** -22 + 1e-38
        assert torch.all((got - act64).abs() <= tol)
    prod = (bits_to_torch(act_bits).float() * up.float()).to(torch.bfloat16)
    assert np.array_equal(a, torch_to_bits(prod))
    q2, s2 = orc.quantize_rows(a, fmt)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


def test_pack_weights_is_the_fragment_permutation(orc):
    """Packed layout: a bijection of the weight bytes onto fragment order,
    zero-padded past K. Byte (n, k) sits in tile (n//16, k//64), chunk
    ((k%64)//16)*16 + n%16, byte k%16; checked on distinct byte values."""
    for N, K in ((32, 128), (48, 80), (16, 16)):
        idx = np.arange(N * K, dtype=np.int64)
        w = (idx % 251).astype(np.uint8)          # position tag
        p = orc.pack_weights(w.reshape(N, K))
        tk = -(-K // 64)
        assert p.size == N * tk * 64
        n, k = np.divmod(idx, K)
        off = ((n // 16) * tk + k // 64) * 1024 + (((k % 64) // 16) * 16 + n % 16) * 16 + k % 16
        assert np.array_equal(p[off], w)
        assert len(np.unique(off)) == N * K
        pad = np.ones(p.size, bool)
        pad[off] = False
        assert not p[pad].any()


@pytest.mark.parametrize("dtype,out_type", [(torch.bfloat16, 0), (torch.float16, 5)])
def test_finish_matches_torch(orc, dtype, out_type):
    """Finish of a stored GEMM result: bias added with torch's 16-bit rounding,
    ReLU exactly, tanh-GeLU within one 16-bit ulp of torch's fp64 function
    (plus the cancellation bound of the fp32 form for negative inputs)."""
    g = torch.Generator().manual_seed(3)
    y = (4 * torch.randn(8, 96, generator=g)).to(dtype)
    b = torch.randn(96, generator=g).to(dtype)
    yb, bb = torch_to_bits(y), torch_to_bits(b)
    biased = (y.float() + b.float()).to(dtype)
    assert np.array_equal(orc.finish(yb, bb, 0, out_type), torch_to_bits(biased))
    assert np.array_equal(orc.finish(yb, None, 0, out_type), yb)
    relu = torch.clamp_min(biased.float(), 0).to(dtype)
    assert np.array_equal(orc.finish(yb, bb, 1, out_type), torch_to_bits(relu))
    ref = torch.nn.functional.gelu(biased.double(), approximate="tanh")
    got = bits_to_torch(orc.finish(yb, bb, 2, out_type), dtype).double()
    ulp = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    tol = ref.abs() * 2 * ulp + biased.double().abs() * 2.0 ** -22 + 1e-30
    assert torch.all((got - ref).abs() <= tol)


def test_cub_sum256_order(orc):
    """The CUB block sum: each of 256 inputs counted exactly once, exact on
    small integers, and it differs from a plain left-to-right fp32 sum on an
    adversarial input (the order is pinned, not just the value)."""
    for c in (0, 1, 31, 32, 200, 255):
        v = np.zeros(256, np.float32)
        v[c] = 5.0
        assert orc.cub_sum256(v) == 5.0
    ints = np.random.default_rng(2).integers(-100, 100, 256).astype(np.float32)
    assert orc.cub_sum256(ints) == float(ints.astype(np.int64).sum())
    # lanes 0, 2, 3 of warp 0 hold 2^24, 1, 1: the stride-1 step forms
    # 1 + 1 = 2 before it meets 2^24 (2^24 + 2 is exact), while a sequential
    # sum rounds 2^24 + 1 back to 2^24 twice.
    v = np.zeros(256, np.float32)
    v[0], v[2], v[3] = 2.0 ** 24, 1.0, 1.0
    assert orc.cub_sum256(v) == 2.0 ** 24 + 2.0  # (1 + 1) formed before meeting 2^24
    seq = np.float32(0)
    for a in v:
        seq = np.float32(seq + a)
    assert float(seq) == 2.0 ** 24


@pytest.mark.parametrize("fmt", [3, 4])
@pytest.mark.parametrize("k", [512, 320, 8])
def test_norm_linear_matches_torch(orc, fmt, k):
    """LayerNorm against torch's fp64 layer_norm (within one bf16 ulp) and the
    oracle's element-wise steps against torch's bf16 rounding given its own
    mean/normalizer; codes = the row quantizer of the normalized row; INT8
    outputs = numpy int64 dot products with the ((acc * sw) * sx) epilogue."""
    rows, n = 5, 24
    g = torch.Generator().manual_seed(k + fmt)
    x = (torch.randn(rows, k, generator=g) * 2 + 0.5).to(torch.bfloat16)
    res = torch.randn(rows, k, generator=g).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(k, generator=g)).to(torch.bfloat16)
    nb = (0.1 * torch.randn(k, generator=g)).to(torch.bfloat16)
    wq, sw = orc.quantize_rows(torch_to_bits((0.05 * torch.randn(n, k, generator=g)).to(torch.bfloat16)), fmt)
    y, nrm, enc, esc, _ = orc.norm_linear(torch_to_bits(x), wq, sw, fmt, norm_weight=torch_to_bits(nw),
                                       norm_bias=torch_to_bits(nb), residual=torch_to_bits(res),
                                       eps=1e-5)
    v = (x.float() + res.float()).to(torch.bfloat16).double()
    ref = torch.nn.functional.layer_norm(v, (k,), nw.double(), nb.double(), eps=1e-5)
    got = bits_to_torch(nrm).double()
    assert torch.all((got - ref).abs() <= ref.abs() * 2.0 ** -7 + 1e-6)
    q2, s2 = orc.quantize_rows(nrm, fmt)
    assert np.array_equal(enc, q2) and np.array_equal(esc, s2)
    if fmt == 4:
        acc = enc.view(np.int8).astype(np.int64) @ wq.view(np.int8).astype(np.int64).T
        d = (acc.astype(np.float32) * sw[None, :]) * esc[:, None]
        assert np.array_equal(y, torch_to_bits(torch.from_numpy(d).to(torch.bfloat16)))
    else:
        table = orc.fp8_decode_table().astype(np.float64)
        ideal = (table[enc] @ table[wq].T) * sw[None, :] * esc[:, None]
        got_y = bits_to_torch(y).double().numpy()
        assert np.linalg.norm(got_y - ideal) / np.linalg.norm(ideal) <= 1e-2


# ---------------------------------------------------------------- sequence producers
ACTS = {1: lambda x: torch.relu(x), 2: lambda x: torch.nn.functional.leaky_relu(x, 0.1),
        3: torch.nn.functional.silu, 4: lambda x: torch.nn.functional.gelu(x),
        5: lambda x: torch.nn.functional.gelu(x, approximate="tanh"),
        6: torch.nn.functional.mish, 7: torch.tanh, 8: torch.sigmoid}


@pytest.mark.parametrize("kind", sorted(ACTS))
def test_act_matches_torch_fp64(orc, kind):
    """ops::activate's set, each within a few fp32 ulp (plus the cancellation
    bound of the fp32 forms) of torch's fp64 function; act(0) = 0 (sigmoid 1/2)."""
    xs = np.concatenate([np.linspace(-30, 30, 2001), [-100.0, -20.5, 19.9, 20.1, 50.0]])
    got = torch.tensor([orc.act(x, kind) for x in xs], dtype=torch.float64)
    ref = ACTS[kind](torch.tensor(xs, dtype=torch.float64))
    tol = ref.abs() * 2.0 ** -21 + torch.tensor(np.abs(xs)) * 2.0 ** -22 + 1e-30
    assert torch.all((got - ref).abs() <= tol), kind
    assert orc.act(0.0, kind) == (0.5 if kind == 8 else 0.0)
    assert orc.act(-3.0, 2, alpha=0.25) == -0.75


def _bf(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).float()


def _rb(t):
    """fp32/fp64 torch tensor -> bf16 (rounded once) -> float."""
    return t.float().to(torch.bfloat16).float()


def test_norm_rows_fusions_match_torch(orc):
    """NormFusion: the 16-bit steps of load / transform reproduced with torch
    given the oracle's statistics; statistics within fp64 bounds; raw = v;
    per-sequence modulation rows; source-row gather and NaN rows."""
    rows, cols, rps = 6, 1000, 3
    g = torch.Generator().manual_seed(11)
    mk = lambda *s, sc=1.0, off=0.0: torch_to_bits((off + sc * torch.randn(*s, generator=g)).to(torch.bfloat16))
    x, res, pb = mk(rows, cols, sc=2.0), mk(rows, cols), mk(cols, sc=0.1)
    gate, shift, scale = mk(2, cols, sc=0.2, off=1.0), mk(2, cols, sc=0.1), mk(2, cols, sc=0.1)
    nw, nb = mk(cols, sc=0.1, off=1.0), mk(cols, sc=0.1)
    q, sc_, u, raw = orc.layer_norm_quantize(
        x, 4, norm_weight=nw, norm_bias=nb, residual=res, projection_bias=pb, gate=gate,
        shift=shift, scale=scale, rows_per_sequence=rps, raw=True)
    seq = torch.arange(rows) // rps
    v = _rb(_rb(_rb(_bf(x) + _bf(pb)) * _bf(gate)[seq]) + _bf(res))
    assert np.array_equal(raw, torch_to_bits(v.to(torch.bfloat16)))
    vd = v.double()
    mean = vd.mean(1, keepdim=True)
    inv = 1 / torch.sqrt(((vd - mean) ** 2).mean(1, keepdim=True) + 1e-5)
    ref = ((vd - mean) * inv * _bf(nw).double() + _bf(nb).double())
    ref = ref * (1 + _bf(scale).double()[seq]) + _bf(shift).double()[seq]
    got = _bf(u).double()
    assert torch.all((got - ref).abs() <= ref.abs() * 2.0 ** -6 + 2e-2)
    # codes = the (pinned) row quantizer of the retained rows
    q2, s2 = orc.quantize_rows(u, 4)
    assert np.array_equal(q, q2) and np.array_equal(sc_, s2)
    # gather: output row r normalizes input row src[r]; bad sources -> NaN, scale 1
    src = np.array([5, 0, -1, 2, 6], np.int32)
    qg, sg, ug, _ = orc.layer_norm_quantize(x, 4, norm_weight=nw, rows=5, source_rows=src)
    direct = orc.norm_rows(x, norm_weight=nw)
    for r, s in enumerate(src):
        if 0 <= s < rows:
            assert np.array_equal(ug[r], direct[s])
        else:
            assert np.all(np.isnan(_bf(ug[r]).numpy())) and sg[r] == 1.0


@pytest.mark.parametrize("group,rotation", [(0, 0), (32, 0), (128, 0), (128, 128), (64, 128)])
def test_layer_norm_quantize_modes(orc, group, rotation):
    """Every encoding mode: codes and scales are the row quantizer's on the
    retained rows."""
    x = synthetic.activations(7, 1024, seed=group + rotation)
    for fmt in (3, 4):
        q, s, u, _ = orc.layer_norm_quantize(x, fmt, group=group, rotation=rotation)
        q2, s2 = orc.quantize_rows(u, fmt, group=group, rotation=rotation)
        assert np.array_equal(q, q2) and np.array_equal(s, s2)


def test_pointwise_matches_torch(orc):
    """The dense Finish steps reproduced with torch's bf16 rounding: bias,
    per-sequence gate and condition, indexed residual (negative -> 0),
    value/residual scales with the contracted fma, output scale, activation
    (pinned above), sequence-tail mask, input repeat; codes = row quantizer."""
    x_rows, repeat, cols, rps, valid = 4, 2, 136, 4, 3
    rows = x_rows * repeat
    g = torch.Generator().manual_seed(5)
    mk = lambda *s, sc=1.0, off=0.0: torch_to_bits((off + sc * torch.randn(*s, generator=g)).to(torch.bfloat16))
    x, b = mk(x_rows, cols, sc=2.0), mk(cols, sc=0.3)
    gate, cond = mk(2, cols, sc=0.2, off=1.0), mk(2, cols, sc=0.5)
    res = mk(3, cols)
    idx = np.array([0, 1, 2, -1, 2, 1, 0, -5], np.int32)
    for kind in (0, 3, 5, 6):
        q, s, out, raw = orc.pointwise_quantize(
            x, 4, bias=b, gate=gate, condition=cond, residual=res, residual_index=idx,
            value_scale=0.75, residual_scale=1.5, output_scale=0.5, activation=kind,
            rows_per_sequence=rps, valid_rows_per_sequence=valid, input_repeat=repeat, raw=True)
        xr = _bf(x)[torch.arange(rows) // repeat]
        seq = torch.arange(rows) // rps
        v = _rb(xr + _bf(b))
        v = _rb(v * _bf(gate)[seq])
        skip = torch.where(torch.tensor(idx)[:, None] >= 0, _bf(res)[torch.tensor(idx).clamp_min(0)],
                           torch.zeros(1))
        v = _rb(torch.tensor(0.75, dtype=torch.float64) * v.double() +
                (torch.tensor(1.5, dtype=torch.float32) * skip).double())
        v = _rb(v + _bf(cond)[seq])
        mask = (torch.arange(rows) % rps >= valid)[:, None]
        v = torch.where(mask, torch.zeros(1), v)
        assert np.array_equal(raw, torch_to_bits(v.to(torch.bfloat16)))
        pre = _rb(v * 0.5)
        act = torch.tensor([[orc.act(float(a), kind) for a in row] for row in pre.tolist()])
        o = torch.where(mask, torch.zeros(1), _rb(act))
        assert np.array_equal(out, torch_to_bits(o.to(torch.bfloat16))), kind
        q2, s2 = orc.quantize_rows(out, 4)
        assert np.array_equal(q, q2) and np.array_equal(s, s2)
    # an index past the residual's rows contributes NaN
    _, _, out, _ = orc.pointwise_quantize(x, 4, residual=res, residual_index=np.array([0, 9, 1, 2], np.int32))
    assert np.all(np.isnan(_bf(out[1]).numpy())) and not np.isnan(_bf(out[0]).numpy()).any()


def _ulps(got, ref):
    """|got - ref| in units of the fp32 spacing at ref (denormal spacing floor)."""
    ref = np.asarray(ref, np.float64)
    sp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    return np.abs(np.asarray(got, np.float64) - ref) / np.maximum(sp, 2.0 ** -149)


def test_qexp_within_one_ulp(orc):
    """The fp32 exponential: within 1 ulp of fp64 exp over its whole finite
    range (incl. subnormal results), exact at 0, inf above / 0 below the
    range, NaN kept."""
    rng = np.random.default_rng(1)
    xs = np.concatenate([rng.uniform(-104, 88.7, 40000), rng.uniform(-1, 1, 20000),
                         np.linspace(-103.9, -87, 3000)]).astype(np.float32)
    got = np.array([orc.qexp(x) for x in xs], np.float32)
    assert _ulps(got, np.exp(xs.astype(np.float64))).max() < 1.0
    assert orc.qexp(0.0) == 1.0
    assert orc.qexp(89.0) == np.inf and orc.qexp(1e4) == np.inf
    assert orc.qexp(-104.0) == 0.0 and orc.qexp(-1e4) == 0.0
    assert np.isnan(orc.qexp(float("nan")))


def test_qtanh_within_two_ulp(orc):
    """The fp32 tanh: within 2 ulp of fp64 tanh on both branches, odd, 1
    beyond 9.1, tanh(0) = 0, NaN kept."""
    rng = np.random.default_rng(2)
    xs = np.concatenate([rng.uniform(-10, 10, 40000), rng.uniform(-0.6, 0.6, 40000),
                         np.float32([0.4999999, 0.5, 0.5000001, 9.0999, 9.1])]).astype(np.float32)
    got = np.array([orc.qtanh(x) for x in xs], np.float32)
    assert _ulps(got, np.tanh(xs.astype(np.float64))).max() < 2.0
    assert all(orc.qtanh(-x) == -orc.qtanh(x) for x in xs[:1000])
    assert orc.qtanh(0.0) == 0.0 and orc.qtanh(12.0) == 1.0 and orc.qtanh(-30.0) == -1.0
    assert np.isnan(orc.qtanh(float("nan")))
