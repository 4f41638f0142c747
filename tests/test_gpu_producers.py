"""GPU parity of the fused quantizing producers through the C ABI
(qlin_quantized_norm, qlin_quantized_gated) against the oracle: quantized
values, scales and the updated residual bit-exact, in every encoding mode,
for bf16/f16, ragged and full row widths (reference quant_norm.cu:14-188,
quant_gated.cu:18-198)."""
import numpy as np
import pytest
import torch

from breeze_tts_cpp_amd import synthetic

pytestmark = pytest.mark.gpu

MODES = [(0, 0), (0, 128), (32, 0), (64, 0), (128, 0), (128, 128), (64, 128)]


def to_dev(bits, dtype, dev):
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).view(dtype).to(dev)


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def rand_bits(shape, dtype, seed, scale=1.0, offset=0.0):
    g = torch.Generator().manual_seed(seed)
    return bits((offset + scale * torch.randn(*shape, generator=g)).to(dtype))


@pytest.mark.parametrize("dtype,src_type", [(torch.bfloat16, 0), (torch.float16, 5)])
@pytest.mark.parametrize("fmt", [3, 4])
@pytest.mark.parametrize("cols", [2048, 1000, 136, 7])
def test_quantized_norm_parity(dev, orc, dtype, src_type, fmt, cols):
    from breeze_tts_cpp_amd import qlinear
    rows = 33
    for update in ("none", "add", "scaled"):
        for gemma in (False, True):
            for group, rot in MODES:
                if rot and cols % 128:
                    continue
                print(f"norm dtype={dtype} fmt={fmt} cols={cols} update={update} gemma={gemma} "
                      f"group={group} rot={rot}", flush=True)
                seed = cols * 7 + group + rot + int(gemma) + len(update)
                x = rand_bits((rows, cols), dtype, seed)
                w = rand_bits((cols,), dtype, seed + 1, 0.1, 1.0)
                u = rand_bits((rows, cols), dtype, seed + 2) if update != "none" else None
                s = rand_bits((cols,), dtype, seed + 3, 0.2, 1.0) if update == "scaled" else None
                res, q, sc, _ = orc.quantized_norm(x, w, fmt, update_bits=u, scale_bits=s,
                                                   eps=1e-5, gemma=gemma, group=group,
                                                   rotation=rot, src_type=src_type)
                xd = to_dev(x, dtype, dev)
                qd, sd = qlinear.quantized_norm(
                    xd, to_dev(w, dtype, dev), fmt,
                    update=None if u is None else to_dev(u, dtype, dev),
                    update_scale=None if s is None else to_dev(s, dtype, dev), eps=1e-5,
                    gemma=gemma, group=group, rotation=rot)
                torch.cuda.synchronize()
                assert np.array_equal(bits(xd), res)
                assert np.array_equal(qd.cpu().numpy(), q)
                assert np.array_equal(sd.cpu().numpy(), sc)


def test_quantized_norm_decode_shapes(dev, orc):
    """The decoder's use (decoder.h:242,271): hidden 2048, residual update,
    M = 1/32/64 and a prefill M = 1024 (sampled check of all rows)."""
    from breeze_tts_cpp_amd import qlinear
    for M in (1, 32, 64, 1024):
        print(f"norm decode M={M}", flush=True)
        x = synthetic.activations(M, 2048, seed=M)
        u = synthetic.activations(M, 2048, seed=M + 1)
        w = rand_bits((2048,), torch.bfloat16, M, 0.05, 1.0)
        for fmt, group, rot in ((4, 0, 0), (4, 128, 128), (3, 128, 128), (3, 0, 0)):
            res, q, sc, _ = orc.quantized_norm(x, w, fmt, update_bits=u, group=group,
                                               rotation=rot)
            xd = to_dev(x, torch.bfloat16, dev)
            qd, sd = qlinear.quantized_norm(xd, to_dev(w, torch.bfloat16, dev), fmt,
                                            update=to_dev(u, torch.bfloat16, dev), group=group,
                                            rotation=rot)
            assert np.array_equal(bits(xd), res)
            assert np.array_equal(qd.cpu().numpy(), q)
            assert np.array_equal(sd.cpu().numpy(), sc)


@pytest.mark.parametrize("dtype,src_type", [(torch.bfloat16, 0), (torch.float16, 5)])
@pytest.mark.parametrize("fmt", [3, 4])
@pytest.mark.parametrize("width", [6144, 8192, 2048, 1000, 9])
def test_quantized_gated_parity(dev, orc, dtype, src_type, fmt, width):
    from breeze_tts_cpp_amd import qlinear
    rows = 17
    for kind in (0, 1):
        for group, rot in MODES:
            if rot and width % 128:
                continue
            print(f"gated dtype={dtype} fmt={fmt} width={width} kind={kind} group={group} "
                  f"rot={rot}", flush=True)
            inp = rand_bits((rows, 2 * width), dtype, width + kind * 3 + group + rot, 2.0)
            q, sc, _ = orc.quantized_gated(inp, kind, fmt, group=group, rotation=rot,
                                           src_type=src_type)
            qd, sd = qlinear.quantized_gated(to_dev(inp, dtype, dev), fmt, kind=kind, group=group,
                                             rotation=rot)
            torch.cuda.synchronize()
            assert np.array_equal(qd.cpu().numpy(), q)
            assert np.array_equal(sd.cpu().numpy(), sc)


def test_quantized_gated_extremes(dev, orc):
    """Saturating activations: e^-x overflows (SiLU -> -0), large gates, zero rows."""
    from breeze_tts_cpp_amd import qlinear
    width = 2048
    g = np.linspace(-120, 120, width, dtype=np.float32)
    rows = np.stack([np.concatenate([g, np.ones(width, np.float32)]),
                     np.concatenate([g[::-1], -np.ones(width, np.float32)]),
                     np.zeros(2 * width, np.float32)])
    inp = synthetic.f32_to_bf16_bits(rows)
    for kind in (0, 1):
        for fmt in (3, 4):
            q, sc, _ = orc.quantized_gated(inp, kind, fmt)
            qd, sd = qlinear.quantized_gated(to_dev(inp, torch.bfloat16, dev), fmt, kind=kind)
            assert np.array_equal(qd.cpu().numpy(), q)
            assert np.array_equal(sd.cpu().numpy(), sc)


@pytest.mark.parametrize("width", [6144, 8192])
def test_quantized_gated_many_rows(dev, orc, width):
    """Above the spread threshold (512 rows) each lane walks several 2048-column
    chunks; both layouts give the oracle's codes and scales."""
    from breeze_tts_cpp_amd import qlinear
    rows = 520
    for kind in (0, 1):
        for group, rot in ((0, 0), (128, 128)):
            print(f"gated many rows width={width} kind={kind} group={group} rot={rot}", flush=True)
            inp = rand_bits((rows, 2 * width), torch.bfloat16, width + kind + group, 2.0)
            q, sc, _ = orc.quantized_gated(inp, kind, 4, group=group, rotation=rot)
            qd, sd = qlinear.quantized_gated(to_dev(inp, torch.bfloat16, dev), 4, kind=kind,
                                             group=group, rotation=rot)
            torch.cuda.synchronize()
            assert np.array_equal(qd.cpu().numpy(), q)
            assert np.array_equal(sd.cpu().numpy(), sc)
