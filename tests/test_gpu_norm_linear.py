"""qlin_norm_linear (LayerNorm -> per-token quantization -> quantized GEMV,
reference normalized_quantized_linear, ops/kernels/sequence/sequence_norm.cu:
260-390, 518-575) on the GPU through the C ABI: outputs, normalized rows,
codes and scales bit-exact against the oracle for INT8 and FP8, bf16/f16,
with and without each fusion, ragged k and channel counts."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
BF16, FP8, I8, F16 = 0, 3, 4, 5


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def dev16(b, dtype, dev):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(dtype).to(dev)


@pytest.mark.parametrize("dtype,src_type", [(torch.bfloat16, BF16), (torch.float16, F16)])
@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("rows,k,n", [(1, 512, 600), (5, 320, 7), (64, 256, 96), (3, 4, 8),
                                      (17, 100, 33), (64, 512, 2040), (300, 128, 1000)])
def test_norm_linear_parity(dev, orc, dtype, src_type, fmt, rows, k, n):
    from breeze_tts_cpp_amd import qlinear
    g = torch.Generator().manual_seed(rows * 31 + k + n + fmt)
    mk = lambda *s, sc=1.0, off=0.0: bits((off + sc * torch.randn(*s, generator=g)).to(dtype))
    x, res, pb = mk(rows, k, sc=2.0, off=0.3), mk(rows, k), mk(k, sc=0.1)
    nw, nb, b = mk(k, sc=0.1, off=1.0), mk(k, sc=0.1), mk(n, sc=0.2)
    gate, shift, scale = mk(1, k, sc=0.3, off=1.0), mk(1, k, sc=0.1), mk(1, k, sc=0.1)
    wq, sw = orc.quantize_rows(mk(n, k, sc=0.05), fmt, src_type=src_type)
    for fused in ((False, False, False, False, 0, False), (True, True, True, True, 1, True),
                  (True, False, True, False, 0, True), (False, True, False, True, 1, False)):
        use_res, use_pb, use_affine, use_bias, act, use_mod = fused
        print(f"norm_linear dtype={dtype} fmt={fmt} rows={rows} k={k} n={n} fused={fused}",
              flush=True)
        fusion = dict(residual=res if use_res else None, projection_bias=pb if use_pb else None,
                      gate=gate if use_mod else None, shift=shift if use_mod else None,
                      scale=scale if use_mod else None)
        y, nrm, enc, esc, raw = orc.norm_linear(
            x, wq, sw, fmt, norm_weight=nw if use_affine else None,
            norm_bias=nb if use_affine else None, bias=b if use_bias else None, act=act,
            eps=1e-5, src_type=src_type, raw=True, **fusion)
        normalized = torch.empty((rows, k), dtype=dtype, device=dev)
        raw_d = torch.empty((rows, k), dtype=dtype, device=dev)
        codes = torch.empty((rows, k), dtype=torch.uint8, device=dev)
        scales = torch.empty((rows,), dtype=torch.float32, device=dev)
        d = lambda a: None if a is None else dev16(a, dtype, dev)
        dfus = {key: d(v) for key, v in fusion.items()}
        yd = qlinear.norm_linear(
            d(x), torch.from_numpy(wq).to(dev), torch.from_numpy(sw).to(dev), fmt,
            norm_weight=d(nw) if use_affine else None, norm_bias=d(nb) if use_affine else None,
            fusion=qlinear.norm_fusion(raw=raw_d, **dfus), bias=d(b) if use_bias else None,
            activation=act, eps=1e-5, normalized=normalized, encoded=(codes, scales))
        torch.cuda.synchronize()
        assert np.array_equal(bits(raw_d), raw)
        assert np.array_equal(bits(normalized), nrm)
        assert np.array_equal(codes.cpu().numpy(), enc)
        assert np.array_equal(scales.cpu().numpy(), esc)
        assert np.array_equal(bits(yd), y)


@pytest.mark.parametrize("fmt", [I8, FP8])
def test_norm_linear_per_sequence_modulation(dev, orc, fmt):
    """gate / shift / scale with one row per sequence (rows_per_sequence = 4)."""
    from breeze_tts_cpp_amd import qlinear
    rows, k, n, rps = 12, 256, 40, 4
    g = torch.Generator().manual_seed(fmt)
    mk = lambda *s, sc=1.0, off=0.0: bits((off + sc * torch.randn(*s, generator=g)).to(torch.bfloat16))
    x = mk(rows, k, sc=2.0)
    gate, shift, scale = mk(3, k, sc=0.3, off=1.0), mk(3, k, sc=0.1), mk(3, k, sc=0.1)
    wq, sw = orc.quantize_rows(mk(n, k, sc=0.05), fmt)
    y, nrm, enc, esc, _ = orc.norm_linear(x, wq, sw, fmt, gate=gate, shift=shift, scale=scale,
                                          rows_per_sequence=rps)
    d = lambda a: dev16(a, torch.bfloat16, dev)
    normalized = torch.empty((rows, k), dtype=torch.bfloat16, device=dev)
    mods = dict(gate=d(gate), shift=d(shift), scale=d(scale))  # alive across the call
    yd = qlinear.norm_linear(d(x), torch.from_numpy(wq).to(dev), torch.from_numpy(sw).to(dev), fmt,
                             fusion=qlinear.norm_fusion(rows_per_sequence=rps, **mods),
                             normalized=normalized)
    torch.cuda.synchronize()
    assert np.array_equal(bits(normalized), nrm)
    assert np.array_equal(bits(yd), y)
