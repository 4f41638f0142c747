"""GPU parity of the sequence-fusion row quantizers through the C ABI against
the oracle: qlin_layer_norm_quantize (reference layer_norm_quantize,
ops/kernels/sequence/sequence_norm.cu:65-200,412-440) and
qlin_pointwise_quantize (reference pointwise_quantize, sequence_pointwise.cu:
149-260,325-357). Codes, scales, retained and raw rows bit-exact in every
encoding mode, for bf16/f16, ragged and vector row widths up to 16384 held in
registers and past it streamed (16391 ... 24576), with
every fusion, the source-row gather and every activation."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
BF16, FP8, I8, F16 = 0, 3, 4, 5
MODES = [(0, 0), (32, 0), (128, 0), (64, 128), (128, 128)]


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def dev16(b, dtype, dev):
    return None if b is None else torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(dtype).to(dev)


def mk(g, dtype, *shape, sc=1.0, off=0.0):
    return bits((off + sc * torch.randn(*shape, generator=g)).to(dtype))


def same_codes(got, want):
    assert np.array_equal(got.cpu().numpy(), want)


@pytest.mark.parametrize("dtype,src_type", [(torch.bfloat16, BF16), (torch.float16, F16)])
@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("cols", [7, 136, 1000, 2048, 6144, 16384, 16392, 20007, 24576])
def test_layer_norm_quantize_parity(dev, orc, dtype, src_type, fmt, cols):
    from breeze_tts_cpp_amd import qlinear
    rows, rps = 6, 3
    g = torch.Generator().manual_seed(cols + fmt)
    x, res, pb = mk(g, dtype, rows, cols, sc=2.0, off=0.2), mk(g, dtype, rows, cols), mk(g, dtype, cols, sc=0.1)
    nw, nb = mk(g, dtype, cols, sc=0.1, off=1.0), mk(g, dtype, cols, sc=0.1)
    gate, shift, scale = (mk(g, dtype, 2, cols, sc=0.2, off=1.0), mk(g, dtype, 1, cols, sc=0.1),
                          mk(g, dtype, 2, cols, sc=0.1))
    for group, rot in MODES:
        if rot and cols % 128:
            continue
        for full in (False, True):
            print(f"layer_norm_quantize dtype={dtype} fmt={fmt} cols={cols} group={group} "
                  f"rot={rot} full={full}", flush=True)
            fus = dict(residual=res, projection_bias=pb, gate=gate, shift=shift, scale=scale) \
                if full else {}
            q, s, u, raw = orc.layer_norm_quantize(
                x, fmt, norm_weight=nw if full else None, norm_bias=nb if full else None,
                group=group, rotation=rot, src_type=src_type, raw=full,
                rows_per_sequence=rps, **fus)
            d = {k: dev16(v, dtype, dev) for k, v in fus.items()}
            retained = torch.empty((rows, cols), dtype=dtype, device=dev)
            raw_d = torch.empty((rows, cols), dtype=dtype, device=dev) if full else None
            fusion = qlinear.norm_fusion(raw=raw_d, rows_per_sequence=rps, **d)
            qd, sd = qlinear.layer_norm_quantize(
                dev16(x, dtype, dev), fmt, norm_weight=dev16(nw, dtype, dev) if full else None,
                norm_bias=dev16(nb, dtype, dev) if full else None, fusion=fusion,
                retained=retained, group=group, rotation=rot)
            torch.cuda.synchronize()
            assert np.array_equal(bits(retained), u)
            if full:
                assert np.array_equal(bits(raw_d), raw)
            same_codes(qd, q)
            assert np.array_equal(sd.cpu().numpy(), s)


@pytest.mark.parametrize("cols", [2048, 17408])
@pytest.mark.parametrize("fmt", [I8, FP8])
def test_layer_norm_quantize_gather(dev, orc, fmt, cols):
    """source_rows: gathered rows, and NaN rows with unit scales for sources
    outside the input."""
    from breeze_tts_cpp_amd import qlinear
    x_rows = 5
    g = torch.Generator().manual_seed(fmt)
    x, res = mk(g, torch.bfloat16, x_rows, cols, sc=2.0), mk(g, torch.bfloat16, x_rows, cols)
    src = np.array([4, 0, -1, 2, 5, 2, 1], np.int32)
    for group in (0, 128):
        print(f"layer_norm_quantize gather fmt={fmt} group={group}", flush=True)
        q, s, u, _ = orc.layer_norm_quantize(x, fmt, rows=len(src), group=group, residual=res,
                                             source_rows=src)
        retained = torch.empty((len(src), cols), dtype=torch.bfloat16, device=dev)
        src_d = torch.from_numpy(src).to(dev)
        res_d = dev16(res, torch.bfloat16, dev)  # alive across the call
        fusion = qlinear.norm_fusion(residual=res_d, source_rows=src_d)
        qd, sd = qlinear.layer_norm_quantize(dev16(x, torch.bfloat16, dev), fmt, fusion=fusion,
                                             rows=len(src), retained=retained, group=group)
        torch.cuda.synchronize()
        assert np.array_equal(bits(retained), u)
        assert np.array_equal(sd.cpu().numpy(), s)
        valid = (src >= 0) & (src < x_rows)
        same_codes(qd[torch.from_numpy(valid).to(dev)], q[valid])


@pytest.mark.parametrize("dtype,src_type", [(torch.bfloat16, BF16), (torch.float16, F16)])
@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("cols", [9, 256, 1000, 4096, 12288, 16391, 20480])
def test_pointwise_quantize_parity(dev, orc, dtype, src_type, fmt, cols):
    from breeze_tts_cpp_amd import qlinear
    x_rows, repeat, rps, valid = 4, 2, 4, 3
    rows = x_rows * repeat
    g = torch.Generator().manual_seed(cols * 3 + fmt)
    x, b = mk(g, dtype, x_rows, cols, sc=2.0), mk(g, dtype, cols, sc=0.3)
    gate, cond = mk(g, dtype, 2, cols, sc=0.2, off=1.0), mk(g, dtype, 1, cols, sc=0.5)
    res = mk(g, dtype, 3, cols)
    idx = np.array([0, 1, 2, -1, 2, 1, 0, -5], np.int32)
    cases = [dict(activation=a) for a in range(9)] + [
        dict(bias=b, gate=gate, condition=cond, residual=res, residual_index=idx, value_scale=0.75,
             residual_scale=1.5, output_scale=0.5, activation=5, rows_per_sequence=rps,
             valid_rows_per_sequence=valid, input_repeat=repeat),
        dict(bias=b, residual=mk(g, dtype, rows, cols), activation=3, input_repeat=repeat)]
    for case in cases:
        for group, rot in (MODES if case.get("input_repeat") else MODES[:2]):
            if rot and cols % 128:
                continue
            tag = {k: v for k, v in case.items() if not isinstance(v, np.ndarray)}
            print(f"pointwise dtype={dtype} fmt={fmt} cols={cols} group={group} rot={rot} {tag}",
                  flush=True)
            q, s, out, raw = orc.pointwise_quantize(x, fmt, group=group, rotation=rot,
                                                    src_type=src_type, raw=True, **case)
            n_rows = out.shape[0]
            dev_args = {k: (torch.from_numpy(v).to(dev) if k == "residual_index" else
                            dev16(v, dtype, dev)) if isinstance(v, np.ndarray) else v
                        for k, v in case.items()}
            raw_d = torch.empty((n_rows, cols), dtype=dtype, device=dev)
            ep = qlinear.epilogue(raw=raw_d, **dev_args)
            retained = torch.empty((n_rows, cols), dtype=dtype, device=dev)
            qd, sd = qlinear.pointwise_quantize(dev16(x, dtype, dev), fmt, ep, retained=retained,
                                                group=group, rotation=rot)
            torch.cuda.synchronize()
            assert np.array_equal(bits(raw_d), raw)
            assert np.array_equal(bits(retained), out)
            same_codes(qd, q)
            assert np.array_equal(sd.cpu().numpy(), s)


@pytest.mark.parametrize("cols", [2048, 18432])
def test_pointwise_quantize_in_place(dev, orc, cols):
    """retained may replace x row for row (ops::linear's output reuse), also
    for streamed rows."""
    from breeze_tts_cpp_amd import qlinear
    g = torch.Generator().manual_seed(9)
    x = mk(g, torch.bfloat16, 32, cols, sc=2.0)
    b = mk(g, torch.bfloat16, cols, sc=0.3)
    q, s, out, _ = orc.pointwise_quantize(x, I8, bias=b, activation=1)
    xd = dev16(x, torch.bfloat16, dev)
    b_d = dev16(b, torch.bfloat16, dev)  # alive across the call
    ep = qlinear.epilogue(bias=b_d, activation=1)
    qd, sd = qlinear.pointwise_quantize(xd, I8, ep, retained=xd)
    torch.cuda.synchronize()
    assert np.array_equal(bits(xd), out)
    same_codes(qd, q)
    assert np.array_equal(sd.cpu().numpy(), s)


def test_sequence_producers_in_a_graph(dev, orc):
    """Graph capture: LayerNorm -> quant, pointwise -> quant and the LayerNorm
    GEMV captured once on a side stream and replayed four times, with eager
    launches and synchronizations between replays and the inputs changed in
    place; every replay equals the oracle on the current inputs."""
    from breeze_tts_cpp_amd import qlinear
    M, H, k, n = 32, 2048, 512, 256
    g = torch.Generator().manual_seed(17)
    bfd = lambda t: t.to(torch.bfloat16).to(dev)
    x, bias = bfd(torch.randn(M, H, generator=g)), bfd(0.3 * torch.randn(H, generator=g))
    xs = bfd(torch.randn(M, k, generator=g))
    wq_np, sw_np = orc.quantize_rows(bits(bfd(0.05 * torch.randn(n, k, generator=g))), I8)
    wq, sw = torch.from_numpy(wq_np).to(dev), torch.from_numpy(sw_np).to(dev)
    lq = torch.empty((M, H), dtype=torch.uint8, device=dev)
    ls = torch.empty((M,), dtype=torch.float32, device=dev)
    pq = torch.empty((M, H), dtype=torch.uint8, device=dev)
    ps = torch.empty((M,), dtype=torch.float32, device=dev)
    y = torch.empty((M, n), dtype=torch.bfloat16, device=dev)
    ep = qlinear.epilogue(bias=bias, activation=qlinear.ACT_SILU)
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        qlinear.layer_norm_quantize(x, I8, values=lq, scales=ls, stream=stream)
        qlinear.pointwise_quantize(x, I8, ep, values=pq, scales=ps, stream=stream)
        qlinear.norm_linear(xs, wq, sw, I8, out=y, stream=stream)
    for replay in range(4):
        print(f"sequence graph replay {replay}", flush=True)
        with torch.no_grad():
            x.copy_(bfd(torch.randn(M, H, generator=g) * (1 + replay)))
            xs.copy_(bfd(torch.randn(M, k, generator=g)))
        qlinear.row_quantize(x, I8)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        xb, xsb = bits(x), bits(xs)
        q, s, _, _ = orc.layer_norm_quantize(xb, I8)
        same_codes(lq, q)
        assert np.array_equal(ls.cpu().numpy(), s)
        q, s, _, _ = orc.pointwise_quantize(xb, I8, bias=bits(bias), activation=3)
        same_codes(pq, q)
        assert np.array_equal(ps.cpu().numpy(), s)
        yo, _, _, _, _ = orc.norm_linear(xsb, wq_np, sw_np, I8)
        assert np.array_equal(bits(y), yo)


@pytest.mark.parametrize("dtype,src_type", [(torch.bfloat16, BF16), (torch.float16, F16)])
@pytest.mark.parametrize("cols", [9, 2048, 6144, 16391, 20480])
def test_pointwise_dense(dev, orc, dtype, src_type, cols):
    """qlin_pointwise (the reference's ops::pointwise, sequence_pointwise.cu:
    281-287): the epilogue's rows, bit-exact against the oracle's retained
    rows, into a new output and in place, with the raw rows, held in
    registers and streamed (past 16384 columns)."""
    from breeze_tts_cpp_amd import qlinear
    x_rows, repeat, rps, valid = 4, 2, 4, 3
    rows = x_rows * repeat
    g = torch.Generator().manual_seed(cols * 5 + src_type)
    x, b = mk(g, dtype, x_rows, cols, sc=2.0), mk(g, dtype, cols, sc=0.3)
    gate, cond = mk(g, dtype, 2, cols, sc=0.2, off=1.0), mk(g, dtype, 1, cols, sc=0.5)
    res = mk(g, dtype, 3, cols)
    idx = np.array([0, 1, 2, -1, 2, 1, 0, -5], np.int32)
    cases = [dict(activation=a) for a in (0, 2, 3, 5)] + [
        dict(bias=b, gate=gate, condition=cond, residual=res, residual_index=idx, value_scale=0.75,
             residual_scale=1.5, output_scale=0.5, activation=5, rows_per_sequence=rps,
             valid_rows_per_sequence=valid, input_repeat=repeat),
        dict(bias=b, residual=mk(g, dtype, x_rows, cols), activation=3)]
    for case in cases:
        tag = {k: v for k, v in case.items() if not isinstance(v, np.ndarray)}
        print(f"pointwise dense dtype={dtype} cols={cols} {tag}", flush=True)
        _, _, out, raw = orc.pointwise_quantize(x, I8, src_type=src_type, raw=True, **case)
        dev_args = {k: (torch.from_numpy(v).to(dev) if k == "residual_index" else
                        dev16(v, dtype, dev)) if isinstance(v, np.ndarray) else v
                    for k, v in case.items()}
        raw_d = torch.empty(out.shape, dtype=dtype, device=dev)
        ep = qlinear.epilogue(raw=raw_d, **dev_args)
        y = qlinear.pointwise(dev16(x, dtype, dev), ep)
        torch.cuda.synchronize()
        assert np.array_equal(bits(y), out)
        assert np.array_equal(bits(raw_d), raw)
        if case.get("input_repeat", 1) == 1:
            xd = dev16(x, dtype, dev)
            qlinear.pointwise(xd, qlinear.epilogue(**dev_args), out=xd)
            torch.cuda.synchronize()
            assert np.array_equal(bits(xd), out)
