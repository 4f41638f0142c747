"""The C++ host interface (include/tts_qlinear.hpp), exercised by the compiled
tests/cpp/test_shim program: host-side metadata and validation on the CPU,
and the reference's load-then-serve sequence (weight quantization,
prepare/seal, ops::linear) on the GPU, checked against the oracle."""
import os
import subprocess

import numpy as np
import pytest

from breeze_tts_cpp_amd import synthetic

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "bin", "test_shim")
BF16, F32, I32, FP8, I8, F16 = 0, 1, 2, 3, 4, 5


def _binary():
    if not os.path.exists(BIN):
        subprocess.run(["make", "-C", os.path.join(ROOT, "tests", "cpp")], check=True,
                       stdout=subprocess.DEVNULL)
    return BIN


def test_host_interface():
    r = subprocess.run([_binary(), "host"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr + r.stdout
    assert "host tests: ok" in r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("calls", ["dense", "rowscaled"])
@pytest.mark.parametrize("mode,M,N,K", [("int8", 16, 2048, 2048), ("group_int8", 32, 512, 1024),
                                        ("int8", 300, 384, 512), ("fp8", 8, 256, 2048)])
def test_linear_end_to_end(dev, orc, tmp_path, mode, M, N, K, calls):
    """Load (quantize_rows of the weights, prepare_quantized, seal) then
    serve through ops::linear: a dense input as layers/linear.cpp:246 passes
    it, or an input already quantized as layers/linear.cpp:179 does."""
    xb = synthetic.activations(M, K, seed=M)
    wb = synthetic.weights(N, K, seed=N)
    xb.tofile(tmp_path / "x.bf16")
    wb.tofile(tmp_path / "w.bf16")
    (tmp_path / "shape.txt").write_text(f"{M} {N} {K} {mode}\n")
    (tmp_path / "calls.txt").write_text(f"{calls}\n")
    print(f"test_shim gpu {mode} M={M} N={N} K={K}", flush=True)
    r = subprocess.run([_binary(), "gpu", str(tmp_path)], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr + r.stdout
    fmt = FP8 if "fp8" in mode else I8
    group = 128 if mode.startswith("group") else 0
    y = np.fromfile(tmp_path / "y.bf16", np.uint16).reshape(M, N)
    wq = np.fromfile(tmp_path / "wq.u8", np.uint8).reshape(N, K)
    wq_ref, sw_ref = orc.quantize_rows(wb, fmt, group=group, rotation=group)
    assert np.array_equal(wq, wq_ref)
    assert np.array_equal(np.fromfile(tmp_path / "sw.f32", np.float32), sw_ref.ravel())
    xq, sx = orc.quantize_rows(xb, fmt, group=group, rotation=group)
    if fmt == FP8:
        ideal = orc.gemm_fp8_ideal(xq, sx, wq_ref, sw_ref)
        got = synthetic.bf16_bits_to_f32(y).astype(np.float64)
        assert np.linalg.norm(got - ideal) / np.linalg.norm(ideal) <= 1e-2
    elif group:
        from breeze_tts_cpp_amd import qlinear
        p = qlinear.plan(M, N, K, fmt, group, group)
        splits, waves, span = qlinear.grouped_partition(p, K)
        ref, _ = orc.gemm_grouped(xq, sx, wq_ref, sw_ref, fmt, group, group, splits, waves, span)
        assert np.array_equal(y, ref)
    else:
        ref = orc.epilogue_i8(orc.gemm_i8_acc(xq, wq_ref), sx, sw_ref)
        assert np.array_equal(y, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("M,width,group", [(32, 6144, 0), (5, 6144, 128), (64, 2048, 0)])
def test_producers_end_to_end(dev, orc, tmp_path, M, width, group):
    """ops::quantized_norm (residual update + RMSNorm, hidden 2048) and
    ops::quantized_gated (SiLU over the gate|up output) through the C++
    interface, against the oracle."""
    x = synthetic.activations(M, 2048, seed=M)
    u = synthetic.activations(M, 2048, seed=M + 1)
    w = synthetic.f32_to_bf16_bits(1.0 + 0.05 * np.random.default_rng(M).standard_normal(2048))
    g = synthetic.activations(M, 2 * width, seed=M + 2)
    for name, a in (("x", x), ("u", u), ("w", w), ("g", g)):
        a.tofile(tmp_path / f"{name}.bf16")
    (tmp_path / "shape.txt").write_text(f"{M} {width} {group}\n")
    print(f"test_shim producers M={M} width={width} group={group}", flush=True)
    r = subprocess.run([_binary(), "producers", str(tmp_path)], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr + r.stdout
    rot = 128 if group else 0
    res, nq, ns, _ = orc.quantized_norm(x, w, I8, update_bits=u, eps=1e-6, group=group,
                                        rotation=rot)
    assert np.array_equal(np.fromfile(tmp_path / "res.bf16", np.uint16).reshape(M, 2048), res)
    assert np.array_equal(np.fromfile(tmp_path / "nq.u8", np.uint8).reshape(M, 2048), nq)
    assert np.array_equal(np.fromfile(tmp_path / "ns.f32", np.float32), ns.ravel())
    gq, gs, _ = orc.quantized_gated(g, 0, I8, group=group, rotation=rot)
    assert np.array_equal(np.fromfile(tmp_path / "gq.u8", np.uint8).reshape(M, width), gq)
    assert np.array_equal(np.fromfile(tmp_path / "gs.f32", np.float32), gs.ravel())


@pytest.mark.gpu
@pytest.mark.parametrize("act", [1, 2])
def test_linear_finish_end_to_end(dev, orc, tmp_path, act):
    """ops::linear with a bias + ReLU / tanh-GeLU epilogue: the fused finish
    on the INT8 GEMM, against the oracle GEMM followed by the oracle finish."""
    M, N, K = 32, 512, 1024
    xb = synthetic.activations(M, K, seed=act)
    wb = synthetic.weights(N, K, seed=act)
    bias = synthetic.f32_to_bf16_bits(np.random.default_rng(act).standard_normal(N) * 0.1)
    xb.tofile(tmp_path / "x.bf16")
    wb.tofile(tmp_path / "w.bf16")
    bias.tofile(tmp_path / "bias.bf16")
    (tmp_path / "shape.txt").write_text(f"{M} {N} {K} int8\n")
    (tmp_path / "finish.txt").write_text(f"{act}\n")
    print(f"test_shim gpu finish act={act}", flush=True)
    r = subprocess.run([_binary(), "gpu", str(tmp_path)], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr + r.stdout
    y = np.fromfile(tmp_path / "y.bf16", np.uint16).reshape(M, N)
    wq, sw = orc.quantize_rows(wb, I8)
    xq, sx = orc.quantize_rows(xb, I8)
    plain = orc.epilogue_i8(orc.gemm_i8_acc(xq, wq), sx, sw, order=0)
    assert np.array_equal(y, orc.finish(plain, bias, act))


@pytest.mark.gpu
@pytest.mark.parametrize("activation,use_residual", [(3, 0), (1, 1), (5, 1), (0, 1)])
def test_linear_dense_epilogue_end_to_end(dev, orc, tmp_path, activation, use_residual):
    """ops::linear with a dense output and an epilogue that is no prepared
    finish (SiLU, or a residual, with no finish prepared): the GEMM, then the
    dense pointwise pass in place, as the reference falls back
    (ops/linear.cpp:68-82). Against the oracle GEMM and the oracle epilogue
    of its stored result."""
    M, N, K = 32, 512, 1024
    xb = synthetic.activations(M, K, seed=activation + 9)
    wb = synthetic.weights(N, K, seed=activation + 9)
    rng = np.random.default_rng(activation)
    bias = synthetic.f32_to_bf16_bits(rng.standard_normal(N) * 0.1)
    residual = synthetic.f32_to_bf16_bits(rng.standard_normal((M, N)))
    for name, a in (("x", xb), ("w", wb), ("bias", bias), ("residual", residual)):
        a.tofile(tmp_path / f"{name}.bf16")
    (tmp_path / "shape.txt").write_text(f"{M} {N} {K} int8\n")
    (tmp_path / "dense.txt").write_text(f"{activation} {use_residual}\n")
    print(f"test_shim gpu dense epilogue act={activation} residual={use_residual}", flush=True)
    r = subprocess.run([_binary(), "gpu", str(tmp_path)], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr + r.stdout
    y = np.fromfile(tmp_path / "y.bf16", np.uint16).reshape(M, N)
    wq, sw = orc.quantize_rows(wb, I8)
    xq, sx = orc.quantize_rows(xb, I8)
    plain = orc.epilogue_i8(orc.gemm_i8_acc(xq, wq), sx, sw, order=0)
    _, _, want, _ = orc.pointwise_quantize(plain, I8, bias=bias,
                                           residual=residual if use_residual else None,
                                           activation=activation)
    assert np.array_equal(y, want)


@pytest.mark.gpu
@pytest.mark.parametrize("activation,use_residual", [(1, 0), (5, 0), (3, 1), (6, 0)])
def test_linear_quantized_output_end_to_end(dev, orc, tmp_path, activation, use_residual):
    """ops::linear with a quantized output (ops/linear.cpp:35-78): a bias +
    ReLU / tanh-GeLU epilogue takes the fused finish then quantize_rows; SiLU,
    Mish or a residual take the GEMM then pointwise_quantize. The stored
    output and the next layer's codes/scales against the oracle."""
    M, N, K = 32, 512, 1024
    xb = synthetic.activations(M, K, seed=activation)
    wb = synthetic.weights(N, K, seed=activation)
    rng = np.random.default_rng(activation)
    bias = synthetic.f32_to_bf16_bits(rng.standard_normal(N) * 0.1)
    res = synthetic.f32_to_bf16_bits(rng.standard_normal((M, N)))
    for name, a in (("x", xb), ("w", wb), ("bias", bias), ("residual", res)):
        a.tofile(tmp_path / f"{name}.bf16")
    (tmp_path / "shape.txt").write_text(f"{M} {N} {K} int8\n")
    (tmp_path / "epilogue.txt").write_text(f"{activation} {use_residual}\n")
    print(f"test_shim gpu quantized output act={activation} residual={use_residual}", flush=True)
    r = subprocess.run([_binary(), "gpu", str(tmp_path)], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr + r.stdout
    y = np.fromfile(tmp_path / "y.bf16", np.uint16).reshape(M, N)
    codes = np.fromfile(tmp_path / "next.u8", np.uint8).reshape(M, N)
    scales = np.fromfile(tmp_path / "next_scales.f32", np.float32)
    wq, sw = orc.quantize_rows(wb, I8)
    xq, sx = orc.quantize_rows(xb, I8)
    plain = orc.epilogue_i8(orc.gemm_i8_acc(xq, wq), sx, sw, order=0)
    if activation in (1, 5) and not use_residual:
        assert np.array_equal(y, orc.finish(plain, bias, 1 if activation == 1 else 2))
        q, s = orc.quantize_rows(y, I8)
    else:
        assert np.array_equal(y, plain)
        q, s, _, _ = orc.pointwise_quantize(plain, I8, bias=bias, activation=activation,
                                            residual=res if use_residual else None)
    assert np.array_equal(codes, q)
    assert np.array_equal(scales, s)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 32])
def test_sequence_end_to_end(dev, orc, tmp_path, M):
    """ops::layer_norm_quantize (K128 groups + H128 rotation) feeding
    ops::linear with a quantized input (group_int8 projection), and
    ops::normalized_linear (LayerNorm + residual -> INT8 GEMV), also with the
    next layer's quantized output, through the C++ interface written as the
    reference's layers/linear.cpp calls it, against the oracle."""
    rng = np.random.default_rng(M)
    x = synthetic.activations(M, 2048, seed=M)
    lw = synthetic.f32_to_bf16_bits(1.0 + 0.05 * rng.standard_normal(2048))
    xs = synthetic.activations(M, 512, seed=M + 1)
    rs = synthetic.activations(M, 512, seed=M + 2)
    ws = synthetic.weights(384, 512, seed=M)
    w2 = synthetic.weights(256, 2048, seed=M + 3)
    for name, a in (("x", x), ("lw", lw), ("xs", xs), ("rs", rs), ("ws", ws), ("w2", w2)):
        a.tofile(tmp_path / f"{name}.bf16")
    (tmp_path / "shape.txt").write_text(f"{M}\n")
    print(f"test_shim sequence M={M}", flush=True)
    r = subprocess.run([_binary(), "sequence", str(tmp_path)], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr + r.stdout
    q, s, _, _ = orc.layer_norm_quantize(x, I8, norm_weight=lw, group=128, rotation=128)
    assert np.array_equal(np.fromfile(tmp_path / "lq.u8", np.uint8).reshape(M, 2048), q)
    assert np.array_equal(np.fromfile(tmp_path / "lqs.f32", np.float32), s.ravel())
    wq, sw = orc.quantize_rows(ws, I8)
    assert np.array_equal(np.fromfile(tmp_path / "wq.u8", np.uint8).reshape(384, 512), wq)
    y, nrm, _, _, _ = orc.norm_linear(xs, wq, sw, I8, residual=rs)
    assert np.array_equal(np.fromfile(tmp_path / "norm.bf16", np.uint16).reshape(M, 512), nrm)
    assert np.array_equal(np.fromfile(tmp_path / "y.bf16", np.uint16).reshape(M, 384), y)
    nq, nqs = orc.quantize_rows(y, I8)
    assert np.array_equal(np.fromfile(tmp_path / "next.u8", np.uint8).reshape(M, 384), nq)
    assert np.array_equal(np.fromfile(tmp_path / "next.f32", np.float32), nqs)
    from breeze_tts_cpp_amd import qlinear
    w2q, sw2 = orc.quantize_rows(w2, I8, group=128, rotation=128)
    p = qlinear.plan(M, 256, 2048, I8, 128, 128)
    ref2, _ = orc.gemm_grouped(q, s, w2q, sw2, I8, 128, 128, *qlinear.grouped_partition(p, 2048))
    assert np.array_equal(np.fromfile(tmp_path / "y2.bf16", np.uint16).reshape(M, 256), ref2)
