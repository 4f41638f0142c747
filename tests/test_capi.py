"""C-ABI boundary checks that need no GPU: the library loads, exports every
entry point declared in include/qlinear.h, and rejects invalid requests with
the documented status before touching the device (the reference throws
std::invalid_argument at the same places: ops/basic.cpp:69-78,
ops/cuda/quantization.cpp:94-102,210-222, quant_grouped.cu:225-233)."""
import ctypes
import os
import re

import pytest

from breeze_tts_cpp_amd import qlinear

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BF16, F32, I32, FP8, I8, F16 = 0, 1, 2, 3, 4, 5
FAKE = 0x10000  # never dereferenced: every call below fails validation first


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "qlinear.h")).read()
    return sorted(set(re.findall(r"\b(qlin_[a-z_]+)\s*\(", text)))


def test_header_exports():
    L = qlinear.load()
    names = declared_symbols()
    assert set(names) == set(qlinear.EXPORTS)
    for name in names:
        assert hasattr(L, name), name
    assert L.qlin_version() >= 100


def status_of(fn, *args):
    return fn(*args)


def test_row_quantize_validation():
    L = qlinear.load()
    q = L.qlin_row_quantize
    ok = dict(src=FAKE, ld=128, rows=2, cols=128, st=BF16, v=FAKE, s=FAKE, fmt=I8, g=0, r=0)

    def call(**kw):
        a = dict(ok, **kw)
        return q(a["src"], a["ld"], a["rows"], a["cols"], a["st"], a["v"], a["s"], a["fmt"],
                 a["g"], a["r"], None)

    assert call(st=F32) == -1
    assert call(fmt=BF16) == -1
    assert call(rows=0) == -1
    assert call(ld=64) == -1
    assert call(src=None) == -1
    assert call(g=48) == -1
    assert call(r=64) == -1
    assert call(cols=192, ld=192, r=128) == -1  # rotation needs cols % 128 == 0
    assert call(src=FAKE + 1) == -2
    assert b"rotation" in L.qlin_last_error() or True


def test_gemm_validation():
    L = qlinear.load()

    def call(M=16, N=64, K=256, fmt=I8, out=BF16, ig=0, wg=0, x=FAKE, y=FAKE, ws=None,
             wsb=0, path=None):
        p = ctypes.byref(path.to_c()) if path else None
        return L.qlin_gemm(p, x, FAKE, FAKE, FAKE, y, M, N, K, fmt, out, ig, wg, ws, wsb, None)

    assert call(fmt=BF16) == -1
    assert call(out=F32) == -1
    assert call(K=200) == -1          # K % 16
    assert call(N=40) == -1           # N % 16
    assert call(K=131072) == -1       # INT8 int32 overflow bound
    assert call(ig=48) == -1
    assert call(x=None) == -1
    assert call(x=FAKE + 4) == -2     # 16-byte operand alignment
    assert call(y=FAKE + 2) == -2
    bad = qlinear.Path(qlinear.KIND_SKINNY, 16, 16, 1, 3)
    assert call(path=bad) == -4
    assert call(path=qlinear.Path(qlinear.KIND_SKINNY, 16, 16, 1, 4)) == -4  # eight waves only
    assert call(path=qlinear.Path(qlinear.KIND_SKINNY, 48, 16, 1, 8)) == -4  # token tiles 16/32/64
    split = qlinear.Path(qlinear.KIND_SKINNY, 16, 16, 2, 8)
    assert call(K=512, path=split) == -3     # split-K needs a workspace
    assert b"workspace" in L.qlin_last_error()
    assert call(K=512, path=split, ws=FAKE, wsb=10) == -3
    T = qlinear.KIND_TILED
    assert call(M=256, path=qlinear.Path(T, 128, 128, 1, 4)) == -4          # no 4-wave 128x128 variant
    assert call(M=256, path=qlinear.Path(T, 128, 256, 1, 2), ig=128, wg=128) == -4  # K groups: no 32x32 tiles
    assert call(M=256, path=qlinear.Path(T, 128, 128, 1, 2)) == -4
    assert call(M=256, path=qlinear.Path(T, 64, 128, 1, 1)) == -4           # 128x64: 4 / 8 waves
    assert call(M=256, path=qlinear.Path(T, 64, 128, 1, 8), ig=32, wg=32) == -4  # small groups: no 128x64
    assert call(M=256, path=qlinear.Path(T, 64, 128, 1, 4), ig=32, wg=32) == -4
    assert call(M=256, path=qlinear.Path(T, 128, 128, 1, 1), ig=32, wg=32) == -4  # small groups: 8 waves
    assert call(M=256, fmt=FP8, path=qlinear.Path(T, 128, 256, 1, 8), ig=64, wg=64) == -4  # FP8: 128x128
    # the 512x128 register-streamed path is disabled (not built)
    assert call(M=256, path=qlinear.Path(T, 128, 512, 1, 4)) == -4
    assert b"disabled" in L.qlin_last_error()
    assert call(M=256, path=qlinear.Path(T, 512, 128, 1, 4)) == -4
    # grid limits are checked before any launch: token tiles on the skinny
    # grid's z dimension (<= 65535), macro tiles on the tiled grid's x (< 2^31)
    assert call(M=1 << 23, N=64, K=256, path=qlinear.Path(qlinear.KIND_SKINNY, 64, 16, 1, 8)) == -4
    assert b"65535" in L.qlin_last_error()
    assert call(M=1 << 30, N=1 << 30, K=16) == -4
    assert b"macro tiles" in L.qlin_last_error()


def test_prefill_plan_rules():
    """The measured tile rules on the BASELINE prefill shapes."""
    shapes = {"qkv": (4096, 2048), "o_proj": (2048, 2048), "gate_up": (12288, 2048),
              "down": (2048, 6144)}

    def tile(M, name, fmt, g=0):
        p = qlinear.plan(M, *shapes[name], fmt, g, g)
        return (p.channels, p.tokens, p.waves)
    # INT8: 256x256 from 192 tiles, 256x128 for long K, else the 128x128 tile
    assert tile(4096, "gate_up", I8) == (256, 256, 8) and tile(4096, "down", I8) == (256, 128, 8)
    assert tile(4096, "qkv", I8) == (256, 256, 8) and tile(1024, "gate_up", I8) == (256, 256, 8)
    assert tile(4096, "o_proj", I8) == (128, 128, 8) and tile(1024, "qkv", I8) == (128, 128, 8)
    assert tile(4096, "gate_up", FP8) == (256, 256, 8) and tile(4096, "down", FP8) == (256, 128, 8)
    assert tile(1024, "gate_up", FP8) == (256, 256, 8)   # 192 tiles, as INT8
    assert tile(4096, "o_proj", FP8) == (128, 128, 8)    # K <= 2048: the 128x128 tile, as INT8
    assert tile(4096, "qkv", I8, 128) == (256, 128, 8) and tile(4096, "qkv", FP8, 128) == (256, 128, 8)
    assert tile(1024, "gate_up", I8, 128) == (128, 128, 8) and tile(1024, "gate_up", FP8, 128) == (128, 128, 8)
    assert tile(4096, "qkv", I8, 32) == (256, 128, 8) and tile(4096, "qkv", FP8, 64) == (128, 128, 8)
    assert tile(4096, "down", I8, 128) == (256, 128, 8) and tile(1024, "gate_up", I8, 64) == (128, 128, 8)
    # half-GPU 128x128 grids (o_proj / down at 1024: 128 tiles) take 128x64 tiles
    assert tile(1024, "down", I8) == (128, 64, 8) and tile(1024, "o_proj", FP8) == (128, 64, 8)
    assert tile(1024, "down", I8, 128) == (128, 64, 8) and tile(1024, "o_proj", FP8, 128) == (128, 64, 8)
    assert tile(1024, "down", I8, 32) == (128, 128, 8)  # small groups: no 128x64 tile


def test_plan_and_workspace():
    p = qlinear.plan(32, 4096, 2048, I8)
    assert p.kind in (qlinear.KIND_SKINNY, qlinear.KIND_TILED)
    assert qlinear.workspace_bytes(p, 32, 4096, 2048, I8) >= 0
    split = qlinear.Path(qlinear.KIND_SKINNY, 32, 16, 4, 8)
    assert qlinear.workspace_bytes(split, 32, 4096, 2048, I8) == 4 * 32 * 4096 * 4
    with pytest.raises(qlinear.QLinearError):
        qlinear.plan(0, 16, 16, I8)


def test_decode_grid_plans():
    """Decode planning puts one workgroup on each of the 256 CUs at the
    BASELINE projections (M=32): tiles x token tiles == 256, slab within LDS."""
    for N, K in ((4096, 2048), (2048, 2048), (12288, 2048), (2048, 6144)):
        p = qlinear.plan(32, N, K, I8)
        assert p.kind == qlinear.KIND_SKINNY
        assert (N // p.channels) * (-(-32 // p.tokens)) == 256, (N, K, p)
        assert p.staged


@pytest.mark.parametrize("fmt,group", [(I8, 0), (qlinear.FP8, 0), (I8, 128), (qlinear.FP8, 128)])
def test_decode_grid_plans_m64(fmt, group):
    """At M=64 the weights under 16 MB take the first tiling (16-token tiles
    before 32, fewest weight rows first) that fits 256 workgroups and stages
    its slab in LDS: qkv moves to 32x32 (16x32 would need 512 workgroups),
    down to 32x16 (the 16x32 slab of K=6144 does not fit), o_proj keeps
    16x32."""
    want = {(4096, 2048): (32, 32), (2048, 2048): (16, 32), (2048, 6144): (32, 16)}
    for (N, K), (tokens, channels) in want.items():
        p = qlinear.plan(64, N, K, fmt, group, group)
        assert p.kind == qlinear.KIND_SKINNY
        assert (p.tokens, p.channels) == (tokens, channels), (N, K, p)
        assert (N // p.channels) * (64 // p.tokens) == 256 and p.staged, (N, K, p)


def test_linear_validation():
    """qlin_linear checks its quantize half, then its GEMM half."""
    L = qlinear.load()

    def call(x=FAKE, ld=2048, st=BF16, xq=FAKE, sx=FAKE, M=32, N=4096, K=2048, fmt=I8,
             out=BF16, ig=0, wg=0, rot=0):
        return L.qlin_linear(None, x, ld, st, xq, sx, FAKE, FAKE, FAKE, M, N, K, fmt, out, ig,
                             wg, rot, None, 0, None)

    assert call(xq=None) == -1                 # scratch activation required
    assert b"scratch" in L.qlin_last_error()
    assert call(st=F32) == -1
    assert call(ld=1024) == -1
    assert call(x=None) == -1
    assert call(rot=64) == -1
    assert call(x=FAKE + 1) == -2


def test_quantized_norm_validation():
    """launch_quantized_norm's checks (reference quant_norm.cu:166-180)."""
    L = qlinear.load()

    def call(res=FAKE, upd=None, scl=None, w=FAKE, st=BF16, rows=4, cols=2048, fmt=I8, g=0, r=0,
             v=FAKE, s=FAKE):
        return L.qlin_quantized_norm(res, upd, scl, w, st, rows, cols, 1e-6, 0, v, s, fmt, g, r,
                                     None)

    assert call(st=F32) == -1
    assert call(fmt=BF16) == -1
    assert call(cols=2049) == -1          # the reference's single-CTA row bound
    assert call(cols=0) == -1
    assert call(rows=0) == -1
    assert call(res=None) == -1
    assert call(w=None) == -1
    assert call(scl=FAKE) == -1           # a scale without an update
    assert call(g=48) == -1
    assert call(cols=200, r=128) == -1
    assert call(res=FAKE + 1) == -2
    assert call(s=FAKE + 2) == -2


def test_quantized_gated_validation():
    """launch_quantized_gated's checks (reference quant_gated.cu:182-191)."""
    L = qlinear.load()

    def call(x=FAKE, st=BF16, rows=4, width=6144, kind=0, v=FAKE, s=FAKE, fmt=I8, g=0, r=0):
        return L.qlin_quantized_gated(x, st, rows, width, kind, v, s, fmt, g, r, None)

    assert call(st=F32) == -1
    assert call(fmt=F16) == -1
    assert call(width=8193) == -1
    assert call(width=0) == -1
    assert call(kind=2) == -1
    assert call(x=None) == -1
    assert call(g=16) == -1
    assert call(width=200, r=128) == -1
    assert call(x=FAKE + 1) == -2


def test_sequence_producer_validation():
    """qlin_layer_norm_quantize / qlin_pointwise_quantize / qlin_norm_linear
    reject what the reference's check_quantized_output, check_norm_shape,
    check_epilogue and normalized_quantized_linear reject
    (ops/kernels/sequence/sequence_internal.cuh:154-197, sequence_norm.cu:
    371-397,518-558, sequence_pointwise.cu:307-324)."""
    L = qlinear.load()
    f = qlinear.qlin_norm_fusion()
    L.qlin_norm_fusion_init(ctypes.byref(f))
    assert f.rows_per_sequence == 1 and not f.residual
    e = qlinear.qlin_epilogue()
    L.qlin_epilogue_init(ctypes.byref(e))
    assert (e.value_scale, e.output_scale, e.residual_scale, e.input_repeat) == (1, 1, 1, 1)
    assert abs(e.alpha - 0.1) < 1e-7 and e.activation == 0 and e.rows_per_sequence == 1

    X, V, S = FAKE, FAKE + 0x100000, FAKE + 0x200000

    def ln(x_rows=4, st=BF16, rows=4, cols=256, fmt=I8, g=0, r=0, fusion=None, eps=1e-5, x=X,
           v=V, s=S):
        return L.qlin_layer_norm_quantize(x, x_rows, st, None, None, eps,
                                          None if fusion is None else ctypes.byref(fusion), None,
                                          rows, cols, v, s, fmt, g, r, None)

    assert ln(st=F32) == -1
    assert ln(fmt=BF16) == -1
    assert ln(r=128, g=0) == -1          # rotation requires group scales
    assert ln(g=128, r=128, cols=200) == -1
    assert ln(x_rows=3) == -1            # rows differ without a gather
    assert ln(eps=0.0) == -1
    assert ln(s=V + 16) == -1            # scales overlap the codes
    bad = qlinear.qlin_norm_fusion()
    L.qlin_norm_fusion_init(ctypes.byref(bad))
    bad.rows_per_sequence = 3
    assert ln(fusion=bad) == -1
    bad.rows_per_sequence = 2
    bad.gate, bad.gate_rows = FAKE + 0x300000, 3   # neither 1 nor 4 / 2 sequences
    assert ln(fusion=bad) == -1
    bad.gate_rows = 2
    bad.source_rows = FAKE + 0x400000  # a gather excludes modulation
    assert ln(fusion=bad) == -1
    assert ln(x=X + 1) == -2

    def pw(x_rows=4, rows=4, cols=256, ep=None, g=0, r=0, x=X, ret=None):
        return L.qlin_pointwise_quantize(x, x_rows, BF16, None if ep is None else ctypes.byref(ep),
                                         ret, rows, cols, V, S, I8, g, r, None)

    assert pw(rows=5) == -1
    assert pw(r=128) == -1
    ep = qlinear.epilogue(input_repeat=2)
    assert pw(ep=ep) == -1                # x_rows * repeat != rows
    assert pw(ep=ep, rows=8, ret=X) == -1  # repeated rows cannot update x in place
    ep = qlinear.epilogue(activation=9)
    assert pw(ep=ep) == -1
    ep = qlinear.epilogue(rows_per_sequence=4, valid_rows_per_sequence=5)
    assert pw(ep=ep) == -1
    ep = qlinear.epilogue()
    ep.residual, ep.residual_rows = FAKE + 0x300000, 3   # dense residual must match rows
    assert pw(ep=ep) == -1
    ep = qlinear.epilogue(rows_per_sequence=2)
    ep.condition, ep.condition_rows = FAKE + 0x300000, 3
    assert pw(ep=ep) == -1

    def nl(k=256, n=64, act=0, fusion=None, y=FAKE + 0x500000):
        return L.qlin_norm_linear(X, None if fusion is None else ctypes.byref(fusion), None, None,
                                  BF16, 4, k, 1e-5, FAKE + 0x600000, FAKE + 0x700000, I8, n, None,
                                  act, y, None, None, None, None)

    assert nl(k=513) == -1
    assert nl(k=6) == -1
    assert nl(act=2) == -1
    gather = qlinear.qlin_norm_fusion()
    L.qlin_norm_fusion_init(ctypes.byref(gather))
    gather.source_rows = FAKE + 0x400000
    assert nl(fusion=gather) == -1
    assert nl(y=X + 2) == -1              # output overlaps the input


def test_noalloc_scratch_limit():
    """qlin_linear_noalloc rejects a shape whose scratch exceeds its fixed
    array before touching the device."""
    L = qlinear.load()
    assert L.qlin_noalloc_scratch_bytes() == 32 << 20
    rc = L.qlin_linear_noalloc(None, FAKE, 16384, BF16, FAKE, FAKE, FAKE, 4096, 16, 16384, I8,
                               BF16, 0, 0, 0, None)
    assert rc == -3 and b"fixed" in L.qlin_last_error()
    # an invalid group is rejected as qlin_linear rejects it, before it sizes
    # the scratch layout
    for ig, wg in ((-1, 0), (96, 128), (128, -128)):
        rc = L.qlin_linear_noalloc(None, FAKE, 2048, BF16, FAKE, FAKE, FAKE, 16, 2048, 2048, I8,
                                   BF16, ig, wg, 0, None)
        assert rc == -1 and b"group" in L.qlin_last_error(), (ig, wg)


def test_measure_library():
    """The streaming-read measurement kernel lives in its own library
    (include/qlin_measure.h), outside the quantized linear ABI, and rejects
    unaligned or ragged buffers before launching."""
    from breeze_tts_cpp_amd import measure
    text = open(os.path.join(ROOT, "include", "qlin_measure.h")).read()
    assert sorted(set(re.findall(r"\b(qlm_[a-z_]+)\s*\(", text))) == ["qlm_stream_read"]
    assert not hasattr(qlinear.load(), "qlin_stream_read")
    L = measure.load()
    assert L.qlm_stream_read(FAKE + 8, 1 << 20, None, None) == -1
    assert L.qlm_stream_read(FAKE, (1 << 20) + 4, None, None) == -1
    assert L.qlm_stream_read(FAKE, 0, None, None) == -1
    assert L.qlm_stream_read(None, 1 << 20, None, None) == -1