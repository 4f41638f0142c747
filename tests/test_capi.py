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
    split = qlinear.Path(qlinear.KIND_SKINNY, 16, 16, 2, 1)
    assert call(K=512, path=split) == -3     # split-K needs a workspace
    assert b"workspace" in L.qlin_last_error()
    assert call(K=512, path=split, ws=FAKE, wsb=10) == -3


def test_plan_and_workspace():
    p = qlinear.plan(32, 4096, 2048, I8)
    assert p.kind in (qlinear.KIND_SKINNY, qlinear.KIND_TILED)
    assert qlinear.workspace_bytes(p, 32, 4096, 2048, I8) >= 0
    split = qlinear.Path(qlinear.KIND_SKINNY, 32, 16, 4, 2)
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
