"""qlin_linear_noalloc (scratch in the library's fixed device array) against
qlin_linear (caller-provided scratch): identical output bits, on consecutive
calls that shrink, across the fused decode, two-launch, split-K and prefill
forms, and under HIP graph replay."""
import numpy as np
import pytest
import torch

from breeze_tts_cpp_amd import synthetic

BF16, F32, I32, FP8, I8, F16 = 0, 1, 2, 3, 4, 5
pytestmark = pytest.mark.gpu


def _bits(y):
    return y.cpu().view(torch.int16).numpy().view(np.uint16)


def _operands(dev, orc, M, N, K, fmt, group, rotation, seed):
    xb = synthetic.activations(M, K, seed=seed)
    wq, sw = orc.quantize_rows(synthetic.weights(N, K, seed=seed + 1), fmt, group=group,
                               rotation=rotation)
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev)
    return x, torch.from_numpy(wq).to(dev), torch.from_numpy(sw).to(dev)


# (M, N, K, fmt, group, rotation, explicit skinny split path?)
CASES = [
    (32, 4096, 2048, I8, 0, 0, False),      # one-launch fused decode form
    (8, 2048, 6144, I8, 0, 0, False),       # quantizer + GEMM
    (1024, 2048, 2048, FP8, 0, 0, False),   # prefill (tiled)
    (48, 512, 2048, I8, 128, 128, True),    # K groups, split-K partials in the array
    (16, 256, 1024, FP8, 0, 0, True),       # per-channel split-K
    (3, 64, 512, I8, 0, 0, False),          # tiny, after larger calls
]


@pytest.mark.parametrize("first,second", [(0, 1), (2, 3), (3, 4), (4, 5), (2, 5)])
def test_noalloc_matches_linear(dev, orc, first, second):
    """Two calls in a row, the second smaller: the array keeps the first
    call's contents, which must not leak into the second result."""
    from breeze_tts_cpp_amd import qlinear
    for idx in (first, second):
        M, N, K, fmt, group, rot, split = CASES[idx]
        print(f"noalloc case {idx}: M={M} N={N} K={K} fmt={fmt} group={group} split={split}",
              flush=True)
        x, wq, sw = _operands(dev, orc, M, N, K, fmt, group, rot, seed=idx + 7)
        path = qlinear.Path(qlinear.KIND_SKINNY, 16, 16, 2, 8, 0) if split else None
        ref = qlinear.linear(x, wq, sw, fmt, group, rot, path=path)
        got = qlinear.linear_noalloc(x, wq, sw, fmt, group, rot, path=path)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(got), _bits(ref)), f"case {idx}"


def test_noalloc_rejects_oversize(dev):
    from breeze_tts_cpp_amd import qlinear
    L = qlinear.load()
    cap = int(L.qlin_noalloc_scratch_bytes())
    M, K = 4096, 16384  # 64 MiB of codes
    assert M * K > cap
    x = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    w = torch.empty((16, K), dtype=torch.uint8, device=dev)
    sw = torch.empty(16, dtype=torch.float32, device=dev)
    with pytest.raises(qlinear.QLinearError) as e:
        qlinear.linear_noalloc(x, w, sw, I8)
    assert e.value.status == -3


def test_noalloc_graph_replay(dev, orc):
    """Captured into a graph and replayed with eager work in between: every
    replay equals the eager qlin_linear result."""
    from breeze_tts_cpp_amd import qlinear
    M, N, K = 32, 2048, 2048
    x, wq, sw = _operands(dev, orc, M, N, K, I8, 0, 0, seed=3)
    ref = _bits(qlinear.linear(x, wq, sw, I8))
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        qlinear.linear_noalloc(x, wq, sw, I8, out=out, stream=s)  # eager first call
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        qlinear.linear_noalloc(x, wq, sw, I8, out=out, stream=s)
    other = _operands(dev, orc, 8, 512, 1024, I8, 0, 0, seed=5)
    for _ in range(3):
        out.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(out), ref)
        qlinear.linear_noalloc(*other, I8)  # eager call between replays
        torch.cuda.synchronize()
