"""The core path inside a HIP graph, as bench.py and a serving loop run it: the
linear (quantize + decode GEMM, split-K with a workspace, K-group FP8), the
prefill GEMM with the fused finish, packed weights, and the fused norm and
gated producers, captured once on a side stream and replayed four times with
the inputs changed in place and eager launches between replays. Every
replay's outputs equal an eager run on the same inputs, bit for bit (the
eager path is the one the parity tests pin against the oracle)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
I8, FP8 = 4, 3


def bits(t):
    return t.contiguous().view(torch.int16 if t.element_size() == 2 else torch.uint8).cpu().numpy()


def test_core_path_in_a_graph(dev):
    from breeze_tts_cpp_amd import qlinear
    from breeze_tts_cpp_amd.qlinear import Path, KIND_SKINNY
    g = torch.Generator().manual_seed(23)
    bf = lambda *s, sc=1.0: (sc * torch.randn(*s, generator=g)).to(torch.bfloat16).to(dev)
    M, Mp, N, K, W = 32, 512, 1024, 2048, 2048
    x, xp, res, upd = bf(M, K), bf(Mp, K), bf(M, K), bf(M, K)
    nw, gu, bias = bf(K, sc=0.1) + 1, bf(M, 2 * W, sc=2.0), bf(N, sc=0.3)
    wq, sw = qlinear.row_quantize(bf(N, K, sc=0.05), I8)
    wq8, sw8 = qlinear.row_quantize(bf(N, K, sc=0.05), FP8, group=128, rotation=128)
    packed = qlinear.pack_weights(wq)
    torch.cuda.synchronize()
    split = Path(KIND_SKINNY, 32, 16, 2, 8)
    ws = torch.empty(qlinear.workspace_bytes(split, M, N, K, I8), dtype=torch.uint8, device=dev)
    outs = {k: torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            for k in ("planned", "split", "packed", "grouped")}
    yp = torch.empty((Mp, N), dtype=torch.bfloat16, device=dev)
    nq = torch.empty((M, K), dtype=torch.uint8, device=dev)
    ns = torch.empty((M,), dtype=torch.float32, device=dev)
    gq = torch.empty((M, W), dtype=torch.uint8, device=dev)
    gs = torch.empty((M,), dtype=torch.float32, device=dev)
    xpq, xps = qlinear.row_quantize(xp, I8)
    res0 = res.clone()
    stream = torch.cuda.Stream()

    def run(o, y_prefill, nqv, nsv, gqv, gsv, s):
        qlinear.linear(x, wq, sw, I8, out=o["planned"], stream=s)
        qlinear.linear(x, wq, sw, I8, path=split, workspace=ws, out=o["split"], stream=s)
        qlinear.linear(x, packed, sw, I8, out=o["packed"], stream=s)
        qlinear.linear(x, wq8, sw8, FP8, group=128, rotation=128, out=o["grouped"], stream=s)
        qlinear.gemm_finish(xpq, xps, wq, sw, I8, bias=bias, activation=2, out=y_prefill,
                            stream=s)
        qlinear.quantized_norm(res, nw, I8, update=upd, values=nqv, scales=nsv, stream=s)
        qlinear.quantized_gated(gu, I8, kind=0, values=gqv, scales=gsv, stream=s)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        run(outs, yp, nq, ns, gq, gs, stream)
    for replay in range(4):
        print(f"core graph replay {replay}", flush=True)
        with torch.no_grad():
            x.copy_(bf(M, K, sc=1 + replay))
            gu.copy_(bf(M, 2 * W, sc=2.0))
            res.copy_(res0)
        qlinear.row_quantize(xp, I8)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = {k: bits(v) for k, v in outs.items()}
        got.update(prefill=bits(yp), nq=bits(nq), ns=ns.cpu().numpy(), gq=bits(gq),
                   gs=gs.cpu().numpy(), res=bits(res))
        # the same work eagerly on the same inputs
        with torch.no_grad():
            res.copy_(res0)
        eo = {k: torch.empty_like(v) for k, v in outs.items()}
        eyp, enq, ens = torch.empty_like(yp), torch.empty_like(nq), torch.empty_like(ns)
        egq, egs = torch.empty_like(gq), torch.empty_like(gs)
        torch.cuda.synchronize()
        run(eo, eyp, enq, ens, egq, egs, torch.cuda.current_stream())
        torch.cuda.synchronize()
        for k, v in eo.items():
            assert np.array_equal(got[k], bits(v)), (replay, k)
        assert np.array_equal(got["prefill"], bits(eyp)), replay
        assert np.array_equal(got["nq"], bits(enq)) and np.array_equal(got["ns"], ens.cpu().numpy())
        assert np.array_equal(got["gq"], bits(egq)) and np.array_equal(got["gs"], egs.cpu().numpy())
        assert np.array_equal(got["res"], bits(res)), replay
        with torch.no_grad():
            res.copy_(res0)
        torch.cuda.synchronize()
