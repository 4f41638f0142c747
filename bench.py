"""Benchmark of the MI355X quantized linear path (BASELINE.json metric:
"INT8/FP8 GEMM TOPS @M=4096 + HBM GB/s @M=32, % of MI355X roofline").

One step = one decode step (M=32 tokens) through the INT8 quantized
projections of a 16-layer 1B-class decoder (hidden 2048, QKV N=4096,
o_proj N=2048, gate_up N=12288, down K=6144; BASELINE config 1 at M=32):
per projection, the quantized branch of ops::linear (qlin_linear): dynamic
per-token activation quantization of the bf16 input into the scratch
activation, then the INT8 GEMM with fused dequant to bf16. The 16 layers hold
distinct weights
(805 MB of int8), so HBM, not the 256 MB Infinity Cache, serves them.
Inputs are resident in HBM before the timed region. The step is captured once
as a HIP graph and replayed.

value = algorithmic bytes per step / step time (GB/s), with per projection
B = N*K + M*K + 4N + 4M + 2*M*N (GEMM) + 3*M*K + 4*M (quantizer).
Also reported: per-projection decode GB/s, prefill (M=4096) INT8/FP8/group TOPS,
the roofline fraction of the dominant kernel and a CPU baseline (the oracle's
multithreaded C restatement) on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
I8_PEAK_TOPS = 5000.0
FP8_PEAK_TFLOPS = 5000.0
LAYERS = 16
M_DECODE = 32
M_PREFILL = 4096


def progress(message):
    """One progress line on stderr (the JSON result goes to stdout)."""
    print(f"[bench {time.strftime('%H:%M:%S')}] {message}", file=sys.stderr, flush=True)


def gemm_bytes(M, N, K, group=0):
    scales = 4 * N * K // group + 4 * M * K // group if group else 4 * N + 4 * M
    return N * K + M * K + scales + 2 * M * N


def quant_bytes(M, K, group=0):
    return 3 * M * K + (4 * M * K // group if group else 4 * M)



def bench_decoder_layer(torch, qlinear, synthetic, dev, stream, layers, args):
    """The same 16 layers' weights in the reference decoder's call order
    (decoder.h:242,271-275,292) at M=32, INT8: residual + RMSNorm -> quant
    (qlin_quantized_norm) -> qkv GEMM; o_proj as a linear (quantize + GEMM);
    residual + RMSNorm -> quant -> gate_up GEMM; SiLU(gate)*up -> quant
    (qlin_quantized_gated) -> down GEMM. Attention itself is outside the path
    (its output is a fixed synthetic tensor). One captured graph of the 16
    layers, timed like the step; bytes = the GEMMs' operands and outputs plus
    each producer's algorithmic bytes."""
    M, H, W = M_DECODE, 2048, 6144
    I8 = qlinear.I8

    def bf(rows, cols, seed):
        return torch.from_numpy(synthetic.activations(rows, cols, seed=seed).view(np.int16)).view(
            torch.bfloat16).to(dev)

    residual, attn = bf(M, H, 11), bf(M, H, 12)
    norm_w = torch.ones(H, dtype=torch.bfloat16, device=dev)
    buf = {
        "xq_h": torch.empty((M, H), dtype=torch.uint8, device=dev),
        "sx": torch.empty((M,), dtype=torch.float32, device=dev),
        "xq_w": torch.empty((M, W), dtype=torch.uint8, device=dev),
        "qkv": torch.empty((M, 4096), dtype=torch.bfloat16, device=dev),
        "o": torch.empty((M, H), dtype=torch.bfloat16, device=dev),
        "gu": torch.empty((M, 2 * W), dtype=torch.bfloat16, device=dev),
        "down": torch.empty((M, H), dtype=torch.bfloat16, device=dev),
    }
    paths = {n: qlinear.plan(M, N, K, I8) for n, (N, K) in synthetic.PROJECTIONS.items()}

    def layer(entry):
        qlinear.quantized_norm(residual, norm_w, I8, update=buf["down"], values=buf["xq_h"],
                               scales=buf["sx"], stream=stream)
        qlinear.gemm(buf["xq_h"], buf["sx"], entry["qkv"]["wq"], entry["qkv"]["sw"], I8,
                     path=paths["qkv"], out=buf["qkv"], stream=stream)
        qlinear.linear(attn, entry["o_proj"]["wq"], entry["o_proj"]["sw"], I8,
                       path=paths["o_proj"], scratch=(buf["xq_h"], buf["sx"]), out=buf["o"],
                       stream=stream)
        qlinear.quantized_norm(residual, norm_w, I8, update=buf["o"], values=buf["xq_h"],
                               scales=buf["sx"], stream=stream)
        qlinear.gemm(buf["xq_h"], buf["sx"], entry["gate_up"]["wq"], entry["gate_up"]["sw"], I8,
                     path=paths["gate_up"], out=buf["gu"], stream=stream)
        qlinear.quantized_gated(buf["gu"], I8, kind=0, values=buf["xq_w"], scales=buf["sx"],
                                stream=stream)
        qlinear.gemm(buf["xq_w"], buf["sx"], entry["down"]["wq"], entry["down"]["sw"], I8,
                     path=paths["down"], out=buf["down"], stream=stream)

    buf["down"].zero_()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for entry in layers:
            layer(entry)
    torch.cuda.synchronize()
    for _ in range(max(3, args.warmup)):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(args.steps):
            graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    gemms = sum(gemm_bytes(M, N, K) for _, (N, K) in synthetic.PROJECTIONS.items())
    norm = 7 * M * H + 2 * H + 4 * M
    gated = 5 * M * W + 4 * M
    layer_bytes = gemms + quant_bytes(M, H) + 2 * norm + gated
    return {"ms_per_step": round(ms, 4), "us_per_layer": round(ms * 1e3 / len(layers), 2),
            "GBps": round(layer_bytes * len(layers) / (ms * 1e-3) / 1e9, 1),
            "layer_bytes": layer_bytes,
            "sequence": "norm->quant, qkv GEMM, o_proj linear, norm->quant, gate_up GEMM, "
                        "SiLU*up->quant, down GEMM"}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--profile", action="store_true",
                    help="short run for rocprofv3 counter passes: a 64 MiB device copy "
                         "(calibrates FETCH_SIZE/WRITE_SIZE), then the decode GEMM graphs "
                         "and one prefill GEMM per format; prints no JSON")
    ap.add_argument("--vendor", action="store_true",
                    help="only the M=4096 comparison with the vendor library's GEMMs "
                         "(hipBLASLt through torch._int_mm / torch._scaled_mm) on the same "
                         "quantized operands; prints one JSON line")
    return ap.parse_args()


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the quantized linear path has no multi-GPU "
              "component in this build; --gpus N with N > 1 is not supported.", file=sys.stderr)
        sys.exit(2)
    import torch

    from breeze_tts_cpp_amd import qlinear, synthetic

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream()
    I8, FP8 = qlinear.I8, qlinear.FP8
    if args.vendor:
        print(json.dumps({"vendor_compare": vendor_compare(torch, qlinear, synthetic, dev,
                                                           stream)}), flush=True)
        return
    projections = list(synthetic.PROJECTIONS.items())

    def bf16_dev(bits):
        return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(dev)

    # ---- operands: 16 layers of distinct int8 weights, quantized on the GPU
    # (load-time weight quantization, io/weights.cpp:80-87).
    layers = []
    with torch.cuda.stream(stream):
        for layer in range(LAYERS):
            entry = {}
            for name, (N, K) in projections:
                wb = synthetic.weights(N, K, seed=1000 + layer) if layer < 2 else None
                if wb is None:  # later layers: cheap distinct weights derived on device
                    base = layers[layer % 2][name]["w_bf16"]
                    w = (base * (1.0 + 0.001 * layer)).contiguous()
                else:
                    w = bf16_dev(wb)
                wq, sw = qlinear.row_quantize(w, I8, stream=stream)
                entry[name] = {"wq": wq, "sw": sw, "N": N, "K": K,
                               "w_bf16": w if layer < 2 else None}
            layers.append(entry)
    torch.cuda.synchronize()
    for entry in layers:
        for v in entry.values():
            v["w_bf16"] = None

    inputs = {}
    for name, (N, K) in projections:
        x = bf16_dev(synthetic.activations(M_DECODE, K, seed=0))
        inputs[name] = {"x": x,
                        "xq": torch.empty((M_DECODE, K), dtype=torch.uint8, device=dev),
                        "sx": torch.empty((M_DECODE,), dtype=torch.float32, device=dev),
                        "y": torch.empty((M_DECODE, N), dtype=torch.bfloat16, device=dev),
                        "path": qlinear.plan(M_DECODE, N, K, I8)}
    for name in inputs:
        p = inputs[name]["path"]
        need = qlinear.workspace_bytes(p, M_DECODE, *synthetic.PROJECTIONS[name], I8)
        inputs[name]["ws"] = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)

    def linear(io, wt):
        qlinear.linear(io["x"], wt["wq"], wt["sw"], I8, path=io["path"],
                       scratch=(io["xq"], io["sx"]), out=io["y"], workspace=io["ws"],
                       stream=stream)

    def step():
        for entry in layers:
            for name, _ in projections:
                linear(inputs[name], entry[name])

    if args.profile:
        profile_run(torch, qlinear, synthetic, dev, stream, layers, inputs, projections)
        return

    # eager reference of one step, then capture the step as a graph
    with torch.cuda.stream(stream):
        step()
    torch.cuda.synchronize()
    eager = {n: inputs[n]["y"].clone() for n in inputs}
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step()
    torch.cuda.synchronize()
    for n in inputs:
        inputs[n]["y"].zero_()
    graph.replay()
    torch.cuda.synchronize()
    for n in inputs:
        assert torch.equal(inputs[n]["y"], eager[n]), f"graph replay differs from eager ({n})"

    progress("decode step")
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(args.steps):
            graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    ms_per_step = start.elapsed_time(end) / args.steps

    step_bytes = LAYERS * sum(gemm_bytes(M_DECODE, N, K) + quant_bytes(M_DECODE, K)
                              for _, (N, K) in projections)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    progress("decoder layer")
    decoder_layer = bench_decoder_layer(torch, qlinear, synthetic, dev, stream, layers, args)

    # ---- per projection, per format and token count: graphs that rotate
    # through >= 640 MB of distinct weights (so HBM, not the 256 MB Infinity
    # Cache, serves them), timed with events on the launch stream: the GEMM on
    # the quantized activations (the dominant kernel) and the whole linear.
    per_proj = {}
    sweep = {}
    for mode, fmt, group, tokens in (("int8", I8, 0, M_DECODE), ("int8", I8, 0, 1),
                                     ("int8", I8, 0, 8), ("int8", I8, 0, 64),
                                     ("fp8", FP8, 0, M_DECODE),
                                     ("group_int8", I8, 128, M_DECODE),
                                     ("group_fp8", FP8, 128, M_DECODE)):
        progress(f"decode sweep {mode} M={tokens}")
        rows = decode_sweep(torch, qlinear, synthetic, dev, stream, fmt, group, tokens,
                            max(5, args.steps // 5))
        if mode == "int8" and tokens == M_DECODE:
            per_proj = rows
        sweep[f"{mode} M={tokens}"] = {
            n: {"gemm_us": r["us_per_launch"], "linear_us": r["linear_us"], "GBps": r["GBps"],
                "frac_hbm": r["frac_hbm"], "stream_us": r["stream_us"], "warm_us": r["warm_us"],
                "frac_of_stream": r["frac_of_stream"], "path": r["path"]}
            for n, r in rows.items()}
    # the dominant kernel: the projection that moves the most bytes (gate_up)
    dominant = max(per_proj, key=lambda n: per_proj[n]["bytes"])
    d = per_proj[dominant]
    roofline = {"bound": "hbm", "kernel": f"skinny_gemm INT8 {dominant} M={M_DECODE}",
                "achieved": d["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(d["GBps"] / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic(dominant),
                "bytes_per_launch": d["bytes"],
                "stream_ceiling_us": d["stream_us"], "frac_of_stream": d["frac_of_stream"]}

    result = {
        "metric": "INT8/FP8 GEMM TOPS @M=4096 + HBM GB/s @M=32, % of MI355X roofline",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,1) activations with 0.5% x20 outlier channels, "
                "N(0,0.02) weights; bf16)",
        "config": {"workload": f"decode step M={M_DECODE}: {LAYERS} layers x "
                               "(qkv 4096x2048, o_proj 2048x2048, gate_up 12288x2048, "
                               "down 2048x6144), per-token INT8 quant + INT8 GEMM + bf16 "
                               "(qlin_linear)",
                   "tokens": M_DECODE, "layers": LAYERS, "format": "int8",
                   "step_bytes": step_bytes},
        "decode_projections": per_proj,
        "decoder_layer": decoder_layer,
        "decode_sweep": sweep,
        "roofline": roofline,
    }

    gpu_prefill_qkv = None
    if not args.no_prefill:
        progress("prefill M=4096")
        detail = bench_prefill(torch, qlinear, synthetic, dev, stream, args)
        # the metric's prefill half as flat scalars, the per-projection rows
        # under prefill_detail
        result["prefill"] = {"M": M_PREFILL}
        for mode, leg in detail.items():
            unit = "TOPS" if mode.endswith("int8") else "TFLOPS"
            result["prefill"][f"{mode}_{unit}"] = leg["TOPS"]
            result["prefill"][f"{mode}_frac_mfma"] = leg["frac_mfma"]
        result["prefill_detail"] = detail
        g = detail["int8"]["projections"]["gate_up"]
        gpu_prefill_qkv = detail["int8"]["projections"]["qkv"]["TOPS"]
        achieved = g["TOPS"]
        result["roofline_mfma"] = {
            "bound": "mfma", "kernel": f"tiled_gemm INT8 gate_up M={M_PREFILL}",
            "achieved": achieved, "peak": I8_PEAK_TOPS, "unit": "TOPS",
            "frac": round(achieved / I8_PEAK_TOPS, 4), "us_per_launch": g["us"],
            "ops_per_launch": 2 * M_PREFILL * g["N"] * g["K"],
            "traffic": measured_prefill_traffic("INT8 gate_up")}
        progress("prefill M=1024")
        result["prefill_m1024"] = bench_prefill(torch, qlinear, synthetic, dev, stream, args,
                                                M=1024)
        progress("producers")
        result["producers"] = bench_producers(torch, qlinear, synthetic, dev, stream, args)

    if not args.no_cpu:
        progress("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(args, value, gpu_prefill_qkv)

    print(json.dumps(result), flush=True)


def decode_sweep(torch, qlinear, synthetic, dev, stream, fmt, group, M, reps):
    """Per projection at M tokens: the GEMM alone and the linear (quantize +
    GEMM, qlin_linear) over distinct weight copies totalling >= 640 MB, each
    graph replayed `reps` times; microseconds per launch. Also the GEMM warm
    (one weight copy, cache-resident) and the streaming-read ceiling over the
    same copies."""
    from breeze_tts_cpp_amd import measure
    rot = 128 if group else 0
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def time_graph(launch, per):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            launch()
        torch.cuda.synchronize()
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            start.record(stream)
            for _ in range(reps):
                g.replay()
            end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) * 1e3 / (reps * per)

    rows = {}
    for name, (N, K) in synthetic.PROJECTIONS.items():
        w = torch.from_numpy(synthetic.weights(N, K, seed=1000).view(np.int16)).view(
            torch.bfloat16).to(dev)
        x = torch.from_numpy(synthetic.activations(M, K, seed=0).view(np.int16)).view(
            torch.bfloat16).to(dev)
        with torch.cuda.stream(stream):
            wq, sw = qlinear.row_quantize(w, fmt, group=group, rotation=rot, stream=stream)
            xq, sx = qlinear.row_quantize(x, fmt, group=group, rotation=rot, stream=stream)
        torch.cuda.synchronize()
        del w
        # distinct copies: the codes with one byte pattern flipped per copy
        # (same sizes and scale layout; the data only has to be distinct)
        copies = max(16, -(-(640 << 20) // (N * K)))
        ws = [wq] + [torch.bitwise_xor(wq, (c * 37) & 0x7f) for c in range(1, copies)]
        path = qlinear.plan(M, N, K, fmt, group, group)
        need = qlinear.workspace_bytes(path, M, N, K, fmt, group, group)
        wsp = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        xs, ss = torch.empty_like(xq), torch.empty_like(sx)
        us = time_graph(lambda: [qlinear.gemm(xq, sx, wc, sw, fmt, input_group=group,
                                              weight_group=group, path=path, out=y,
                                              workspace=wsp, stream=stream) for wc in ws],
                        len(ws))
        us_linear = time_graph(lambda: [qlinear.linear(x, wc, sw, fmt, group, rot, path=path,
                                                       scratch=(xs, ss), out=y, workspace=wsp,
                                                       stream=stream) for wc in ws], len(ws))
        # warm (cache-resident): the first copy 16 times in a row, so L2 and
        # the Infinity Cache serve the weights after the first launch
        us_warm = time_graph(lambda: [qlinear.gemm(xq, sx, ws[0], sw, fmt, input_group=group,
                                                   weight_group=group, path=path, out=y,
                                                   workspace=wsp, stream=stream)
                                      for _ in range(16)], 16)
        # the streaming-read ceiling: the same weight copies read once each
        # by the plain 16-byte-load kernel (qlin_stream_read), same replay
        us_stream = time_graph(lambda: [measure.stream_read(wc, stream=stream) for wc in ws],
                               len(ws))
        b = gemm_bytes(M, N, K, group)
        rows[name] = {"N": N, "K": K, "us_per_launch": round(us, 3), "bytes": b,
                      "GBps": round(b / (us * 1e-6) / 1e9, 1),
                      "frac_hbm": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                      "path": [path.kind, path.tokens, path.channels, path.splits, path.waves,
                               path.staged],
                      "linear_us": round(us_linear, 3), "weight_copies": copies,
                      "stream_us": round(us_stream, 3), "warm_us": round(us_warm, 3),
                      "frac_of_stream": round(us_stream / us, 4)}
        del ws
        torch.cuda.empty_cache()
    return rows


def measured_traffic(name):
    """HBM bytes per launch of the decode linear for projection `name`, from the
    committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary
    (profiles/hbm_traffic_decode_linear.md, copy-kernel calibrated: a row per
    projection in its first table, the last column the scaled bytes per
    dispatch; the later streaming-read table, whose rows carry the same
    projection names, is not read); None when that summary has no row for
    it."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_decode_linear.md")
    if not os.path.exists(path):
        return None
    found = None
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        # rows are labelled by projection, optionally followed by a note in
        # parentheses ("qkv (one launch)"); the first matching row is the
        # decode linear's
        if len(cells) >= 3 and cells[0].split(" (")[0] == name:
            try:
                found = int(cells[-1].replace(",", ""))
            except ValueError:
                found = None
            break
    return found


def measured_prefill_traffic(label):
    """HBM bytes per launch (scaled FETCH_SIZE + WRITE_SIZE) of the prefill
    GEMM labelled `label` ("INT8 gate_up", ...) in the committed counter
    summary profiles/mfma_util_prefill.md (its last two columns); None when
    the summary has no such row."""
    path = os.path.join(ROOT, "profiles", "mfma_util_prefill.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 3 and cells[0] == label:
            try:
                return int(cells[-2].replace(",", "")) + int(cells[-1].replace(",", ""))
            except ValueError:
                return None
    return None


def profile_run(torch, qlinear, synthetic, dev, stream, layers, inputs, projections):
    """Kernels for counter passes, in this order: one 64 MiB copy (known
    traffic: 64 MiB read + 64 MiB written), the streaming-read kernel over 16
    copies of each projection's weight bytes (two passes), 5 rounds of each projection's
    16-layer decode linear (qlin_linear, fused at M=32), then one M=4096 INT8,
    FP8, group_int8 and group_fp8 GEMM per projection."""
    from breeze_tts_cpp_amd import measure
    src = torch.empty(64 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    # the streaming-read ceiling kernel over each projection's weight bytes,
    # 16 distinct copies each (so they come from HBM)
    for name, (N, K) in projections:
        copies = [torch.empty(N * K, dtype=torch.uint8, device=dev).fill_(c) for c in range(16)]
        torch.cuda.synchronize()
        # two passes: the first also pays for writing the fills' dirty lines
        # back from the caches; the second is the measurement
        for _ in range(2):
            for buf in copies:
                measure.stream_read(buf, stream=stream)
            torch.cuda.synchronize()
        del copies
    for name, (N, K) in projections:
        io = inputs[name]
        for _ in range(5):
            for entry in layers:
                qlinear.linear(io["x"], entry[name]["wq"], entry[name]["sw"], qlinear.I8,
                               path=io["path"], scratch=(io["xq"], io["sx"]), out=io["y"],
                               stream=stream)
    torch.cuda.synchronize()
    M = M_PREFILL
    for fmt, group in ((qlinear.I8, 0), (qlinear.FP8, 0), (qlinear.I8, 128), (qlinear.FP8, 128)):
        rot = 128 if group else 0
        for name, (N, K) in projections:
            x = torch.from_numpy(synthetic.activations(M, K, seed=1).view(np.int16)).view(
                torch.bfloat16).to(dev)
            w = torch.from_numpy(synthetic.weights(N, K, seed=1).view(np.int16)).view(
                torch.bfloat16).to(dev)
            xq, sx = qlinear.row_quantize(x, fmt, group=group, rotation=rot, stream=stream)
            wq, sw = qlinear.row_quantize(w, fmt, group=group, rotation=rot, stream=stream)
            qlinear.gemm(xq, sx, wq, sw, fmt, input_group=group, weight_group=group,
                         stream=stream)
            torch.cuda.synchronize()


def bench_prefill(torch, qlinear, synthetic, dev, stream, args, M=M_PREFILL):
    """M=4096 INT8, FP8, group_int8 and group_fp8 GEMMs over the four
    projections: TOPS = 2*M*N*K / kernel time. Per format, the four projections'
    graphs (10 GEMMs each) are built, warmed up together for about 30 replays
    each (the clock settles upward under sustained MFMA load), then timed in
    5 interleaved rounds of 3 replays; each projection reports its median."""
    import statistics
    out = {}
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps, rounds, per_round = 10, 5, 3
    modes = (("int8", qlinear.I8, 0), ("fp8", qlinear.FP8, 0), ("group_int8", qlinear.I8, 128),
             ("group_fp8", qlinear.FP8, 128))
    for fmt_name, fmt, group in modes:
        legs = {}
        rot = 128 if group else 0
        for name, (N, K) in synthetic.PROJECTIONS.items():
            x = torch.from_numpy(synthetic.activations(M, K, seed=1).view(np.int16)).view(
                torch.bfloat16).to(dev)
            w = torch.from_numpy(synthetic.weights(N, K, seed=1).view(np.int16)).view(
                torch.bfloat16).to(dev)
            with torch.cuda.stream(stream):
                xq, sx = qlinear.row_quantize(x, fmt, group=group, rotation=rot, stream=stream)
                wq, sw = qlinear.row_quantize(w, fmt, group=group, rotation=rot, stream=stream)
                y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
                path = qlinear.plan(M, N, K, fmt, group, group)
                need = qlinear.workspace_bytes(path, M, N, K, fmt, group, group)
                ws = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for _ in range(reps):
                    qlinear.gemm(xq, sx, wq, sw, fmt, input_group=group, weight_group=group,
                                 path=path, out=y, workspace=ws, stream=stream)
            legs[name] = {"graph": g, "N": N, "K": K, "path": path, "keep": (xq, sx, wq, sw, y, ws),
                          "us": []}
            del x, w
        torch.cuda.synchronize()
        for _ in range(30):
            for leg in legs.values():
                leg["graph"].replay()
        torch.cuda.synchronize()
        for r in range(rounds):
            order = list(legs) if r % 2 == 0 else list(reversed(legs))
            for name in order:
                with torch.cuda.stream(stream):
                    start.record(stream)
                    for _ in range(per_round):
                        legs[name]["graph"].replay()
                    end.record(stream)
                torch.cuda.synchronize()
                legs[name]["us"].append(start.elapsed_time(end) * 1e3 / (per_round * reps))
        rows = {}
        total_ops, total_us = 0, 0.0
        for name, leg in legs.items():
            us = statistics.median(leg["us"])
            ops = 2 * M * leg["N"] * leg["K"]
            total_ops += ops
            total_us += us
            p = leg["path"]
            rows[name] = {"N": leg["N"], "K": leg["K"], "us": round(us, 2),
                          "TOPS": round(ops / (us * 1e-6) / 1e12, 1),
                          "path": [p.kind, p.tokens, p.channels, p.splits, p.waves]}
        del legs
        tops = total_ops / (total_us * 1e-6) / 1e12
        peak = I8_PEAK_TOPS if fmt == qlinear.I8 else FP8_PEAK_TFLOPS
        out[fmt_name] = {"TOPS": round(tops, 1), "frac_mfma": round(tops / peak, 4),
                         "peak": peak, "projections": rows}
    return out


def vendor_compare(torch, qlinear, synthetic, dev, stream, M=M_PREFILL):
    """The vendor library's GEMMs on this build's quantized operands (the same
    synthetic activations and weights as the prefill legs), timed beside the
    planned qlin GEMM the same way (graphs of 10 calls, warm-up, 5
    interleaved rounds, medians): INT8 torch._int_mm (int8 x int8 -> int32,
    no dequant epilogue, so it does less work than qlin's bf16 output) and FP8
    torch._scaled_mm with row-wise scales and bf16 output (the same contract
    as qlin's FP8 GEMM). Both run on hipBLASLt on this image."""
    import statistics
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps, rounds = 10, 5
    out = {}
    for fmt_name, fmt in (("int8", qlinear.I8), ("fp8", qlinear.FP8)):
        rows, legs = {}, {}
        for name, (N, K) in synthetic.PROJECTIONS.items():
            x = torch.from_numpy(synthetic.activations(M, K, seed=1).view(np.int16)).view(
                torch.bfloat16).to(dev)
            w = torch.from_numpy(synthetic.weights(N, K, seed=1).view(np.int16)).view(
                torch.bfloat16).to(dev)
            with torch.cuda.stream(stream):
                xq, sx = qlinear.row_quantize(x, fmt, stream=stream)
                wq, sw = qlinear.row_quantize(w, fmt, stream=stream)
                y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            torch.cuda.synchronize()
            if fmt == qlinear.I8:
                a8, b8 = xq.view(torch.int8), wq.view(torch.int8)
                vendor = lambda a8=a8, b8=b8: torch._int_mm(a8, b8.t())
            else:
                a8, b8 = xq.view(torch.float8_e4m3fn), wq.view(torch.float8_e4m3fn)
                sa, sb = sx.view(M, 1), sw.view(1, N)
                vendor = lambda a8=a8, b8=b8, sa=sa, sb=sb: torch._scaled_mm(
                    a8, b8.t(), scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)
            ours = lambda xq=xq, sx=sx, wq=wq, sw=sw, y=y: qlinear.gemm(
                xq, sx, wq, sw, fmt, out=y, stream=stream)
            for leg, fn in (("vendor", vendor), ("qlin", ours)):
                with torch.cuda.stream(stream):
                    fn()
                torch.cuda.synchronize()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=stream):
                    for _ in range(reps):
                        fn()
                legs[(name, leg)] = {"graph": g, "ops": 2 * M * N * K, "us": [],
                                     "keep": (xq, sx, wq, sw, y)}
        torch.cuda.synchronize()
        for _ in range(30):
            for leg in legs.values():
                leg["graph"].replay()
        torch.cuda.synchronize()
        for r in range(rounds):
            for key in (list(legs) if r % 2 == 0 else list(reversed(legs))):
                with torch.cuda.stream(stream):
                    start.record(stream)
                    legs[key]["graph"].replay()
                    end.record(stream)
                torch.cuda.synchronize()
                legs[key]["us"].append(start.elapsed_time(end) * 1e3 / reps)
        totals = {"vendor": [0, 0.0], "qlin": [0, 0.0]}
        for (name, leg), v in legs.items():
            us = statistics.median(v["us"])
            rows.setdefault(name, {})[leg + "_us"] = round(us, 2)
            totals[leg][0] += v["ops"]
            totals[leg][1] += us
        out[fmt_name] = {k: round(o / (u * 1e-6) / 1e12, 1) for k, (o, u) in totals.items()}
        out[fmt_name]["unit"] = "TOPS" if fmt == qlinear.I8 else "TFLOPS"
        out[fmt_name]["projections"] = rows
        del legs
    out["vendor_ops"] = {"int8": "torch._int_mm, int32 output (no dequant epilogue)",
                         "fp8": "torch._scaled_mm, row-wise fp32 scales, bf16 output"}
    return out


def bench_producers(torch, qlinear, synthetic, dev, stream, args):
    """The fused quantizing producers at the decoder's shapes (hidden 2048,
    FFN 6144; INT8 per-token): residual update + RMSNorm -> quant,
    SiLU(gate) * up -> quant, LayerNorm -> quant and bias + tanh-GeLU -> quant
    at M=32 and M=4096, and LayerNorm -> quantized GEMV at k=512. Algorithmic
    bytes: norm reads x, update (2MK each) and weight (2K), writes the
    residual (2MK), codes (MK) and scales (4M); gated reads gate|up (4MW),
    writes codes (MW) and scales (4M); LayerNorm / pointwise read x (2MK) and
    one [K] vector (2K), write codes (MK) and scales (4M)."""
    out = {}
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    H, W = 2048, 6144

    def timed(launch, reps=20, n_rep=5):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for _ in range(reps):
                launch()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            start.record(stream)
            for _ in range(n_rep):
                g.replay()
            end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) * 1e3 / (n_rep * reps)

    for M in (M_DECODE, M_PREFILL):
        def bf(shape, seed):
            return torch.from_numpy(synthetic.activations(shape[0], shape[1], seed=seed).view(
                np.int16)).view(torch.bfloat16).to(dev)
        x, u, gu = bf((M, H), 1), bf((M, H), 2), bf((M, 2 * W), 3)
        w = torch.ones(H, dtype=torch.bfloat16, device=dev)
        nq = torch.empty((M, H), dtype=torch.uint8, device=dev)
        gq = torch.empty((M, W), dtype=torch.uint8, device=dev)
        ns = torch.empty((M,), dtype=torch.float32, device=dev)
        gs = torch.empty((M,), dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        us_n = timed(lambda: qlinear.quantized_norm(x, w, qlinear.I8, update=u, values=nq,
                                                    scales=ns, stream=stream))
        us_g = timed(lambda: qlinear.quantized_gated(gu, qlinear.I8, kind=0, values=gq,
                                                     scales=gs, stream=stream))
        # LayerNorm -> quant (no fusions) and the linear output's pointwise
        # epilogue (bias + tanh-GeLU) -> quant, at the decoder's hidden size.
        bias = bf((1, H), 4).reshape(H)
        lq = torch.empty((M, H), dtype=torch.uint8, device=dev)
        ls = torch.empty((M,), dtype=torch.float32, device=dev)
        ep = qlinear.epilogue(bias=bias, activation=qlinear.ACT_GELU_TANH)
        us_l = timed(lambda: qlinear.layer_norm_quantize(x, qlinear.I8, norm_weight=w,
                                                         values=lq, scales=ls, stream=stream))
        us_p = timed(lambda: qlinear.pointwise_quantize(x, qlinear.I8, ep, values=lq, scales=ls,
                                                        stream=stream))
        b_n = 7 * M * H + 2 * H + 4 * M
        b_g = 5 * M * W + 4 * M
        b_l = 3 * M * H + 2 * H + 4 * M
        b_p = 3 * M * H + 2 * H + 4 * M
        leg = lambda us, b: {"us": round(us, 2), "bytes": b, "GBps": round(b / (us * 1e-6) / 1e9, 1)}
        out[f"M={M}"] = {"quantized_norm": leg(us_n, b_n), "quantized_gated": leg(us_g, b_g),
                         "layer_norm_quantize": leg(us_l, b_l),
                         "pointwise_quantize": leg(us_p, b_p)}
    # LayerNorm -> quantized GEMV for a small-hidden projection (k = 512,
    # n = 2048, INT8): reads x (2·rows·k) and the weights (n·k + 4n), writes y.
    rows, k, n = M_DECODE, 512, 2048
    xs = torch.from_numpy(synthetic.activations(rows, k, seed=7).view(np.int16)).view(
        torch.bfloat16).to(dev)
    wq = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev).view(torch.uint8)
    sw = torch.full((n,), 1e-3, dtype=torch.float32, device=dev)
    y = torch.empty((rows, n), dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    us_nl = timed(lambda: qlinear.norm_linear(xs, wq, sw, qlinear.I8, out=y, stream=stream))
    b_nl = n * k + 4 * n + 2 * rows * k + 2 * rows * n
    out[f"norm_linear rows={rows} k={k} n={n}"] = {
        "us": round(us_nl, 2), "bytes": b_nl, "GBps": round(b_nl / (us_nl * 1e-6) / 1e9, 1)}
    return out


def cpu_baseline(args, gpu_value, gpu_prefill=None):
    """The oracle's multithreaded C restatement of quant + GEMM + dequant
    (oracle/qlinear_oracle.c, orc_cpu_qlinear; the x86-64-v4 build on an
    AVX-512 host) timed on bounded samples of the BASELINE configs, about
    20 s in all, median rep of each:
    - INT8 per-token, one layer's four projections at M=32 (1 of the step's
      16 layers; this is `value`, in the step's GB/s of algorithmic bytes);
    - FP8 and group_int8 (H128 rotation, K128 groups) one layer at M=32, GB/s;
    - INT8 prefill: the qkv projection at M=4096, TOPS."""
    from breeze_tts_cpp_amd import synthetic
    from oracle import oracle

    threads = args.cpu_threads or min(16, os.cpu_count() or 1)
    _, isa = oracle.cpu_lib()

    def timed(jobs, seconds):
        for job in jobs[:1]:
            oracle.cpu_qlinear(*job, threads=threads, fast=True)  # warm-up
        times = []
        t_end = time.time() + seconds
        while len(times) < 3 or (time.time() < t_end and len(times) < 1000):
            t0 = time.perf_counter()
            for job in jobs:
                oracle.cpu_qlinear(*job, threads=threads, fast=True)
            times.append(time.perf_counter() - t0)
        return float(np.median(times)), len(times)

    def layer(fmt, group):
        jobs, total = [], 0
        for name, (N, K) in synthetic.PROJECTIONS.items():
            wq, sw = oracle.quantize_rows(synthetic.weights(N, K, seed=1000), fmt, group=group,
                                          rotation=group)
            jobs.append((synthetic.activations(M_DECODE, K, seed=0), wq, sw, fmt, group, group))
            total += gemm_bytes(M_DECODE, N, K, group) + quant_bytes(M_DECODE, K, group)
        return jobs, total

    out = {}
    jobs, total = layer(oracle.I8, 0)
    t, reps = timed(jobs, 8.0)
    gbs = total / t / 1e9
    sample = [f"INT8 one layer (4 projections, M={M_DECODE}) of the {LAYERS}-layer step, "
              f"median of {reps} reps"]
    for mode, fmt, group in (("fp8", oracle.FP8, 0), ("group_int8", oracle.I8, 128)):
        jobs, total = layer(fmt, group)
        t, reps = timed(jobs, 4.0)
        out[f"{mode}_GBps"] = round(total / t / 1e9, 2)
        sample.append(f"{mode} one layer M={M_DECODE} ({reps} reps)")
    N, K = synthetic.PROJECTIONS["qkv"]
    wq, sw = oracle.quantize_rows(synthetic.weights(N, K, seed=1000), oracle.I8)
    t, reps = timed([(synthetic.activations(M_PREFILL, K, seed=0), wq, sw, oracle.I8, 0, 0)], 6.0)
    out["prefill_int8_qkv_TOPS"] = round(2 * M_PREFILL * N * K / t / 1e12, 3)
    sample.append(f"INT8 qkv M={M_PREFILL} ({reps} reps)")
    ratio = f"; GPU/CPU = {round(gpu_value / gbs, 1)}x (decode step)"
    if gpu_prefill:
        ratio += f", {round(gpu_prefill / out['prefill_int8_qkv_TOPS'], 1)}x (INT8 prefill)"
    return {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "isa": isa, **out, "sample": "; ".join(sample) + ratio}


if __name__ == "__main__":
    main()
