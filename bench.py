"""Benchmark of the quantized matvec path on one MI355X.

Metric: "quant matvec weight-GB/s (% HBM peak) at 8B shapes;
M=512 GEMM int8 TOPS".

One step = one decode pass over the Llama-3-8B Q4_K_M layer set (config 2):
32 layers x 7 matrices (wq, wk, wo, ffn_gate, ffn_up: Q4_K; wv, ffn_down:
Q6_K), batch 1, each launch converting its f32 activation to Q8_K inside the
kernel, in the reference engine's order (engine.c:317-378). Matrices that
read the same activation share a launch (q/k/v, gate/up: 4 launches per
layer; --unfused gives one launch per matrix). The pass is captured in a HIP
graph; 4,444,913,664 weight bytes are streamed per pass.
value = weight bytes / pass time (GB/s). Weights are seeded synthetic GGUF
blocks (random fields, f16 scales in the configured ranges), activations
N(0,1); both are resident in HBM before timing starts.

Extra fields: the dominant kernel's roofline (Q4_K matvec, per-launch HIP
events), the M=512 prefill GEMM (config 3) in TOPS, the other formats'
matvec rates at configs 0, 1 and 4 (batch 1 and 8), the decode attention
over an f16 KV cache at the 8B shape (positions 511 and 4095), and the
reference's own AVX2 gemv (oracle/_ref, through its lane pool) on a bounded
sample of the same weights on the host cores.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-gemm]
                    [--no-configs] [--no-attn] [--profile gemm|traffic|configs|attn]
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

HBM_PEAK_GBS = 8000.0           # MI355X HBM3E, GB/s
# HBM bytes per gate_up launch measured by rocprofv3 FETCH_SIZE / WRITE_SIZE
# in runs of their own (counters cannot be collected in a timed run),
# scaled by the factors a 64 MiB copy gives (2.00 and 1.00); see
# profiles/matvec_gate_up_traffic.md for the commands and raw values.
GATE_UP_TRAFFIC_BYTES = 2.00 * 32454.0 * 1024 + 1.00 * 112.0 * 1024
INT8_PEAK_TOPS = 5033.0         # MI355X dense int8 MFMA, TOPS (256 CU x 2.4 GHz x 8192)
F16_PEAK_TFLOPS = 2516.5        # MI355X dense f16 MFMA, TFLOP/s (half the int8 rate)
N_LAYERS = 32


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-gemm", action="store_true", help="skip the M=512 GEMM")
    ap.add_argument("--no-prefill", action="store_true",
                    help="skip the M=512 prefill pass over the 32 layers")
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--unfused", action="store_true",
                    help="one launch per matrix instead of fused q/k/v and gate/up launches")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the per-format matvec measurements (configs 0, 1, 4)")
    ap.add_argument("--no-attn", action="store_true", help="skip the decode attention")
    ap.add_argument("--profile", choices=("gemm", "traffic", "configs", "attn", "prefill", "batch8",
                                          "calib"),
                    help="run one workload for a profiler and exit: the GEMM M sweep, "
                         "a 64 MiB copy plus 12 gate/up launches (HBM counter runs), "
                         "the per-format matvec measurements, the decode attention, "
                         "the M=512 prefill pass over 32 layers and the batch-8 decode step, "
                         "the batch-8 decode step alone, or the HBM calibration "
                         "(a 4 GiB streaming read and the decode pass's launches read-only)")
    return ap.parse_args()


def build_layers(dev, rng, keep_host_layers):
    """Upload 32 distinct layers; return device weights and the host bytes of
    the first `keep_host_layers` layers (for the CPU baseline)."""
    import siphon_amd as sa
    from siphon_amd import synth
    layers, host = [], []
    for il in range(N_LAYERS):
        mats = {}
        hl = {}
        for (name, wt, n_out, n_in) in synth.LLAMA3_8B_LAYER:
            d_range = (1e-4, 2e-3) if wt == sa.Q6_K else (1e-4, 4e-3)
            W = synth.make_weights(wt, n_out, n_in, rng, d_range=d_range)
            mats[name] = dev.upload(wt, n_out, n_in, W)
            if il < keep_host_layers:
                hl[name] = W
        layers.append(mats)
        if il < keep_host_layers:
            host.append(hl)
    return layers, host


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every GPU box here has one MI355X and the "
              f"path is single-GPU by design (requested --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)
    import torch
    import siphon_amd as sa
    from siphon_amd import synth

    torch.cuda.init()
    dev = sa.Device(0)
    rng = np.random.default_rng(args.seed)
    if args.profile:
        stream = torch.cuda.Stream()
        if args.profile == "gemm":
            out = bench_gemm(dev, torch, stream, rng)
        elif args.profile == "calib":
            out = profile_calibration(dev, torch, stream)
        elif args.profile == "prefill":
            layers, _ = build_layers(dev, rng, 0)
            out = bench_prefill_pass(dev, torch, stream, layers)
            out["decode_batch8"] = bench_batch_decode(dev, torch, stream, layers)
        elif args.profile == "batch8":
            layers, _ = build_layers(dev, rng, 0)
            out = bench_batch_decode(dev, torch, stream, layers)
        elif args.profile == "configs":
            out = bench_configs(dev, torch, stream, rng)
        elif args.profile == "attn":
            out = bench_attention(dev, torch, stream)
        else:
            out = profile_traffic(dev, torch, stream, rng)
        dev.close()
        print(json.dumps(out), flush=True)
        return
    t0 = time.time()
    cpu_layers = 0 if args.no_cpu else 2
    layers, host_layers = build_layers(dev, rng, cpu_layers)
    log(f"uploaded 32 layers in {time.time() - t0:.1f} s")
    pass_bytes = sum(l[name].gguf_bytes for l in layers for name in l)

    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    # activations: one f32 vector per (layer, stage), N(0,1), resident in HBM
    acts = [[torch.randn(n, device="cuda") for n in (4096, 4096, 4096, 14336)]
            for _ in range(N_LAYERS)]
    outs = {name: torch.empty(n_out, device="cuda")
            for (name, _, n_out, _) in synth.LLAMA3_8B_LAYER}
    stage_of = {"wq": 0, "wk": 0, "wv": 0, "wo": 1, "ffn_gate": 2, "ffn_up": 2, "ffn_down": 3}
    # launches per layer: matrices that share an activation run in one launch
    # (q/k/v and gate/up), in the reference engine's order
    groups = [("qkv", ("wq", "wk", "wv")), ("wo", ("wo",)), ("gate_up", ("ffn_gate", "ffn_up")),
              ("down", ("ffn_down",))]
    if args.unfused:
        groups = [(n, (n,)) for n in ("wq", "wk", "wv", "wo", "ffn_gate", "ffn_up", "ffn_down")]

    def decode_pass(events=None):
        for il in range(N_LAYERS):
            for label, names in groups:
                ws = [layers[il][n] for n in names]
                x = acts[il][stage_of[names[0]]]
                if events is not None:
                    e0 = torch.cuda.Event(enable_timing=True)
                    e1 = torch.cuda.Event(enable_timing=True)
                    e0.record(stream)
                if len(ws) == 1:
                    dev.gemv_dev(ws[0], x.data_ptr(), outs[names[0]].data_ptr(), ws[0].n_out, sp)
                else:
                    dev.gemv_multi_dev(ws, x.data_ptr(), [outs[n].data_ptr() for n in names], sp)
                if events is not None:
                    e1.record(stream)
                    nbytes = sum(w.gguf_bytes + 4 * w.n_out for w in ws) + 4 * ws[0].n_in
                    events.append((label, nbytes, e0, e1))

    # eager reference output, then capture the pass in a graph
    with torch.cuda.stream(stream):
        decode_pass()
    torch.cuda.synchronize()
    eager = {k: v.clone() for k, v in outs.items()}
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        decode_pass()
    for _ in range(3):  # replays must reproduce the eager results exactly
        graph.replay()
        torch.cuda.synchronize()
        for k in outs:
            assert torch.equal(outs[k], eager[k]), f"graph replay differs on {k}"

    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    ms_per_step = elapsed * 1e3 / args.steps
    value = pass_bytes / (elapsed / args.steps) / 1e9

    # roofline of the dominant kernel (the gate+up launch: Q4_K, 66 MB, the
    # largest share of the pass). Each launch kind of the pass is captured in
    # a graph of its own (its 32 launches over the 32 layers, back to back on
    # the launch stream) and timed with HIP events on that stream over
    # several replays: the average launch duration, as a kernel trace shows.
    per = {}
    for label, names in groups:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for il in range(N_LAYERS):
                ws = [layers[il][n] for n in names]
                x = acts[il][stage_of[names[0]]]
                if len(ws) == 1:
                    dev.gemv_dev(ws[0], x.data_ptr(), outs[names[0]].data_ptr(), ws[0].n_out, sp)
                else:
                    dev.gemv_multi_dev(ws, x.data_ptr(), [outs[n].data_ptr() for n in names], sp)
        g.replay()
        torch.cuda.synchronize()
        reps = 10
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            with torch.cuda.stream(stream):
                g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * N_LAYERS)
        ws = [layers[0][n] for n in names]
        nbytes = sum(w.gguf_bytes + 4 * w.n_out for w in ws) + 4 * ws[0].n_in
        per[label] = (nbytes, us)
        del g
    probe = probe_floors(dev, torch, stream,
                         {label: sum(layers[0][n].gguf_bytes for n in names)
                          for label, names in groups})
    dom = "gate_up" if "gate_up" in per else "ffn_gate"
    nbytes, us = per[dom]
    achieved = nbytes / (us * 1e-6) / 1e9
    roofline = {
        "kernel": f"sihip::matvec_kernel<Q4_K,Q4_K,1> ({dom} launch, 32 per pass)",
        "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "avg_launch_us": round(us, 2),
        "algorithmic_bytes_per_launch": nbytes,
        "traffic": round(GATE_UP_TRAFFIC_BYTES) if dom == "gate_up" else None,
        "traffic_over_algorithmic": (round(GATE_UP_TRAFFIC_BYTES / nbytes, 4)
                                     if dom == "gate_up" else None),
        "per_launch_us": {k: round(v[1], 2) for k, v in per.items()},
        "per_launch_GBs": {k: round(v[0] / (v[1] * 1e-6) / 1e9, 1) for k, v in per.items()},
        # the read-only probe over the same weight bytes, launched the same
        # way (32 launches of the kind back to back in one graph): the floor
        # of a launch of that size, and each kind's time over it
        "per_launch_probe_us": {k: round(v, 2) for k, v in probe.items()},
        "per_launch_over_probe": {k: round(per[k][1] / probe[k], 3) for k in per},
    }

    result = {
        "metric": "quant matvec weight-GB/s (% HBM peak) at 8B shapes; M=512 GEMM int8 TOPS",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "q4_K/q6_K x q8_K (int8 dot, f32 acc)",
        "data": "synthetic (seeded random GGUF blocks, N(0,1) activations)",
        "config": {"workload": "Llama-3-8B Q4_K_M decode layer set, 32 layers x 7 matvecs, "
                               "batch 1, HIP graph", "weight_bytes_per_step": pass_bytes,
                   "launches_per_layer": len(groups),
                   "hbm_frac": round(value / HBM_PEAK_GBS, 4)},
        "roofline": roofline,
    }

    if not args.no_gemm:
        result["gemm_m512"] = bench_gemm(dev, torch, stream, rng)
    if not args.no_prefill:
        result["prefill_pass"] = bench_prefill_pass(dev, torch, stream, layers)
        result["decode_batch8"] = bench_batch_decode(dev, torch, stream, layers)
    if not args.no_attn:
        result["attention"] = bench_attention(dev, torch, stream)
    if not args.no_configs:
        for l in layers:  # the per-format runs upload their own matrices
            for w in l.values():
                w.free()
        layers = []
        result["configs"] = bench_configs(dev, torch, stream, rng)

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(host_layers, pass_bytes)
        result["cpu_baseline"]["gpu_over_cpu"] = round(value / result["cpu_baseline"]["value"], 1)

    for l in layers:
        for w in l.values():
            w.free()
    dev.close()
    print(json.dumps(result), flush=True)


def bench_attention(dev, torch, stream, positions=(511, 4095)):
    """Decode attention over the f16 KV cache at Llama-3-8B's shape (32
    query heads, 8 KV heads, head_dim 128, n_ctx 4096): the launches of one
    layer (two up to 1024 positions, three beyond), the 32 layers' caches (537 MB, past the 256 MB MALL) in one
    HIP graph. Algorithmic bytes per layer: the K and V slices read (2 x 8 x
    n x 128 x 2 B), the query and output (2 x 32 x 128 x 4 B)."""
    n_head, n_kv, hd, n_ctx = 32, 8, 128, 4096
    sp = stream.cuda_stream
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    caches = [(torch.randn(n_kv * n_ctx * hd, device="cuda", generator=g).half(),
               torch.randn(n_kv * hd * n_ctx, device="cuda", generator=g).half())
              for _ in range(N_LAYERS)]
    q = torch.randn(N_LAYERS, n_head * hd, device="cuda", generator=g)
    out = torch.empty(N_LAYERS, n_head * hd, device="cuda")
    kq = float(1.0 / np.sqrt(hd))
    res = {"shape": {"n_head": n_head, "n_head_kv": n_kv, "head_dim": hd, "n_ctx": n_ctx}}
    for pos in positions:
        def layer_pass():
            for il in range(N_LAYERS):
                k, v = caches[il]
                dev.attn_decode_dev(q[il].data_ptr(), k.data_ptr(), v.data_ptr(), n_head, n_kv,
                                    hd, n_ctx, pos, kq, out[il].data_ptr(), None, None, sp)
        with torch.cuda.stream(stream):
            layer_pass()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            layer_pass()
        graph.replay()
        torch.cuda.synchronize()
        reps = 10
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            with torch.cuda.stream(stream):
                graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * N_LAYERS)
        nbytes = 2 * n_kv * (pos + 1) * hd * 2 + 2 * n_head * hd * 4
        # up to 1024 positions the softmax runs inside the value launch
        res[f"pos{pos}"] = {"us_per_layer": round(us, 2), "launches": 2 if pos < 1024 else 3,
                            "kv_bytes": nbytes,
                            "GBs": round(nbytes / (us * 1e-6) / 1e9, 1),
                            "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        del graph
    return res


def bench_gemm(dev, torch, stream, rng, rotate_bytes=512 << 20):
    """Config 3: Q4_K W[14336 x 4096] x X[M x 4096] -> Y[M x 14336], M = 512
    headline and the sweep {64, 128, 512, 2048}. Each call quantizes X to Q8_K
    rows and runs the MFMA GEMM; enough weight copies rotate that more than
    `rotate_bytes` of GGUF bytes (fewer than any GEMM-ordered copy holds)
    stream between two reads of one copy, so the 256 MB Infinity Cache cannot
    serve them. The first call per copy builds its GEMM-ordered copy; three
    untimed passes over the copies precede the four timed ones (a copy's
    kernel time drifts down by up to 13% over the first hundred calls after
    a pause, so a short window would time the drift, not the sustained
    rate)."""
    import siphon_amd as sa
    from siphon_amd import synth
    n_out, n_in = 14336, 4096
    W = synth.make_weights(sa.Q4_K, n_out, n_in, rng)
    copies = -(-rotate_bytes // W.nbytes) + 1
    ws = [dev.upload(sa.Q4_K, n_out, n_in, W) for _ in range(copies)]
    sp = stream.cuda_stream
    sweep = {}
    for M in (64, 128, 512, 2048):
        X = torch.randn(M, n_in, device="cuda")
        Y = torch.empty(M, n_out, device="cuda")
        with torch.cuda.stream(stream):
            for _ in range(3):
                for w in ws:
                    dev.gemm_dev(w, X.data_ptr(), M, Y.data_ptr(), sp)
        torch.cuda.synchronize()
        reps = 4 * len(ws)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        with torch.cuda.stream(stream):
            for i in range(reps):
                dev.gemm_dev(ws[i % len(ws)], X.data_ptr(), M, Y.data_ptr(), sp)
        e1.record(stream)
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) / 1e3 / reps
        tops = 2.0 * M * n_out * n_in / t / 1e12
        sweep[str(M)] = {"us_per_call": round(t * 1e6, 1), "TOPS": round(tops, 1),
                         "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
        del X, Y
    for w in ws:
        w.free()
    # the other matrix-core formats at the same shape, M = 512 (not
    # configured by the baseline: how far the Q4_K prefill path carries;
    # F16 runs on the f16 MFMAs, whose dense peak is half the int8 one)
    formats = {}
    M = 512
    X = torch.randn(M, n_in, device="cuda")
    Y = torch.empty(M, n_out, device="cuda")
    for wt in (sa.Q5_K, sa.Q2_K, sa.Q3_K, sa.Q6_K, sa.Q4_0, sa.Q5_0, sa.Q8_0, sa.F16):
        Wf = synth.make_weights(wt, n_out, n_in, rng)
        wf = [dev.upload(wt, n_out, n_in, Wf) for _ in range(-(-rotate_bytes // Wf.nbytes) + 1)]
        with torch.cuda.stream(stream):
            for _ in range(3):
                for w in wf:
                    dev.gemm_dev(w, X.data_ptr(), M, Y.data_ptr(), sp)
        torch.cuda.synchronize()
        reps = 4 * len(wf)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        with torch.cuda.stream(stream):
            for i in range(reps):
                dev.gemm_dev(wf[i % len(wf)], X.data_ptr(), M, Y.data_ptr(), sp)
        e1.record(stream)
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) / 1e3 / reps
        tops = 2.0 * M * n_out * n_in / t / 1e12
        formats[sa.NAMES[wt]] = {"us_per_call": round(t * 1e6, 1), "TOPS": round(tops, 1),
                                 "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
        if wt == sa.F16:  # f16 MFMAs: also against the dense f16 peak
            formats[sa.NAMES[wt]]["frac_f16_peak"] = round(tops / F16_PEAK_TFLOPS, 4)
        for w in wf:
            w.free()
    del X, Y
    head = sweep["512"]
    return {"value": head["TOPS"], "unit": "TOPS", "M": 512, "shape": [n_out, n_in],
            "copies": copies,
            "us_per_call": head["us_per_call"], "sweep": sweep, "other_formats_m512": formats,
            "roofline": {"bound": "mfma", "achieved": head["TOPS"], "peak": INT8_PEAK_TOPS,
                         "unit": "TOP/s", "frac": head["frac_int8_peak"]}}


def bench_prefill_pass(dev, torch, stream, layers, M=512, reps=5):
    """Prefill of a 512-token prompt through the 32 decode-pass layers: the
    7 matrices of each layer in engine order on M = 512 activation rows
    (N(0,1), resident in HBM), the matrices that share an activation (q/k/v,
    gate/up) in one gemm_multi_dev call (the activation quantized once), the
    others one gemm_dev call each: 128 calls in one HIP graph. The GEMM
    copies are built first, as load-time placement builds them. TOPS = 2 M x
    (weights' n_out x n_in summed) / pass time; per matrix kind, its 32
    single gemm_dev calls in a graph of their own give the average call time
    (activation quantization included)."""
    import siphon_amd as sa
    from siphon_amd import synth
    sp = stream.cuda_stream
    for l in layers:
        for w in l.values():
            w.prepare_gemm()
    names = [n for (n, _, _, _) in synth.LLAMA3_8B_LAYER]
    X = {n_in: torch.randn(M, n_in, device="cuda") for n_in in (4096, 14336)}
    Y = {n: torch.empty(M, layers[0][n].n_out, device="cuda") for n in names}

    def calls(il, name):
        w = layers[il][name]
        dev.gemm_dev(w, X[w.n_in].data_ptr(), M, Y[name].data_ptr(), sp)

    groups = [("wq", "wk", "wv"), ("wo",), ("ffn_gate", "ffn_up"), ("ffn_down",)]

    def run_pass():
        for il in range(N_LAYERS):
            for grp in groups:
                if len(grp) == 1:
                    calls(il, grp[0])
                else:
                    ws = [layers[il][n] for n in grp]
                    dev.gemm_multi_dev(ws, X[ws[0].n_in].data_ptr(), M,
                                       [Y[n].data_ptr() for n in grp], sp)

    with torch.cuda.stream(stream):
        run_pass()
    torch.cuda.synchronize()
    eager = {n: y.clone() for n, y in Y.items()}
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        run_pass()
    for _ in range(2):  # replays must reproduce the eager results exactly
        g.replay()
        torch.cuda.synchronize()
        for n in names:
            assert torch.equal(Y[n], eager[n]), f"prefill graph replay differs on {n}"
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        with torch.cuda.stream(stream):
            g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    pass_ms = e0.elapsed_time(e1) / reps
    ops = sum(2.0 * M * w.n_out * w.n_in for l in layers for w in l.values())
    tops = ops / (pass_ms * 1e-3) / 1e12
    del g
    per = {}
    for n in names:
        gn = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gn, stream=stream):
            for il in range(N_LAYERS):
                calls(il, n)
        gn.replay()
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(reps):
            with torch.cuda.stream(stream):
                gn.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * N_LAYERS)
        w = layers[0][n]
        t = 2.0 * M * w.n_out * w.n_in / (us * 1e-6) / 1e12
        per[n] = {"type": sa.NAMES[w.type],
                  "shape": [w.n_out, w.n_in], "us_per_call": round(us, 1), "TOPS": round(t, 1),
                  "frac_int8_peak": round(t / INT8_PEAK_TOPS, 4)}
        del gn
    dom = max(per, key=lambda k: per[k]["us_per_call"])
    return {"M": M, "layers": N_LAYERS, "calls_per_pass": N_LAYERS * len(groups), "matrices_per_pass": N_LAYERS * len(names),
            "ms_per_pass": round(pass_ms, 3), "TOPS": round(tops, 1),
            "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
            "tokens_per_s": round(M / (pass_ms * 1e-3), 1),
            "per_matrix": per,
            "roofline": {"kernel": f"{dom} GEMM ({per[dom]['type']})", "bound": "mfma",
                         "achieved": per[dom]["TOPS"], "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
                         "frac": per[dom]["frac_int8_peak"]}}


def bench_batch_decode(dev, torch, stream, layers, M=8, reps=20, warmup=5):
    """A decode step of M sequences at once through the 32 decode-pass
    layers: per layer q/k/v and gate/up in one gemm_multi_dev call each
    (activation quantized once), wo and down one gemm_dev call, on M
    activation rows resident in HBM; 128 calls in one HIP graph, replays
    checked against the eager results. tokens/s = M / pass time; GB/s = the
    pass's GGUF weight bytes / pass time (each weight streamed once per
    step, whatever M). `warmup` untimed replays precede the `reps` timed
    ones."""
    from siphon_amd import synth
    sp = stream.cuda_stream
    for l in layers:
        for w in l.values():
            w.prepare_gemm()
    names = [n for (n, _, _, _) in synth.LLAMA3_8B_LAYER]
    X = {n_in: torch.randn(M, n_in, device="cuda") for n_in in (4096, 14336)}
    Y = {n: torch.empty(M, layers[0][n].n_out, device="cuda") for n in names}
    groups = [("wq", "wk", "wv"), ("wo",), ("ffn_gate", "ffn_up"), ("ffn_down",)]

    def run_pass():
        for il in range(N_LAYERS):
            for grp in groups:
                ws = [layers[il][n] for n in grp]
                if len(ws) == 1:
                    dev.gemm_dev(ws[0], X[ws[0].n_in].data_ptr(), M, Y[grp[0]].data_ptr(), sp)
                else:
                    dev.gemm_multi_dev(ws, X[ws[0].n_in].data_ptr(), M,
                                       [Y[n].data_ptr() for n in grp], sp)

    with torch.cuda.stream(stream):
        run_pass()
    torch.cuda.synchronize()
    eager = {n: y.clone() for n, y in Y.items()}
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        run_pass()
    for _ in range(2):
        g.replay()
        torch.cuda.synchronize()
        for n in names:
            assert torch.equal(Y[n], eager[n]), f"batch decode graph replay differs on {n}"
    for _ in range(warmup):  # untimed, back to back like the timed replays
        with torch.cuda.stream(stream):
            g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        with torch.cuda.stream(stream):
            g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    del g
    pass_ms = e0.elapsed_time(e1) / reps
    nbytes = sum(w.gguf_bytes for l in layers for w in l.values())
    gbs = nbytes / (pass_ms * 1e-3) / 1e9
    return {"M": M, "layers": N_LAYERS, "calls_per_pass": N_LAYERS * len(groups),
            "ms_per_pass": round(pass_ms, 4), "tokens_per_s": round(M / (pass_ms * 1e-3), 1),
            "weight_GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}


def _config_shapes():
    """Configs 0, 1 and 4 of the benchmark plan: (label, type, n_out, n_in,
    batches). Config 1's Q6_K head uses n_in 1024 (Q6_K needs a multiple of
    256; the 896-wide head of that model cannot be Q6_K)."""
    import siphon_amd as sa
    shapes = [("cfg0 Q4_K 5632x2048", sa.Q4_K, 5632, 2048, (1,)),
              ("cfg0 Q4_0 5632x2048", sa.Q4_0, 5632, 2048, (1, 8)),
              ("cfg1 Q8_0 4864x896", sa.Q8_0, 4864, 896, (1,)),
              ("cfg1 Q6_K head 151936x1024", sa.Q6_K, 151936, 1024, (1,)),
              ("cfg1 Q8_0 head 151936x896", sa.Q8_0, 151936, 896, (1,))]
    for wt in (sa.Q2_K, sa.Q3_K, sa.Q5_K, sa.Q5_0, sa.F16):
        nm = sa.NAMES[wt]
        shapes += [(f"cfg4 {nm} attn 5120x5120", wt, 5120, 5120, (1, 8)),
                   (f"cfg4 {nm} kv 1024x5120", wt, 1024, 5120, (1, 8)),
                   (f"cfg4 {nm} ffn_up 27648x5120", wt, 27648, 5120, (1, 8)),
                   (f"cfg4 {nm} ffn_down 5120x27648", wt, 5120, 27648, (1, 8))]
    return shapes


def bench_configs(dev, torch, stream, rng, rotate_bytes=512 << 20):
    """Per-format matvec rates at the other configs' shapes, batch 1 (and 8
    for config 4). Enough copies of each matrix rotate that more than
    `rotate_bytes` stream between two reads of one copy, so the 256 MB
    Infinity Cache cannot serve them; the launches over all copies are one
    HIP graph, replayed; rate = weight bytes / average launch time."""
    from siphon_amd import synth
    sp = stream.cuda_stream
    out = {}
    for label, wt, n_out, n_in, batches in _config_shapes():
        W = synth.make_weights(wt, n_out, n_in, rng)
        copies = max(2, -(-rotate_bytes // W.nbytes) + 1)
        ws = [dev.upload(wt, n_out, n_in, W) for _ in range(copies)]
        del W
        entry = {"bytes": ws[0].gguf_bytes, "copies": copies}
        for M in batches:
            X = torch.randn(M, n_in, device="cuda")
            Y = torch.empty(M, n_out, device="cuda")

            def run():
                for w in ws:
                    if M == 1:
                        dev.gemv_dev(w, X.data_ptr(), Y.data_ptr(), n_out, sp)
                    else:
                        dev.gemm_dev(w, X.data_ptr(), M, Y.data_ptr(), sp)
            with torch.cuda.stream(stream):
                run()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                run()
            g.replay()
            torch.cuda.synchronize()
            reps = max(3, int(2e9 // (copies * ws[0].gguf_bytes)))
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(reps):
                with torch.cuda.stream(stream):
                    g.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (reps * copies)
            gbs = ws[0].gguf_bytes / (us * 1e-6) / 1e9
            entry[f"batch{M}"] = {"us_per_call": round(us, 2), "GB/s": round(gbs, 1),
                                  "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
            del g, X, Y
        for w in ws:
            w.free()
        # the read-only probe over the same bytes, rotated the same way: the
        # floor of a launch of that size
        probe = probe_rotated(dev, torch, stream, entry["bytes"], copies)
        entry["probe_us"] = round(probe, 2)
        for k in list(entry):
            if k.startswith("batch"):
                entry[k]["over_probe"] = round(entry[k]["us_per_call"] / probe, 3)
        out[label] = entry
    return out


def probe_rotated(dev, torch, stream, nbytes, copies):
    """The read-only probe (sihip_probe_read_dev) over nbytes, `copies`
    launches over consecutive slices of one buffer in one HIP graph (as
    bench_configs rotates its weight copies past the MALL), timed with HIP
    events on the launch stream: average microseconds per launch."""
    sp = stream.cuda_stream
    sink = torch.zeros(4096, dtype=torch.int32, device="cuda")
    span = (nbytes + 255) // 256 * 256
    nb16 = nbytes // 16 * 16
    buf = torch.ones((copies * span + 4095) // 4, dtype=torch.int32, device="cuda")

    def run():
        for i in range(copies):
            dev.probe_read_dev(buf.data_ptr() + i * span, nb16, sink.data_ptr(), sp)
    with torch.cuda.stream(stream):
        run()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        run()
    g.replay()
    torch.cuda.synchronize()
    reps = max(3, int(2e9 // (copies * nbytes)))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        with torch.cuda.stream(stream):
            g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * copies)
    del g, buf
    torch.cuda.empty_cache()  # see probe_floors
    return us


def probe_floors(dev, torch, stream, sizes, reps=10):
    """For each launch kind (label: bytes per launch), the library's
    read-only probe (sihip_probe_read_dev: nontemporal 16-byte loads, four
    in flight per thread) over that many bytes, 32 launches over consecutive
    slices of one buffer (past the 256 MB MALL) in one HIP graph, timed with
    HIP events on the launch stream: average microseconds per launch."""
    sp = stream.cuda_stream
    sink = torch.zeros(4096, dtype=torch.int32, device="cuda")
    span = max(sizes.values())
    buf = torch.ones((N_LAYERS * span + 4095) // 4, dtype=torch.int32, device="cuda")
    out = {}
    for label, nb in sizes.items():
        def run():
            for il in range(N_LAYERS):
                dev.probe_read_dev(buf.data_ptr() + il * span, nb, sink.data_ptr(), sp)
        with torch.cuda.stream(stream):
            run()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            run()
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            with torch.cuda.stream(stream):
                g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        out[label] = e0.elapsed_time(e1) * 1e3 / (reps * N_LAYERS)
        del g
    del buf
    # hand the probe's buffer (2.1 GB) back to the device: kept in torch's
    # cache, it made the batch-8 step measured after it 3% slower (1.71
    # against 1.66 ms, one box), the library's GEMM copies then being
    # allocated around it
    torch.cuda.empty_cache()
    return out


def profile_calibration(dev, torch, stream, reps=10):
    """HBM ceilings the decode pass is measured against, with the library's
    read-only probe kernel (sihip_probe_read_dev):
    - one streaming read of 4 GiB per launch: the rate HBM gives a long
      read;
    - the decode pass's launch structure with nothing but reads: per layer
      four launches of the q/k/v, wo, gate/up and down weight bytes of the
      Llama-3-8B Q4_K_M layer, 32 layers over consecutive slices of one
      4.44 GB buffer (past the 256 MB MALL), 128 launches in one HIP graph.
    Each time is the average over `reps` launches or graph replays, with
    HIP events on the launch stream."""
    import siphon_amd as sa
    from siphon_amd import synth
    sp = stream.cuda_stream
    sink = torch.zeros(4096, dtype=torch.int32, device="cuda")
    big = 4 << 30
    buf = torch.ones(big // 4, dtype=torch.int32, device="cuda")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    dev.probe_read_dev(buf.data_ptr(), big, sink.data_ptr(), sp)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(reps):
        dev.probe_read_dev(buf.data_ptr(), big, sink.data_ptr(), sp)
    e1.record(stream)
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) / 1e3 / reps
    stream_gbs = big / t / 1e9
    del buf
    shapes = {n: (wt, o, i) for (n, wt, o, i) in synth.LLAMA3_8B_LAYER}
    wb = {n: sa.row_bytes(wt, i) * o for n, (wt, o, i) in shapes.items()}
    groups = [("qkv", ("wq", "wk", "wv")), ("wo", ("wo",)), ("gate_up", ("ffn_gate", "ffn_up")),
              ("down", ("ffn_down",))]
    sizes = [sum(wb[n] for n in names) for _, names in groups]
    layer_bytes = sum(sizes)
    buf = torch.ones((N_LAYERS * layer_bytes + 4095) // 4, dtype=torch.int32, device="cuda")
    base = buf.data_ptr()

    def run_pass():
        off = 0
        for _ in range(N_LAYERS):
            for nb in sizes:
                dev.probe_read_dev(base + off, nb, sink.data_ptr(), sp)
                off += nb

    with torch.cuda.stream(stream):
        run_pass()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        run_pass()
    g.replay()
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(reps):
        with torch.cuda.stream(stream):
            g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    pass_ms = e0.elapsed_time(e1) / reps
    pass_gbs = N_LAYERS * layer_bytes / (pass_ms * 1e-3) / 1e9
    del g, buf
    floors = probe_floors(dev, torch, stream, dict(zip([g[0] for g in groups], sizes)), reps)
    return {"probe_us_per_launch_kind": {k: round(v, 2) for k, v in floors.items()},"stream_read": {"bytes": big, "ms": round(t * 1e3, 3), "GB/s": round(stream_gbs, 1),
                            "hbm_frac": round(stream_gbs / HBM_PEAK_GBS, 4)},
            "pass_read_only": {"launches": N_LAYERS * len(sizes), "bytes": N_LAYERS * layer_bytes,
                               "launch_bytes": dict(zip([g[0] for g in groups], sizes)),
                               "ms": round(pass_ms, 4), "GB/s": round(pass_gbs, 1),
                               "hbm_frac": round(pass_gbs / HBM_PEAK_GBS, 4)}}


def profile_traffic(dev, torch, stream, rng):
    """For the HBM counter runs (FETCH_SIZE, WRITE_SIZE): three 64 MiB
    device copies (calibration: the counters' bytes per dispatch against a
    known size), then 12 fused gate/up launches over 6 distinct weight
    pairs (793 MB, more than the Infinity Cache)."""
    import siphon_amd as sa
    from siphon_amd import synth
    a = torch.ones(16 << 20, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    W = synth.make_weights(sa.Q4_K, 14336, 4096, rng)
    pairs = [[dev.upload(sa.Q4_K, 14336, 4096, W) for _ in range(2)] for _ in range(6)]
    x = torch.randn(4096, device="cuda")
    ys = [torch.empty(14336, device="cuda") for _ in range(2)]
    for r in range(2):
        for ws in pairs:
            dev.gemv_multi_dev(ws, x.data_ptr(), [y.data_ptr() for y in ys], stream.cuda_stream)
    torch.cuda.synchronize()
    for ws in pairs:
        for w in ws:
            w.free()
    return {"copy_bytes": 2 * (64 << 20), "gate_up_launches": 12,
            "gate_up_weight_bytes": 2 * 33030144}


def host_cpus():
    """Lanes for the CPU baseline: every CPU this process may run on (its
    affinity set, the host's share granted to the job), one lane each; and a
    description of the host: CPU model, logical CPUs and physical cores of
    the machine, and the affinity count."""
    allowed = len(os.sched_getaffinity(0))
    model, phys = "unknown", set()
    try:
        cur = {}
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name" and model == "unknown":
                model = v
            if k in ("physical id", "core id"):
                cur[k] = v
            if not line.strip() and cur:
                phys.add((cur.get("physical id"), cur.get("core id")))
                cur = {}
    except OSError:
        pass
    return allowed, {"cpu_model": model, "host_logical_cpus": os.cpu_count(),
                     "host_physical_cores": len(phys) or None, "affinity_cpus": allowed}


def cpu_baseline(host_layers, pass_bytes, budget_s=10.0):
    """The reference's own AVX2 gemv (compiled from the reference sources into
    oracle/_ref) through its lane pool, on a bounded sample of the same
    workload: the 7 matrices of the first 2 layers (278 MB of weights),
    visited round-robin (so consecutive calls do not re-read a cached
    matrix) until about `budget_s` seconds of gemv time; GB/s = sample bytes
    / sum over matrices of the median call time. Falls back to the CPU
    oracle (kind "port") where the reference checker was not built."""
    from oracle import siq
    ref = siq.Reference.load()
    kind = "reference" if ref is not None else "port"
    lanes, host = host_cpus()
    from siphon_amd import synth
    shapes = {name: (wt, n_out, n_in) for (name, wt, n_out, n_in) in synth.LLAMA3_8B_LAYER}
    rng = np.random.default_rng(7)
    items = []
    for hl in host_layers:
        for name, W in hl.items():
            wt, n_out, n_in = shapes[name]
            items.append((wt, W, n_out, n_in, rng.standard_normal(n_in).astype(np.float32), []))
    oracle = siq.Oracle() if ref is None else None
    spent = 0.0
    t_start = time.time()
    while spent < budget_s or min(len(it[5]) for it in items) < 3:
        for (wt, W, n_out, n_in, x, times) in items:
            if ref is not None:
                _, secs = ref.gemv_timed(wt, W, n_out, n_in, x, lanes, 1)
                t = float(secs[0])
            else:
                t1 = time.perf_counter()
                oracle.gemv(wt, W, n_out, n_in, x, lanes)
                t = time.perf_counter() - t1
            times.append(t)
            spent += t
        if time.time() - t_start > 6 * budget_s:
            break
    total_bytes = sum(it[1].nbytes for it in items)
    total_s = sum(float(np.median(it[5])) for it in items)
    gbs = total_bytes / total_s / 1e9
    return {"value": round(gbs, 2), "unit": "GB/s", "cores": lanes, "kind": kind, **host,
            "impl": ("avx2" if ref.avx2 else "scalar") if ref is not None else "oracle",
            "sample": f"{len(host_layers)} layers x 7 matrices ({total_bytes} weight bytes), "
                      f"round-robin gemv calls (quantize + dots) through a {lanes}-lane pool, "
                      f"{min(len(it[5]) for it in items)}+ calls per matrix, "
                      f"{spent:.1f} s of gemv time, median per matrix",
            "pass_ms_estimate": round(pass_bytes / (gbs * 1e9) * 1e3, 1)}


if __name__ == "__main__":
    main()
