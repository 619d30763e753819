"""Benchmark of the MoE layer forward on one MI355X.

Default workload (the decode configuration the metric is quoted on): one MoE
layer, d=1024, 16 routed experts, top-2, SwiGLU hidden 2048, Int8 expert
weights (per-16 absmax/127 block scales), fp32 router, a batch of 32 tokens
with N(0,1) activations resident in HBM; weights N(0, 0.02), seed 0.  A step
is one layer forward (router, top-k, dispatch, gate/up, down, combine).
Four copies of the layer's weights (4 x 126 MB) are used round-robin so the
256 MB Infinity Cache cannot hold the weight set.

Other workloads (--workload): c2 with --tokens 1/8/32; c3 (FP4 prefill,
d=1024, 64+1 experts, top-6, h=512, T=4096); c4 (Int8 prefill, d=2048, 128
experts, top-8, h=768, T=16384, Zipf(1.2) router-bias skew); c5d / c5p (24
blocks RMSNorm + MoE + residual, d=2048, 64+1 experts, top-4, h=1024, FP4,
T=64 / T=8192; four distinct seeded weight sets cycled over the 24 layers,
every layer with its own resident copy).

--adapters R times a training step instead: forward and backward through
the host API with rank-R adapters on every layer of the mixture.

Prints one JSON line.  `value` comes from the timed steps (synchronised on
both sides, no per-kernel events).  `roofline` is for the dominant kernel:
HBM-bound gemv_gateup (decode) or MFMA-bound mfma_gateup (prefill); achieved
= algorithmic bytes or FLOPs per launch / mean launch time, the mean taken by
one HIP event pair (torch.cuda.Event on the stream the kernels run on) around
a burst of back-to-back relaunches of that kernel over every resident layer
copy, which keeps per-launch event skew out of the figure.  A further pass
with an event pair around every kernel gives the per-kernel breakdown in
`detail`.  `cpu_baseline` times the
CPU restatement of the reference algorithm (oracle/, float64, the
reference's SplitAcrossThreads policy) on a bounded sample of the same
workload on the host cores."""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE-layer tokens/s @1 GPU; achieved HBM GB/s & MFMA util vs peak"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
MFMA_FP32_PEAK_TFLOPS = 157.3

WORKLOADS = {
    "c2": dict(d=1024, E=16, k=2, h=2048, S=0, prec="int8", T=32, layers=1, copies=4, seed=0),
    "c3": dict(d=1024, E=64, k=6, h=512, S=1, prec="fp4", T=4096, layers=1, copies=1, seed=3),
    "c4": dict(d=2048, E=128, k=8, h=768, S=0, prec="int8", T=16384, layers=1, copies=1, seed=4, zipf=0.6),
    "c5d": dict(d=2048, E=64, k=4, h=1024, S=1, prec="fp4", T=64, layers=24, copies=1, seed=5, sets=4),
    "c5p": dict(d=2048, E=64, k=4, h=1024, S=1, prec="fp4", T=8192, layers=24, copies=1, seed=5, sets=4),
}


def weight_bytes_per_value(prec):
    return {"int8": 1.0, "fp4": 0.5, "fp32": 4.0}[prec]


def expert_bytes(c, rows, width):
    """Reference-format bytes of one rows x width matrix (codes + scales)."""
    b = weight_bytes_per_value(c["prec"])
    scales = 0 if c["prec"] == "fp32" else rows * ((width + 15) // 16) * 4
    return int(rows * width * b) + scales


def gateup_bytes(c, load, T):
    """Algorithmic HBM bytes of one gate/up launch: gate and up matrices of
    every expert with load > 0 (plus shared experts), the token rows read
    (fp32) and hidden rows written (fp32)."""
    active = int(np.count_nonzero(load)) + c["S"]
    return active * 2 * expert_bytes(c, c["h"], c["d"]) + T * c["d"] * 4 + (int(load.sum()) + c["S"] * T) * c["h"] * 4


def step_bytes(c, load, T):
    active = int(np.count_nonzero(load)) + c["S"]
    per_expert = 2 * expert_bytes(c, c["h"], c["d"]) + expert_bytes(c, c["d"], c["h"])
    return active * per_expert + c["E"] * c["d"] * 4 + c["E"] * 8 + 2 * T * c["d"] * 4


def gateup_flops(c, load, T):
    """Useful FLOPs of one gate/up launch: 2 * rows * (2h) * d."""
    rows = int(load.sum()) + c["S"] * T
    return 2.0 * rows * 2 * c["h"] * c["d"]


def layer_flops(c, T):
    return 2.0 * T * (c["E"] * c["d"] + (c["k"] + c["S"]) * 3 * c["d"] * c["h"])


def make_specs(gt, c):
    from tests.moe_fixtures import FLOAT32, FP4, INT8, make_moe, zipf_router_bias
    prec = {"int8": INT8, "fp4": FP4, "fp32": FLOAT32}[c["prec"]]
    bias = zipf_router_bias(c["E"], 1.2, seed=c["seed"], scale=c["zipf"]) if "zipf" in c else None
    sets = c.get("sets", 1)
    return [make_moe(gt.encode_rows, d=c["d"], h=c["h"], E=c["E"], k=c["k"], S=c["S"], precision=prec,
                     router_precision=FLOAT32, seed=c["seed"] + 101 * i, router_bias=bias) for i in range(sets)]


def host_cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_baseline(c, specs, budget_s):
    """The CPU restatement of the reference forward on the host cores, timed
    on a bounded sample of the workload's tokens."""
    import oracle
    cores = host_cores()
    tokens = min(c["T"], 32)
    x = np.random.default_rng(0).normal(size=(tokens, c["d"]))
    reps, t0 = 0, time.perf_counter()
    while True:
        if c["layers"] > 1:
            norms = [np.ones(c["d"])] * c["layers"]
            layers = [specs[i % len(specs)] for i in range(c["layers"])]
            oracle.stack_forward(layers, norms, x, threads=cores)
        else:
            oracle.moe_forward(specs[0], x, threads=cores)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    what = f"{c['layers']}-layer stack" if c["layers"] > 1 else "layer"
    return {"value": tokens * reps / el, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{reps} forwards of the {what} over {tokens} of the workload's tokens "
                      f"(float64 restatement, SplitAcrossThreads over {cores} threads), {el:.1f} s"}


def traffic_from_profiles(key):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        entry = json.load(f).get(key)
    return None if entry is None else entry.get("bytes_per_launch")


def transposed_bytes(c, load, T):
    """Algorithmic HBM bytes of the backward's three transposed products over
    the compressed rows (down, gate, up): every active expert's three
    matrices once, the gradients read and the input-side gradients written
    (fp32)."""
    active = int(np.count_nonzero(load)) + c["S"]
    P = int(load.sum()) + c["S"] * T
    per_expert = 2 * expert_bytes(c, c["h"], c["d"]) + expert_bytes(c, c["d"], c["h"])
    return active * per_expert + P * (c["d"] + c["h"] + 2 * c["h"] + c["h"] + 2 * c["d"]) * 4


def adapter_bench(args, c):
    """--adapters R: one training step of a layer whose every layer carries a
    rank-R adapter (alpha 2R): forward and backward through the host API
    (float64 rows in and out over PCIe, as the reference's Forward and
    Backward take them).  The roofline is for the transposed product over
    the compressed rows, timed by the library's per-kernel events."""
    import gotransformers_amd as gt
    from oracle import lora
    T, d = c["T"], c["d"]
    spec = make_specs(gt, c)[0]
    ctx = gt.Context(0)
    m = gt.MixtureOfExperts.from_spec(ctx, spec)
    m.add_adapters(args.adapters, 2.0 * args.adapters, seed=1)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((T, d))
    G = rng.uniform(-1, 1, (T, d))
    steps = args.steps or 50
    warmup = args.warmup if args.warmup is not None else 5
    for _ in range(warmup):
        m.forward(x)
        m.backward(G)
    t0 = time.perf_counter()
    for _ in range(steps):
        m.forward(x)
        m.backward(G)
    ms = (time.perf_counter() - t0) * 1e3 / steps
    load = m.last_expert_load()
    ctx.timing(True)
    ctx.timing_reset()
    n_detail = min(steps, 20)
    for _ in range(n_detail):
        m.forward(x)
        m.backward(G)
    times = ctx.timing_read()
    ctx.timing(False)
    m.destroy()
    ctx.close()
    tr_ms, tr_calls = times["rows_transposed"]
    per_step_s = tr_ms / n_detail / 1e3
    P = int(load.sum()) + c["S"] * T
    if T * c["k"] > 8 * c["E"]:  # many positions per expert: bound by arithmetic (fp32-exact products)
        work = 2.0 * P * 3 * c["d"] * c["h"]
        achieved = work / per_step_s / 1e12
        roof = {"bound": "mfma", "achieved": achieved, "peak": MFMA_FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": achieved / MFMA_FP32_PEAK_TFLOPS}
    else:
        work = transposed_bytes(c, load, T)
        achieved = work / per_step_s / 1e9
        roof = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": achieved / HBM_PEAK_GBS}
    roof.update({"traffic": None, "kernel": "rows_transposed", "algorithmic_per_step": work,
                 "mean_launch_us": tr_ms / tr_calls * 1e3, "launches_per_step": tr_calls / n_detail})
    cpu = None
    if not args.no_cpu:
        ads = lora.make_adapters(spec, args.adapters, 2.0 * args.adapters, np.random.default_rng(1))
        tokens = min(T, 8)
        reps, t0 = 0, time.perf_counter()
        while True:
            _, st = lora.forward(spec, ads, x[:tokens])
            lora.backward(spec, ads, st, G[:tokens], lora.zero_grads(spec, ads))
            reps += 1
            el = time.perf_counter() - t0
            if el >= args.cpu_seconds:
                break
        cpu = {"value": tokens * reps / el, "unit": "tokens/s", "cores": host_cores(), "kind": "port",
               "sample": f"{reps} forward+backward steps of the float64 adapter restatement (numpy) over "
                         f"{tokens} tokens, {el:.1f} s"}
    line = {
        "metric": "MoE-layer adapter training tokens/s (forward + backward, host API) @1 GPU",
        "value": T / (ms / 1e3), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"{args.workload} layer with rank-{args.adapters} adapters on every layer, T={T}",
                   "tokens": T, "d_model": d, "routed_experts": c["E"], "shared_experts": c["S"],
                   "top_k": c["k"], "expert_hidden": c["h"], "expert_weights": f"{c['prec']} per-16 fp32 scales"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "detail": {"kernel_ms_per_step_events": {k: v[0] / n_detail for k, v in sorted(times.items())}},
    }
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="c2", choices=sorted(WORKLOADS))
    ap.add_argument("--tokens", type=int, default=None)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--graph", action="store_true", help="replay each step as a recorded HIP graph")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run one 1 GiB device copy (for PMC byte-counter calibration)")
    ap.add_argument("--adapters", type=int, default=0,
                    help="time a training step (forward + backward) with rank-R adapters on every layer")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: --gpus {args.gpus} is not supported "
              f"(the path is measured at one GPU's share; DESIGN.md describes how it would shard)",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import gotransformers_amd as gt

    c = dict(WORKLOADS[args.workload])
    if args.tokens:
        c["T"] = args.tokens
    if args.adapters:
        if c["layers"] != 1:
            print("--adapters measures a single layer (c2, c3 or c4)", file=sys.stderr)
            sys.exit(2)
        adapter_bench(args, c)
        return
    T, d = c["T"], c["d"]
    prefill_like = T * c["k"] > 8 * c["E"]
    steps = args.steps or (400 if not prefill_like and c["layers"] == 1 else 30 if c["layers"] == 1 else 10)
    warmup = args.warmup if args.warmup is not None else max(3, steps // 10)
    warmup = max(warmup, c["copies"])  # every weight copy has run a forward before the relaunch burst

    specs = make_specs(gt, c)
    ctx = gt.Context(0)
    n_obj = c["copies"] * c["layers"]
    layers = [gt.MixtureOfExperts.from_spec(ctx, specs[i % len(specs)]) for i in range(n_obj)]
    if c["layers"] > 1:
        for m in layers:
            m.set_norm_weights(np.ones(d))
    g = torch.Generator(device="cpu").manual_seed(0)
    x0 = torch.randn(T, d, generator=g, dtype=torch.float32).cuda()
    x = x0.clone()
    y = torch.empty(T, d, dtype=torch.float32, device="cuda")

    # a stream of our own (default priority): its handle is non-null, so the
    # library launches on it and torch events recorded on it bracket our kernels
    stream = torch.cuda.Stream()
    sptr = stream.cuda_stream
    torch.cuda.set_stream(stream)

    graphs = []
    if args.graph:  # the step recorded once per weight copy and replayed as a HIP graph
        if c["layers"] > 1:
            graphs = [gt.Graph.capture_stack(layers, T, x.data_ptr(), path=gt.PATH_AUTO)]
        else:
            graphs = [gt.Graph.capture_forward(m, T, x.data_ptr(), y.data_ptr(), path=gt.PATH_AUTO)
                      for m in layers]

    def step(i):
        if c["layers"] > 1:
            x.copy_(x0)
            if graphs:
                graphs[0].launch(stream=sptr)
            else:
                gt.stack_forward_device(layers, T, x.data_ptr(), path=gt.PATH_AUTO, stream=sptr)
        elif graphs:
            graphs[i % c["copies"]].launch(stream=sptr)
        else:
            layers[i % c["copies"]].forward_device(T, x.data_ptr(), y.data_ptr(), path=gt.PATH_AUTO, stream=sptr)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    path = layers[0].last_path
    load = layers[0].last_expert_load()

    # timed region: K steps bracketed by synchronisation (no per-kernel events)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_plain = (t1 - t0) * 1e3 / steps

    # the dominant kernel: a burst of relaunches of the last forward's
    # gate/up kernel on the same stream, rotating through every resident
    # layer (so weight reads keep missing the Infinity Cache), bracketed by
    # one HIP event pair
    n_burst = max(len(layers), (200 if path == gt.PATH_FP32 else 20) // len(layers) * len(layers))
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for m in layers:
        m.relaunch(gt.KERNEL_GATEUP, stream=sptr)
    ev0.record(stream)
    for i in range(n_burst):
        layers[i % len(layers)].relaunch(gt.KERNEL_GATEUP, stream=sptr)
    ev1.record(stream)
    ev1.synchronize()
    kmean_s = ev0.elapsed_time(ev1) / n_burst / 1e3
    klaunch = n_burst

    # per-kernel breakdown: event pairs around every kernel over a few steps
    ctx.timing(True)
    ctx.timing_reset()
    n_detail = min(steps, 50)
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    for i in range(n_detail):
        step(i)
    torch.cuda.synchronize()
    t3 = time.perf_counter()
    times = ctx.timing_read()
    ctx.timing(False)
    ms_events = (t3 - t2) * 1e3 / n_detail

    if args.copy_calibration:
        a = torch.empty(1 << 28, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()

    decode = path == gt.PATH_FP32
    dominant = "gemv_gateup" if decode else "mfma_gateup"
    key = f"{dominant}/{args.workload}_t{T}"
    if decode:
        per_launch = gateup_bytes(c, load, T)
        achieved = per_launch / kmean_s / 1e9
        roof = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": achieved / HBM_PEAK_GBS, "traffic": traffic_from_profiles(key)}
    else:
        per_launch = gateup_flops(c, load, T)
        achieved = per_launch / kmean_s / 1e12
        roof = {"bound": "mfma", "achieved": achieved, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": achieved / MFMA_BF16_PEAK_TFLOPS, "traffic": traffic_from_profiles(key)}
    roof.update({"kernel": dominant, "algorithmic_per_launch": per_launch, "mean_launch_us": kmean_s * 1e6,
                 "launches": klaunch})

    for g in graphs:
        g.destroy()
    for m in layers:
        m.destroy()
    ctx.close()

    cpu = None if args.no_cpu else cpu_baseline(c, specs, args.cpu_seconds)

    names = {"c2": "C2 decode: MoE layer", "c3": "C3 prefill: MoE layer", "c4": "C4 skewed prefill: MoE layer",
             "c5d": "C5 decode: 24-block stack", "c5p": "C5 prefill: 24-block stack"}
    workload = (f"{names[args.workload]} d={d} E={c['E']}+{c['S']} shared k={c['k']} h={c['h']} "
                f"{c['prec']} experts, T={T}")
    step_layers = c["layers"]
    line = {
        "metric": METRIC,
        "value": T / (ms_plain / 1e3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_plain,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if decode else "bf16",
        "data": "synthetic",
        "config": {"workload": workload, "tokens": T, "d_model": d, "routed_experts": c["E"],
                   "shared_experts": c["S"], "top_k": c["k"], "expert_hidden": c["h"],
                   "expert_weights": f"{c['prec']} per-16 fp32 scales", "layers_per_step": step_layers,
                   "weight_copies": c["copies"],
                   "path": "fp32 dequant-GEMV" if decode else "bf16 MFMA grouped GEMM",
                   "hip_graph": bool(graphs)},
        "roofline": roof,
        "cpu_baseline": cpu,
        "detail": {
            "ms_per_step_with_kernel_events": ms_events,
            "kernel_ms_per_step_events": {k: v[0] / n_detail for k, v in sorted(times.items())},
            "active_experts_layer0": int(np.count_nonzero(load)),
            "step_algorithmic_bytes": step_bytes(c, load, T) * step_layers,
            "step_hbm_frac": step_bytes(c, load, T) * step_layers / (ms_plain / 1e3) / 1e9 / HBM_PEAK_GBS,
            "step_flops": layer_flops(c, T) * step_layers,
            "step_mfma_frac": layer_flops(c, T) * step_layers / (ms_plain / 1e3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
        },
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
