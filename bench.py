"""Benchmark of the MoE forward path on one MI355X.

Default workload (the largest configuration that fits one GPU): a stack of
24 blocks x <- x + MoE(RMSNorm(x)), each MoE layer d=2048, 64 routed experts
plus 1 shared expert, top-4, SwiGLU hidden 1024, FP4 expert weights (per-16
absmax/6 fp32 block scales), fp32 router; a prefill chunk of 8192 tokens
with N(0,1) activations resident in HBM; weights N(0, 0.02) from seeded
generators (four distinct weight sets cycled over the 24 layers, every layer
with its own resident copy, 7.4 GB).  A step is one pass of the 24-block
stack over the chunk (RMSNorm, router, top-k, dispatch, gate/up, down,
combine and residual per block).

`value` is tokens per second from the median of the per-step durations,
each bracketed by a HIP event pair on the stream the kernels run on (the
residual stream's reset before each step is outside the events).  The steps
are enqueued behind a bounded spin kernel, so they run back to back and the
events time the device rather than the host's enqueue of few-microsecond
launches.  The line also reports the mean over the same steps and the host's
time to enqueue one step (which the spin hides: a step whose enqueue takes
longer than its device time is host-bound without a captured graph).

`roofline` is for the dominant kernel (the MFMA grouped gate/up GEMM on the
prefill path, the dequant-GEMV gate/up on the decode path): achieved =
algorithmic FLOPs or bytes per launch / mean launch time, the mean taken by
HIP event pairs around rotations of back-to-back relaunches of that kernel:
on the decode path one relaunch per resident layer per rotation (the pass
over the layers a step makes, so the kernel runs as hot as in the steps),
each rotation behind a short spin, about 200 launches in all; on the prefill
path one rotation of 20-24 launches, no spin; `step_frac` is the whole step's algorithmic work
over the step time against the same peak.  `traffic` is the HBM bytes per
launch measured by rocprofv3 FETCH_SIZE / WRITE_SIZE passes for the same
workload, read from profiles/traffic.json and reported only when the
kernel sources it was measured on are the ones built now (null otherwise).

`detail.workloads` repeats the measurement, without CPU baseline, for the
other configurations: the decode chunk of the same stack (T=64), one Int8
decode layer (d=1024, 16 experts, top-2, h=2048) at T=1, 8 and 32, each
rotating over enough resident weight copies that the gate/up bytes of the
experts a step can activate, times the copies, come to at least 768 MB (three
times the 256 MB Infinity Cache; 77 copies at T=1, 10 at T=8 and T=32), so
every step and every relaunch reads its weights from HBM,
one FP4 prefill layer (d=1024, 64+1 experts, top-6, h=512, T=4096) and one
Int8 prefill layer with Zipf(1.2) router-bias skew (d=2048, 128 experts,
top-8, h=768, T=16384).  --workload picks another headline; --no-detail
skips the rest.

`cpu_baseline` times the CPU restatement of the reference algorithm
(oracle/, float64, the reference's SplitAcrossThreads policy) on a bounded
sample of the headline workload's tokens, on all host cores and on one.

--adapters R times a training step instead: forward and backward through
the host API with rank-R adapters on every layer of the mixture."""
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
    "c2": dict(d=1024, E=16, k=2, h=2048, S=0, prec="int8", T=32, layers=1, copies=None, seed=0),
    "c3": dict(d=1024, E=64, k=6, h=512, S=1, prec="fp4", T=4096, layers=1, copies=1, seed=3),
    "c4": dict(d=2048, E=128, k=8, h=768, S=0, prec="int8", T=16384, layers=1, copies=1, seed=4, zipf=0.6),
    "c5d": dict(d=2048, E=64, k=4, h=1024, S=1, prec="fp4", T=64, layers=24, copies=1, seed=5, sets=4),
    "c5p": dict(d=2048, E=64, k=4, h=1024, S=1, prec="fp4", T=8192, layers=24, copies=1, seed=5, sets=4),
}


# Single-layer decode workloads rotate over this many bytes of the experts a
# step can activate (three times the 256 MB Infinity Cache), so that no step
# and no relaunch finds its weights in the cache.
CACHE_DEFEAT_BYTES = 768 << 20


def weight_copies(c):
    """Resident weight copies a workload rotates over: one for stacks (every
    layer has its own copy) and prefill layers (every expert is read per
    step, bytes far beyond the cache); for a decode layer enough copies that
    the gate/up bytes of the min(T*k, E) + S experts a step can activate,
    times the copies, reach CACHE_DEFEAT_BYTES."""
    if c.get("copies"):
        return c["copies"]
    if c["layers"] > 1 or c["T"] * c["k"] > 8 * c["E"]:
        return 1
    active = min(c["T"] * c["k"], c["E"]) + c["S"]
    per_copy = active * 2 * expert_bytes(c, c["h"], c["d"])
    return max(4, -(-CACHE_DEFEAT_BYTES // per_copy))


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


def step_bytes(c, loads, T):
    """Algorithmic HBM bytes of one step: per layer, the three matrices of
    every expert with load > 0 plus the shared experts, the router, and the
    token rows in and out (fp32)."""
    per_expert = 2 * expert_bytes(c, c["h"], c["d"]) + expert_bytes(c, c["d"], c["h"])
    total = 0
    for load in loads:
        active = int(np.count_nonzero(load)) + c["S"]
        total += active * per_expert + c["E"] * c["d"] * 4 + c["E"] * 8 + 2 * T * c["d"] * 4
    return total


def gateup_flops(c, load, T):
    """Useful FLOPs of one gate/up launch: 2 * rows * (2h) * d."""
    rows = int(load.sum()) + c["S"] * T
    return 2.0 * rows * 2 * c["h"] * c["d"]


def layer_flops(c, T):
    return 2.0 * T * (c["E"] * c["d"] + (c["k"] + c["S"]) * 3 * c["d"] * c["h"])


def make_specs(gt, c):
    """The workload's distinct weight sets, each expert drawn N(0, 0.02) from
    its own seeded generator and encoded on a thread pool."""
    from tests.moe_fixtures import FLOAT32, FP4, INT8, make_moe_parallel, zipf_router_bias
    prec = {"int8": INT8, "fp4": FP4, "fp32": FLOAT32}[c["prec"]]
    bias = zipf_router_bias(c["E"], 1.2, seed=c["seed"], scale=c["zipf"]) if "zipf" in c else None
    sets = c.get("sets", 1)
    return [make_moe_parallel(gt.encode_rows, d=c["d"], h=c["h"], E=c["E"], k=c["k"], S=c["S"], precision=prec,
                              router_precision=FLOAT32, seed=c["seed"] + 101 * i, router_bias=bias,
                              threads=min(16, host_cores())) for i in range(sets)]


def host_cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_once(c, specs, budget_s, threads, tokens):
    """The CPU restatement of the reference forward (float64, the
    reference's SplitAcrossThreads policy over `threads` threads), timed on
    `tokens` of the workload's tokens for about budget_s seconds."""
    import oracle
    x = np.random.default_rng(0).normal(size=(tokens, c["d"]))
    reps, t0 = 0, time.perf_counter()
    while True:
        if c["layers"] > 1:
            norms = [np.ones(c["d"])] * c["layers"]
            layers = [specs[i % len(specs)] for i in range(c["layers"])]
            oracle.stack_forward(layers, norms, x, threads=threads)
        else:
            oracle.moe_forward(specs[0], x, threads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    what = f"{c['layers']}-block stack" if c["layers"] > 1 else "layer"
    return {"value": tokens * reps / el, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{reps} forward(s) of the {what} over {tokens} of the workload's tokens "
                      f"(float64 restatement, SplitAcrossThreads over {threads} thread(s)), {el:.1f} s"}


def cpu_baseline(c, specs, budget_s):
    """All host cores, then one core (half the budget each), with the CPU model."""
    cores = host_cores()
    allc = cpu_baseline_once(c, specs, budget_s / 2, cores, min(c["T"], 32))
    one = cpu_baseline_once(c, specs, budget_s / 2, 1, min(c["T"], 4 if c["layers"] > 1 else 8))
    allc["cpu_model"] = cpu_model()
    allc["one_core"] = one
    return allc


# the sources a kernel is built from (its measured traffic and profiles hold
# for these bytes only); also the kernels' routing neighbours for the
# decode profiles
TRAFFIC_SOURCES = {
    "mfma_gateup": ["experts_mfma.hip", "mfma.h", "common.h"],
    "gemv_gateup": ["experts_gemv.hip", "common.h"],
    "route": ["route.hip", "kernels.h", "common.h", "mfma.h"],
}


def sources_digest(kernel):
    import hashlib
    h = hashlib.sha256()
    for name in TRAFFIC_SOURCES[kernel]:
        with open(os.path.join(ROOT, "gotransformers_amd", "csrc", name), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def traffic_from_profiles(kernel, key):
    """HBM bytes per launch of `kernel` measured (rocprofv3 FETCH_SIZE and
    WRITE_SIZE passes) on workload `key`, if it was measured on the kernel
    sources built now; None otherwise."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        entry = json.load(f).get(key)
    if entry is None or entry.get("sources") != sources_digest(kernel):
        return None
    return entry.get("bytes_per_launch")


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




NAMES = {"c2": "C2 decode: MoE layer", "c3": "C3 prefill: MoE layer", "c4": "C4 skewed prefill: MoE layer",
         "c5d": "C5 decode: 24-block stack", "c5p": "C5 prefill: 24-block stack"}


def workload_name(key, c):
    return (f"{NAMES[key]} d={c['d']} E={c['E']}+{c['S']} shared k={c['k']} h={c['h']} "
            f"{c['prec']} experts, T={c['T']}")


def build_layers(gt, ctx, c, specs):
    n_obj = c["copies"] * c["layers"]
    layers = [gt.MixtureOfExperts.from_spec(ctx, specs[i % len(specs)]) for i in range(n_obj)]
    if c["layers"] > 1:
        for m in layers:
            m.set_norm_weights(np.ones(c["d"]))
    return layers


# Shader-clock cycles of the spin kernel that holds a stream while the host
# enqueues timed work behind it: the enqueue of a few-microsecond launch costs
# the host about as long as the launch runs, so without it the events would
# time the host (under a kernel tracer, several times as long).  About 33 ms
# at 2.4 GHz ahead of the timed steps, 10 ms ahead of each relaunch rotation.
HOLD_STEPS = 80_000_000
HOLD_ROTATION = 25_000_000


def hold_queue(torch, cycles=HOLD_STEPS):
    """A bounded spin on the current stream."""
    torch.cuda._sleep(cycles)


def measure(gt, torch, ctx, c, key, layers, steps, warmup, stream, graph=False, n_detail=20):
    """One workload on resident layers: per-step event times, the dominant
    kernel's relaunch burst and the per-kernel breakdown."""
    T, d = c["T"], c["d"]
    sptr = stream.cuda_stream
    g = torch.Generator(device="cpu").manual_seed(0)
    x0 = torch.randn(T, d, generator=g, dtype=torch.float32).cuda()
    x = x0.clone()
    y = torch.empty(T, d, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    graphs = []
    if graph:  # the step recorded once per weight copy and replayed as a HIP graph
        if c["layers"] > 1:
            graphs = [gt.Graph.capture_stack(layers, T, x.data_ptr(), path=gt.PATH_AUTO)]
        else:
            graphs = [gt.Graph.capture_forward(m, T, x.data_ptr(), y.data_ptr(), path=gt.PATH_AUTO)
                      for m in layers]

    def prepare(i):
        if c["layers"] > 1:
            x.copy_(x0)  # the stack updates x in place

    def step(i):
        if c["layers"] > 1:
            if graphs:
                graphs[0].launch(stream=sptr)
            else:
                gt.stack_forward_device(layers, T, x.data_ptr(), path=gt.PATH_AUTO, stream=sptr)
        elif graphs:
            graphs[i % c["copies"]].launch(stream=sptr)
        else:
            layers[i % c["copies"]].forward_device(T, x.data_ptr(), y.data_ptr(), path=gt.PATH_AUTO, stream=sptr)

    with torch.cuda.stream(stream):
        for i in range(warmup):
            prepare(i)
            step(i)
        torch.cuda.synchronize()
        path = layers[0].last_path
        loads = [m.last_expert_load() for m in layers[:c["layers"]]]

        # timed steps: an event pair on the kernels' stream around each step,
        # all enqueued behind a spin kernel so that the steps then run back to
        # back, as a captured graph would run them (the host's enqueue time is
        # outside the events; enqueue_ms is what it costs per step)
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        torch.cuda.synchronize()
        hold_queue(torch)
        t0 = time.perf_counter()
        for i in range(steps):
            prepare(i)
            evs[i][0].record(stream)
            step(i)
            evs[i][1].record(stream)
        enqueue_ms = (time.perf_counter() - t0) * 1e3 / steps
        torch.cuda.synchronize()
        step_ms = np.array([a.elapsed_time(b) for a, b in evs])

        # the dominant kernel: rotations of relaunches of each layer's gate/up
        # kernel of its last forward over every resident layer (so weight
        # reads keep missing the Infinity Cache), one event pair around each
        # rotation, each rotation behind a short spin.  One rotation is one
        # pass over the resident layers, as the steps make it: a long
        # back-to-back burst of the kernel alone runs hotter than the steps
        # do, and its later launches slow down (about 15% at C5 decode).
        # (prefill: one rotation of at least 20 launches and no spin: its
        # launches take hundreds of microseconds each, far longer than their
        # enqueue, and a rotation right after a spin, with the chip idle
        # meanwhile, measured 15-20% slower than the same kernel in the steps)
        if path == gt.PATH_FP32:
            per_rot, rotations = len(layers), max(1, -(-200 // len(layers)))
        else:
            per_rot, rotations = max(len(layers), 20 // len(layers) * len(layers)), 1
        for m in layers:
            m.relaunch(gt.KERNEL_GATEUP, stream=sptr)
        rot_ms = []
        for _ in range(rotations):
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            if path == gt.PATH_FP32:
                hold_queue(torch, HOLD_ROTATION)
            ev0.record(stream)
            for i in range(per_rot):
                layers[i % len(layers)].relaunch(gt.KERNEL_GATEUP, stream=sptr)
            ev1.record(stream)
            rot_ms.append((ev0, ev1))
        torch.cuda.synchronize()
        n_burst = rotations * per_rot
        kmean_s = sum(a.elapsed_time(b) for a, b in rot_ms) / n_burst / 1e3

        # per-kernel breakdown: the library's event pair around every kernel
        ctx.timing(True)
        ctx.timing_reset()
        n_detail = min(steps, n_detail)
        for i in range(n_detail):
            prepare(i)
            step(i)
        times = ctx.timing_read()
        ctx.timing(False)
    for gr in graphs:
        gr.destroy()

    decode = path == gt.PATH_FP32
    med_s = float(np.median(step_ms)) / 1e3
    if decode:
        kernel = "gemv_gateup"
        per_launch = gateup_bytes(c, loads[0], T)
        achieved = per_launch / kmean_s / 1e9
        step_work = step_bytes(c, loads, T) * (1 if c["layers"] > 1 else 1)
        roof = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": achieved / HBM_PEAK_GBS}
        step_achieved = step_work / med_s / 1e9
    else:
        kernel = "mfma_gateup"
        per_launch = gateup_flops(c, loads[0], T)
        achieved = per_launch / kmean_s / 1e12
        step_work = layer_flops(c, T) * c["layers"]
        roof = {"bound": "mfma", "achieved": achieved, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": achieved / MFMA_BF16_PEAK_TFLOPS}
        step_achieved = step_work / med_s / 1e12
    roof.update({"traffic": traffic_from_profiles(kernel, f"{kernel}/{key}_t{T}"), "kernel": kernel,
                 "algorithmic_per_launch": per_launch, "mean_launch_us": kmean_s * 1e6, "launches": n_burst,
                 "step_achieved": step_achieved, "step_frac": step_achieved / roof["peak"],
                 "step_algorithmic": step_work})
    return {
        "path": path, "decode": decode, "loads": loads, "ms_median": med_s * 1e3,
        "ms_mean": float(step_ms.mean()), "ms_min": float(step_ms.min()), "ms_max": float(step_ms.max()),
        "enqueue_ms": enqueue_ms, "value": T / med_s, "roofline": roof,
        "kernel_ms_per_step": {k: v[0] / n_detail for k, v in sorted(times.items())},
    }


def summary(key, c, r):
    roof = r["roofline"]
    return {"workload": workload_name(key, c), "tokens_per_s": r["value"], "ms_per_step_median": r["ms_median"],
            "ms_per_step_mean": r["ms_mean"], "path": "fp32 dequant-GEMV" if r["decode"] else "bf16 MFMA grouped GEMM",
            "kernel": roof["kernel"], "kernel_us": roof["mean_launch_us"], "bound": roof["bound"],
            "kernel_achieved": roof["achieved"], "kernel_frac": roof["frac"], "traffic": roof["traffic"],
            "step_achieved": roof["step_achieved"], "step_frac": roof["step_frac"], "unit": roof["unit"],
            "kernel_ms_per_step": r["kernel_ms_per_step"],
            "active_experts_layer0": int(np.count_nonzero(r["loads"][0])),
            "weight_copies": c["copies"], "rotated_gateup_weight_bytes": rotated_bytes(c, r)}


def rotated_bytes(c, r):
    """Gate/up weight bytes of the active experts over every resident copy
    or layer the steps and relaunch bursts rotate through (each layer's
    realised routing)."""
    per_layer = [(int(np.count_nonzero(l)) + c["S"]) * 2 * expert_bytes(c, c["h"], c["d"]) for l in r["loads"]]
    return int(sum(per_layer) * c["copies"])


def measure_host_api(gt, c, layers, reps=200):
    """The drop-in's own call path, as go/mixtureofexperts/gpu_unix.go makes it
    for every Forward: gtmoe_set_balance_biases, gtmoe_forward (float64 rows
    in over PCIe, float64 rows out, blocking until they are back) and
    gtmoe_last_routing of the cached routing state (chosen experts, gates,
    load, rows for each expert and their offsets), through ctypes on
    preallocated buffers, rotating over the resident layers.  Wall clock per
    Forward, and per call when each is repeated alone."""
    import ctypes as C
    lib = gt.library()
    T, d, k, E = c["T"], c["d"], c["k"], c["E"]
    x = np.random.default_rng(1).standard_normal((T, d))
    y = np.empty_like(x)
    bal = np.zeros(E)
    chosen, rows = np.empty(T * k, np.int32), np.empty(T * k, np.int32)
    gates = np.empty(T * k)
    load, offs = np.empty(E, np.int32), np.empty(E + 1, np.int32)
    got = C.c_int32()
    px, py, pb = x.ctypes.data, y.ctypes.data, bal.ctypes.data
    pc, pg, pl, pr, po = (a.ctypes.data for a in (chosen, gates, load, rows, offs))
    handles = [m.handle for m in layers]

    def balance(h):
        return lib.gtmoe_set_balance_biases(h, pb)

    def forward(h):
        return lib.gtmoe_forward(h, T, px, None, py, 0)

    def routing(h):
        return lib.gtmoe_last_routing(h, C.byref(got), pc, pg, pl, pr, po)

    def run(calls, n):
        for i in range(len(handles)):  # every layer once first
            for f in calls:
                assert f(handles[i]) == 0
        t0 = time.perf_counter()
        for i in range(n):
            h = handles[i % len(handles)]
            for f in calls:
                if f(h) != 0:
                    raise RuntimeError("host API call failed")
        return (time.perf_counter() - t0) / n * 1e6

    per_forward = run((balance, forward, routing), reps)
    parts = {"set_balance_biases": run((balance,), reps), "forward": run((forward,), reps)}
    # gtmoe_last_routing alone reads the same forward's state again (the
    # dispatch tables, once built, are not rebuilt)
    parts["last_routing_after_forward"] = per_forward - parts["set_balance_biases"] - parts["forward"]
    return {"us_per_forward": per_forward, "us_per_call": parts, "layers_rotated": len(handles), "reps": reps,
            "tokens_per_s": T / (per_forward / 1e6)}


def run_detail(gt, torch, ctx, stream, keys, shared, args):
    """The other workloads, each on its own resident layers (the C5 decode
    chunk reuses the stack of the C5 prefill headline when it was built)."""
    out = []
    for key, tokens in keys:
        c = dict(WORKLOADS[key])
        if tokens:
            c["T"] = tokens
        c["copies"] = weight_copies(c)
        reuse = shared.get(c.get("seed"), None) if key in ("c5d", "c5p") else None
        layers = reuse if reuse is not None else build_layers(gt, ctx, c, make_specs(gt, c))
        steps = 50 if c["layers"] > 1 or c["T"] * c["k"] > 8 * c["E"] else 200
        host = None
        try:
            r = measure(gt, torch, ctx, c, key, layers, steps, max(5, c["copies"]), stream)
            if key == "c2" and c["T"] in (1, 32) or key == "c5d":
                # the Go drop-in's per-Forward calls on one layer of this shape
                host = measure_host_api(gt, dict(c, layers=1), layers[:c["layers"] * c["copies"]])
                host["device_us_per_layer"] = r["ms_median"] * 1e3 / c["layers"]
        finally:
            if reuse is None:
                for m in layers:
                    m.destroy()
        s = summary(key, c, r)
        if host:
            s["host_api"] = host
        if key == "c4":
            load = np.sort(r["loads"][0])[::-1]
            s["realized_load_desc_first8"] = load[:8].tolist()
            s["realized_load_median"] = int(np.median(load))
            s["realized_load_min"] = int(load[-1])
        out.append(s)
        print(f"detail {key} T={c['T']}: {s['tokens_per_s']:.0f} tokens/s, {s['kernel']} "
              f"{s['kernel_frac'] * 100:.1f}% of peak, step {s['step_frac'] * 100:.1f}%", file=sys.stderr, flush=True)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="c5p", choices=sorted(WORKLOADS))
    ap.add_argument("--tokens", type=int, default=None)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-detail", action="store_true", help="measure the headline workload only")
    ap.add_argument("--graph", action="store_true", help="replay each step as a recorded HIP graph")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run one 1 GiB device copy (for PMC byte-counter calibration)")
    ap.add_argument("--adapters", type=int, default=0,
                    help="time a training step (forward + backward) with rank-R adapters on every layer")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: --gpus {args.gpus} is not supported "
              f"(the path is measured at one GPU's share: a layer's experts, router and shared experts on one "
              f"device)",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import gotransformers_amd as gt

    key = args.workload
    c = dict(WORKLOADS[key])
    if args.tokens:
        c["T"] = args.tokens
    c["copies"] = weight_copies(c)
    if args.adapters:
        if c["layers"] != 1:
            print("--adapters measures a single layer (c2, c3 or c4)", file=sys.stderr)
            sys.exit(2)
        adapter_bench(args, c)
        return
    T, d = c["T"], c["d"]
    steps = args.steps or (200 if c["layers"] == 1 and T * c["k"] <= 8 * c["E"] else 50)
    warmup = args.warmup if args.warmup is not None else max(3, min(10, steps // 10))
    warmup = max(warmup, c["copies"])  # every weight copy has run a forward before the relaunch burst

    specs = make_specs(gt, c)
    ctx = gt.Context(0)
    # a stream of our own (default priority): the library launches on it and
    # the events recorded on it bracket our kernels
    stream = torch.cuda.Stream()
    layers = build_layers(gt, ctx, c, specs)
    r = measure(gt, torch, ctx, c, key, layers, steps, warmup, stream, graph=args.graph)

    if args.copy_calibration:
        a = torch.empty(1 << 28, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        del a, b

    detail_workloads = []
    if not args.no_detail:
        plan = [("c5d", None), ("c5p", None), ("c2", 1), ("c2", 8), ("c2", 32), ("c3", None), ("c4", None)]
        plan = [(k, t) for k, t in plan if not (k == key and (t or WORKLOADS[k]["T"]) == T)]
        shared = {c["seed"]: layers} if key in ("c5d", "c5p") else {}
        detail_workloads = run_detail(gt, torch, ctx, stream, plan, shared, args)
    for m in layers:
        m.destroy()
    ctx.close()

    cpu = None if args.no_cpu else cpu_baseline(c, specs, args.cpu_seconds)

    decode = r["decode"]
    line = {
        "metric": METRIC,
        "value": r["value"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": r["ms_median"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if decode else "bf16",
        "data": "synthetic",
        "config": {"workload": workload_name(key, c), "tokens": T, "d_model": d, "routed_experts": c["E"],
                   "shared_experts": c["S"], "top_k": c["k"], "expert_hidden": c["h"],
                   "expert_weights": f"{c['prec']} per-16 fp32 scales", "layers_per_step": c["layers"],
                   "weight_copies": c["copies"], "rotated_gateup_weight_bytes": rotated_bytes(c, r),
                   "path": "fp32 dequant-GEMV" if decode else "bf16 MFMA grouped GEMM",
                   "hip_graph": bool(args.graph), "step_timing": "median of per-step HIP event pairs; steps enqueued behind a spin kernel, so they run back to back"},
        "roofline": r["roofline"],
        "cpu_baseline": cpu,
        "detail": {
            "ms_per_step_mean": r["ms_mean"], "ms_per_step_min": r["ms_min"], "ms_per_step_max": r["ms_max"],
            "host_enqueue_ms_per_step": r["enqueue_ms"],
            "kernel_ms_per_step_events": r["kernel_ms_per_step"],
            "active_experts_layer0": int(np.count_nonzero(r["loads"][0])),
            "workloads": detail_workloads,
        },
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
