"""Benchmark of the MoE layer forward on one MI355X.

Workload (the decode configuration the metric is quoted on): one MoE layer,
d=1024, 16 routed experts, top-2, SwiGLU hidden 2048, Int8 expert weights
(per-16 absmax/127 block scales), fp32 router, a batch of 32 tokens with
N(0,1) activations resident in HBM; weights N(0, 0.02), seed 0.  A step is
one layer forward (router, top-k, dispatch, gate/up, down, combine).

Four copies of the layer's weights (4 x 126 MB) are used round-robin so the
256 MB Infinity Cache cannot hold the weight set: the gate/up and down
kernels read their weights from HBM.

Prints one JSON line.  `roofline` is for the dominant kernel (gemv_gateup):
achieved = algorithmic bytes per launch / mean launch time from HIP events
recorded around every kernel of the timed region.  `cpu_baseline` times the
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
D, E, K, H = 1024, 16, 2, 2048
COPIES = 4


def expert_specs(gt, seed):
    """Encoded weights of one layer (same arrays for every copy)."""
    from tests.moe_fixtures import FLOAT32, INT8, make_moe
    return make_moe(gt.encode_rows, d=D, h=H, E=E, k=K, S=0, precision=INT8, router_precision=FLOAT32, seed=seed)


def gateup_bytes(load, tokens):
    """Algorithmic HBM bytes of one gemv_gateup launch: gate and up rows
    (Int8 codes + fp32 scale per 16) of every expert with load > 0, the
    token rows it reads (fp32) and the hidden rows it writes (fp32)."""
    active = int(np.count_nonzero(load))
    weights = active * 2 * H * (D + D // 16 * 4)
    return weights + tokens * D * 4 + int(load.sum()) * H * 4


def step_bytes(load, tokens):
    """Algorithmic HBM bytes of a whole layer forward (for the extra
    whole-step fraction): router, all weights of active experts, inputs,
    outputs."""
    active = int(np.count_nonzero(load))
    per_expert = 3 * D * H + 3 * D * H // 16 * 4
    return active * per_expert + E * D * 4 + E * 8 + 2 * tokens * D * 4


def cpu_baseline(spec, tokens, budget_s):
    import oracle
    cores = os.cpu_count() or 1
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        pass
    x = np.random.default_rng(0).normal(size=(tokens, D))
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.moe_forward(spec, x, threads=cores)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return {"value": tokens * reps / el, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{reps} forwards of the same layer at T={tokens} (float64 restatement, "
                      f"SplitAcrossThreads over {cores} threads), {el:.1f} s"}


def traffic_from_profiles(workload_key):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        data = json.load(f)
    entry = data.get(workload_key)
    return None if entry is None else entry.get("bytes_per_launch")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--tokens", type=int, default=32)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run one 1 GiB device copy (for PMC byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: --gpus {args.gpus} is not supported "
              f"(the path is measured at one GPU's share; see DESIGN.md for sharding)", file=sys.stderr)
        sys.exit(2)

    import torch
    import gotransformers_amd as gt

    T = args.tokens
    spec = expert_specs(gt, seed=0)
    ctx = gt.Context(0)
    layers = [gt.MixtureOfExperts.from_spec(ctx, spec) for _ in range(COPIES)]
    g = torch.Generator(device="cpu").manual_seed(0)
    x = torch.randn(T, D, generator=g, dtype=torch.float32).cuda()
    y = torch.empty(T, D, dtype=torch.float32, device="cuda")

    def step(i):
        layers[i % COPIES].forward_device(T, x.data_ptr(), y.data_ptr(), path=gt.PATH_AUTO)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    path = layers[0].last_path
    load = layers[0].last_expert_load()

    # timed region: K steps, per-kernel HIP events on the layer's stream
    ctx.timing(True)
    ctx.timing_reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    times = ctx.timing_read()
    ctx.timing(False)
    ms_per_step = (t1 - t0) * 1e3 / args.steps

    # the same K steps without per-kernel events (launch overhead of events excluded)
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    t3 = time.perf_counter()
    ms_plain = (t3 - t2) * 1e3 / args.steps

    if args.copy_calibration:
        a = torch.empty(1 << 28, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()

    dominant = "gemv_gateup" if path == gt.PATH_FP32 else "mfma_gateup"
    kms, klaunch = times.get(dominant, (float("nan"), 1))
    kmean_s = kms / klaunch / 1e3
    gbytes = gateup_bytes(load, T)
    achieved = gbytes / kmean_s / 1e9
    workload = f"C2 decode: MoE layer d={D} E={E} k={K} h={H} Int8 experts, T={T}"
    traffic = traffic_from_profiles(f"{dominant}/c2_int8_t{T}")
    step_total_ms = sum(v[0] for v in times.values()) / args.steps

    for m in layers:
        m.destroy()
    ctx.close()

    cpu = None if args.no_cpu else cpu_baseline(spec, T, args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": T / (ms_plain / 1e3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_plain,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": workload, "tokens": T, "d_model": D, "routed_experts": E, "top_k": K,
                   "expert_hidden": H, "expert_weights": "Int8 per-16 fp32 scales", "weight_copies": COPIES,
                   "path": "fp32 dequant-GEMV" if path == gt.PATH_FP32 else "bf16 MFMA"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic, "kernel": dominant,
                     "algorithmic_bytes_per_launch": gbytes, "mean_launch_us": kmean_s * 1e6},
        "cpu_baseline": cpu,
        "detail": {
            "ms_per_step_with_kernel_events": ms_per_step,
            "kernel_ms_per_step": {k: v[0] / args.steps for k, v in sorted(times.items())},
            "sum_of_kernel_ms_per_step": step_total_ms,
            "active_experts": int(np.count_nonzero(load)),
            "step_algorithmic_bytes": step_bytes(load, T),
            "step_hbm_frac": step_bytes(load, T) / (ms_plain / 1e3) / 1e9 / HBM_PEAK_GBS,
        },
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
