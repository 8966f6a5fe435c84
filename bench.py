#!/usr/bin/env python3
"""Benchmark of the PTO-WSP data-parallel tile path on one MI355X.

Default workload (the headline bandwidth config):
the README rmsnorm tile kernel over X[16, 8192, 16, 128] fp32 ~ N(0,1)
(1 GiB in, 1 GiB out), workload P(batch=16) x P(tiles=8192), schedule
round_robin(4) + TaskWindow(8192, STALL), compiled with
``compile(target="hip_gfx950")``.  A step is one ``execute()`` of the
compiled program over resident device buffers; K steps are timed between
``torch.cuda.synchronize()`` calls.

Besides the headline line's fields, ``configs`` reports every BASELINE
config this build runs (GB/s or TFLOP/s, fraction of the MI355X peak),
and ``cpu_baseline`` times this repository's C restatement of the
reference cpu_sim artifact (oracle/, 1 thread) on the same inputs.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME|all] [--no-cpu]
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "pto-wsp_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
METRIC = "GB/s & TFLOP/s as % of MI355X roofline per config, 1 GPU, vs cpu_sim wall"

CONFIGS = {
    "rmsnorm_quickstart": {"kind": "rmsnorm", "shape": (1, 2, 16, 128), "sigma": 1.0, "seed": 0,
                           "baseline_config": 0},
    "rmsnorm_bw": {"kind": "rmsnorm", "shape": (16, 8192, 16, 128), "sigma": 1.0, "seed": 0, "baseline_config": 1},
    "softmax": {"kind": "softmax", "shape": (8, 4096, 32, 512), "sigma": 3.0, "seed": 0, "baseline_config": 2},
}
HEADLINE = "rmsnorm_bw"


def make_workload(kind, X, Y):
    from pto_wsp import (DType, Dense, DispatchPolicy, In, Out, P, TaskWindow, Tensor, Tile, WindowMode,
                         kernel, pto, workload)

    f32 = DType.F32
    B, NT, R, C = tuple(X.shape)
    Xt = Tensor(data=X, shape=tuple(X.shape), dtype=f32)
    Yt = Tensor(data=Y, shape=tuple(Y.shape), dtype=f32)
    if kind == "rmsnorm":
        @kernel
        def rmsnorm_tile(x: In[Tile[R, C, f32]], out: Out[Tile[R, C, f32]]):
            sq = pto.mul(x, x)
            mean_sq = pto.rowmean(sq)
            inv = pto.rsqrt(mean_sq)
            pto.store(out, pto.mul(x, inv))

        body = rmsnorm_tile
    else:
        @kernel
        def softmax_tile(x: In[Tile[R, C, f32]], out: Out[Tile[R, C, f32]]):
            m = pto.rowmax(x)
            e = pto.exp(pto.sub(x, m))
            pto.store(out, pto.div(e, pto.rowsum(e)))

        body = softmax_tile

    batch, tiles = Dense[B](), Dense[NT]()

    @workload
    def wl():
        for b in P(batch):
            for t in P(tiles):
                body[b, t](x=Xt[b][t], out=Yt[b][t])

    return (wl().dispatch(DispatchPolicy.round_robin(num_aicpus=4))
            .task_graph(window=TaskWindow(8192, "tasks", WindowMode.STALL)))


def load_traffic(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/<name>_traffic.json), if committed."""
    path = os.path.join(ROOT, "profiles", f"{name}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("traffic_bytes")


def run_gpu(name, steps, warmup):
    import torch

    cfg = CONFIGS[name]
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(cfg["seed"])
    x = torch.randn(cfg["shape"], generator=gen, device=dev, dtype=torch.float32) * cfg["sigma"]
    y = torch.empty_like(x)
    prog = make_workload(cfg["kind"], x, y).compile(target="hip_gfx950")
    for _ in range(warmup):
        prog.execute()
        prog.synchronize()
    torch.cuda.synchronize()
    kernel_ms = []
    t0 = time.perf_counter()
    for _ in range(steps):
        prog.execute()
        prog.synchronize()
        kernel_ms.append(prog.stats.device_time_ms)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1000.0
    nbytes = 2 * x.numel() * 4
    ms_step = wall_ms / steps
    k_ms = sum(kernel_ms) / len(kernel_ms)
    achieved = nbytes / (k_ms * 1e-3) / 1e9
    return {
        "x": x, "y": y, "prog": prog,
        "ms_per_step": ms_step,
        "kernel_ms": k_ms,
        "gbps": nbytes / (ms_step * 1e-3) / 1e9,
        "achieved_gbps": achieved,
        "frac": achieved / HBM_PEAK_GBS,
        "bytes": nbytes,
        "tasks": prog.stats.task_count,
        "total_cycles": prog.stats.total_cycles,
    }


def run_cpu(name, x, budget_s=12.0, max_reps=8):
    """The oracle (C restatement of cpu_sim, 1 thread) on the same input."""
    import numpy as np

    from oracle.runner import run_workload

    cfg = CONFIGS[name]
    xh = x.detach().cpu().numpy()
    yh = np.zeros_like(xh)
    times = []
    t_start = time.perf_counter()
    while len(times) < max_reps and (time.perf_counter() - t_start) < budget_s:
        t0 = time.perf_counter()
        run_workload(make_workload(cfg["kind"], xh, yh))
        times.append(time.perf_counter() - t0)
    sec = sum(times) / len(times)
    nbytes = 2 * xh.nbytes
    return {"value": nbytes / sec / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"the full {name} workload X{list(cfg['shape'])}, {len(times)} run(s) of "
                      f"{sec:.2f} s each, wall clock around the oracle call, 1 of {len(os.sched_getaffinity(0))} cores",
            "y": yh}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="all", help=f"one of {list(CONFIGS)} or 'all'")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only; --gpus must be 1", file=sys.stderr)
        sys.exit(2)

    import torch

    if not os.path.exists(os.path.join(ROOT, "pto-wsp_amd", "pto_wsp", "libptowsp_hip.so")):
        import __graft_entry__

        __graft_entry__.build()
    assert torch.cuda.is_available(), "bench.py needs a GPU"

    names = list(CONFIGS) if args.config == "all" else [args.config]
    head = HEADLINE if HEADLINE in names else names[0]
    per = {}
    main_res = None
    cpu = None
    for name in names:
        steps = args.steps if name == head else max(3, args.steps // 4)
        r = run_gpu(name, steps, args.warmup)
        entry = {"baseline_config": CONFIGS[name]["baseline_config"], "shape": list(CONFIGS[name]["shape"]),
                 "kernel_ms": round(r["kernel_ms"], 5), "ms_per_step": round(r["ms_per_step"], 5),
                 "achieved": round(r["achieved_gbps"], 1), "unit": "GB/s", "peak": HBM_PEAK_GBS,
                 "frac": round(r["frac"], 4), "tasks": r["tasks"], "total_cycles": r["total_cycles"]}
        if not args.no_cpu and name in (head, "softmax"):
            c = run_cpu(name, r["x"], budget_s=12.0 if name == head else 6.0)
            import numpy as np

            same = bool(np.allclose(r["y"].cpu().numpy(), c.pop("y"), rtol=1e-5, atol=1e-6))
            entry["cpu_sim_port_gbps"] = round(c["value"], 4)
            entry["matches_cpu_sim"] = same
            if name == head:
                cpu = c
        per[name] = entry
        if name == head:
            main_res = r
        del r
        torch.cuda.empty_cache()

    cfg = CONFIGS[head]
    line = {
        "metric": METRIC,
        "value": round(main_res["gbps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_res["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (torch.randn on device, seeded)",
        "config": {"workload": f"{head}: rmsnorm_tile Tile[16,128,F32] over X{list(cfg['shape'])}, "
                               "P(batch=16) x P(tiles=8192), round_robin(4), TaskWindow(8192, STALL)",
                   "baseline_config": cfg["baseline_config"], "bytes_per_step": main_res["bytes"],
                   "target": "hip_gfx950"},
        "roofline": {"bound": "hbm", "achieved": round(main_res["achieved_gbps"], 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(main_res["frac"], 4), "traffic": load_traffic(head)},
        "cpu_baseline": cpu,
        "configs": per,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
