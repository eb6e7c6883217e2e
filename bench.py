"""Throughput of the reflector-free batched QR on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 4] [--no-cpu] [--no-geqrf]

A step is one factorization of the configuration's whole batch (inputs resident in HBM,
outputs written to preallocated buffers, no host synchronisation inside).  Prints one JSON
line.  Default workload: BASELINE configuration 4, 256 x 512 x 512 fp32, six pathology
classes cycled (synthetic, seeded).
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import platform
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "matrices/sec + % fp32-MFMA roofline, batched QR n=512 fp32 (1 GPU)"
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0


def _events_ms(fn, reps: int, stream) -> float:
    """Average ms of fn() over reps calls, timed with HIP events on `stream`."""
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        fn()
    stop.record(stream)
    stop.synchronize()
    return start.elapsed_time(stop) / reps


def _cpu_name() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(A_cpu: torch.Tensor, classes: int, budget_s: float = 10.0):
    """The oracle (torch-CPU restatement of the reference, fp32) on a bounded sample."""
    from oracle import rnr as orc

    # torch's own intra-op thread count (OMP_NUM_THREADS where set).  It is deliberately not
    # changed: calling torch.set_num_threads at all makes this image's MKL batched sgetrf fail
    # (SLASWP parameter error, then a hang) on these inputs.
    cores = torch.get_num_threads()
    sample = A_cpu[: max(1, classes)].contiguous()
    orc.custom_kernel(sample[:1])  # warm-up
    t0 = time.perf_counter()
    reps = 0
    while reps < 1 or time.perf_counter() - t0 < budget_s:
        orc.custom_kernel(sample)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    torch.geqrf(sample)
    t1 = time.perf_counter()
    greps = 0
    while greps < 3 or time.perf_counter() - t1 < 2.0:
        torch.geqrf(sample)
        greps += 1
    dtg = (time.perf_counter() - t1) / greps
    return {
        "value": sample.shape[0] / dt,
        "unit": "matrices/s",
        "cores": cores,
        "kind": "port",
        "sample": f"first {sample.shape[0]} matrices of the same batch (every class), "
                  f"{reps} repetitions in {dt * reps:.1f} s; CPU: {_cpu_name()}",
        "torch_geqrf_cpu": sample.shape[0] / dtg,
    }


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=4)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-geqrf", action="store_true")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (the batch is independent per matrix; "
              "multi-GPU sharding is a design note, not implemented)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)

    wl = importlib.import_module("qr-contest_amd.workloads")
    rnr = importlib.import_module("qr-contest_amd.reflection_no_reflectors")
    native = importlib.import_module("qr-contest_amd._native")
    cfg = wl.CONFIGS[args.config]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    A_cpu = wl.make_batch(args.config)
    A = A_cpu.to(dev)
    plan = rnr.QRPlan(cfg.batch, cfg.n, dev)
    stream = torch.cuda.current_stream(dev)

    for _ in range(args.warmup):
        plan.run(A)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ms_ev = _events_ms(lambda: plan.run(A), args.steps, stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ms = ms_ev
    mats_per_s = cfg.batch / (ms / 1e3)
    nominal_tflops = cfg.nominal_flops_per_matrix * cfg.batch / (ms / 1e3) / 1e12
    gbs = cfg.bytes_per_matrix * cfg.batch / (ms / 1e3) / 1e9

    # validity of what was timed: gates on one matrix per class of the last step's output
    from oracle import checker
    k = min(cfg.batch, 6)
    H, tau = plan.H[:k].cpu(), plan.tau[:k].cpu()
    fr, og, ft, ot, ok = checker.check(A_cpu[:k], H, tau)
    info_ok = int(plan.info.abs().sum().item()) == 0

    # the path's kernels one at a time, through the single-launch stage entry points
    stages = {}
    lib = native.lib()
    Lb = torch.empty_like(A)
    perm = torch.empty(cfg.batch, cfg.n, dtype=torch.int32, device=dev)
    ws_lu = torch.empty(native.workspace_bytes("lu", cfg.batch, cfg.n), dtype=torch.uint8, device=dev)
    nn = cfg.n * cfg.n

    def run_lu():
        native.check("rnr_lu_f32", lib.rnr_lu_f32(A.data_ptr(), cfg.batch, cfg.n, nn, Lb.data_ptr(),
                                                  perm.data_ptr(), ws_lu.data_ptr(), ws_lu.numel(),
                                                  stream.cuda_stream))
    Yb = plan.H.clone()
    s_b = torch.empty(cfg.batch, cfg.n, device=dev)
    t_b = torch.empty(cfg.batch, cfg.n, device=dev)

    def run_chart():
        native.check("rnr_chart_f32", lib.rnr_chart_f32(Yb.data_ptr(), cfg.batch, cfg.n, s_b.data_ptr(),
                                                        t_b.data_ptr(), stream.cuda_stream))
    run_lu(); run_chart()
    torch.cuda.synchronize()
    reps = max(3, args.steps // 2)
    stages["k_lu_pivot_ms"] = _events_ms(run_lu, reps, stream)
    stages["k_lu_chart_ms"] = _events_ms(run_chart, reps, stream)

    n3 = float(cfg.n) ** 3
    lu_flops = 2.0 / 3.0 * n3 * cfg.batch
    lu_tflops = lu_flops / (stages["k_lu_pivot_ms"] / 1e3) / 1e12

    gpu_geqrf = None
    if not args.no_geqrf:
        try:
            torch.geqrf(A)
            torch.cuda.synchronize()
            g_ms = _events_ms(lambda: torch.geqrf(A), 3, stream)
            gpu_geqrf = {"matrices_per_s": cfg.batch / (g_ms / 1e3), "ms_per_batch": g_ms}
        except Exception as e:  # reported, not fatal
            gpu_geqrf = {"error": repr(e)[:200]}

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(A_cpu, classes=24 if cfg.n <= 512 else 2)

    out = {
        "metric": METRIC,
        "value": mats_per_s,
        "unit": "matrices/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic, seeded (qr-contest_amd/workloads.py make_batch)",
        "config": {"workload": cfg.name, "batch": cfg.batch, "n": cfg.n},
        "roofline": {
            "bound": "mfma",
            "achieved": lu_tflops,
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": lu_tflops / PEAK_FP32_MFMA_TFLOPS,
            "traffic": None,
            "kernel": "k_lu<true> (partial-pivot LU, (2/3) n^3 flops per matrix)",
        },
        "path": {
            "nominal_tflops": nominal_tflops,
            "nominal_frac_fp32_mfma": nominal_tflops / PEAK_FP32_MFMA_TFLOPS,
            "hbm_gbs_algorithmic": gbs,
            "wall_ms_per_step": wall_ms,
        },
        "stages_ms": stages,
        "gates": {"factor_max": fr, "factor_gate": ft, "ortho_max": og, "ortho_gate": ot,
                  "checked": k, "pass": bool(ok.all()) and info_ok},
        "gpu_torch_geqrf": gpu_geqrf,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
