"""Throughput of the reflector-free batched QR on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 4] [--no-cpu] [--no-geqrf]

A step is one factorization of the configuration's whole batch (inputs resident in HBM,
outputs written to preallocated buffers, no host synchronisation inside).  Prints one JSON
line.  Default workload: BASELINE configuration 4, 256 x 512 x 512 fp32, six pathology
classes cycled (synthetic, seeded).
"""
from __future__ import annotations

import argparse
import ctypes
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


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_headline_256x512.md")
# bench kernel label -> the kernel symbol in the rocprofv3 counter summary
# rocprofv3 symbols of each reported kernel and their launches per step
PROFILE_SYMBOL = {"k_trsm": [("rnr::k_trsm<true, 128>", 2)], "k_chol": [("rnr::k_chol", 2)],
                  "k_lu<true> (LU)": [("rnr::k_lu<true, 64, 1, false>", 1)],
                  "k_lu<false> (chart)": [("rnr::k_lu<false, 64, 1, false>", 1)],
                  "k_tn_upper": [("rnr::k_tn_upper<128, false, false, true, 16, true>", 1),
                                 ("rnr::k_tn_upper<128, false, false, true, 16, false>", 1),
                                 ("rnr::k_tn_upper<128, true, true, true, 16, false>", 1)]}


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` (mean over its launches in one step) from the committed
    rocprofv3 FETCH/WRITE summary (headline workload only), or None."""
    syms = PROFILE_SYMBOL.get(kernel)
    if not syms:
        return None
    per = {}
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic "):
                    name, val = line[len("traffic "):].rsplit(" ", 1)
                    per[name] = int(val)
    except OSError:
        return None
    if not all(s in per for s, _ in syms):
        return None
    return int(sum(per[s] * c for s, c in syms) / sum(c for _, c in syms))


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
    ap.add_argument("--no-gates", action="store_true",
                    help="skip the float64 gate check of the output (profiling runs)")
    ap.add_argument("--no-aux", action="store_true",
                    help="skip the generator and Q-consumer timings")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 256 MiB device copy three times (the known-size kernel that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes)")
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

    if args.copy_calibration:
        x = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        del x, y

    t_gen = time.perf_counter()
    A_cpu = wl.make_batch(args.config)
    host_gen_ms = (time.perf_counter() - t_gen) * 1e3
    t_h2d = time.perf_counter()
    A = A_cpu.to(dev)
    torch.cuda.synchronize()
    h2d_ms = (time.perf_counter() - t_h2d) * 1e3
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

    # validity of what was timed: the contest gates on every matrix of the last step's output,
    # evaluated in float64 on the GPU (rnr_check_f64), outside the timed region
    gates = None
    if not args.no_gates:
        chk = importlib.import_module("qr-contest_amd.check")
        torch.cuda.synchronize()
        t_chk = time.perf_counter()
        fr, og, ft, ot, ok = chk.check(A, plan.H, plan.tau)
        ratio, _, ok_col = chk.check_percol(A, plan.H, plan.tau)
        torch.cuda.synchronize()
        chk_ms = (time.perf_counter() - t_chk) * 1e3
        info_ok = int(plan.info.abs().sum().item()) == 0
        gates = {"factor_max": fr, "factor_gate": ft, "ortho_max": og, "ortho_gate": ot,
                 "percol_max": ratio, "checked": cfg.batch, "checker": "rnr_check_f64 (GPU, float64)",
                 "checker_ms": chk_ms, "pass": bool(ok.all()) and bool(ok_col.all()) and info_ok}

    # the steps either side of the path: the input generators and the Q consumers
    aux = None
    if not args.no_aux:
        gen = importlib.import_module("qr-contest_amd.generate")
        hh = importlib.import_module("qr-contest_amd.householder")
        gen.device_batch(args.config, device=dev)
        torch.cuda.synchronize()
        t_dg = time.perf_counter()
        gen.device_batch(args.config, device=dev)
        torch.cuda.synchronize()
        dev_gen_ms = (time.perf_counter() - t_dg) * 1e3
        Hc, tc = plan.H.clone(), plan.tau.clone()
        hh.householder_product(Hc, tc)
        torch.cuda.synchronize()
        orgqr_ms = _events_ms(lambda: hh.householder_product(Hc, tc), 3, stream)
        C = torch.randn(cfg.batch, cfg.n, 64, device=dev)
        hh.ormqr(Hc, tc, C, transpose=True)
        torch.cuda.synchronize()
        ormqr_ms = _events_ms(lambda: hh.ormqr(Hc, tc, C, transpose=True), 3, stream)
        cmpm = importlib.import_module("qr-contest_amd.comparator")
        cmpm.hh_geqrf(A)
        torch.cuda.synchronize()
        hh_ms = _events_ms(lambda: cmpm.hh_geqrf(A), 3, stream)
        aux = {"householder_comparator": {"ms_per_batch": hh_ms, "matrices_per_s": cfg.batch / (hh_ms / 1e3),
                                          "source": "rnr_hh_geqrf_f32 (blocked Householder, geqrf layout; "
                                                    "benchmark only, not the product path)"},
               "generator": {"device_ms": dev_gen_ms, "host_ms": host_gen_ms, "host_to_device_ms": h2d_ms,
                             "device_source": "rnr_generate_f32 (Philox4x32-10, float64 Haar factors)",
                             "host_source": "workloads.make_batch (torch CPU, float64)"},
               "orgqr": {"ms_per_batch": orgqr_ms, "matrices_per_s": cfg.batch / (orgqr_ms / 1e3)},
               "ormqr_qt_64cols": {"ms_per_batch": ormqr_ms}}

    # per-kernel times of the live path: rnr_qr_f32_timed records an event before each launch
    lib = native.lib()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(native.RNR_QR_TIMED_EVENTS)]
    for e in evs:
        e.record(stream)  # creates the underlying hipEvent
    handles = (ctypes.c_void_p * len(evs))(*[e.cuda_event for e in evs])
    nn = cfg.n * cfg.n
    stage_ms = {k: 0.0 for k in native.QR_STAGES}
    reps = max(3, args.steps)
    torch.cuda.synchronize()
    for _ in range(reps):
        st = lib.rnr_qr_f32_timed(A.data_ptr(), cfg.batch, cfg.n, nn, plan.H.data_ptr(), plan.tau.data_ptr(),
                                  plan.info.data_ptr(), plan.ws.data_ptr(), plan.ws.numel(), stream.cuda_stream,
                                  handles, len(evs))
        native.check("rnr_qr_f32_timed", st)
        evs[-1].synchronize()
        for i, k in enumerate(native.QR_STAGES):
            stage_ms[k] += evs[i].elapsed_time(evs[i + 1]) / reps

    # algorithmic flops per matrix of each launch (minimal counts, not what the kernel executes)
    n3 = float(cfg.n) ** 3
    flops = {"lu": 2 / 3 * n3, "gram_L": n3 / 3, "chol_1": n3 / 3, "trsm_1": n3, "gram_Q1": n3,
             "chol_2": n3 / 3, "trsm_2": n3, "chart": 2 / 3 * n3, "closure": n3}
    kernels = {"k_lu<true> (LU)": ["lu"], "k_lu<false> (chart)": ["chart"], "k_chol": ["chol_1", "chol_2"],
               "k_trsm": ["trsm_1", "trsm_2"], "k_tn_upper": ["gram_L", "gram_Q1", "closure"]}
    per_kernel = {}
    for name, ks in kernels.items():
        t = sum(stage_ms[k] for k in ks)
        f = sum(flops[k] for k in ks) * cfg.batch
        per_kernel[name] = {"ms_per_step": t, "launches": len(ks), "avg_launch_us": 1e3 * t / len(ks),
                            "tflops": f / (t / 1e3) / 1e12}
    dom = max(per_kernel, key=lambda k: per_kernel[k]["ms_per_step"])
    dom_tflops = per_kernel[dom]["tflops"]

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
            "achieved": dom_tflops,
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": dom_tflops / PEAK_FP32_MFMA_TFLOPS,
            "traffic": measured_traffic(dom) if args.config == 4 else None,
            "traffic_source": os.path.relpath(TRAFFIC_FILE, ROOT) if args.config == 4 else None,
            "kernel": dom,
        },
        "path": {
            "nominal_tflops": nominal_tflops,
            "nominal_frac_fp32_mfma": nominal_tflops / PEAK_FP32_MFMA_TFLOPS,
            "hbm_gbs_algorithmic": gbs,
            "wall_ms_per_step": wall_ms,
        },
        "stages_ms": stage_ms,
        "kernels": per_kernel,
        "gates": gates,
        "aux": aux,
        "gpu_torch_geqrf": gpu_geqrf,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
