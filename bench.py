"""Benchmark of the headline hot path: TensorProduct fwd + full VJP on MI355X.

Workload (BASELINE.json metric): TensorProduct(C=128, m_max=6, parity="full"),
N = 131072 rows, fp32, x, y ~ N(0, 1) and a materialised ones cotangent, all
resident in HBM before timing.  One step = the compiled module's forward plus
``torch.autograd.grad(out, (x, y, weight), ones)`` (dx, dy, dw), as in the
reference's protocol (benchmarks/eqx/scripts/benchmark.py:88-100).

Prints one JSON line.  ``value`` is rows/s of the whole step; ``roofline`` is
the dominant kernel (the fused backward) on its algorithmic bytes
4 * (5 N W + 2 P_w) divided by its own duration, timed with HIP events
recorded around that kernel on its stream (o2mi_kernel_timing);
``cpu_baseline`` is the reference's CPU PyTorch algebra (oracle/cpu_port.py)
timed on the host cores over a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for entry in (REPO / "ictc-o2-hp_amd", REPO):
    if str(entry) not in sys.path:
        sys.path.insert(0, str(entry))

HBM_PEAK_GBS = 8000.0                      # MI355X HBM3E, published
A100_PUBLISHED_ROWS_S = 2171940.0          # complete_matrix.csv:385 (A100, 60.348 ms)


def _args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--rows", type=int, default=131072)
    p.add_argument("--channels", type=int, default=128)
    p.add_argument("--m-max", type=int, default=6)
    p.add_argument("--parity", default="full", choices=("canonical", "full"))
    p.add_argument("--no-compile", action="store_true", help="eager module instead of torch.compile")
    p.add_argument("--cpu-seconds", type=float, default=15.0,
                   help="time budget of the CPU-baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    return p.parse_args()


def _cpu_baseline(channels, m_max, parity, width, budget_s):
    """Reference CPU algebra (fp32, autograd) on 2048-row chunks of the workload."""
    import numpy as np
    import torch
    from oracle.cpu_port import CPUPort

    cores = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(cores)
    port = CPUPort(channels, m_max, parity)
    rng = np.random.default_rng(0)
    chunk = 2048
    x = rng.standard_normal((chunk, width)).astype(np.float32)
    y = rng.standard_normal((chunk, width)).astype(np.float32)
    w = (rng.standard_normal(port.plan.weight_numel) * 0.02).astype(np.float32)
    g = np.ones((chunk, width), dtype=np.float32)
    port.forward_vjp(x[:64], y[:64], w, g[:64])         # warm-up
    rows, start = 0, time.perf_counter()
    while True:
        port.forward_vjp(x, y, w, g)
        rows += chunk
        elapsed = time.perf_counter() - start
        if elapsed >= budget_s or rows >= 16 * chunk:
            break
    return {"value": rows / elapsed, "unit": "rows/s", "cores": cores, "kind": "port",
            "sample": f"{rows} rows in {chunk}-row chunks of C{channels} m{m_max} {parity}, "
                      f"fp32 forward + autograd dx/dy/dw, {elapsed:.1f} s"}


def _traffic(path: Path, key: str):
    """Measured HBM bytes per launch of the dominant kernel, if profiled."""
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get(key, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def main():
    args = _args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); "
              f"got --gpus {args.gpus}", file=sys.stderr)
        raise SystemExit(2)
    import torch
    from ictc_o2_hp import TensorProduct, _native

    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    torch.set_float32_matmul_precision("highest")
    device = torch.device("cuda:0")
    _native.library()

    torch.manual_seed(34527)
    module = TensorProduct(args.channels, args.m_max, parity=args.parity).to(device)
    width, pw, n = module.representation_dimension, module.weight.numel(), args.rows
    gen = torch.Generator(device=device).manual_seed(78211)
    x = torch.randn((n, width), device=device, generator=gen).requires_grad_()
    y = torch.randn((n, width), device=device, generator=gen).requires_grad_()
    cot = torch.ones((n, width), device=device)
    run = module if args.no_compile else torch.compile(module, fullgraph=True, dynamic=False)

    def step():
        out = run(x, y)
        return torch.autograd.grad(out, (x, y, module.weight), cot)

    for _ in range(max(1, args.warmup)):
        step()
    torch.cuda.synchronize()
    _native.kernel_timing_read()              # drop warm-up records
    _native.kernel_timing(True)
    start_evt = torch.cuda.Event(enable_timing=True)
    stop_evt = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start_evt.record()
    for _ in range(args.steps):
        step()
    stop_evt.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    _native.kernel_timing(False)
    fwd_ms, fwd_n, bwd_ms, bwd_n = _native.kernel_timing_read()
    ms_per_step = start_evt.elapsed_time(stop_evt) / args.steps

    alg_step = 4.0 * (8.0 * n * width + 3.0 * pw)
    alg_bwd = 4.0 * (5.0 * n * width + 2.0 * pw)
    alg_fwd = 4.0 * (3.0 * n * width + pw)
    bwd_avg = bwd_ms / max(1, bwd_n)
    fwd_avg = fwd_ms / max(1, fwd_n)
    achieved = alg_bwd / (bwd_avg * 1e-3) / 1e9
    workload = f"TensorProduct C{args.channels} m{args.m_max} {args.parity} N={n} fwd+full VJP"
    record = {
        "metric": "fwd+full-VJP rows/s, N=131072 C128 m_max=6 full parity; achieved HBM GB/s",
        "value": n / (ms_per_step * 1e-3),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": (n / (ms_per_step * 1e-3)) / A100_PUBLISHED_ROWS_S
        if (n, args.channels, args.m_max, args.parity) == (131072, 128, 6, "full") else None,
        "dtype": "f32",
        "data": "synthetic: x, y ~ N(0,1) (seeded), ones cotangent, default-initialised weights",
        "config": {"workload": workload, "rows": n, "channels": args.channels,
                   "m_max": args.m_max, "parity": args.parity, "width": width,
                   "weights": pw, "compiled": not args.no_compile},
        "achieved_step_GBps": alg_step / (ms_per_step * 1e-3) / 1e9,
        "step_roofline_frac": alg_step / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "kernels_ms": {"forward": fwd_avg, "backward": bwd_avg,
                       "forward_GBps": alg_fwd / (fwd_avg * 1e-3) / 1e9,
                       "launches": [fwd_n, bwd_n]},
        "wall_ms_per_step": wall_ms / args.steps,
        "roofline": {"bound": "hbm", "kernel": "tp_backward_kernel", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": _traffic(REPO / "profiles" / "traffic.json",
                                         f"backward_C{args.channels}_m{args.m_max}_{args.parity}_N{n}")},
    }
    del x, y, cot
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        record["cpu_baseline"] = _cpu_baseline(args.channels, args.m_max, args.parity, width,
                                               args.cpu_seconds)
    print(json.dumps(record), flush=True)


if __name__ == "__main__":
    main()
