"""Benchmark of the headline hot path: TensorProduct fwd + full VJP on MI355X.

``--workload radial`` and ``--workload uvu`` measure BASELINE.json configs[4]
(RadialUvuTensorProduct chain) and configs[3] (UvuTensorProduct, at a row
count that fits one GPU) with the same JSON fields; the default is the
headline TensorProduct workload below.

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
    p.add_argument("--workload", default="tp", choices=("tp", "radial", "uvu"))
    p.add_argument("--copy-probe", action="store_true",
                   help="after the run, copy 512 MiB 3 times with an elementwise kernel "
                        "(reference traffic for HBM counter calibration)")
    p.add_argument("--edges", type=int, default=1048576, help="radial workload: edges")
    p.add_argument("--uvu-rows", type=int, default=16384,
                   help="uvu workload: rows (65536 needs 524 GB of per-row weights)")
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
        if elapsed >= budget_s:
            break
    return {"value": rows / elapsed, "unit": "rows/s", "cores": cores, "kind": "port",
            "cpu": _cpu_model(),
            "sample": f"{rows} rows in {chunk}-row chunks of C{channels} m{m_max} {parity}, "
                      f"fp32 forward + autograd dx/dy/dw, {elapsed:.1f} s"}


def _cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def _sample_stats(samples):
    """Median and inter-quartile range of per-step times (ms)."""
    import statistics
    if not samples:
        return None, None
    q = statistics.quantiles(samples, n=4) if len(samples) >= 2 else [samples[0]] * 3
    return statistics.median(samples), q[2] - q[0]


def _traffic(path: Path, key: str):
    """Measured HBM bytes per launch of the dominant kernel, if profiled."""
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get(key, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def _timed_steps(torch, step, steps, warmup):
    """Warm up, then time `steps` steps with events on torch's current stream
    (the stream every kernel of the step is launched on)."""
    from ictc_o2_hp import _native
    for _ in range(max(1, warmup)):
        step()
    torch.cuda.synchronize()
    _native.kernel_timing_read_kinds()          # drop warm-up records
    _native.kernel_timing(True)
    events = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    events[0].record()
    for i in range(steps):
        step()
        events[i + 1].record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    _native.kernel_timing(False)
    kinds = _native.kernel_timing_read_kinds()
    samples = [events[i].elapsed_time(events[i + 1]) for i in range(steps)]
    return events[0].elapsed_time(events[-1]) / steps, wall_ms / steps, kinds, samples


def _radial_chain(torch, device, edges, nodes=65536, channels=64, m_max=4, hidden=64):
    """gather x from nodes, Bessel(8) radial features with a cosine
    cutoff -> MLP 8->64->64 (SiLU) -> fused final affine + V=1 uvu product."""
    import math
    from ictc_o2_hp import RadialUvuTensorProduct, UvuTensorProduct

    tp = UvuTensorProduct(channels, 1, m_max, parity="canonical", shared_weights=False)
    trunk = torch.nn.Sequential(torch.nn.Linear(8, hidden), torch.nn.SiLU(),
                                torch.nn.Linear(hidden, hidden), torch.nn.SiLU())
    radial_out = torch.nn.Linear(hidden, tp.weight_numel)

    class Chain(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.trunk = trunk
            self.radial = RadialUvuTensorProduct(tp, radial_out)

        def forward(self, node_feats, src, basis, angular):
            return self.radial(node_feats[src], angular, self.trunk(basis))

    chain = Chain().to(device)
    gen = torch.Generator(device=device).manual_seed(4242)
    node_feats = torch.randn((nodes, tp.input1_dimension), device=device, generator=gen)
    node_feats.requires_grad_()
    src = torch.randint(0, nodes, (edges,), device=device, generator=gen)
    r = 0.5 + 4.5 * torch.rand((edges, 1), device=device, generator=gen)
    cutoff = 5.0
    n = torch.arange(1, 9, device=device, dtype=torch.float32)
    envelope = 0.5 * (torch.cos(math.pi * r / cutoff) + 1.0)
    basis = math.sqrt(2.0 / cutoff) * torch.sin(n * math.pi * r / cutoff) / r * envelope
    phi = 2.0 * math.pi * torch.rand((edges, 1), device=device, generator=gen)
    parts = [torch.ones_like(phi)]
    for m in range(1, m_max + 1):
        parts += [torch.cos(m * phi), torch.sin(m * phi)]
    angular = torch.cat(parts, dim=1).contiguous()
    return chain, tp, node_feats, src, basis.contiguous(), angular


def _radial_cpu_baseline(channels, m_max, hidden, budget_s):
    """The radial oracle (numpy fp64 restatement of the reference algebra):
    affine + uvu forward and its full VJP on 512-edge chunks."""
    import numpy as np
    from oracle import uvu_oracle as U

    cores = min(16, len(os.sched_getaffinity(0)))
    plan = U.UvuOraclePlan(channels, 1, m_max, parity="canonical")
    rng = np.random.default_rng(0)
    chunk = 512
    x = rng.standard_normal((chunk, plan.width1))
    y = rng.standard_normal((chunk, plan.width2))
    h = rng.standard_normal((chunk, hidden))
    a = rng.standard_normal((plan.weight_numel, hidden)) / 8.0
    b = rng.standard_normal(plan.weight_numel)
    g = rng.standard_normal((chunk, plan.width1))
    edges, start = 0, time.perf_counter()
    while True:
        U.radial_forward(plan, x, y, h, a, b)
        U.radial_backward(plan, x, y, h, a, b, g)
        edges += chunk
        elapsed = time.perf_counter() - start
        if elapsed >= budget_s:
            break
    return {"value": edges / elapsed, "unit": "edges/s", "cores": cores, "kind": "port",
            "sample": f"{edges} edges in {chunk}-edge chunks, radial affine + uvu C{channels} "
                      f"m{m_max} canonical forward and VJP (x, y, hidden, alpha, bias), "
                      f"numpy fp64, {elapsed:.1f} s"}


def radial_main(args):
    import torch
    from ictc_o2_hp import _native

    torch.backends.cuda.matmul.allow_tf32 = False
    torch.set_float32_matmul_precision("highest")
    device = torch.device("cuda:0")
    _native.library()
    torch.manual_seed(2024)
    edges = args.edges
    chain, tp, node_feats, src, basis, angular = _radial_chain(torch, device, edges)
    run = chain if args.no_compile else torch.compile(chain, fullgraph=True, dynamic=False)
    params = [node_feats] + list(chain.parameters())
    cot = torch.ones((edges, tp.input1_dimension), device=device)

    def step():
        out = run(node_feats, src, basis, angular)
        return torch.autograd.grad(out, params, cot)

    ms_per_step, wall_ms, kinds, samples = _timed_steps(torch, step, args.steps, args.warmup)
    median, iqr = _sample_stats(samples)
    pw, hidden, width = tp.weight_numel, 64, tp.input1_dimension
    gemm = 2.0 * edges * pw * hidden                      # one affine map over all edges
    per = {k: kinds[k][0] / max(1, kinds[k][1]) for k in kinds}
    flops = {"radial_forward": gemm, "radial_backward": 2 * gemm, "radial_weight": gemm}
    tflops = {k: flops[k] / (per[k] * 1e-3) / 1e12 for k in flops if per[k] > 0}
    dominant = max(flops, key=lambda k: per[k])
    peak = 157.3
    record = {
        "metric": "radial chain fwd + full VJP edges/s (configs[4]); matrix-core TFLOP/s",
        "value": edges / (ms_per_step * 1e-3), "unit": "edges/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: random src/r/phi (seeded), random-init MLP 8->64->64 and final "
                "affine, ones cotangent",
        "config": {"workload": f"RadialUvuTensorProduct C64 m4 canonical E={edges} "
                               "(gather from 65536 nodes, MLP 8->64->64 SiLU) fwd+full VJP",
                   "edges": edges, "channels": 64, "m_max": 4, "hidden": hidden,
                   "weights_per_edge": pw, "compiled": not args.no_compile},
        "ms_per_step_median": median, "ms_per_step_iqr": iqr,
        "kernels_ms": per, "kernels_TFLOPs": tflops, "wall_ms_per_step": wall_ms,
        "roofline": {"bound": "mfma", "kernel": dominant,
                     "achieved": tflops.get(dominant), "peak": peak, "unit": "TFLOP/s",
                     "frac": (tflops.get(dominant) or 0.0) / peak, "traffic": None},
    }
    del chain, node_feats, basis, angular, cot
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        record["cpu_baseline"] = _radial_cpu_baseline(64, 4, hidden, args.cpu_seconds)
    print(json.dumps(record), flush=True)


def uvu_main(args):
    """configs[3] at a row count that fits one GPU: UvuTensorProduct C1=128,
    C2=32, m4 full, per-row weights N(0, 1/sqrt(C2)), fwd + VJP with dw."""
    import torch
    from ictc_o2_hp import UvuTensorProduct, _native

    device = torch.device("cuda:0")
    _native.library()
    n = args.uvu_rows
    module = UvuTensorProduct(128, 32, 4, parity="full", shared_weights=False).to(device)
    gen = torch.Generator(device=device).manual_seed(3131)
    x = torch.randn((n, module.input1_dimension), device=device, generator=gen)
    y = torch.randn((n, module.input2_dimension), device=device, generator=gen)
    w = torch.randn((n, module.weight_numel), device=device, generator=gen) / (32 ** 0.5)
    for t in (x, y, w):
        t.requires_grad_()
    cot = torch.ones_like(x)
    run = module if args.no_compile else torch.compile(module, fullgraph=True, dynamic=False)

    def step():
        return torch.autograd.grad(run(x, y, w), (x, y, w), cot)

    ms_per_step, wall_ms, _, samples = _timed_steps(torch, step, args.steps, args.warmup)
    median, iqr = _sample_stats(samples)
    w1, w2, pw = module.input1_dimension, module.input2_dimension, module.weight_numel
    # Algorithmic bytes: forward reads x, y, w, writes out; backward reads x, y,
    # w, g and writes dx, dy, dw.
    alg = 4.0 * n * (2 * w1 + w2 + pw + w1) + 4.0 * n * (3 * w1 + w2 + pw + w1 + w2 + pw)
    achieved = alg / (ms_per_step * 1e-3) / 1e9
    record = {
        "metric": "uvu fwd + VJP rows/s (configs[3] shape, reduced N); step HBM GB/s",
        "value": n / (ms_per_step * 1e-3), "unit": "rows/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: x, y ~ N(0,1), w ~ N(0, 1/sqrt(32)) per row (seeded), ones cotangent",
        "config": {"workload": f"UvuTensorProduct C128 V32 m4 full N={n} per-row weights "
                               "fwd+VJP (x, y, w)", "rows": n, "weights_per_row": pw},
        "ms_per_step_median": median, "ms_per_step_iqr": iqr,
        "wall_ms_per_step": wall_ms,
        "roofline": {"bound": "hbm", "kernel": "uvu step", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": None},
    }
    print(json.dumps(record), flush=True)


def main():
    args = _args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); "
              f"got --gpus {args.gpus}", file=sys.stderr)
        raise SystemExit(2)
    if args.workload != "tp":
        (radial_main if args.workload == "radial" else uvu_main)(args)
        return _copy_probe(args)
    tp_main(args)
    _copy_probe(args)


def _copy_probe(args):
    """out = src * 1 over 2^27 floats: 512 MiB read + 512 MiB written per launch."""
    if not args.copy_probe:
        return
    import torch
    src = torch.ones(1 << 27, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()


def tp_main(args):
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

    ms_per_step, wall_ms, kinds, samples = _timed_steps(torch, step, args.steps, args.warmup)
    wall_ms *= args.steps
    median, iqr = _sample_stats(samples)
    (fwd_ms, fwd_n), (bwd_ms, bwd_n) = kinds["tp_forward"], kinds["tp_backward"]

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
        "ms_per_step_median": median,
        "ms_per_step_iqr": iqr,
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
