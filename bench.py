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
    p.add_argument("--no-stream-ceiling", action="store_true",
                   help="skip the HBM streaming-ceiling probe (tp workload)")
    p.add_argument("--workload", default="tp",
                   choices=("tp", "radial", "uvu", "uvu-rows", "uvu-shared", "grid", "radial-grid",
                            "force"),
                   help="grid: every configs[2] point (and configs[1]) as HIP-graph replays; "
                        "radial-grid: the reference's published radial-chain points; "
                        "force: a second-order (force-loss) step through the TP")
    p.add_argument("--grid-out", default=None, help="grid: also write the records to this file")
    p.add_argument("--radial-point", default=None,
                   help="radial-grid: only this 'edges,channels' point (e.g. 131072,64)")
    p.add_argument("--grid-set", default="configs2", choices=("configs2", "all"),
                   help="grid: BASELINE.json configs[2] (96 points) or every published point (240)")
    p.add_argument("--grid-rows", default=None,
                   help="grid: only these row counts (comma-separated), e.g. 16384,32768")
    p.add_argument("--copy-probe", action="store_true",
                   help="after the run, copy 512 MiB 3 times with an elementwise kernel "
                        "(reference traffic for HBM counter calibration)")
    p.add_argument("--edges", type=int, default=1048576, help="radial workload: edges")
    p.add_argument("--torch-gather", action="store_true",
                   help="radial workload: gather node features with torch indexing (atomic "
                        "scatter-add backward) instead of the fused left_index gather")
    p.add_argument("--channels-in2", type=int, default=1,
                   help="uvu-shared workload: copies V of the second input (default 1; with "
                        "V > 1 the shape is C128 m4 full, 65,536 rows unless --rows is given)")
    p.add_argument("--uvu-rows", type=int, default=16384,
                   help="uvu workload: rows (65536 needs 524 GB of per-row weights)")
    return p.parse_args()


def _cpu_threads():
    """Host threads for the CPU baseline: every core in this process's affinity
    mask, bounded by OMP_NUM_THREADS when the host declares its CPU share there
    (the GPU boxes give one GPU's job 16 cores of a larger mask)."""
    cores = len(os.sched_getaffinity(0))
    declared = os.environ.get("OMP_NUM_THREADS", "")
    if declared.isdigit() and int(declared) > 0:
        cores = min(cores, int(declared))
    return cores


def _one_piece(port, rows, seed):
    """Seconds of one fp32 forward + autograd VJP over `rows` rows in one piece."""
    import numpy as np
    rng = np.random.default_rng(seed)
    width = port.plan.width
    x = rng.standard_normal((rows, width)).astype(np.float32)
    y = rng.standard_normal((rows, width)).astype(np.float32)
    w = (rng.standard_normal(port.plan.weight_numel) * 0.02).astype(np.float32)
    g = np.ones((rows, width), dtype=np.float32)
    port.forward_vjp(x[:64], y[:64], w, g[:64])         # warm-up
    start = time.perf_counter()
    port.forward_vjp(x, y, w, g)
    return time.perf_counter() - start


def _cpu_baseline(channels, m_max, parity, width, budget_s):
    """Reference CPU algebra (fp32, autograd) on 2048-row chunks of the workload,
    plus BASELINE.json configs[0] (C32 m2 canonical, N=4096) and configs[1]
    (C128 m6 full, N=6400) each timed in one piece."""
    import numpy as np
    import torch
    from oracle.cpu_port import CPUPort

    cores = _cpu_threads()
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
    pieces = {}
    for name, (c, m, par, n) in (("configs0", (32, 2, "canonical", 4096)),
                                 ("configs1", (128, 6, "full", 6400))):
        seconds = _one_piece(CPUPort(c, m, par), n, 1)
        pieces[name] = {"rows": n, "ms": seconds * 1e3, "rows_per_s": n / seconds,
                        "workload": f"C{c} m{m} {par}, fp32 forward + autograd dx/dy/dw"}
    return {"value": rows / elapsed, "unit": "rows/s", "cores": cores, "kind": "port",
            "cpu": _cpu_model(), "affinity_cores": len(os.sched_getaffinity(0)),
            "sample": f"{rows} rows in {chunk}-row chunks of C{channels} m{m_max} {parity}, "
                      f"fp32 forward + autograd dx/dy/dw, {elapsed:.1f} s",
            "one_piece": pieces}


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


def _stream_ceiling(rows, width):
    """Best GB/s of plain 3-read/2-write and 2-read/1-write row streams on this
    GPU (ictc-o2-hp_amd/bin/o2mi_stream_probe, a child process), or None."""
    import subprocess
    probe = REPO / "ictc-o2-hp_amd" / "bin" / "o2mi_stream_probe"
    if not probe.exists():
        return None
    width = width if width <= 4096 and width % 4 == 0 else 3328
    try:
        proc = subprocess.run([str(probe), str(rows), str(width)], capture_output=True,
                              text=True, timeout=120)
        return json.loads(proc.stdout) if proc.returncode == 0 else None
    except (OSError, ValueError, subprocess.TimeoutExpired):
        return None


def _traffic(path: Path, key: str):
    """Measured HBM bytes per launch of the dominant kernel, if profiled."""
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get(key, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def _timed_steps(torch, step, steps, warmup):
    """Warm up, then three passes of `steps` steps on torch's current stream
    (the stream every kernel of the step is launched on), each bracketed by
    synchronizes:

    1. the timed region of ``value``: one HIP event pair around all steps and
       nothing between the steps;
    2. one event after every step, for the per-step median and IQR;
    3. the library's per-kernel HIP event pairs (o2mi_kernel_timing) around
       every main kernel, for the kernel durations behind ``roofline``.

    Each recorded event puts a few microseconds between the launches around
    it, so the per-step and per-kernel events are kept out of pass 1.
    Returns (ms per step of pass 1, wall ms per step of pass 1, per-kernel
    records of pass 3, per-step samples of pass 2)."""
    from ictc_o2_hp import _native
    for _ in range(max(1, warmup)):
        step()
    torch.cuda.synchronize()
    _native.kernel_timing_read_kinds()          # drop warm-up records

    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        step()
    stop.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms_per_step = start.elapsed_time(stop) / steps

    events = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    events[0].record()
    for i in range(steps):
        step()
        events[i + 1].record()
    torch.cuda.synchronize()
    samples = [events[i].elapsed_time(events[i + 1]) for i in range(steps)]

    _native.kernel_timing(True)
    torch.cuda.synchronize()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    _native.kernel_timing(False)
    kinds = _native.kernel_timing_read_kinds()
    return ms_per_step, wall_ms / steps, kinds, samples


def _radial_chain(torch, device, edges, nodes=65536, channels=64, m_max=4, hidden=64,
                  fused_gather=True):
    """gather x from nodes, Bessel(8) radial features with a cosine
    cutoff -> MLP 8->64->64 (SiLU) -> fused final affine + V=1 uvu product.
    ``fused_gather``: the radial kernels read node rows through ``left_index``
    (table gradient summed in a fixed order); otherwise ``node_feats[src]``."""
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
            if fused_gather:
                return self.radial(node_feats, angular, self.trunk(basis), left_index=src)
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

    cores = _cpu_threads()
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
    chain, tp, node_feats, src, basis, angular = _radial_chain(
        torch, device, edges, fused_gather=not args.torch_gather)
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
                   "gather": "torch indexing" if args.torch_gather else "fused left_index",
                   "edges": edges, "channels": 64, "m_max": 4, "hidden": hidden,
                   "weights_per_edge": pw, "compiled": not args.no_compile},
        "ms_per_step_median": median, "ms_per_step_iqr": iqr,
        "kernels_ms": per, "kernels_TFLOPs": tflops, "wall_ms_per_step": wall_ms,
        "roofline": {"bound": "mfma", "kernel": dominant,
                     "achieved": tflops.get(dominant), "peak": peak, "unit": "TFLOP/s",
                     "frac": (tflops.get(dominant) or 0.0) / peak,
                     "traffic": _traffic(REPO / "profiles" / "traffic.json",
                                         f"{dominant}_C64_m4_canonical_E{edges}"
                                         + ("" if not args.torch_gather else "_torch_gather"))},
    }
    del chain, node_feats, basis, angular, cot
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        record["cpu_baseline"] = _radial_cpu_baseline(64, 4, hidden, args.cpu_seconds)
    print(json.dumps(record), flush=True)


def uvu_main(args, v=32):
    """configs[3] at a row count that fits one GPU: UvuTensorProduct C1=128,
    C2=32, m4 full, per-row weights N(0, 1/sqrt(C2)), fwd + VJP with dw.  With
    v = 1 (workload uvu-rows) the same with one copy of the second input: the
    per-row weights a radial network feeds (configs[4]'s op with external
    weights), not a BASELINE metric."""
    import torch
    from ictc_o2_hp import UvuTensorProduct, _native

    device = torch.device("cuda:0")
    _native.library()
    n = args.uvu_rows
    module = UvuTensorProduct(128, v, 4, parity="full", shared_weights=False).to(device)
    gen = torch.Generator(device=device).manual_seed(3131)
    x = torch.randn((n, module.input1_dimension), device=device, generator=gen)
    y = torch.randn((n, module.input2_dimension), device=device, generator=gen)
    w = torch.randn((n, module.weight_numel), device=device, generator=gen) / (v ** 0.5)
    for t in (x, y, w):
        t.requires_grad_()
    cot = torch.ones_like(x)
    run = module if args.no_compile else torch.compile(module, fullgraph=True, dynamic=False)

    def step():
        return torch.autograd.grad(run(x, y, w), (x, y, w), cot)

    ms_per_step, wall_ms, kinds, samples = _timed_steps(torch, step, args.steps, args.warmup)
    median, iqr = _sample_stats(samples)
    w1, w2, pw = module.input1_dimension, module.input2_dimension, module.weight_numel
    # Algorithmic bytes per launch: the forward reads x, y, w and writes out;
    # the backward reads x, g, y, w and writes dx, dy, dw.
    alg_fwd = 4.0 * n * (2 * w1 + w2 + pw)
    alg_bwd = 4.0 * n * (3 * w1 + 2 * w2 + 2 * pw)
    per = {k: kinds[k][0] / max(1, kinds[k][1]) for k in ("uvu_forward", "uvu_backward")}
    bwd_gbs = alg_bwd / (per["uvu_backward"] * 1e-3) / 1e9 if per["uvu_backward"] else None
    kernel = "uvu_row_backward_kernel" if v == 32 else "radial_backward_streamed_kernel (per-row)"
    record = {
        "metric": ("uvu fwd + VJP rows/s (configs[3] shape, reduced N); step HBM GB/s" if v == 32
                   else f"uvu per-row V={v} fwd + VJP rows/s; step HBM GB/s"),
        "value": n / (ms_per_step * 1e-3), "unit": "rows/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": f"synthetic: x, y ~ N(0,1), w ~ N(0, 1/sqrt({v})) per row (seeded), ones "
                "cotangent",
        "config": {"workload": f"UvuTensorProduct C128 V{v} m4 full N={n} per-row weights "
                               "fwd+VJP (x, y, w)", "rows": n, "weights_per_row": pw},
        "ms_per_step_median": median, "ms_per_step_iqr": iqr,
        "wall_ms_per_step": wall_ms,
        "achieved_step_GBps": (alg_fwd + alg_bwd) / (ms_per_step * 1e-3) / 1e9,
        "kernels_ms": {"forward": per["uvu_forward"], "backward": per["uvu_backward"],
                       "forward_GBps": alg_fwd / (per["uvu_forward"] * 1e-3) / 1e9
                       if per["uvu_forward"] else None},
        "roofline": {"bound": "hbm", "kernel": kernel, "achieved": bwd_gbs,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": bwd_gbs / HBM_PEAK_GBS if bwd_gbs else None,
                     "traffic": _traffic(REPO / "profiles" / "traffic.json",
                                         f"uvu_backward_C128_V{v}_m4_full_N{n}")},
    }
    print(json.dumps(record), flush=True)


def uvu_shared_main(args):
    """UvuTensorProduct in the reference's default mode (shared trainable
    weights), compiled, forward + gradients of x, y and the weights with a ones
    cotangent.  V = 1: the example of its docs/UVU.md (C128, m6, full first
    input, canonical second input, 16,384 rows).  V = --channels-in2 > 1: C128,
    m4, full parity, 65,536 rows.  Not a BASELINE metric."""
    import torch
    from ictc_o2_hp import UvuTensorProduct, _native

    device = torch.device("cuda:0")
    _native.library()
    v = args.channels_in2
    torch.manual_seed(7)
    if v == 1:
        n = args.rows if args.rows != 131072 else 16384
        module = UvuTensorProduct(128, 1, 6, parity="full", parity_in2="canonical").to(device)
        shape = "C128 V1 m6 full/canonical"
        metric = "uvu shared-weight V=1 fwd + VJP rows/s (docs/UVU.md example shape)"
    else:
        n = args.rows if args.rows != 131072 else 65536
        module = UvuTensorProduct(128, v, 4, parity="full").to(device)
        shape = f"C128 V{v} m4 full"
        metric = f"uvu shared-weight V={v} fwd + VJP rows/s"
    x = torch.randn(n, module.input1_dimension, device=device, requires_grad=True)
    y = torch.randn(n, module.input2_dimension, device=device, requires_grad=True)
    cot = torch.ones_like(x)
    run = module if args.no_compile else torch.compile(module, fullgraph=True, dynamic=False)

    def step():
        return torch.autograd.grad(run(x, y), (x, y, module.weight), cot)

    ms_per_step, wall_ms, kinds, samples = _timed_steps(torch, step, args.steps, args.warmup)
    median, iqr = _sample_stats(samples)
    w1, w2 = module.input1_dimension, module.input2_dimension
    per = {k: kinds[k][0] / max(1, kinds[k][1]) for k in ("uvu_forward", "uvu_backward")}
    alg_fwd, alg_bwd = 4.0 * n * (2 * w1 + w2), 4.0 * n * (3 * w1 + 2 * w2)
    record = {
        "metric": metric,
        "value": n / (ms_per_step * 1e-3), "unit": "rows/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: x, y ~ N(0,1) (seeded), default-initialised shared weights, "
                "ones cotangent",
        "config": {"workload": f"UvuTensorProduct {shape} shared weights N={n} fwd+VJP "
                               f"(x, y, w)", "rows": n,
                   "paths": module.weight_numel // (128 * v)},
        "ms_per_step_median": median, "ms_per_step_iqr": iqr, "wall_ms_per_step": wall_ms,
        "kernels_ms": {"forward": per["uvu_forward"], "backward": per["uvu_backward"]},
        "kernels_GBps": {"forward": alg_fwd / (per["uvu_forward"] * 1e-3) / 1e9
                         if per["uvu_forward"] else None,
                         "backward": alg_bwd / (per["uvu_backward"] * 1e-3) / 1e9
                         if per["uvu_backward"] else None},
    }
    print(json.dumps(record), flush=True)


def force_main(args):
    """Force-loss step through TensorProduct (C, m_max, parity from the flags;
    rows default 16,384): E = sum(out * out), F = dE/dx with create_graph,
    then the gradients of sum(F^2) with respect to y and the weights, i.e. the
    TP's second order.  Not a BASELINE metric: the reference computes this
    order with its PyTorch algebra."""
    import torch
    from ictc_o2_hp import TensorProduct, _native

    device = torch.device("cuda:0")
    _native.library()
    n = args.rows if args.rows != 131072 else 16384
    torch.manual_seed(5)
    module = TensorProduct(args.channels, args.m_max, parity=args.parity).to(device)
    x = torch.randn(n, module.representation_dimension, device=device, requires_grad=True)
    y = torch.randn_like(x, requires_grad=True)

    def step():
        out = module(x, y)
        (forces,) = torch.autograd.grad((out * out).sum(), x, create_graph=True)
        return torch.autograd.grad(forces.square().sum(), (y, module.weight))

    torch.cuda.reset_peak_memory_stats(device)
    ms_per_step, wall_ms, kinds, samples = _timed_steps(torch, step, args.steps, args.warmup)
    median, iqr = _sample_stats(samples)
    record = {
        "metric": "TP force-loss step rows/s (second order)", "value": n / (ms_per_step * 1e-3),
        "unit": "rows/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms_per_step, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: x, y ~ N(0,1) (seeded), default-initialised weights",
        "config": {"workload": f"TensorProduct C{args.channels} m{args.m_max} {args.parity} "
                               f"N={n}: forces by create_graph, grads of sum(F^2) wrt y, w",
                   "rows": n},
        "ms_per_step_median": median, "ms_per_step_iqr": iqr, "wall_ms_per_step": wall_ms,
        "kernel_launches": {k: kinds[k][1] for k in ("tp_forward", "tp_backward")},
        "peak_allocated_MiB": torch.cuda.max_memory_allocated(device) / 2**20,
    }
    print(json.dumps(record), flush=True)


# Published A100 times (ms) of the reference's TensorProduct, forward and
# forward + full VJP, for every point of its benchmark matrix
# (benchmarks/eqx/results/complete_matrix.csv, candidate_ms, 4 significant
# digits): "N C m_max parity fwd fwd+VJP".  configs[2] is the subset
# C in {32, 64, 128, 256}, m_max in {1, 4, 6}.
A100_GRID = (
    "16384 32 1 c 0.05837 0.3021; 16384 32 1 f 0.0809 0.4424; 16384 32 2 c 0.07782 0.4035;"
    "16384 32 2 f 0.1106 0.6948; 16384 32 3 c 0.09677 0.556; 16384 32 3 f 0.1669 0.9969;"
    "16384 32 4 c 0.2002 0.9032; 16384 32 4 f 0.2074 1.376; 16384 32 5 c 0.2724 1.248;"
    "16384 32 5 f 0.2381 1.857; 16384 32 6 c 0.3594 1.688; 16384 32 6 f 0.2816 2.399;"
    "16384 64 1 c 0.07424 0.3492; 16384 64 1 f 0.1188 0.6359; 16384 64 2 c 0.1024 0.5207;"
    "16384 64 2 f 0.1782 1.125; 16384 64 3 c 0.1393 0.7578; 16384 64 3 f 0.2775 1.718;"
    "16384 64 4 c 0.1889 1.378; 16384 64 4 f 0.3471 2.5; 16384 64 5 c 0.2222 1.892;"
    "16384 64 5 f 0.4116 3.539; 16384 64 6 c 0.2586 2.533; 16384 64 6 f 0.4864 4.596;"
    "16384 96 1 c 0.09114 0.4229; 16384 96 1 f 0.1618 0.8479; 16384 96 2 c 0.1311 0.6861;"
    "16384 96 2 f 0.2596 1.597; 16384 96 3 c 0.1772 1.036; 16384 96 3 f 0.3973 2.583;"
    "16384 96 4 c 0.2591 2.028; 16384 96 4 f 0.4966 3.702; 16384 96 5 c 0.3082 2.896;"
    "16384 96 5 f 0.5934 5.299; 16384 96 6 c 0.3594 3.901; 16384 96 6 f 0.706 5.953;"
    "16384 128 1 c 0.09984 0.4654; 16384 128 1 f 0.1966 1.03; 16384 128 2 c 0.1536 0.7839;"
    "16384 128 2 f 0.322 2.085; 16384 128 3 c 0.2186 1.228; 16384 128 3 f 0.4818 3.319;"
    "16384 128 4 c 0.3267 2.537; 16384 128 4 f 0.6528 4.884; 16384 128 5 c 0.3901 3.63;"
    "16384 128 5 f 0.7726 6.97; 16384 128 6 c 0.4552 4.674; 16384 128 6 f 0.9083 7.824;"
    "16384 256 1 c 0.1587 0.6886; 16384 256 1 f 0.3564 1.977; 16384 256 2 c 0.255 1.401;"
    "16384 256 2 f 0.5811 4.064; 16384 256 3 c 0.3732 2.338; 16384 256 3 f 0.9272 6.568;"
    "16384 256 4 c 0.6001 4.964; 16384 256 4 f 1.225 9.202; 16384 256 5 c 0.7322 6.709;"
    "16384 256 5 f 1.488 11.87; 16384 256 6 c 0.8663 9.286; 16384 256 6 f 1.761 15.26;"
    "32768 32 1 c 0.07526 0.3784; 32768 32 1 f 0.1188 0.6472; 32768 32 2 c 0.1034 0.5765;"
    "32768 32 2 f 0.1782 1.12; 32768 32 3 c 0.1393 0.8351; 32768 32 3 f 0.2755 1.727;"
    "32768 32 4 c 0.3569 1.67; 32768 32 4 f 0.3523 2.5; 32768 32 5 c 0.4992 2.382;"
    "32768 32 5 f 0.4137 3.563; 32768 32 6 c 0.6666 3.237; 32768 32 6 f 0.4931 4.575;"
    "32768 64 1 c 0.1004 0.4685; 32768 64 1 f 0.1961 1.029; 32768 64 2 c 0.1541 0.7895;"
    "32768 64 2 f 0.3052 2.087; 32768 64 3 c 0.2166 1.235; 32768 64 3 f 0.4951 3.309;"
    "32768 64 4 c 0.3256 2.549; 32768 64 4 f 0.6385 4.836; 32768 64 5 c 0.3901 3.665;"
    "32768 64 5 f 0.7644 6.647; 32768 64 6 c 0.4552 4.909; 32768 64 6 f 0.898 8.37;"
    "32768 96 1 c 0.13 0.6093; 32768 96 1 f 0.279 1.529; 32768 96 2 c 0.2094 1.133;"
    "32768 96 2 f 0.469 3.092; 32768 96 3 c 0.299 1.898; 32768 96 3 f 0.7219 4.756;"
    "32768 96 4 c 0.4639 3.931; 32768 96 4 f 0.9324 6.53; 32768 96 5 c 0.5632 5.186;"
    "32768 96 5 f 1.121 8.926; 32768 96 6 c 0.6646 7.652; 32768 96 6 f 1.331 11.48;"
    "32768 128 1 c 0.1541 0.683; 32768 128 1 f 0.3512 1.973; 32768 128 2 c 0.256 1.386;"
    "32768 128 2 f 0.5775 3.96; 32768 128 3 c 0.3763 2.328; 32768 128 3 f 0.9078 5.755;"
    "32768 128 4 c 0.598 4.947; 32768 128 4 f 1.252 9.512; 32768 128 5 c 0.725 6.499;"
    "32768 128 5 f 1.477 11.8; 32768 128 6 c 0.853 8.595; 32768 128 6 f 1.744 15.11;"
    "32768 256 1 c 0.2668 1.231; 32768 256 1 f 0.6651 3.859; 32768 256 2 c 0.4526 2.654;"
    "32768 256 2 f 1.132 7.51; 32768 256 3 c 0.6953 4.549; 32768 256 3 f 1.814 11.41;"
    "32768 256 4 c 1.148 9.051; 32768 256 4 f 2.386 16.63; 32768 256 5 c 1.406 12.68;"
    "32768 256 5 f 2.923 23.5; 32768 256 6 c 1.671 17.1; 32768 256 6 f 3.454 30.36;"
    "65536 32 1 c 0.1019 0.514; 65536 32 1 f 0.1997 1.059; 65536 32 2 c 0.1567 0.8945;"
    "65536 32 2 f 0.3036 2.066; 65536 32 3 c 0.2166 1.416; 65536 32 3 f 0.4946 3.326;"
    "65536 32 4 c 0.6666 3.218; 65536 32 4 f 0.6451 4.84; 65536 32 5 c 0.9492 4.652;"
    "65536 32 5 f 0.766 6.524; 65536 32 6 c 1.284 6.345; 65536 32 6 f 0.9062 7.769;"
    "65536 64 1 c 0.1536 0.6856; 65536 64 1 f 0.3507 1.964; 65536 64 2 c 0.2575 1.388;"
    "65536 64 2 f 0.5652 3.877; 65536 64 3 c 0.3768 2.332; 65536 64 3 f 0.9277 6.338;"
    "65536 64 4 c 0.599 4.97; 65536 64 4 f 1.214 8.309; 65536 64 5 c 0.7255 7.138;"
    "65536 64 5 f 1.464 11.82; 65536 64 6 c 0.8571 8.773; 65536 64 6 f 1.728 14.96;"
    "65536 96 1 c 0.212 0.9928; 65536 96 1 f 0.5202 2.959; 65536 96 2 c 0.3635 2.141;"
    "65536 96 2 f 0.8837 6.052; 65536 96 3 c 0.5381 3.656; 65536 96 3 f 1.403 8.78;"
    "65536 96 4 c 0.8817 7.183; 65536 96 4 f 1.802 12.58; 65536 96 5 c 1.07 10.02;"
    "65536 96 5 f 2.178 17.73; 65536 96 6 c 1.265 13.56; 65536 96 6 f 2.588 22.79;"
    "65536 128 1 c 0.2627 1.217; 65536 128 1 f 0.6661 3.844; 65536 128 2 c 0.4598 2.649;"
    "65536 128 2 f 1.115 7.506; 65536 128 3 c 0.6932 4.514; 65536 128 3 f 1.748 11.21;"
    "65536 128 4 c 1.146 9.765; 65536 128 4 f 2.443 16.65; 65536 128 5 c 1.395 12.68;"
    "65536 128 5 f 2.883 23.26; 65536 128 6 c 1.645 17.1; 65536 128 6 f 3.419 30.09;"
    "65536 256 1 c 0.4844 2.359; 65536 256 1 f 1.286 7.639; 65536 256 2 c 0.8407 5.17;"
    "65536 256 2 f 2.166 14.24; 65536 256 3 c 1.316 7.719; 65536 256 3 f 3.561 22.47;"
    "65536 256 4 c 2.248 17.67; 65536 256 4 f 4.714 33.17; 65536 256 5 c 2.755 25.17;"
    "65536 256 5 f 5.762 47.22; 65536 256 6 c 3.275 34.41; 65536 256 6 f 6.844 60.81;"
    "131072 32 1 c 0.1536 0.7808; 131072 32 1 f 0.3533 1.988; 131072 32 2 c 0.2601 1.617;"
    "131072 32 2 f 0.5663 4.032; 131072 32 3 c 0.3773 2.714; 131072 32 3 f 0.917 6.525;"
    "131072 32 4 c 1.28 6.234; 131072 32 4 f 1.23 9.547; 131072 32 5 c 1.845 9.143;"
    "131072 32 5 f 1.47 11.66; 131072 32 6 c 2.519 11.82; 131072 32 6 f 1.742 15.08;"
    "131072 64 1 c 0.2642 1.216; 131072 64 1 f 0.6656 3.829; 131072 64 2 c 0.4608 2.647;"
    "131072 64 2 f 1.083 7.902; 131072 64 3 c 0.6881 4.505; 131072 64 3 f 1.794 11.13;"
    "131072 64 4 c 1.147 9.641; 131072 64 4 f 2.37 16.43; 131072 64 5 c 1.396 12.78;"
    "131072 64 5 f 2.862 23.24; 131072 64 6 c 1.648 17.17; 131072 64 6 f 3.376 30.12;"
    "131072 96 1 c 0.3758 1.88; 131072 96 1 f 1.006 5.414; 131072 96 2 c 0.6641 4.163;"
    "131072 96 2 f 1.732 10.72; 131072 96 3 c 1.021 6.283; 131072 96 3 f 2.746 17.13;"
    "131072 96 4 c 1.705 13.77; 131072 96 4 f 3.547 24.69; 131072 96 5 c 2.093 19.97;"
    "131072 96 5 f 4.283 35.23; 131072 96 6 c 2.474 26.81; 131072 96 6 f 5.101 45.51;"
    "131072 128 1 c 0.4782 2.322; 131072 128 1 f 1.297 7.608; 131072 128 2 c 0.8607 5.134;"
    "131072 128 2 f 2.16 14.34; 131072 128 3 c 1.329 7.715; 131072 128 3 f 3.423 22.19;"
    "131072 128 4 c 2.244 17.49; 131072 128 4 f 4.799 33.18; 131072 128 5 c 2.742 25.24;"
    "131072 128 5 f 5.7 46.73; 131072 128 6 c 3.238 34.17; 131072 128 6 f 6.778 60.35;"
    "131072 256 1 c 0.9185 4.545; 131072 256 1 f 2.531 13.86; 131072 256 2 c 1.614 9.164;"
    "131072 256 2 f 4.236 28.46; 131072 256 3 c 2.579 15.32; 131072 256 3 f 6.652 45.07;"
    "131072 256 4 c 4.454 35.3; 131072 256 4 f 9.351 66.2; 131072 256 5 c 5.465 50.43;"
    "131072 256 5 f 11.42 95.81; 131072 256 6 c 6.479 68.71; 131072 256 6 f 13.54 124.1;"
)


def _a100_grid():
    table = {}
    for item in "".join(A100_GRID).split(";"):
        if item.strip():
            n, c, m, par, fwd, both = item.split()
            table[(int(n), int(c), int(m), "full" if par == "f" else "canonical")] = (
                float(fwd), float(both))
    return table


def _graph_step(torch, step, check):
    """Capture `step` in a HIP graph; replay it three times, each checked
    bitwise against `check` (the eager result), with eager work between."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(outs, check):
            if not torch.equal(got, want):
                raise RuntimeError("graph replay differs from the eager step")
        step()                                  # eager work between replays
    return graph


def _replay_ms(torch, graph, samples=20):
    import statistics
    for _ in range(3):
        graph.replay()
    events = [torch.cuda.Event(enable_timing=True) for _ in range(samples + 1)]
    torch.cuda.synchronize()
    events[0].record()
    for i in range(samples):
        graph.replay()
        events[i + 1].record()
    torch.cuda.synchronize()
    return statistics.median(events[i].elapsed_time(events[i + 1]) for i in range(samples))


def grid_main(args):
    """configs[2] (and configs[1]): forward and forward + full VJP of every
    (N, C, m_max, parity) point, each step captured in a HIP graph and timed
    as the median of 20 replays; kernel times from eager steps."""
    import torch
    from ictc_o2_hp import TensorProduct, _native

    torch.backends.cuda.matmul.allow_tf32 = False
    device = torch.device("cuda:0")
    _native.library()
    a100 = _a100_grid()
    if args.grid_set == "configs2":
        a100 = {k: v for k, v in a100.items() if k[1] in (32, 64, 128, 256) and k[2] in (1, 4, 6)}
    points = sorted(a100) + [(6400, 128, 6, "full")]
    if args.grid_rows:
        keep = {int(v) for v in args.grid_rows.split(",")}
        points = [pt for pt in points if pt[0] in keep]
    records = []
    for n, c, m, parity in points:
        torch.manual_seed(34527)
        module = TensorProduct(c, m, parity=parity).to(device)
        width, pw = module.representation_dimension, module.weight.numel()
        gen = torch.Generator(device=device).manual_seed(78211)
        x = torch.randn((n, width), device=device, generator=gen).requires_grad_()
        y = torch.randn((n, width), device=device, generator=gen).requires_grad_()
        cot = torch.ones((n, width), device=device)
        params = (x, y, module.weight)

        def both():
            return torch.autograd.grad(module(x, y), params, cot)

        def forward():
            with torch.no_grad():
                return (module(x, y),)

        eager_both, eager_fwd = both(), forward()
        g_both = _graph_step(torch, both, eager_both)
        g_fwd = _graph_step(torch, forward, eager_fwd)
        both_ms, fwd_ms = _replay_ms(torch, g_both), _replay_ms(torch, g_fwd)
        _, _, kinds, _ = _timed_steps(torch, both, 5, 1)
        kf = kinds["tp_forward"][0] / max(1, kinds["tp_forward"][1])
        kb = kinds["tp_backward"][0] / max(1, kinds["tp_backward"][1])
        alg = 4.0 * (8.0 * n * width + 3.0 * pw)
        ref = a100.get((n, c, m, parity))
        rec = {"rows": n, "channels": c, "m_max": m, "parity": parity, "width": width,
               "fwd_ms": fwd_ms, "fwd_vjp_ms": both_ms, "rows_per_s": n / (both_ms * 1e-3),
               "step_GBps": alg / (both_ms * 1e-3) / 1e9,
               "kernel_fwd_ms": kf, "kernel_bwd_ms": kb,
               "kernel_fwd_GBps": 4.0 * (3.0 * n * width + pw) / (kf * 1e-3) / 1e9,
               "kernel_bwd_GBps": 4.0 * (5.0 * n * width + 2.0 * pw) / (kb * 1e-3) / 1e9,
               "a100_fwd_ms": ref[0] if ref else None, "a100_fwd_vjp_ms": ref[1] if ref else None,
               "speedup_fwd_vjp": (ref[1] / both_ms) if ref else None}
        records.append(rec)
        print(json.dumps(rec), flush=True)
        del g_both, g_fwd, eager_both, eager_fwd, x, y, cot, module
        torch.cuda.empty_cache()
    if args.grid_out:
        Path(args.grid_out).write_text(json.dumps(records, indent=1))


# The reference's published radial chain (docs/RADIAL_PERFORMANCE.md:17-26, :37-52; A100,
# torch.compile): Linear(16,64)-SiLU-Linear(64,64)-SiLU-Linear(64,P*C,bias=False) -> V=1
# uvu TP, first/output full parity, angular canonical, m_max 6, per-edge inputs (no gather).
# (edges, C) -> (forward ms, full VJP ms).
A100_RADIAL = {
    (131072, 64): (25.991, 114.167), (16384, 64): (3.660, 13.159),
    (131072, 256): (102.812, 410.604), (32768, 128): (12.808, 50.896),
    (32768, 64): (6.212, 27.778), (65536, 64): (13.015, 56.530),
    (32768, 256): (25.843, 100.963), (131072, 128): (51.236, 208.039),
}


def radial_grid_main(args):
    """The reference's radial-chain benchmark points: compiled forward and full
    VJP (x, angular, basis and every network parameter), median of 11 samples
    after 20 warm-ups, as in docs/RADIAL_PERFORMANCE.md:3-11."""
    import statistics
    import torch
    from ictc_o2_hp import RadialUvuTensorProduct, UvuTensorProduct, _native, radial_ops

    torch.backends.cuda.matmul.allow_tf32 = False
    torch.set_float32_matmul_precision("highest")
    device = torch.device("cuda:0")
    _native.library()
    records = []
    points = sorted(A100_RADIAL.items(), key=lambda kv: kv[0][::-1])
    if args.radial_point:
        want = tuple(int(v) for v in args.radial_point.split(","))
        points = [kv for kv in points if kv[0] == want]
    for (edges, c), (ref_fwd, ref_vjp) in points:
        torch.manual_seed(7)
        tp = UvuTensorProduct(c, 1, 6, parity="full", parity_in2="canonical",
                              shared_weights=False)
        trunk = torch.nn.Sequential(torch.nn.Linear(16, 64), torch.nn.SiLU(),
                                    torch.nn.Linear(64, 64), torch.nn.SiLU())
        radial = RadialUvuTensorProduct(tp, torch.nn.Linear(64, tp.weight_numel, bias=False))

        class Chain(torch.nn.Module):
            def __init__(self):
                super().__init__()
                self.trunk, self.radial = trunk, radial

            def forward(self, x, angular, basis):
                return self.radial(x, angular, self.trunk(basis))

        chain = Chain().to(device)
        gen = torch.Generator(device=device).manual_seed(edges + c)
        x = torch.randn(edges, tp.input1_dimension, device=device, generator=gen)
        angular = torch.randn(edges, tp.input2_dimension, device=device, generator=gen)
        basis = torch.randn(edges, 16, device=device, generator=gen)
        for t in (x, angular, basis):
            t.requires_grad_()
        cot = torch.randn(edges, tp.input1_dimension, device=device, generator=gen)
        run = torch.compile(chain, fullgraph=True, dynamic=False)
        params = [x, angular, basis] + list(chain.parameters())

        def forward():
            return run(x, angular, basis)

        def full_vjp():
            return torch.autograd.grad(run(x, angular, basis), params, cot)

        times = {}
        for name, fn in (("forward", forward), ("full_vjp", full_vjp)):
            for _ in range(20):
                fn()
            torch.cuda.synchronize()
            samples = []
            for _ in range(11):
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record()
                fn()
                e1.record()
                torch.cuda.synchronize()
                samples.append(e0.elapsed_time(e1))
            times[name] = statistics.median(samples)
        rec = {"edges": edges, "channels": c, "paths": tp.weight_numel // c,
               "fused_kernels": radial_ops.fused_plan(tp._kernel_metadata_id, 64) is not None,
               "forward_ms": times["forward"], "full_vjp_ms": times["full_vjp"],
               "a100_forward_ms": ref_fwd, "a100_full_vjp_ms": ref_vjp,
               "speedup_forward": ref_fwd / times["forward"],
               "speedup_full_vjp": ref_vjp / times["full_vjp"]}
        records.append(rec)
        print(json.dumps(rec), flush=True)
        del chain, run, x, angular, basis, cot
        torch.cuda.empty_cache()
    if args.grid_out:
        Path(args.grid_out).write_text(json.dumps(records, indent=1))


def main():
    args = _args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); "
              f"got --gpus {args.gpus}", file=sys.stderr)
        raise SystemExit(2)
    if args.workload == "grid":
        return grid_main(args)
    if args.workload == "radial-grid":
        return radial_grid_main(args)
    if args.workload == "force":
        return force_main(args)
    if args.workload == "uvu-shared":
        return uvu_shared_main(args)
    if args.workload == "uvu-rows":
        return uvu_main(args, v=1)
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

    peak_mib = torch.cuda.max_memory_allocated() / 2**20
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
        "peak_allocated_MiB": peak_mib,
        "roofline": {"bound": "hbm", "kernel": "tp_backward_kernel", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": _traffic(REPO / "profiles" / "traffic.json",
                                         f"backward_C{args.channels}_m{args.m_max}_{args.parity}_N{n}")},
    }
    del x, y, cot
    torch.cuda.empty_cache()
    if not args.no_stream_ceiling:
        ceiling = _stream_ceiling(n, width)
        if ceiling:
            record["stream_ceiling"] = ceiling
            record["roofline"]["frac_of_stream_ceiling"] = achieved / ceiling["read3_write2_GBps"]
            record["kernels_ms"]["forward_frac_of_stream_ceiling"] = (
                alg_fwd / (fwd_avg * 1e-3) / 1e9 / ceiling["read2_write1_GBps"])
    if not args.no_cpu_baseline:
        record["cpu_baseline"] = _cpu_baseline(args.channels, args.m_max, args.parity, width,
                                               args.cpu_seconds)
    print(json.dumps(record), flush=True)


if __name__ == "__main__":
    main()
