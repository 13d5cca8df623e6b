"""Qualification at the benchmarked sizes: every BASELINE.json configs[2]
family, configs[3] and configs[4] at their full launch geometry against the
fp64 oracles (gate: normalized max error <= 1e-5).

The reference qualifies each configs[2] family at N = 131072 against fp64
before it times anything (benchmarks/eqx/scripts/run_scan.py:49-58,
validate_math.py:13-110).  Here each case runs the kernels on the whole
tensor; rows (edges) are independent, so a random subset of them is compared
with the oracle, and the sums over rows (TP dw, radial dalpha / dbias and the
node-table gradient) come from a cotangent that is zero outside the subset,
which makes the oracle's sums over the subset the exact expected values.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import o2_oracle as O
from oracle import uvu_oracle as U

TOL = 1e-5
pytestmark = pytest.mark.gpu


def _subset(n, count, seed):
    rows = torch.randperm(n, generator=torch.Generator().manual_seed(seed))[:count]
    return rows.sort().values.cuda()


def _np(t, rows=None):
    t = t.detach()
    if rows is not None:
        t = t[rows]
    return t.double().cpu().numpy()


# N x C x m_max x parity.  Every (C, m_max, parity) family at the
# smallest and the largest N of the grid; all C are even, so the channel-major
# float2-access kernels of each family run (every family of the grid, including
# M1 full, M4 canonical and M6 canonical).
GRID = [(c, m, parity, n) for c in (32, 64, 128, 256) for m in (1, 4, 6)
        for parity in ("canonical", "full") for n in (16384, 131072)]


@pytest.mark.parametrize("channels,m_max,parity,n_rows", GRID)
def test_configs2_family_at_full_size(channels, m_max, parity, n_rows):
    from ictc_o2_hp import TensorProduct
    print(f"qualification TP C{channels} m{m_max} {parity} N={n_rows}", flush=True)
    torch.manual_seed(channels + 10 * m_max)
    module = TensorProduct(channels, m_max, parity=parity).cuda()
    gen = torch.Generator(device="cuda").manual_seed(n_rows + channels * 31 + m_max)
    width = module.representation_dimension
    x = torch.randn((n_rows, width), device="cuda", generator=gen).requires_grad_()
    y = torch.randn((n_rows, width), device="cuda", generator=gen).requires_grad_()
    g = torch.randn((n_rows, width), device="cuda", generator=gen)
    rows = _subset(n_rows, 256, n_rows + channels)
    mask = torch.zeros((n_rows, 1), device="cuda")
    mask[rows] = 1.0
    g = g * mask
    # The float2-access variant needs even rows and 8-byte aligned tensors.
    assert (parity == "full" or channels % 2 == 0) and x.data_ptr() % 8 == 0
    out = module(x, y)
    dx, dy, dw = torch.autograd.grad(out, (x, y, module.weight), g)
    torch.cuda.synchronize()
    plan = O.OraclePlan(channels, m_max, parity)
    w = _np(module.weight)
    xs, ys, gs = _np(x, rows), _np(y, rows), _np(g, rows)
    ref_dx, ref_dy, ref_dw = O.backward(plan, xs, ys, w, gs)
    errors = {
        "out": O.normalized_error(O.forward(plan, xs, ys, w), _np(out, rows)),
        "dx": O.normalized_error(ref_dx, _np(dx, rows)),
        "dy": O.normalized_error(ref_dy, _np(dy, rows)),
        "dw": O.normalized_error(ref_dw, _np(dw)),
    }
    assert max(errors.values()) <= TOL, errors


def test_configs3_uvu_per_row_weights_at_benchmark_size():
    """configs[3] (C128, V32, m4 full, per-row weights N(0, 1/sqrt(32))) at the
    benchmarked N = 16384: w and dw are 65.5 GB each.  Per-row dw rows are
    independent, so 32 random rows of out, dx, dy and dw are compared."""
    from ictc_o2_hp import UvuTensorProduct
    print("qualification uvu C128 V32 m4 full N=16384", flush=True)
    n = 16384
    module = UvuTensorProduct(128, 32, 4, parity="full", shared_weights=False,
                              internal_weights=False).cuda()
    gen = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn((n, module.input1_dimension), device="cuda", generator=gen).requires_grad_()
    y = torch.randn((n, module.input2_dimension), device="cuda", generator=gen).requires_grad_()
    w = torch.randn((n, module.weight_numel), device="cuda", generator=gen)
    w.mul_(1.0 / math.sqrt(32)).requires_grad_()
    g = torch.randn((n, module.input1_dimension), device="cuda", generator=gen)
    out = module(x, y, w)
    dx, dy, dw = torch.autograd.grad(out, (x, y, w), g)
    torch.cuda.synchronize()
    rows = _subset(n, 32, 33)
    plan = U.UvuOraclePlan(128, 32, 4, parity="full")
    xs, ys, ws, gs = _np(x, rows), _np(y, rows), _np(w, rows), _np(g, rows)
    ref_dx, ref_dy, ref_dw = U.backward(plan, xs, ys, ws, gs, shared=False)
    errors = {
        "out": O.normalized_error(U.forward(plan, xs, ys, ws, shared=False), _np(out, rows)),
        "dx": O.normalized_error(ref_dx, _np(dx, rows)),
        "dy": O.normalized_error(ref_dy, _np(dy, rows)),
        "dw": O.normalized_error(ref_dw, _np(dw, rows)),
    }
    assert max(errors.values()) <= TOL, errors


def _configs4_inputs(edges, nodes, seed):
    from ictc_o2_hp import RadialUvuTensorProduct, UvuTensorProduct
    torch.manual_seed(seed)
    tp = UvuTensorProduct(64, 1, 4, parity="canonical", shared_weights=False).cuda()
    radial_out = torch.nn.Linear(64, tp.weight_numel).cuda()
    module = RadialUvuTensorProduct(tp, radial_out)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    table = torch.randn((nodes, tp.input1_dimension), device="cuda", generator=gen)
    src = torch.randint(0, nodes, (edges,), device="cuda", generator=gen)
    phi = 2.0 * math.pi * torch.rand((edges, 1), device="cuda", generator=gen)
    parts = [torch.ones_like(phi)]
    for m in range(1, 5):
        parts += [torch.cos(m * phi), torch.sin(m * phi)]
    angular = torch.cat(parts, dim=1).contiguous()
    hidden = torch.nn.functional.silu(torch.randn((edges, 64), device="cuda", generator=gen))
    g = torch.randn((edges, tp.input1_dimension), device="cuda", generator=gen)
    return tp, radial_out, module, table, src, angular, hidden, g


def test_configs4_radial_at_benchmark_size():
    """E = 1,048,576 edges, C64 m4 canonical, H64, node rows
    gathered from 65,536 nodes through the fused left_index read.  256 random
    edges: out, dangular, dhidden on those edges; the node-table gradient,
    dalpha and dbias from a cotangent that is zero on every other edge."""
    from ictc_o2_hp import radial_ops
    print("qualification radial C64 m4 canonical H64 E=1048576 gathered", flush=True)
    edges, nodes = 1 << 20, 65536
    tp, linear, module, table, src, angular, hidden, g = _configs4_inputs(edges, nodes, 4)
    assert radial_ops.fused_plan(tp._kernel_metadata_id, 64) is not None
    rows = _subset(edges, 256, 44)
    mask = torch.zeros((edges, 1), device="cuda")
    mask[rows] = 1.0
    g = g * mask
    table.requires_grad_()
    angular.requires_grad_()
    hidden.requires_grad_()
    out = module(table, angular, hidden, left_index=src)
    dtable, dang, dhid, dalpha, dbias = torch.autograd.grad(
        out, (table, angular, hidden, linear.weight, linear.bias), g)
    torch.cuda.synchronize()
    plan = U.UvuOraclePlan(64, 1, 4, parity="canonical")
    idx = src[rows].cpu().numpy()
    args = (plan, _np(table), idx, _np(angular, rows), _np(hidden, rows), _np(linear.weight),
            _np(linear.bias))
    ref_out = U.radial_gather_forward(*args)
    ref = U.radial_gather_backward(*args, _np(g, rows))
    errors = {
        "out": O.normalized_error(ref_out, _np(out, rows)),
        "dtable": O.normalized_error(ref[0], _np(dtable)),
        "dangular": O.normalized_error(ref[1], _np(dang, rows)),
        "dhidden": O.normalized_error(ref[2], _np(dhid, rows)),
        "dalpha": O.normalized_error(ref[3], _np(dalpha)),
        "dbias": O.normalized_error(ref[4], _np(dbias)),
    }
    assert max(errors.values()) <= TOL, errors


def test_configs4_radial_full_size_is_reproducible():
    """configs[4] at full size with a dense cotangent: two backward passes give
    bitwise equal gradients (fixed-order sums, no atomics)."""
    print("qualification radial E=1048576 bitwise reproducibility", flush=True)
    edges, nodes = 1 << 20, 65536
    tp, linear, module, table, src, angular, hidden, g = _configs4_inputs(edges, nodes, 5)
    for t in (table, angular, hidden):
        t.requires_grad_()
    results = []
    for _ in range(2):
        out = module(table, angular, hidden, left_index=src)
        grads = torch.autograd.grad(out, (table, angular, hidden, linear.weight, linear.bias), g)
        results.append([out.detach(), *grads])
    torch.cuda.synchronize()
    for a, b in zip(*results):
        assert torch.equal(a, b)
