"""GPU parity of the gathered radial input and the deterministic row gather /
scatter-add (HIP kernels through the C ABI) against the fp64 oracle.

Gate: normalized max error <= 1e-5 (the reference's gate) for float arithmetic;
the gather is checked bitwise, and the scatter-add bitwise against a float32
sum of each table row's edges in increasing edge order (its documented order).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import uvu_oracle as U
from oracle.o2_oracle import normalized_error

TOL = 1e-5
pytestmark = pytest.mark.gpu


def _sequential_f32(rows, index, n):
    """Each table row's edges summed in increasing edge order, in float32."""
    out = np.zeros((n, rows.shape[1]), dtype=np.float32)
    for e in np.argsort(index, kind="stable"):
        i = index[e]
        if 0 <= i < n:
            out[i] = np.float32(out[i] + rows[e])
    return out


@pytest.mark.parametrize("width", [576, 7])
def test_gather_rows_bitwise(width):
    from ictc_o2_hp import gather_rows
    print(f"gather width={width}", flush=True)
    rng = np.random.default_rng(10)
    table = rng.standard_normal((300, width)).astype(np.float32)
    index = rng.integers(-5, 310, size=1000)
    got = gather_rows(torch.from_numpy(table).cuda(), torch.from_numpy(index).cuda())
    assert np.array_equal(got.cpu().numpy(), U.gather(table, index))


@pytest.mark.parametrize("width", [576, 9])
def test_scatter_add_rows_fixed_order(width):
    from ictc_o2_hp import scatter_add_rows
    print(f"scatter width={width}", flush=True)
    rng = np.random.default_rng(11)
    rows = rng.standard_normal((3000, width)).astype(np.float32)
    index = rng.integers(-3, 200, size=3000)
    got = scatter_add_rows(torch.from_numpy(rows).cuda(), torch.from_numpy(index).cuda(), 200)
    got = got.cpu().numpy()
    assert np.array_equal(got, _sequential_f32(rows, index, 200))
    ref = U.scatter_add(rows.astype(np.float64), index, 200)
    assert normalized_error(ref, got) <= TOL


def test_scatter_add_rows_reproducible_and_adjoint():
    from ictc_o2_hp import gather_rows, scatter_add_rows
    torch.manual_seed(12)
    table = torch.randn(5000, 576, device="cuda", dtype=torch.float64).float()
    index = torch.randint(0, 5000, (200000,), device="cuda")
    rows = torch.randn(200000, 576, device="cuda")
    a = scatter_add_rows(rows, index, 5000)
    b = scatter_add_rows(rows, index, 5000)
    assert torch.equal(a, b)
    terms = gather_rows(table, index).double() * rows.double()
    lhs, rhs = terms.sum(), (table.double() * a.double()).sum()
    assert abs(float(lhs - rhs)) <= 1e-6 * float(terms.abs().sum())
    # Autograd of each is the other.
    t = table.clone().requires_grad_()
    (g,) = torch.autograd.grad(gather_rows(t, index), t, rows)
    assert torch.equal(g, a)


def _build(c, m, hidden, seed, bias=True):
    from ictc_o2_hp import RadialUvuTensorProduct, UvuTensorProduct
    tp = UvuTensorProduct(c, 1, m, parity="canonical", shared_weights=False).cuda()
    linear = torch.nn.Linear(hidden, tp.weight_numel, bias=bias).cuda()
    rng = np.random.default_rng(seed + 1)
    with torch.no_grad():
        linear.weight.copy_(torch.from_numpy(rng.standard_normal(linear.weight.shape)
                                             / np.sqrt(hidden)))
        if bias:
            linear.bias.copy_(torch.from_numpy(rng.standard_normal(linear.bias.shape) * 0.5))
    plan = U.UvuOraclePlan(c, 1, m, parity="canonical")
    return tp, linear, RadialUvuTensorProduct(tp, linear), plan


def _gathered_case(c, m, hidden, nodes, edges, seed, low=0, high=None, wrt_roles=5):
    print(f"gathered radial C={c} m={m} H={hidden} nodes={nodes} edges={edges} seed={seed}",
          flush=True)
    tp, linear, module, plan = _build(c, m, hidden, seed)
    rng = np.random.default_rng(seed)
    table = rng.standard_normal((nodes, plan.width1)).astype(np.float32)
    index = rng.integers(low, nodes if high is None else high, size=edges)
    y = rng.standard_normal((edges, plan.width2)).astype(np.float32)
    h = rng.standard_normal((edges, hidden)).astype(np.float32)
    g = rng.standard_normal((edges, plan.width1)).astype(np.float32)
    tt, yt, ht = (torch.from_numpy(a).cuda().requires_grad_() for a in (table, y, h))
    it = torch.from_numpy(index).cuda()
    out = module(tt, yt, ht, left_index=it)
    params = (tt, yt, ht, linear.weight, linear.bias)[:wrt_roles]
    grads = torch.autograd.grad(out, params, torch.from_numpy(g).cuda())
    torch.cuda.synchronize()
    alpha = linear.weight.detach().double().cpu().numpy()
    b = linear.bias.detach().double().cpu().numpy()
    args = (plan, table.astype(np.float64), index, y.astype(np.float64), h.astype(np.float64),
            alpha, b)
    assert normalized_error(U.radial_gather_forward(*args), out.detach().cpu().numpy()) <= TOL
    ref = U.radial_gather_backward(*args, g.astype(np.float64))
    for r, a in zip(ref, grads):
        assert a.shape == r.shape
        assert normalized_error(r, a.double().cpu().numpy()) <= TOL
    return tp, linear, module, (tt, it, yt, ht, torch.from_numpy(g).cuda()), out, grads


def test_configs4_structure_gathered_fused():
    from ictc_o2_hp import radial_ops, scatter_add_rows
    tp, linear, module, (tt, it, yt, ht, g), out, grads = _gathered_case(64, 4, 64, 2000, 5000, 20)
    assert radial_ops.fused_plan(tp._kernel_metadata_id, 64) is not None
    # Same arithmetic as the kernels on materialised rows; the table adjoint is
    # the fixed-order sum of those rows' adjoints.
    left = tt.detach()[it].requires_grad_()
    ref_out = module(left, yt, ht)
    assert torch.equal(out, ref_out)
    ref_grads = torch.autograd.grad(ref_out, (left, yt, ht, linear.weight, linear.bias), g)
    assert torch.equal(grads[0], scatter_add_rows(ref_grads[0], it, tt.shape[0]))
    for a, b in zip(grads[1:], ref_grads[1:]):
        assert torch.equal(a, b)


def test_gathered_out_of_range_and_ragged():
    _gathered_case(32, 2, 16, 100, 131, 21, low=-4, high=106)
    _gathered_case(16, 1, 8, 7, 1, 22)


def test_gathered_composed_structure():
    from ictc_o2_hp import radial_ops
    tp, *_ = _gathered_case(24, 2, 8, 50, 300, 23)     # C % 16 != 0: no fused kernel
    assert radial_ops.fused_plan(tp._kernel_metadata_id, 8) is None


def test_gathered_roles_subset():
    _gathered_case(32, 2, 16, 64, 200, 24, wrt_roles=1)     # table only
    _gathered_case(32, 2, 16, 64, 200, 25, wrt_roles=3)     # table, angular, hidden


def test_gathered_empty_edges():
    tp, linear, module, _ = _build(32, 2, 16, 26)
    table = torch.randn(10, tp.input1_dimension, device="cuda", requires_grad=True)
    index = torch.zeros(0, dtype=torch.int64, device="cuda")
    y = torch.randn(0, tp.input2_dimension, device="cuda", requires_grad=True)
    h = torch.randn(0, 16, device="cuda", requires_grad=True)
    out = module(table, y, h, left_index=index)
    assert out.shape == (0, tp.input1_dimension)
    gt, ga, gb = torch.autograd.grad(out, (table, linear.weight, linear.bias),
                                     torch.zeros_like(out))
    assert torch.count_nonzero(gt) == 0 and torch.count_nonzero(ga) == 0
    assert torch.count_nonzero(gb) == 0


def test_gathered_reproducible():
    tp, linear, module, _ = _build(64, 4, 64, 27)
    torch.manual_seed(27)
    table = torch.randn(3000, tp.input1_dimension, device="cuda", requires_grad=True)
    index = torch.randint(0, 3000, (20000,), device="cuda")
    y = torch.randn(20000, tp.input2_dimension, device="cuda")
    h = torch.randn(20000, 64, device="cuda")
    g = torch.randn(20000, tp.input1_dimension, device="cuda")
    params = (table, linear.weight, linear.bias)
    first = torch.autograd.grad(module(table, y, h, left_index=index), params, g)
    second = torch.autograd.grad(module(table, y, h, left_index=index), params, g)
    for a, b in zip(first, second):
        assert torch.equal(a, b)


def test_gathered_torch_compile_fullgraph():
    tp, linear, module, _ = _build(32, 2, 16, 28)
    torch.manual_seed(28)
    table = torch.randn(40, tp.input1_dimension, device="cuda", requires_grad=True)
    index = torch.randint(0, 40, (96,), device="cuda")
    y = torch.randn(96, tp.input2_dimension, device="cuda", requires_grad=True)
    h = torch.randn(96, 16, device="cuda", requires_grad=True)
    g = torch.randn(96, tp.input1_dimension, device="cuda")

    def run(t, i, yy, hh):
        return module(t, yy, hh, left_index=i)

    compiled = torch.compile(run, fullgraph=True, dynamic=False)
    params = (table, y, h, linear.weight, linear.bias)
    eager = torch.autograd.grad(run(table, index, y, h), params, g)
    comp = torch.autograd.grad(compiled(table, index, y, h), params, g)
    for a, b in zip(eager, comp):
        assert torch.equal(a, b)


@pytest.mark.parametrize("c,hidden", [(16, 8), (24, 8)])   # fused, composed
def test_gathered_double_backward(c, hidden):
    from ictc_o2_hp import RadialUvuTensorProduct, UvuTensorProduct
    print(f"gathered double backward C={c} H={hidden}", flush=True)
    tp, linear, module, _ = _build(c, 2, hidden, 29)
    torch.manual_seed(29)
    table = torch.randn(6, tp.input1_dimension, device="cuda", requires_grad=True)
    index = torch.randint(0, 6, (20,), device="cuda")
    y = torch.randn(20, tp.input2_dimension, device="cuda", requires_grad=True)
    h = torch.randn(20, hidden, device="cuda", requires_grad=True)

    def second_order(mod, lin, tt, ii, yy, hh):
        loss = mod(tt, yy, hh, left_index=ii).square().sum()
        gt, gh = torch.autograd.grad(loss, (tt, hh), create_graph=True)
        return torch.autograd.grad(gt.square().sum() + gh.sum(), (tt, yy, lin.weight, lin.bias))

    got = second_order(module, linear, table, index, y, h)
    tp64 = UvuTensorProduct(c, 1, 2, parity="canonical", shared_weights=False).double()
    lin64 = torch.nn.Linear(hidden, tp64.weight_numel).double()
    with torch.no_grad():
        lin64.weight.copy_(linear.weight.double().cpu())
        lin64.bias.copy_(linear.bias.double().cpu())
    ref_module = RadialUvuTensorProduct(tp64, lin64)
    t64, y64, h64 = (v.detach().double().cpu().requires_grad_() for v in (table, y, h))
    want = second_order(ref_module, lin64, t64, index.cpu(), y64, h64)
    for r, a in zip(want, got):
        assert normalized_error(r.detach().numpy(), a.double().cpu().numpy()) <= TOL


def test_message_passing_gather_and_aggregate():
    """left_index (fused gather) and out_index (deterministic edge -> node sum)
    together, at the configs[4] structure, against the oracle; reproducible."""
    from ictc_o2_hp import radial_ops
    print("message passing C64 m4 H64 nodes=1500 edges=6000", flush=True)
    tp, linear, module, plan = _build(64, 4, 64, 31)
    assert radial_ops.fused_plan(tp._kernel_metadata_id, 64) is not None
    rng = np.random.default_rng(31)
    nodes, edges = 1500, 6000
    table = rng.standard_normal((nodes, plan.width1)).astype(np.float32)
    src = rng.integers(0, nodes, size=edges)
    dst = rng.integers(0, nodes, size=edges)
    y = rng.standard_normal((edges, plan.width2)).astype(np.float32)
    h = rng.standard_normal((edges, 64)).astype(np.float32)
    g = rng.standard_normal((nodes, plan.width1)).astype(np.float32)
    tt, yt, ht = (torch.from_numpy(a).cuda().requires_grad_() for a in (table, y, h))
    st, dt = torch.from_numpy(src).cuda(), torch.from_numpy(dst).cuda()
    params = (tt, yt, ht, linear.weight, linear.bias)

    def run():
        out = module(tt, yt, ht, left_index=st, out_index=dt, out_rows=nodes)
        return (out, *torch.autograd.grad(out, params, torch.from_numpy(g).cuda()))

    first, second = run(), run()
    for a, b in zip(first, second):
        assert torch.equal(a, b)
    alpha = linear.weight.detach().double().cpu().numpy()
    bias = linear.bias.detach().double().cpu().numpy()
    args = (plan, table.astype(np.float64), src, y.astype(np.float64), h.astype(np.float64),
            alpha, bias)
    want = U.scatter_add(U.radial_gather_forward(*args), dst, nodes)
    assert normalized_error(want, first[0].detach().cpu().numpy()) <= TOL
    ref = U.radial_gather_backward(*args, U.gather(g.astype(np.float64), dst))
    for r, a in zip(ref, first[1:]):
        assert normalized_error(r, a.double().cpu().numpy()) <= TOL
