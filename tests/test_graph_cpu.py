"""Gathered radial input and deterministic row scatter-add: oracle pins, CPU
paths and C-ABI argument checks (no GPU needed)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import uvu_oracle as U
from oracle.o2_oracle import normalized_error


def _loop_gather(table, index):
    out = np.zeros((len(index), table.shape[1]))
    for e, i in enumerate(index):
        if 0 <= i < table.shape[0]:
            out[e] = table[i]
    return out


def _loop_scatter(rows, index, n):
    out = np.zeros((n, rows.shape[1]))
    for e, i in enumerate(index):
        if 0 <= i < n:
            out[i] += rows[e]
    return out


def test_oracle_gather_scatter_brute_force():
    rng = np.random.default_rng(0)
    table = rng.standard_normal((7, 5))
    index = np.array([3, 0, 6, 3, 3, -1, 7, 2, 100, 0])
    rows = rng.standard_normal((len(index), 5))
    assert np.array_equal(U.gather(table, index), _loop_gather(table, index))
    assert np.allclose(U.scatter_add(rows, index, 7), _loop_scatter(rows, index, 7),
                       rtol=0, atol=1e-15)


def test_oracle_scatter_is_the_adjoint_of_gather():
    rng = np.random.default_rng(1)
    table = rng.standard_normal((11, 4))
    index = rng.integers(-2, 13, size=40)
    rows = rng.standard_normal((40, 4))
    lhs = np.sum(U.gather(table, index) * rows)
    rhs = np.sum(table * U.scatter_add(rows, index, 11))
    assert abs(lhs - rhs) <= 1e-12 * (1 + abs(lhs))
    # A scatter into the neighbouring row breaks the identity.
    wrong = U.scatter_add(rows, np.where(index >= 0, index + 1, index), 12)[:11]
    assert abs(np.sum(table * wrong) - lhs) > 1e-3


def test_oracle_gathered_radial_table_gradient_finite_differences():
    plan = U.UvuOraclePlan(2, 1, 1, parity="canonical")
    rng = np.random.default_rng(2)
    nodes, edges, hidden = 3, 6, 3
    table = rng.standard_normal((nodes, plan.width1))
    index = np.array([0, 2, 2, 1, 0, 2])
    y = rng.standard_normal((edges, plan.width2))
    h = rng.standard_normal((edges, hidden))
    alpha = rng.standard_normal((plan.weight_numel, hidden))
    bias = rng.standard_normal(plan.weight_numel)
    g = rng.standard_normal((edges, plan.width1))
    dtable = U.radial_gather_backward(plan, table, index, y, h, alpha, bias, g)[0]
    eps = 1e-6
    fd = np.zeros_like(table)
    for r in range(nodes):
        for c in range(plan.width1):
            tp, tm = table.copy(), table.copy()
            tp[r, c] += eps
            tm[r, c] -= eps
            fp = np.sum(g * U.radial_gather_forward(plan, tp, index, y, h, alpha, bias))
            fm = np.sum(g * U.radial_gather_forward(plan, tm, index, y, h, alpha, bias))
            fd[r, c] = (fp - fm) / (2 * eps)
    assert np.allclose(dtable, fd, rtol=1e-6, atol=1e-7)


def test_graph_ops_cpu_match_oracle_and_gradcheck():
    from ictc_o2_hp import gather_rows, scatter_add_rows
    rng = np.random.default_rng(3)
    table = torch.from_numpy(rng.standard_normal((9, 6))).requires_grad_()
    index = torch.tensor([4, 4, 0, 8, -3, 9, 2, 4])
    rows = torch.from_numpy(rng.standard_normal((8, 6))).requires_grad_()
    assert np.array_equal(gather_rows(table, index).detach().numpy(),
                          U.gather(table.detach().numpy(), index.numpy()))
    assert np.allclose(scatter_add_rows(rows, index, 9).detach().numpy(),
                       U.scatter_add(rows.detach().numpy(), index.numpy(), 9), atol=1e-14)
    assert torch.autograd.gradcheck(lambda t: gather_rows(t, index), (table,))
    assert torch.autograd.gradcheck(lambda r: scatter_add_rows(r, index, 9), (rows,))
    assert torch.autograd.gradgradcheck(lambda t: gather_rows(t, index), (table,))
    with pytest.raises(ValueError):
        gather_rows(table, index.reshape(2, 4))
    with pytest.raises(ValueError):
        scatter_add_rows(rows, index[:3], 9)
    with pytest.raises(ValueError):
        gather_rows(table, index.float())


def _radial_module(c, m, hidden, dtype=torch.float64, seed=0):
    from ictc_o2_hp import RadialUvuTensorProduct, UvuTensorProduct
    torch.manual_seed(seed)
    tp = UvuTensorProduct(c, 1, m, parity="canonical", shared_weights=False).to(dtype)
    lin = torch.nn.Linear(hidden, tp.weight_numel).to(dtype)
    return tp, lin, RadialUvuTensorProduct(tp, lin)


def test_module_left_index_cpu_matches_oracle():
    tp, lin, module = _radial_module(4, 2, 5)
    plan = U.UvuOraclePlan(4, 1, 2, parity="canonical")
    rng = np.random.default_rng(4)
    nodes, edges = 7, 23
    table = torch.from_numpy(rng.standard_normal((nodes, plan.width1))).requires_grad_()
    index = torch.from_numpy(rng.integers(0, nodes, size=edges))
    y = torch.from_numpy(rng.standard_normal((edges, plan.width2))).requires_grad_()
    h = torch.from_numpy(rng.standard_normal((edges, 5))).requires_grad_()
    g = rng.standard_normal((edges, plan.width1))
    out = module(table, y, h, left_index=index)
    grads = torch.autograd.grad(out, (table, y, h, lin.weight, lin.bias), torch.from_numpy(g))
    args = (plan, table.detach().numpy(), index.numpy(), y.detach().numpy(),
            h.detach().numpy(), lin.weight.detach().numpy(), lin.bias.detach().numpy())
    assert normalized_error(U.radial_gather_forward(*args), out.detach().numpy()) <= 1e-12
    for r, a in zip(U.radial_gather_backward(*args, g), grads):
        assert normalized_error(r, a.numpy()) <= 1e-12


def test_module_left_index_validation():
    tp, lin, module = _radial_module(4, 1, 3)
    table = torch.randn(5, tp.input1_dimension, dtype=torch.float64)
    index = torch.tensor([0, 1, 4])
    y = torch.randn(3, tp.input2_dimension, dtype=torch.float64)
    h = torch.randn(3, 3, dtype=torch.float64)
    module(table, y, h, left_index=index)
    with pytest.raises(ValueError):
        module(table[:, :-1], y, h, left_index=index)
    with pytest.raises(ValueError):
        module(table, y[:2], h, left_index=index)
    with pytest.raises(ValueError):
        module(table, y, h[:, :2], left_index=index)
    with pytest.raises(ValueError):
        module(table, y, h, left_index=index.float())
    with pytest.raises(ValueError):
        module(table.unsqueeze(0), y, h, left_index=index)


def test_rows_c_abi_argument_checks():
    from ictc_o2_hp import _native
    lib = _native.library()
    assert lib.o2mi_rows_gather_f32(None, 0, None, -1, 4, None, None) != 0
    assert lib.o2mi_rows_gather_f32(None, 0, None, 0, 4, None, None) == 0
    assert lib.o2mi_rows_gather_f32(None, 0, None, 5, 4, None, None) != 0
    assert lib.o2mi_rows_segment_sum_f32(None, 0, 4, None, None, -1, None, None) != 0
    assert lib.o2mi_rows_segment_sum_f32(None, 0, 4, None, None, 0, None, None) == 0
    assert lib.o2mi_rows_segment_sum_f32(None, 3, 4, None, None, 2, None, None) != 0
    handle = ctypes.c_void_p()
    assert lib.o2mi_radial_plan_create(64, 4, 0, 4, 0, 64, ctypes.byref(handle)) == 0
    try:
        # A table of 2^31 bytes or more is refused before any launch.
        big = (1 << 31) // (4 * 576)
        status = lib.o2mi_radial_forward_gather_f32(handle, None, big + 1, None, None, None,
                                                    None, None, None, None, 1, None)
        assert status == -2
        assert b"2 GiB" in lib.o2mi_last_error()
    finally:
        lib.o2mi_radial_plan_destroy(handle)


def test_module_out_index_cpu_matches_oracle():
    tp, lin, module = _radial_module(4, 2, 5, seed=5)
    plan = U.UvuOraclePlan(4, 1, 2, parity="canonical")
    rng = np.random.default_rng(5)
    nodes, edges = 9, 31
    table = torch.from_numpy(rng.standard_normal((nodes, plan.width1))).requires_grad_()
    src = torch.from_numpy(rng.integers(0, nodes, size=edges))
    dst = torch.from_numpy(rng.integers(-1, nodes + 1, size=edges))   # includes dropped ones
    y = torch.from_numpy(rng.standard_normal((edges, plan.width2))).requires_grad_()
    h = torch.from_numpy(rng.standard_normal((edges, 5))).requires_grad_()
    g = rng.standard_normal((nodes, plan.width1))
    out = module(table, y, h, left_index=src, out_index=dst, out_rows=nodes)
    assert out.shape == (nodes, plan.width1)
    grads = torch.autograd.grad(out, (table, y, h, lin.weight, lin.bias), torch.from_numpy(g))
    args = (plan, table.detach().numpy(), src.numpy(), y.detach().numpy(),
            h.detach().numpy(), lin.weight.detach().numpy(), lin.bias.detach().numpy())
    want = U.scatter_add(U.radial_gather_forward(*args), dst.numpy(), nodes)
    assert normalized_error(want, out.detach().numpy()) <= 1e-12
    # Adjoint of the scatter: the node cotangent gathered per edge.
    ref = U.radial_gather_backward(*args, U.gather(g, dst.numpy()))
    for r, a in zip(ref, grads):
        assert normalized_error(r, a.numpy()) <= 1e-12
    # Without left_index the per-edge rows are given directly.
    left = table.detach()[src]
    direct = module(left, y, h, out_index=dst, out_rows=nodes)
    assert torch.allclose(direct, out, atol=1e-12)
    with pytest.raises(ValueError):
        module(table, y, h, left_index=src, out_index=dst)
    with pytest.raises(ValueError):
        module(table, y, h, left_index=src, out_index=dst[:3], out_rows=nodes)
