"""CPU checks of the uvu plan, the uvu oracle and the module surface.

The oracle is pinned by the reference's recorded tables and vectors
(tests/golden/uvu_*), by finite differences of its forward, by the bilinear
adjoint identity, and by planted mistakes that must fail those pins.
"""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import uvu_oracle as U
from oracle.o2_oracle import normalized_error

TABLES = json.loads((GOLDEN / "uvu_tables.json").read_text())

PLAN_ARGS = {
    "c128_v32_m4_full": (128, 32, 4, {"parity": "full"}),
    "c64_v1_m4_canonical": (64, 1, 4, {"parity": "canonical"}),
    "c128_v1_m6_full_in2canonical": (128, 1, 6, {"parity": "full", "parity_in2": "canonical"}),
    "c3_v2_m2_full": (3, 2, 2, {"parity": "full"}),
    "c4_v1_m4_canonical": (4, 1, 4, {"parity": "canonical"}),
    "c3_v1_m6_full_in2canonical": (3, 1, 6, {"parity": "full", "parity_in2": "canonical"}),
    "c2_v3_m3_canonical_in2full_m2_path": (2, 3, 3, {"parity": "canonical", "parity_in2": "full",
                                                     "m_max_in2": 2,
                                                     "path_normalization": "path"}),
    "c2_v2_m1_full_norm_element": (2, 2, 1, {"parity": "full", "normalization": "norm",
                                             "path_normalization": "element"}),
}
SHARED = {"c3_v2_m2_full": True, "c4_v1_m4_canonical": False, "c3_v1_m6_full_in2canonical": False,
          "c2_v3_m3_canonical_in2full_m2_path": False, "c2_v2_m1_full_norm_element": True}


def _token(key):
    if key[0] == "scalar":
        return "0e" if key[1] == 1 else "0o"
    return str(key[1])


@pytest.mark.parametrize("name", sorted(PLAN_ARGS))
def test_module_plan_matches_reference_tables(name):
    from ictc_o2_hp import ReferenceUvuTensorProduct
    c, v, m, kw = PLAN_ARGS[name]
    table = TABLES[name]
    module = ReferenceUvuTensorProduct(c, v, m, **kw)
    assert [list(p) for p in module.paths] == table["paths"]
    assert [[_token(e.key), e.copy, e.offset, e.dim] for e in module.entries_in1] == \
        table["entries_in1"]
    assert [[_token(e.key), e.copy, e.offset, e.dim] for e in module.entries_in2] == \
        table["entries_in2"]
    assert module.input1_dimension == table["input1_dimension"]
    assert module.input2_dimension == table["input2_dimension"]
    assert module.weight_numel == table["weight_numel"]
    np.testing.assert_allclose(np.array(module._coefficient_values),
                               np.array(table["coefficients"]), rtol=0, atol=1e-14)


@pytest.mark.parametrize("name", sorted(PLAN_ARGS))
def test_oracle_plan_matches_reference_tables(name):
    c, v, m, kw = PLAN_ARGS[name]
    table = TABLES[name]
    plan = U.UvuOraclePlan(c, v, m, **kw)
    assert [list(p) for p in plan.paths] == table["paths"]
    assert plan.width1 == table["input1_dimension"] and plan.width2 == table["input2_dimension"]
    assert plan.weight_numel == table["weight_numel"]
    np.testing.assert_allclose(plan.padded().reshape(-1, 8), np.array(table["coefficients"]),
                               rtol=0, atol=1e-14)


@pytest.mark.parametrize("name", sorted(SHARED))
def test_oracle_matches_reference_vectors(name, golden_uvu):
    c, v, m, kw = PLAN_ARGS[name]
    plan = U.UvuOraclePlan(c, v, m, **kw)
    x, y, w, g = (golden_uvu[f"{name}/{k}"] for k in ("x", "y", "w", "g"))
    out = U.forward(plan, x, y, w, SHARED[name])
    dx, dy, dw = U.backward(plan, x, y, w, g, SHARED[name])
    for key, value in (("out", out), ("dx", dx), ("dy", dy), ("dw", dw)):
        np.testing.assert_allclose(value, golden_uvu[f"{name}/{key}"], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("name", sorted(SHARED))
def test_reference_module_matches_reference_vectors(name, golden_uvu):
    from ictc_o2_hp import ReferenceUvuTensorProduct, UvuTensorProduct
    c, v, m, kw = PLAN_ARGS[name]
    for cls in (ReferenceUvuTensorProduct, UvuTensorProduct):
        module = cls(c, v, m, shared_weights=SHARED[name], internal_weights=False, **kw).double()
        x, y, w = (torch.from_numpy(golden_uvu[f"{name}/{k}"]).requires_grad_()
                   for k in ("x", "y", "w"))
        out = module(x, y, w)
        grads = torch.autograd.grad(out, (x, y, w), torch.from_numpy(golden_uvu[f"{name}/g"]))
        for key, value in zip(("out", "dx", "dy", "dw"), (out.detach(), *grads)):
            np.testing.assert_allclose(value.numpy(), golden_uvu[f"{name}/{key}"], rtol=1e-12,
                                       atol=1e-12)


def _random(plan, n, shared, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, plan.width1))
    y = rng.standard_normal((n, plan.width2))
    w = rng.standard_normal((plan.weight_numel,) if shared else (n, plan.weight_numel))
    g = rng.standard_normal((n, plan.width1))
    return x, y, w, g


@pytest.mark.parametrize("shared", [True, False])
def test_oracle_backward_finite_differences(shared):
    plan = U.UvuOraclePlan(2, 2, 2, parity="full", path_normalization="path")
    x, y, w, g = _random(plan, 3, shared, 11)
    dx, dy, dw = U.backward(plan, x, y, w, g, shared)
    eps = 1e-6

    def loss(xx, yy, ww):
        return float(np.sum(U.forward(plan, xx, yy, ww, shared) * g))

    for arr, grad, which in ((x, dx, 0), (y, dy, 1), (w, dw, 2)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            args = [x.copy(), y.copy(), w.copy()]
            args[which][idx] += eps
            up = loss(*args)
            args[which][idx] -= 2 * eps
            num[idx] = (up - loss(*args)) / (2 * eps)
        np.testing.assert_allclose(grad, num, rtol=1e-6, atol=1e-7)


def test_oracle_adjoint_identity():
    """<g, f(x, y, w)> = <dx, x> = <dy, y> = <dw, w>: f is linear in each argument."""
    plan = U.UvuOraclePlan(5, 3, 3, parity="canonical", parity_in2="full")
    x, y, w, g = _random(plan, 7, False, 12)
    dx, dy, dw = U.backward(plan, x, y, w, g, False)
    value = np.sum(U.forward(plan, x, y, w, False) * g)
    for a, b in ((dx, x), (dy, y), (dw, w)):
        assert abs(np.sum(a * b) - value) <= 1e-10 * max(1.0, abs(value))


def test_oracle_shared_equals_broadcast_per_row():
    plan = U.UvuOraclePlan(4, 2, 2, parity="full")
    x, y, w, g = _random(plan, 6, True, 13)
    rows = np.broadcast_to(w, (6, w.size)).copy()
    np.testing.assert_allclose(U.forward(plan, x, y, w, True), U.forward(plan, x, y, rows, False))
    shared = U.backward(plan, x, y, w, g, True)
    per_row = U.backward(plan, x, y, rows, g, False)
    np.testing.assert_allclose(shared[0], per_row[0])
    np.testing.assert_allclose(shared[1], per_row[1])
    np.testing.assert_allclose(shared[2], per_row[2].sum(axis=0))


def test_planted_mistakes_fail_the_pins(golden_uvu, monkeypatch):
    """A wrong copy basis or a dropped path normalisation must fail the golden vectors."""
    name = "c2_v3_m3_canonical_in2full_m2_path"
    c, v, m, kw = PLAN_ARGS[name]
    x, y, w = (golden_uvu[f"{name}/{k}"] for k in ("x", "y", "w"))
    expected = golden_uvu[f"{name}/out"]
    monkeypatch.setattr(U, "_J", np.array([[0.0, 1.0], [-1.0, 0.0]]))
    wrong = U.forward(U.UvuOraclePlan(c, v, m, **kw), x, y, w, False)
    assert normalized_error(expected, wrong) > 1e-3
    monkeypatch.undo()
    unscaled = dict(kw, path_normalization="none")
    wrong = U.forward(U.UvuOraclePlan(c, v, m, **unscaled), x, y, w, False)
    assert normalized_error(expected, wrong) > 1e-3


def test_radial_oracle_chain_rule():
    plan = U.UvuOraclePlan(3, 1, 2, parity="canonical")
    rng = np.random.default_rng(14)
    n, h = 4, 5
    x = rng.standard_normal((n, plan.width1))
    y = rng.standard_normal((n, plan.width2))
    hidden = rng.standard_normal((n, h))
    alpha = rng.standard_normal((plan.weight_numel, h))
    bias = rng.standard_normal(plan.weight_numel)
    g = rng.standard_normal((n, plan.width1))
    dx, dy, dh, da, db = U.radial_backward(plan, x, y, hidden, alpha, bias, g)
    eps = 1e-6

    def loss(hh, aa, bb):
        return float(np.sum(U.radial_forward(plan, x, y, hh, aa, bb) * g))

    for arr, grad, which in ((hidden, dh, 0), (alpha, da, 1), (bias, db, 2)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            args = [hidden.copy(), alpha.copy(), bias.copy()]
            args[which][idx] += eps
            up = loss(*args)
            args[which][idx] -= 2 * eps
            num[idx] = (up - loss(*args)) / (2 * eps)
        np.testing.assert_allclose(grad, num, rtol=1e-6, atol=1e-7)
    assert U.radial_backward(plan, x, y, hidden, alpha, None, g)[4] is None


def test_kernel_metadata_ranges():
    from ictc_o2_hp.uvu_o2 import ReferenceUvuTensorProduct, kernel_metadata
    module = ReferenceUvuTensorProduct(3, 2, 3, parity="full", parity_in2="canonical")
    info, order1, order2 = kernel_metadata(module.entries_in1, module.entries_in2, module.paths,
                                           3, 2)
    p, nx, ny = len(module.paths), len(module.entries_in1), len(module.entries_in2)
    assert info.shape == (p + 2 * nx + ny, 7) and info.dtype == np.int32
    assert sorted(order1) == list(range(p)) and sorted(order2) == list(range(p))
    for base, order, role in ((p, list(range(p)), 2), (p + nx, order1, 0),
                              (p + 2 * nx, order2, 1)):
        count = ny if role == 1 else nx
        covered = []
        for index in range(count):
            begin, end = info[base + index, 2:4]
            covered += [order[q] for q in range(begin, end)]
            assert all(module.paths[order[q]][role] == index for q in range(begin, end))
        assert sorted(covered) == list(range(p))
    for q, (i, j, k) in enumerate(module.paths):
        assert info[q, 6] == q * 3 * 2
        assert info[q, 0] == module.entries_in1[i].offset
        assert info[q, 1] == module.entries_in2[j].offset
        assert info[q, 2] == module.entries_in1[k].offset


def test_module_validation_and_weights():
    from ictc_o2_hp import UvuTensorProduct
    with pytest.raises(ValueError):
        UvuTensorProduct(0, 1, 2)
    with pytest.raises(ValueError):
        UvuTensorProduct(4, 1, 2, parity="odd")
    with pytest.raises(ValueError):
        UvuTensorProduct(4, 1, 2, normalization="none")
    with pytest.raises(ValueError):
        UvuTensorProduct(4, 1, 2, path_normalization="all")
    with pytest.raises(ValueError):
        UvuTensorProduct(4, 1, 2, shared_weights=False, internal_weights=True)
    module = UvuTensorProduct(4, 2, 2)
    assert module.weight.shape == (module.weight_numel,)
    assert module.parameter_count == module.weight_numel
    assert list(module.state_dict()) == ["weight"]
    x = torch.randn(3, module.input1_dimension)
    y = torch.randn(3, module.input2_dimension)
    with pytest.raises(ValueError):
        module(x[:, :-1], y)
    with pytest.raises(ValueError):
        module(x, y[:2])
    with pytest.raises(ValueError):
        module(x, y, torch.randn(module.weight_numel + 1))
    assert module.weight_view_for_path(1).shape == (4, 2)
    with pytest.raises(IndexError):
        module.weight_view_for_path(len(module.paths))
    external = UvuTensorProduct(4, 2, 2, shared_weights=False)
    assert external.parameter_count == 0
    with pytest.raises(ValueError):
        external(x, y)
    batched = external(x.reshape(3, 1, -1), y.reshape(3, 1, -1),
                       torch.randn(3, 1, external.weight_numel))
    assert batched.shape == (3, 1, module.input1_dimension)


def test_double_cast_restores_exact_coefficients():
    from ictc_o2_hp import UvuTensorProduct
    module = UvuTensorProduct(2, 1, 3, path_normalization="path")
    exact = torch.tensor(module._coefficient_values, dtype=torch.float64).reshape(-1, 2, 2, 2)
    module.half().double()
    assert torch.equal(module._coefficients, exact)
