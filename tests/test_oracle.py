"""Pins the CPU oracle (oracle/o2_oracle.py) before it is trusted as the checker.

Each oracle function is checked against something independent of its own
formula: the reference's recorded tables and vectors (tests/golden/), the
reference's recorded structural counts, finite differences, the bilinear
adjoint identity and O(2) equivariance.  ``test_planted_*`` plant plausible
mistakes in the oracle (on the CPU) and show that a check above catches them.
"""
from __future__ import annotations

import json
import math

import numpy as np
import pytest

from oracle import o2_oracle as O
from oracle.cpu_port import CPUPort

from conftest import GOLDEN


def _tables():
    return json.loads((GOLDEN / "cg_tables.json").read_text())


def _cg_mismatches(tables) -> int:
    bad = 0
    for key, table in tables.items():
        m, parity, norm = key.split("/")
        plan = O.OraclePlan(1, int(m), parity, norm)
        tokens = [[("0e" if k == ("scalar", 1) else "0o" if k == ("scalar", -1) else str(k[1]))
                   for k in path] for path in plan.paths]
        assert tokens == table["paths"], key
        assert [list(s) for s in plan.weight_slices] == table["weight_offsets"], key
        for cg, ref in zip(plan.cgs, table["terms"]):
            dense = np.zeros_like(cg)
            for k, comp in enumerate(ref):
                for i, j, c in comp:
                    dense[i, j, k] = c
            bad += int(np.abs(dense - cg).max() > 1e-13)
    return bad


def test_coupling_closed_form_matches_reference_tables():
    """All 36 (m_max 0..8, parity, normalization) path lists, weight offsets and
    coupling tables recorded from the reference's fast_o2 sparse extraction."""
    assert _cg_mismatches(_tables()) == 0


def test_planted_basis_sign_mistake_is_caught(monkeypatch):
    """A plausible convention slip (plain +cos/+sin harmonics for every m)."""
    monkeypatch.setattr(O, "_basis_sign", lambda m: 1.0)
    assert _cg_mismatches(_tables()) > 0


def test_planted_odd_scalar_orientation_is_caught(monkeypatch):
    """J versus J^T for the odd scalar (o2_math.py:310-333)."""
    original = O.raw_coupling

    def flipped(k1, k2, k3):
        c = original(k1, k2, k3)
        if (k1 == ("scalar", -1)) != (k2 == ("scalar", -1)) and k3[0] == "freq":
            c = -c
        return c

    monkeypatch.setattr(O, "raw_coupling", flipped)
    assert _cg_mismatches(_tables()) > 0


def test_structure_matches_recorded_qualification_families():
    """(paths, parameters, width) of the reference's 60 recorded families."""
    records = json.loads((GOLDEN / "qualification_structure.json").read_text())
    assert len(records) == 60
    for r in records:
        plan = O.OraclePlan(r["C"], r["m_max"], r["parity"])
        assert (len(plan.paths), plan.weight_numel, plan.width) == \
            (r["paths"], r["parameters"], r["width"]), r["source"]


def _cases(golden):
    return sorted({k.split("/")[0] for k in golden.files})


def _plan_of(name):
    c, m, parity, norm = name.split("_")
    return O.OraclePlan(int(c[1:]), int(m[1:]), parity, norm)


def test_forward_and_vjp_match_reference_vectors(golden_tp):
    """The reference's einsum algebra run in fp64 on stored inputs."""
    for name in _cases(golden_tp):
        plan = _plan_of(name)
        x, y, g, w = (golden_tp[f"{name}/{k}"] for k in ("x", "y", "g", "weight"))
        got = [O.forward(plan, x, y, w), *O.backward(plan, x, y, w, g)]
        for key, value in zip(("out", "dx", "dy", "dw"), got):
            assert O.normalized_error(golden_tp[f"{name}/{key}"], value) < 1e-13, (name, key)


def test_planted_routing_mistake_is_caught(golden_tp, monkeypatch):
    """Routing scalar outputs to copy 1 instead of copy 0 of frequency inputs."""
    def routing(self, path):
        k1, k2, k3 = self.path_index[path]
        o = np.arange(self.blocks[k3].mul)
        m1, m2 = self.blocks[k1].mul, self.blocks[k2].mul
        r1 = (o + (m1 - self.blocks[k3].mul if m1 > self.blocks[k3].mul else 0)) % m1
        r2 = (o + (m2 - self.blocks[k3].mul if m2 > self.blocks[k3].mul else 0)) % m2
        return r1, r2

    monkeypatch.setattr(O.OraclePlan, "routing", routing)
    name = "c17_m3_full_component"
    plan = _plan_of(name)
    x, y, w = (golden_tp[f"{name}/{k}"] for k in ("x", "y", "weight"))
    assert O.normalized_error(golden_tp[f"{name}/out"], O.forward(plan, x, y, w)) > 1e-3


@pytest.mark.parametrize("channels,m_max,parity,norm", [(2, 2, "full", "component"),
                                                        (3, 3, "canonical", "norm"),
                                                        (1, 4, "full", "norm")])
def test_vjp_finite_differences(channels, m_max, parity, norm):
    plan = O.OraclePlan(channels, m_max, parity, norm)
    rng = np.random.default_rng(channels * 10 + m_max)
    x, y, g = (rng.standard_normal((3, plan.width)) for _ in range(3))
    w = rng.standard_normal(plan.weight_numel)
    dx, dy, dw = O.backward(plan, x, y, w, g)

    def loss(a, b, c):
        return float((O.forward(plan, a, b, c) * g).sum())

    eps = 1e-6
    for grad, which in ((dx, 0), (dy, 1), (dw, 2)):
        direction = rng.standard_normal(grad.shape)
        args_p = [x, y, w]
        args_m = [x, y, w]
        args_p[which] = args_p[which] + eps * direction
        args_m[which] = args_m[which] - eps * direction
        numeric = (loss(*args_p) - loss(*args_m)) / (2 * eps)
        assert math.isclose(numeric, float((grad * direction).sum()), rel_tol=1e-6, abs_tol=1e-8)


def test_bilinear_adjoint_identity():
    """out is linear in each of x, y, w: <f(dx_dir, y, w), g> = <dx_dir, dx>."""
    plan = O.OraclePlan(5, 5, "full")
    rng = np.random.default_rng(3)
    x, y, g, u = (rng.standard_normal((7, plan.width)) for _ in range(4))
    w, v = rng.standard_normal(plan.weight_numel), rng.standard_normal(plan.weight_numel)
    dx, dy, dw = O.backward(plan, x, y, w, g)
    assert math.isclose((O.forward(plan, u, y, w) * g).sum(), (u * dx).sum(), rel_tol=1e-12)
    assert math.isclose((O.forward(plan, x, u, w) * g).sum(), (u * dy).sum(), rel_tol=1e-12)
    assert math.isclose((O.forward(plan, x, y, v) * g).sum(), (v * dw).sum(), rel_tol=1e-12)


def _act(plan, flat, theta, reflect):
    """O(2) action in the public copy bases (native_o2.py:224-247, o2_math.py:187-216)."""
    det = -1.0 if reflect else 1.0
    blocks = plan.unpack(flat)
    out = []
    for b, v in zip(plan.blocks, blocks):
        if b.key[0] == "scalar":
            out.append(v * (1.0 if b.key[1] == 1 else det))
            continue
        m = b.key[1]
        c, s = math.cos(m * theta), math.sin(m * theta)
        r = np.array([[c, -det * s], [s, det * c]])
        v = v.copy()
        v[:, :plan.C] = v[:, :plan.C] @ r.T
        if plan.full:
            v[:, plan.C:] = v[:, plan.C:] @ (det * r).T
        out.append(v)
    return plan.pack(out)


@pytest.mark.parametrize("parity", ["canonical", "full"])
@pytest.mark.parametrize("reflect", [False, True])
def test_forward_is_o2_equivariant(parity, reflect):
    plan = O.OraclePlan(3, 4, parity)
    rng = np.random.default_rng(11)
    x, y = rng.standard_normal((5, plan.width)), rng.standard_normal((5, plan.width))
    w = rng.standard_normal(plan.weight_numel)
    theta = 0.7316
    lhs = O.forward(plan, _act(plan, x, theta, reflect), _act(plan, y, theta, reflect), w)
    rhs = _act(plan, O.forward(plan, x, y, w), theta, reflect)
    assert np.abs(lhs - rhs).max() < 1e-12


@pytest.mark.parametrize("parity,layout", [("canonical", 1), ("full", 2)])
def test_component_major_layout_is_a_permutation(parity, layout):
    plan = O.OraclePlan(4, 3, parity)
    rng = np.random.default_rng(5)
    x, y = rng.standard_normal((6, plan.width)), rng.standard_normal((6, plan.width))
    w = rng.standard_normal(plan.weight_numel)
    to_layout = lambda a: plan.pack(plan.unpack(a, 0), layout)
    assert np.array_equal(plan.pack(plan.unpack(to_layout(x), layout), 0), x)
    out = O.forward(plan, to_layout(x), to_layout(y), w, layout)
    assert np.allclose(out, to_layout(O.forward(plan, x, y, w)), rtol=0, atol=1e-13)


def test_cpu_port_matches_reference_vectors(golden_tp):
    for name in _cases(golden_tp):
        c, m, parity, norm = name.split("_")
        port = CPUPort(int(c[1:]), int(m[1:]), parity, norm)
        got = port.forward_vjp(*(golden_tp[f"{name}/{k}"] for k in ("x", "y", "weight", "g")))
        for key, value in zip(("out", "dx", "dy", "dw"), got):
            assert O.normalized_error(golden_tp[f"{name}/{key}"], value.double().numpy()) < 1e-6


def test_normalized_error_metric():
    """max|ref - act| / max(1e-7, max|ref|, max|act|) (support.py:33-35)."""
    assert O.normalized_error(np.array([2.0, -4.0]), np.array([2.0, -3.0])) == 0.25
    assert O.normalized_error(np.zeros(3), np.zeros(3)) == 0.0
    assert O.normalized_error(np.array([0.0]), np.array([1e-8])) == pytest.approx(0.1)
