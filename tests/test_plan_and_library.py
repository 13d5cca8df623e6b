"""Host-side plan, compiled tables and the C ABI surface (no GPU needed)."""
from __future__ import annotations

import ctypes
import json
import re
import subprocess
import sys

import numpy as np
import pytest

from conftest import GOLDEN, REPO
from oracle import o2_oracle as O


@pytest.fixture(scope="session")
def lib():
    """The in-tree library, built first if this checkout has none yet."""
    from ictc_o2_hp import _native
    if not _native.LIBRARY_PATH.exists():
        subprocess.run([sys.executable, str(REPO / "ictc-o2-hp_amd" / "build_native.py")],
                       check=True)
    return _native.library()


def test_plan_matches_reference_tables():
    from ictc_o2_hp.plan import TPPlan
    tables = json.loads((GOLDEN / "cg_tables.json").read_text())
    for key, table in tables.items():
        m, parity, norm = key.split("/")
        plan = TPPlan(1, int(m), parity, norm)
        assert [list(o) for o in plan.weight_offsets] == table["weight_offsets"], key
        assert plan.width == table["width"], key
        for path, ref in zip(plan.table, table["terms"]):
            mine = [(t.i, t.j, t.k) for t in path.terms]
            theirs = [(i, j, k) for k, comp in enumerate(ref) for i, j, _ in comp]
            assert mine == theirs, key
            coef = [t.coefficient for t in path.terms]
            ref_coef = [c for comp in ref for _, _, c in comp]
            assert np.allclose(coef, ref_coef, rtol=0, atol=1e-14), key


def test_plan_agrees_with_oracle_for_many_channels():
    from ictc_o2_hp.plan import TPPlan
    for c, m, parity in ((17, 3, "full"), (128, 6, "full"), (5, 4, "canonical"), (2, 0, "full")):
        plan, oracle = TPPlan(c, m, parity), O.OraclePlan(c, m, parity)
        assert plan.width == oracle.width
        assert plan.weight_numel == oracle.weight_numel
        assert list(plan.weight_offsets) == [tuple(s) for s in oracle.weight_slices]
        for cg, ref in zip(plan.cg, oracle.cgs):
            assert np.abs(cg - ref).max() < 1e-14


def test_kernel_table_magnitudes_are_uniform():
    from ictc_o2_hp.plan import kernel_table
    for m in range(0, 9):
        for parity in ("canonical", "full"):
            for norm in ("component", "norm"):
                _, paths = kernel_table(m, parity, norm)
                mags = {round(p[4], 12) for p in paths}
                expected = {1.0, round(2 ** -0.5, 12)} if norm == "component" else \
                    {1.0, round(2 ** -0.5, 12), 0.5}
                assert mags <= expected, (m, parity, norm, mags)


def test_element_offsets_match_layout_rules():
    """triton_o2.py:110-121 addressing for layouts 0, 1, 2."""
    from ictc_o2_hp.plan import TPPlan
    plan = TPPlan(3, 2, "full")
    oracle = O.OraclePlan(3, 2, "full")
    index = np.arange(plan.width, dtype=float)[None, :]
    for layout in (0, 2):
        blocks = oracle.unpack(index, layout)
        for k, block in enumerate(plan.blocks):
            for ch in range(block.multiplicity):
                for comp in range(block.irrep_dimension):
                    assert plan.element_offset(k, ch, comp, layout) == blocks[k][0, ch, comp]


def test_compiled_tables_equal_host_plan(lib):
    from ictc_o2_hp import _native
    from ictc_o2_hp.plan import kernel_table
    for m in range(0, 7):
        for parity in ("canonical", "full"):
            for norm in ("component", "norm"):
                keys, paths = kernel_table(m, parity, norm)
                cpaths, mags, terms = _native.compiled_table(m, parity, norm)
                assert len(cpaths) == len(paths)
                cursor = 0
                for row, mag, path in zip(cpaths, mags, paths):
                    k1, k2, k3, wstart, magnitude, pterms = path
                    assert tuple(row[:4]) == (k1, k2, k3, wstart)
                    assert row[4] == cursor and row[5] == len(pterms)
                    assert row[6] == keys[k3][1]
                    assert mag == np.float32(magnitude)
                    assert [tuple(t) for t in terms[cursor:cursor + len(pterms)]] == list(pterms)
                    cursor += len(pterms)


def test_library_exports_every_declared_symbol(lib):
    header = (REPO / "include" / "ictc_o2_hp_amd.h").read_text()
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(o2mi_\w+)\s*\(", header, re.M)
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name


def test_plan_create_validates_arguments(lib):
    from ictc_o2_hp import _native
    handle = ctypes.c_void_p()
    assert lib.o2mi_tp_plan_create(0, 2, 0, 0, 0, ctypes.byref(handle)) == -1
    assert lib.o2mi_tp_plan_create(8, -1, 0, 0, 0, ctypes.byref(handle)) == -1
    assert lib.o2mi_tp_plan_create(8, 2, 3, 0, 0, ctypes.byref(handle)) == -1
    assert lib.o2mi_tp_plan_create(8, 2, 1, 0, 1, ctypes.byref(handle)) == -1   # layout/parity
    assert lib.o2mi_tp_plan_create(8, 99, 1, 0, 0, ctypes.byref(handle)) == -2  # beyond the limit
    assert b"table-driven" in lib.o2mi_last_error()
    plan = _native.TPNativePlan(128, 6, "full", "component", 0)
    assert (plan.width, plan.weight_numel) == (3328, 19712)
    plan = _native.TPNativePlan(5, 4, "canonical", "norm", 1)
    assert (plan.width, plan.weight_numel) == (45, 155)


def test_tp_ops_refuse_mismatched_shapes_before_launch(lib):
    """o2_forward / o2_backward check every operand's shape against the plan
    (x, y, cotangent [N, W]; weight P_w) before any device work."""
    import torch
    from ictc_o2_hp import TensorProduct, ops
    tp = TensorProduct(4, 2, parity="full")
    w = tp.weight.detach()
    x = torch.zeros(3, tp.representation_dimension)
    meta = (tp._weight_path_info, tp._weight_path_coefficients, tp._metadata_id)
    bad = [
        (x, x[:2], w, x),                      # right rows differ
        (x, x, w[:-1], x),                     # weight too short
        (x, x, w, x[:, :-1]),                  # cotangent width
        (x[:, :-1], x[:, :-1], w, x[:, :-1]),  # width not the plan's
    ]
    for left, right, weight, grad in bad:
        with pytest.raises(ValueError, match="shapes do not match"):
            ops.o2_backward(left, right, weight, grad, *meta)
    with pytest.raises(ValueError, match="shapes do not match"):
        ops.o2_forward(x, x[:2], w, *meta)
    with pytest.raises(ValueError, match="shapes do not match"):
        ops.o2_forward(x, x, w[:-1], *meta)


def test_plans_beyond_compiled_orders_are_table_driven(lib):
    """Plans beyond the compiled orders (m_max >= 9) are created table-driven
    (width and P_w from the selection rules, equal to the host plan); the key
    limit is 48."""
    from ictc_o2_hp import _native
    from ictc_o2_hp.plan import TPPlan
    for c, m, parity in ((16, 7, "full"), (5, 8, "canonical"), (3, 10, "full"),
                         (4, 9, "canonical"), (2, 46, "full"), (2, 47, "canonical"),
                         (32, 6, "full")):
        native = _native.TPNativePlan(c, m, parity, "component", 0)
        host = TPPlan(c, m, parity)
        assert (native.width, native.weight_numel) == (host.width, host.weight_numel)
        assert native.compiled == (m <= 8)
    for m, parity in ((47, 1), (48, 0)):
        handle = ctypes.c_void_p()
        assert lib.o2mi_tp_plan_create(2, m, parity, 0, 0, ctypes.byref(handle)) == -2
