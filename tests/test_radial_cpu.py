"""CPU checks of RadialUvuTensorProduct: construction contract, the composed
path against the radial oracle, and the fused-structure table."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import uvu_oracle as U
from oracle.o2_oracle import normalized_error


def _modules(c=4, m=2, parity="canonical", parity_in2=None, hidden=8, bias=True, **kw):
    from ictc_o2_hp import RadialUvuTensorProduct, UvuTensorProduct
    tp = UvuTensorProduct(c, 1, m, parity=parity, parity_in2=parity_in2, shared_weights=False,
                          **kw)
    linear = torch.nn.Linear(hidden, tp.weight_numel, bias=bias)
    return tp, linear, RadialUvuTensorProduct(tp, linear)


def test_constructor_contract():
    from ictc_o2_hp import RadialUvuTensorProduct, UvuTensorProduct
    tp = UvuTensorProduct(4, 1, 2, shared_weights=False)
    with pytest.raises(TypeError):
        RadialUvuTensorProduct(torch.nn.Linear(2, 2), torch.nn.Linear(2, tp.weight_numel))
    with pytest.raises(ValueError):
        RadialUvuTensorProduct(UvuTensorProduct(4, 2, 2, shared_weights=False),
                               torch.nn.Linear(3, 4 * 2 * 10))
    with pytest.raises(ValueError):
        RadialUvuTensorProduct(UvuTensorProduct(4, 1, 2), torch.nn.Linear(3, tp.weight_numel))
    with pytest.raises(TypeError):
        RadialUvuTensorProduct(tp, torch.nn.Sequential(torch.nn.Linear(3, tp.weight_numel)))
    with pytest.raises(ValueError):
        RadialUvuTensorProduct(tp, torch.nn.Linear(3, tp.weight_numel + 1))
    module = RadialUvuTensorProduct(tp, torch.nn.Linear(3, tp.weight_numel))
    # External-weight TPs keep an empty persistent "weight" buffer (uvu_o2.py:156).
    assert sorted(module.state_dict()) == ["radial_out.bias", "radial_out.weight", "tp.weight"]
    assert module.tp is tp


def test_forward_validation():
    tp, linear, module = _modules()
    x = torch.randn(5, tp.input1_dimension)
    y = torch.randn(5, tp.input2_dimension)
    h = torch.randn(5, 8)
    with pytest.raises(ValueError):
        module(x[:, :-1], y, h)
    with pytest.raises(ValueError):
        module(x, y[:4], h)
    with pytest.raises(ValueError):
        module(x, y, h[:, :-1])
    with pytest.raises(TypeError):
        module(x.long(), y.long(), h.long())
    with pytest.raises(ValueError):
        module(x.double(), y, h)


@pytest.mark.parametrize("bias", [True, False])
def test_composed_path_matches_oracle(bias):
    tp, linear, module = _modules(c=3, m=3, parity="full", parity_in2="canonical", hidden=5,
                                  bias=bias, path_normalization="path")
    module = module.double()
    plan = U.UvuOraclePlan(3, 1, 3, parity="full", parity_in2="canonical",
                           path_normalization="path")
    rng = np.random.default_rng(3)
    x = rng.standard_normal((7, plan.width1))
    y = rng.standard_normal((7, plan.width2))
    h = rng.standard_normal((7, 5))
    g = rng.standard_normal((7, plan.width1))
    xt, yt, ht = (torch.from_numpy(a).requires_grad_() for a in (x, y, h))
    out = module(xt, yt, ht)
    params = [linear.weight] + ([linear.bias] if bias else [])
    grads = torch.autograd.grad(out, [xt, yt, ht, *params], torch.from_numpy(g))
    alpha = linear.weight.detach().numpy()
    b = linear.bias.detach().numpy() if bias else None
    ref_out = U.radial_forward(plan, x, y, h, alpha, b)
    ref = U.radial_backward(plan, x, y, h, alpha, b, g)
    assert normalized_error(ref_out, out.detach().numpy()) <= 1e-12
    for r, a in zip([v for v in ref if v is not None], grads):
        assert normalized_error(r, a.numpy()) <= 1e-12


def test_batch_shapes_on_cpu():
    tp, linear, module = _modules()
    x = torch.randn(2, 3, tp.input1_dimension)
    y = torch.randn(2, 3, tp.input2_dimension)
    h = torch.randn(2, 3, 8)
    out = module(x, y, h)
    assert out.shape == x.shape
    flat = module(x.reshape(6, -1), y.reshape(6, -1), h.reshape(6, -1))
    assert torch.allclose(out.reshape(6, -1), flat)


def test_fused_structure_table():
    """Every m_max <= 6 structure with equal angular orders has fused kernels;
    the generated traversal orders are permutations grouped as the kernels
    assume, and the double-buffered alpha chunks fit in LDS."""
    import build_native
    from ictc_o2_hp.uvu_o2 import ReferenceUvuTensorProduct
    names = {build_native._radial_name(*s) for s in build_native.RADIAL_STRUCTURES}
    assert "R4c4c" in names                      # configs[4]: C64, m4, canonical
    assert "R6f6c" in names                      # the reference's radial benchmark
    assert len(names) == 28
    for m, parity, m2, parity2 in build_native.RADIAL_STRUCTURES:
        tp = ReferenceUvuTensorProduct(16, 1, m, parity=parity, m_max_in2=m2,
                                       parity_in2=parity2, shared_weights=False)
        lds = 4 * (8 * len(tp.paths) + 2 * build_native.RADIAL_CHUNK * 16 * (1 + 68))
        assert lds <= 160 * 1024


def test_generated_orders_group_paths(tmp_path):
    """fwd groups paths by output entry and bwd by first-input entry (each group
    contiguous, so one entry of accumulators is live); wgt is a permutation."""
    import re
    import build_native
    build_native.generate_radial(tmp_path)
    text = (tmp_path / "o2mi_radial_plans.h").read_text()
    text = text[text.index("struct R6f6c {"):]
    text = text[:text.index("\n};\n")]
    paths = [tuple(map(int, t)) for t in
             re.findall(r"\{(\d+), (\d+), (\d+), \d+, \d+\}", text.split("paths[kPaths] = ")[1]
                        .split(";")[0])]
    orders = {k: list(map(int, re.search(k + r"\[kPaths\] = \{([^}]*)\}", text)
                          .group(1).split(", "))) for k in ("fwd", "bwd", "wgt")}
    assert len(paths) == 254
    for key, role in (("fwd", 2), ("bwd", 0), ("wgt", 1)):
        order = orders[key]
        assert sorted(order) == list(range(254))
        keys = [paths[p][role] for p in order]
        seen, last = set(), None
        for k in keys:                            # contiguous groups
            assert k == last or k not in seen
            seen.add(k)
            last = k


def test_library_exports_radial_symbols():
    from ictc_o2_hp import _native
    try:
        lib = _native.library()
    except _native.NativeLibraryError:
        pytest.skip("library not built")
    for name in ("o2mi_radial_plan_create", "o2mi_radial_plan_destroy", "o2mi_radial_paths",
                 "o2mi_radial_forward_f32", "o2mi_radial_backward_workspace_bytes",
                 "o2mi_radial_backward_f32"):
        assert hasattr(lib, name)


def test_radial_plan_create_validation():
    import ctypes
    from ictc_o2_hp import _native
    try:
        lib = _native.library()
    except _native.NativeLibraryError:
        pytest.skip("library not built")
    handle = ctypes.c_void_p()
    assert lib.o2mi_radial_plan_create(64, 4, 0, 4, 0, 64, ctypes.byref(handle)) == 0
    assert lib.o2mi_radial_paths(handle) == 31
    assert lib.o2mi_radial_plan_destroy(handle) == 0
    assert lib.o2mi_radial_plan_create(24, 4, 0, 4, 0, 64, ctypes.byref(handle)) == -2
    assert lib.o2mi_radial_plan_create(64, 4, 0, 4, 0, 66, ctypes.byref(handle)) == -2
    assert lib.o2mi_radial_plan_create(64, 4, 0, 4, 0, 128, ctypes.byref(handle)) == -2
    # m_max 6, full / canonical: 254 paths, streamed kernels.
    assert lib.o2mi_radial_plan_create(64, 6, 1, 6, 0, 64, ctypes.byref(handle)) == 0
    assert lib.o2mi_radial_paths(handle) == 254
    assert lib.o2mi_radial_plan_destroy(handle) == 0
    assert lib.o2mi_radial_plan_create(64, 6, 1, 6, 1, 64, ctypes.byref(handle)) == 0
    assert lib.o2mi_radial_paths(handle) == 508
    assert lib.o2mi_radial_plan_destroy(handle) == 0
    assert lib.o2mi_radial_plan_create(64, 7, 0, 7, 0, 64, ctypes.byref(handle)) == -2
    assert lib.o2mi_radial_plan_create(0, 4, 0, 4, 0, 64, ctypes.byref(handle)) == -1
    assert lib.o2mi_radial_plan_create(64, 4, 2, 4, 0, 64, ctypes.byref(handle)) == -1
    assert lib.o2mi_radial_backward_workspace_bytes(None, 10, 31) == 0


def test_uvu_plan_create_validation():
    """Plans of the plan-specialised uvu kernels (shared weights 1 <= V <= 8,
    per-row weights V = 1) and the argument checks that precede any GPU call."""
    import ctypes
    from ictc_o2_hp import _native
    try:
        lib = _native.library()
    except _native.NativeLibraryError:
        pytest.skip("library not built")
    handle = ctypes.c_void_p()
    for v in (1, 2, 3, 8):
        assert lib.o2mi_uvu_shared_plan_create(64, v, 4, 0, 4, 0, ctypes.byref(handle)) == 0
        assert lib.o2mi_radial_paths(handle) == 31
        assert lib.o2mi_radial_plan_destroy(handle) == 0
    assert lib.o2mi_uvu_shared_plan_create(32, 4, 6, 1, 6, 1, ctypes.byref(handle)) == 0
    assert lib.o2mi_radial_paths(handle) == 508
    assert lib.o2mi_radial_plan_destroy(handle) == 0
    assert lib.o2mi_uvu_shared_plan_create(64, 9, 4, 0, 4, 0, ctypes.byref(handle)) == -2
    assert lib.o2mi_uvu_shared_plan_create(24, 1, 4, 0, 4, 0, ctypes.byref(handle)) == -2
    assert lib.o2mi_uvu_shared_plan_create(64, 2, 7, 0, 7, 0, ctypes.byref(handle)) == -2
    assert lib.o2mi_uvu_shared_plan_create(64, 0, 4, 0, 4, 0, ctypes.byref(handle)) == -1
    assert lib.o2mi_uvu_shared_plan_create(64, 1, 4, 3, 4, 0, ctypes.byref(handle)) == -1
    # Per-row weights need V = 1; zero rows are a no-op.
    v1, v2 = ctypes.c_void_p(), ctypes.c_void_p()
    assert lib.o2mi_uvu_shared_plan_create(64, 1, 4, 0, 4, 0, ctypes.byref(v1)) == 0
    assert lib.o2mi_uvu_shared_plan_create(64, 2, 4, 0, 4, 0, ctypes.byref(v2)) == 0
    assert lib.o2mi_uvu_rows_forward_f32(v2, None, None, None, None, None, 10, None) == -2
    assert lib.o2mi_uvu_rows_forward_f32(v1, None, None, None, None, None, 0, None) == 0
    assert lib.o2mi_uvu_rows_forward_f32(v1, None, None, None, None, None, 10, None) == -1
    assert lib.o2mi_uvu_rows_backward_f32(v1, None, None, None, None, None, None, None, None,
                                          None, 0, 10, 8, None) == -1
    assert lib.o2mi_uvu_rows_backward_f32(v2, None, None, None, None, None, None, None, None,
                                          None, 0, 10, 7, None) == -2
    for h in (v1, v2):
        assert lib.o2mi_radial_plan_destroy(h) == 0


def test_compiled_coupling_signs_hold_for_every_normalization(tmp_path):
    """The fused kernels compile each path's non-zero coupling slots (mask) and
    their signs (neg) and read one magnitude per path at run time.  For every
    fused structure and every normalization the module's couplings must have
    exactly those slots and signs, and one magnitude per path."""
    import re
    import build_native
    from ictc_o2_hp.uvu_o2 import UvuLayout, uvu_plan
    build_native.generate_radial(tmp_path)
    text = (tmp_path / "o2mi_radial_plans.h").read_text()
    for m, p1, m2, p2 in build_native.RADIAL_STRUCTURES:
        name = build_native._radial_name(m, p1, m2, p2)
        body = text[text.index(f"struct {name} {{"):]
        body = body[:body.index("\n};\n")]
        rows = [tuple(map(int, t)) for t in re.findall(
            r"\{(\d+), (\d+), (\d+), (\d+), (\d+)\}", body.split("paths[kPaths] = ")[1].split(";")[0])]
        first, second = UvuLayout.build(5, m, p1), UvuLayout.build(3, m2, p2)
        for norm in ("component", "norm"):
            for pnorm in ("none", "element", "path"):
                paths, coef = uvu_plan(first.entries, second.entries, norm, pnorm, 3)
                assert len(paths) == len(rows)
                for (i, j, k), cg, (ri, rj, rk, mask, neg) in zip(paths, coef, rows):
                    assert (i, j, k) == (ri, rj, rk)
                    flat = cg.reshape(-1)     # slot = out * 4 + in1 * 2 + in2
                    nz = np.abs(flat) > 1e-12
                    assert sum(1 << s for s in range(8) if nz[s]) == mask
                    assert sum(1 << s for s in range(8) if flat[s] < -1e-12) == neg
                    mags = np.abs(flat[nz])
                    assert np.allclose(mags, mags[0], rtol=1e-12)
