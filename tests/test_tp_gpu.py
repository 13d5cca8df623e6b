"""GPU parity of the HIP TensorProduct kernels against the fp64 oracle.

Bar (the reference's gate, benchmarks/eqx/scripts/support.py:33-35 and
validate_math.py:72-75): normalized max error <= 1e-5 for out, dx, dy and dw.
Large shapes compare a random subset of rows for out / dx / dy (rows are
independent) and obtain dw from a cotangent that is zero outside the subset,
so the oracle's dw over that subset is the exact expected value while the
kernels run with the full launch geometry.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import o2_oracle as O

TOL = 1e-5

pytestmark = pytest.mark.gpu


def _module(channels, m_max, parity, normalization="component", layout_cls=None, seed=0):
    from ictc_o2_hp import ComponentMajorTensorProduct, TensorProduct
    torch.manual_seed(seed)
    cls = layout_cls or TensorProduct
    return cls(channels, m_max, parity=parity, normalization=normalization).cuda()


def _run(module, x, y, g):
    xt = torch.from_numpy(x).float().cuda().requires_grad_()
    yt = torch.from_numpy(y).float().cuda().requires_grad_()
    out = module(xt, yt)
    dx, dy, dw = torch.autograd.grad(out, (xt, yt, module.weight),
                                     torch.from_numpy(g).float().cuda())
    torch.cuda.synchronize()
    return [t.detach().double().cpu().numpy() for t in (out, dx, dy, dw)]


def _check(plan, module, x, y, g, rows=None, layout=0):
    print(f"case C={plan.C} M={plan.M} {plan.parity} {plan.normalization} N={x.shape[0]} "
          f"layout={layout}", flush=True)
    w = module.weight.detach().double().cpu().numpy()
    if rows is not None:
        g = g.copy()
        mask = np.zeros(x.shape[0], bool)
        mask[rows] = True
        g[~mask] = 0.0
    out, dx, dy, dw = _run(module, x, y, g)
    sel = slice(None) if rows is None else rows
    ref_out = O.forward(plan, x[sel], y[sel], w, layout)
    ref_dx, ref_dy, ref_dw = O.backward(plan, x[sel], y[sel], w, g[sel], layout)
    errors = {
        "out": O.normalized_error(ref_out, out[sel]),
        "dx": O.normalized_error(ref_dx, dx[sel]),
        "dy": O.normalized_error(ref_dy, dy[sel]),
        "dw": O.normalized_error(ref_dw, dw),
    }
    assert all(np.isfinite(a).all() for a in (out, dx, dy, dw))
    assert max(errors.values()) <= TOL, errors
    return errors


CASES = [
    # C, M, parity, normalization, N
    (32, 2, "canonical", "component", 4096),   # configs[0] shape
    (17, 3, "full", "component", 37),          # odd C, odd N (reproduction_check.json)
    (32, 1, "canonical", "component", 37),
    (32, 6, "full", "component", 37),
    (4, 6, "full", "norm", 5),
    (3, 1, "canonical", "norm", 1),
    (2, 0, "full", "component", 9),
    (5, 4, "canonical", "component", 300),     # odd C canonical: unaligned rows
    (64, 4, "full", "component", 1000),
    (130, 2, "full", "component", 70),         # 260 lanes: two tiles, partial second tile
    (300, 1, "canonical", "component", 40),    # 300 lanes: two tiles
    (256, 6, "full", "component", 33),         # 512 lanes, C256 m6 full
]


@pytest.mark.parametrize("channels,m_max,parity,normalization,n_rows", CASES)
def test_parity_small(channels, m_max, parity, normalization, n_rows):
    rng = np.random.default_rng(1000 + channels * 7 + m_max)
    plan = O.OraclePlan(channels, m_max, parity, normalization)
    module = _module(channels, m_max, parity, normalization)
    x, y, g = (rng.standard_normal((n_rows, plan.width)) for _ in range(3))
    _check(plan, module, x, y, g)


def test_parity_config1_subset():
    """C128, m6, full, N=6400 (checked on 512 random rows)."""
    rng = np.random.default_rng(6400)
    plan = O.OraclePlan(128, 6, "full")
    module = _module(128, 6, "full")
    x, y, g = (rng.standard_normal((6400, plan.width)) for _ in range(3))
    rows = np.sort(rng.choice(6400, 512, replace=False))
    _check(plan, module, x, y, g, rows=rows)


@pytest.mark.parametrize("parity", ["canonical", "full"])
def test_component_major_layouts(parity):
    from ictc_o2_hp import ComponentMajorTensorProduct
    rng = np.random.default_rng(77)
    plan = O.OraclePlan(24, 3, parity)
    module = _module(24, 3, parity, layout_cls=ComponentMajorTensorProduct)
    x, y, g = (rng.standard_normal((150, plan.width)) for _ in range(3))
    _check(plan, module, x, y, g, layout=1 if parity == "canonical" else 2)


def test_golden_vectors(golden_tp):
    """The reference's own fp64 outputs on stored inputs (tests/golden/tp_vectors.npz)."""
    from ictc_o2_hp import TensorProduct
    names = sorted({k.split("/")[0] for k in golden_tp.files})
    for name in names:
        c, m, parity, norm = name.split("_")
        module = TensorProduct(int(c[1:]), int(m[1:]), parity=parity, normalization=norm).cuda()
        with torch.no_grad():
            module.weight.copy_(torch.from_numpy(golden_tp[f"{name}/weight"]).float())
        got = _run(module, golden_tp[f"{name}/x"], golden_tp[f"{name}/y"],
                   golden_tp[f"{name}/g"])
        for key, value in zip(("out", "dx", "dy", "dw"), got):
            err = O.normalized_error(golden_tp[f"{name}/{key}"], value)
            assert err <= TOL, (name, key, err)


def test_empty_rows():
    module = _module(16, 3, "full")
    x = torch.zeros(0, module.representation_dimension, device="cuda", requires_grad=True)
    y = torch.zeros_like(x, requires_grad=True)
    out = module(x, y)
    assert out.shape == x.shape
    dx, dy, dw = torch.autograd.grad(out, (x, y, module.weight), torch.zeros_like(out))
    assert dx.shape == x.shape and dy.shape == y.shape
    assert torch.count_nonzero(dw).item() == 0


def test_backward_is_bitwise_reproducible():
    module = _module(128, 6, "full")
    gen = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(3000, module.representation_dimension, device="cuda", generator=gen)
    y = torch.randn(x.shape, device="cuda", generator=gen)
    g = torch.randn(x.shape, device="cuda", generator=gen)
    results = []
    for _ in range(3):
        xt, yt = x.clone().requires_grad_(), y.clone().requires_grad_()
        out = module(xt, yt)
        results.append(torch.autograd.grad(out, (xt, yt, module.weight), g))
    for other in results[1:]:
        for a, b in zip(results[0], other):
            assert torch.equal(a, b)


def test_dw_additive_over_row_partitions():
    """Full-size-style check: dw over all rows equals the sum of dw over a
    partition of the rows, each computed with its own launch geometry."""
    module = _module(64, 6, "full")
    gen = torch.Generator(device="cuda").manual_seed(9)
    n = 20000
    x = torch.randn(n, module.representation_dimension, device="cuda", generator=gen)
    y = torch.randn(x.shape, device="cuda", generator=gen)
    g = torch.randn(x.shape, device="cuda", generator=gen)

    def dw_of(a, b, c):
        a = a.clone().requires_grad_()
        return torch.autograd.grad(module(a, b), module.weight, c)[0].double()

    whole = dw_of(x, y, g)
    parts = sum(dw_of(x[s:e], y[s:e], g[s:e]) for s, e in ((0, 7), (7, 5000), (5000, n)))
    err = (whole - parts).abs().max().item() / max(whole.abs().max().item(), 1e-7)
    assert err <= TOL, err


def test_batch_shapes_and_noncontiguous():
    from ictc_o2_hp import TensorProduct
    torch.manual_seed(3)
    module = TensorProduct(8, 2, parity="full").cuda()
    w = module.representation_dimension
    base = torch.randn(4, 6, 2 * w, device="cuda")
    x = base[..., :w]          # non-contiguous view
    y = torch.randn(4, 6, w, device="cuda")
    out = module(x, y)
    ref = module(x.contiguous().reshape(-1, w), y.reshape(-1, w)).reshape(4, 6, w)
    assert out.shape == (4, 6, w)
    assert torch.equal(out, ref)


def test_torch_compile_fullgraph():
    from ictc_o2_hp import TensorProduct
    torch.manual_seed(4)
    module = TensorProduct(32, 4, parity="full").cuda()
    compiled = torch.compile(module, fullgraph=True, dynamic=False)
    x = torch.randn(257, module.representation_dimension, device="cuda", requires_grad=True)
    y = torch.randn_like(x, requires_grad=True)
    g = torch.randn_like(x)
    eager = torch.autograd.grad(module(x, y), (x, y, module.weight), g)
    out = compiled(x, y)
    comp = torch.autograd.grad(out, (x, y, module.weight), g)
    for a, b in zip(eager, comp):
        assert torch.allclose(a, b, rtol=0, atol=0)


def test_double_backward_matches_fp64():
    from ictc_o2_hp import TensorProduct
    torch.manual_seed(6)
    module = TensorProduct(6, 2, parity="full").cuda()
    x = torch.randn(11, module.representation_dimension, device="cuda", requires_grad=True)
    y = torch.randn_like(x, requires_grad=True)
    out = module(x, y)
    (gx,) = torch.autograd.grad(out.square().sum(), x, create_graph=True)
    (hx,) = torch.autograd.grad(gx.sum(), y)
    module64 = TensorProduct(6, 2, parity="full").double()
    module64.weight.data.copy_(module.weight.data.double().cpu())
    x64 = x.detach().double().cpu().requires_grad_()
    y64 = y.detach().double().cpu().requires_grad_()
    module64.internal_compute_dtype = torch.float64
    out64 = module64(x64, y64)
    (gx64,) = torch.autograd.grad(out64.square().sum(), x64, create_graph=True)
    (hx64,) = torch.autograd.grad(gx64.sum(), y64)
    assert O.normalized_error(hx64.numpy(), hx.double().cpu().numpy()) <= TOL


def _orders_1_to_3(module, x, y):
    """First VJP of a loss whose cotangent depends on the output, second order
    with cotangents on all three first-order results, and third order."""
    out = module(x, y)
    e = (out * out.roll(1, 0)).sum()
    gx, gy, gw = torch.autograd.grad(e, (x, y, module.weight), create_graph=True)
    s = gx.square().sum() + (gy * y).sum() + gw.square().sum()
    hx, hy, hw = torch.autograd.grad(s, (x, y, module.weight), create_graph=True)
    t = hx.sum() + hy.square().sum() + (hw * hw.flip(0)).sum()
    return (gx, gy, gw, hx, hy, hw) + torch.autograd.grad(t, (x, y, module.weight))


@pytest.mark.parametrize("parity,layout", [("full", "tp"), ("canonical", "component")])
def test_second_and_third_order_match_fp64(parity, layout):
    """The second order is built from the kernel ops by multilinearity; the
    orders above compose through the same ops."""
    from ictc_o2_hp import ComponentMajorTensorProduct, TensorProduct
    cls = TensorProduct if layout == "tp" else ComponentMajorTensorProduct
    torch.manual_seed(7)
    module = cls(8, 3, parity=parity).cuda()
    with torch.no_grad():
        module.weight.normal_()
    x = torch.randn(37, module.representation_dimension, device="cuda", requires_grad=True)
    y = torch.randn_like(x, requires_grad=True)
    print(f"case orders 1-3 {cls.__name__} {parity}", flush=True)
    got = _orders_1_to_3(module, x, y)
    module64 = cls(8, 3, parity=parity).double()
    module64.weight.data.copy_(module.weight.data.double().cpu())
    module64.internal_compute_dtype = torch.float64
    x64 = x.detach().double().cpu().requires_grad_()
    y64 = y.detach().double().cpu().requires_grad_()
    want = _orders_1_to_3(module64, x64, y64)
    for name, r, a in zip(("gx", "gy", "gw", "hx", "hy", "hw", "tx", "ty", "tw"), want, got):
        assert O.normalized_error(r.detach().numpy(), a.detach().double().cpu().numpy()) <= TOL, name


def test_native_library_is_loaded():
    """The GPU path must run the in-tree HIP library (no silent fallback)."""
    from ictc_o2_hp import _native
    lib = _native.library()
    assert "ictc_o2_hp_amd" in lib.o2mi_version().decode()
    module = _module(8, 1, "canonical")
    x = torch.randn(3, module.representation_dimension, device="cuda")
    module(x, x)
    import os
    maps = open(f"/proc/{os.getpid()}/maps").read()
    assert _native.LIBRARY_NAME in maps


def _normalized_error_t(ref: torch.Tensor, got: torch.Tensor) -> float:
    """The reference's metric (oracle normalized_error) on device tensors."""
    scale = max(1e-7, ref.abs().max().item(), got.abs().max().item())
    return (ref - got.to(ref.dtype)).abs().max().item() / scale


def _headline_inputs(seed):
    module = _module(128, 6, "full", seed=seed)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    n = 131072
    x = torch.randn(n, module.representation_dimension, device="cuda", generator=gen)
    y = torch.randn(x.shape, device="cuda", generator=gen)
    g = torch.randn(x.shape, device="cuda", generator=gen)
    return module, x, y, g


def test_headline_full_size_rows_vs_oracle():
    """BASELINE headline shape (N=131072, C128 m6 full) at its full launch
    geometry: 256 random rows against the fp64 oracle, dw from a cotangent
    that is zero outside those rows (so the oracle's dw over them is exact)."""
    print("case headline N=131072 C128 m6 full, 256-row oracle subset", flush=True)
    module, x, y, g = _headline_inputs(131)
    rows = torch.randperm(x.shape[0], generator=torch.Generator().manual_seed(131))[:256]
    rows = rows.sort().values.cuda()
    mask = torch.zeros(x.shape[0], 1, device="cuda")
    mask[rows] = 1.0
    g = g * mask
    xr, yr = x.clone().requires_grad_(), y.clone().requires_grad_()
    out = module(xr, yr)
    dx, dy, dw = torch.autograd.grad(out, (xr, yr, module.weight), g)
    plan = O.OraclePlan(128, 6, "full")
    w = module.weight.detach().double().cpu().numpy()
    xs, ys, gs = (t[rows].double().cpu().numpy() for t in (x, y, g))
    ref_dx, ref_dy, ref_dw = O.backward(plan, xs, ys, w, gs)
    errors = {
        "out": O.normalized_error(O.forward(plan, xs, ys, w),
                                  out.detach()[rows].double().cpu().numpy()),
        "dx": O.normalized_error(ref_dx, dx[rows].double().cpu().numpy()),
        "dy": O.normalized_error(ref_dy, dy[rows].double().cpu().numpy()),
        "dw": O.normalized_error(ref_dw, dw.double().cpu().numpy()),
    }
    assert max(errors.values()) <= TOL, errors


def test_headline_full_size_every_row_vs_fp64_algebra():
    """BASELINE headline shape, every row and the full dw: the kernels against
    the PyTorch algebra (the reference's fast_o2.py map, pinned to the oracle
    on the CPU) evaluated in float64 on the GPU in row chunks."""
    from ictc_o2_hp.torch_algebra import flat_forward
    print("case headline N=131072 C128 m6 full, all rows vs fp64 algebra", flush=True)
    module, x, y, g = _headline_inputs(132)
    xr, yr = x.clone().requires_grad_(), y.clone().requires_grad_()
    out = module(xr, yr)
    dx, dy, dw = torch.autograd.grad(out, (xr, yr, module.weight), g)
    plan = module._plan
    w64 = module.weight.detach().double().requires_grad_()
    worst = {"out": 0.0, "dx": 0.0, "dy": 0.0}
    dw64 = torch.zeros_like(w64)
    for s in range(0, x.shape[0], 16384):
        e = s + 16384
        a = x[s:e].double().requires_grad_()
        b = y[s:e].double().requires_grad_()
        ref = flat_forward(a, b, w64, plan)
        ra, rb, rw = torch.autograd.grad(ref, (a, b, w64), g[s:e].double())
        dw64 += rw
        for name, r, got in (("out", ref.detach(), out[s:e]), ("dx", ra, dx[s:e]),
                             ("dy", rb, dy[s:e])):
            worst[name] = max(worst[name], _normalized_error_t(r, got))
        del ref, ra, rb, a, b
    worst["dw"] = _normalized_error_t(dw64, dw)
    assert max(worst.values()) <= TOL, worst


def test_component_major_matches_reference_layout_vectors():
    """The component-major kernels (layouts 1 and 2) against the reference's
    component-major product on its stored inputs (tests/golden/layout_vectors.npz)."""
    from conftest import GOLDEN
    from ictc_o2_hp import ComponentMajorTensorProduct
    data = np.load(GOLDEN / "layout_vectors.npz")
    for name in sorted({k.split("/")[0] for k in data.files}):
        print(f"case component-major reference vectors {name}", flush=True)
        c, m, parity, norm = name.split("_")
        module = ComponentMajorTensorProduct(int(c[1:]), int(m[1:]), parity=parity,
                                             normalization=norm).cuda()
        with torch.no_grad():
            module.weight.copy_(torch.from_numpy(data[f"{name}/weight"]).float())
        got = _run(module, data[f"{name}/x"], data[f"{name}/y"], data[f"{name}/g"])
        for key, value in zip(("out", "dx", "dy", "dw"), got):
            assert O.normalized_error(data[f"{name}/{key}"], value) <= TOL, (name, key)


# m_max above the benchmark grid: compiled plans up to m8 (m8 full has 136
# paths), beyond that the table-driven kernels, which read the module's
# path_info / path_coefficients tables (the reference JIT-specialises any
# m_max, triton_o2.py:1098-1132).
HIGH_ORDER = [
    # C, M, parity, normalization, N, layout class
    (16, 7, "full", "component", 300, None),
    (16, 8, "canonical", "component", 257, None),
    (12, 8, "full", "norm", 130, None),
    (5, 7, "canonical", "norm", 40, None),           # odd C
    (24, 7, "full", "component", 64, "component_major"),
    (6, 8, "canonical", "norm", 33, "component_major"),
    # several 128-lane tiles per row (LDS-staged forward weights, 128-lane
    # backward tiles), the last one partial
    (80, 7, "full", "component", 70, None),
    (128, 8, "full", "norm", 37, None),
    (72, 7, "full", "component", 21, "component_major"),
    (200, 8, "canonical", "component", 45, None),
    # table-driven
    (9, 10, "full", "norm", 33, None),
    (16, 9, "canonical", "component", 129, None),
    (8, 9, "full", "component", 70, None),
    (7, 9, "canonical", "component", 50, "component_major"),
    (4, 10, "full", "norm", 20, "component_major"),
]


@pytest.mark.parametrize("channels,m_max,parity,normalization,n_rows,layout", HIGH_ORDER)
def test_high_order_plans_match_oracle(channels, m_max, parity, normalization, n_rows, layout):
    from ictc_o2_hp import ComponentMajorTensorProduct
    print(f"case high order C{channels} m{m_max} {parity} {normalization} N{n_rows} "
          f"layout {layout}", flush=True)
    rng = np.random.default_rng(700 + channels + m_max)
    plan = O.OraclePlan(channels, m_max, parity, normalization)
    cls = ComponentMajorTensorProduct if layout else None
    module = _module(channels, m_max, parity, normalization, layout_cls=cls)
    assert module._on_kernels(torch.zeros(1, device="cuda"))
    x, y, g = (rng.standard_normal((n_rows, plan.width)) for _ in range(3))
    lay = 0 if not layout else (1 if parity == "canonical" else 2)
    _check(plan, module, x, y, g, layout=lay)


@pytest.mark.parametrize("channels,m_max,parity", [(32, 8, "full"), (32, 9, "canonical")])
def test_high_order_rows_at_scale(channels, m_max, parity):
    """N = 65536 (many blocks and row groups; compiled m8 full, table-driven
    m9): 256 random rows against the oracle, dw from a cotangent masked to
    them."""
    print(f"case high order at scale C{channels} m{m_max} {parity}", flush=True)
    rng = np.random.default_rng(7007 + m_max)
    plan = O.OraclePlan(channels, m_max, parity)
    module = _module(channels, m_max, parity)
    n = 65536
    x, y, g = (rng.standard_normal((n, plan.width)) for _ in range(3))
    rows = np.sort(rng.choice(n, 256, replace=False))
    _check(plan, module, x, y, g, rows=rows)


@pytest.mark.parametrize("channels,m_max,parity,normalization,layout", [
    (16, 8, "full", "component", 0),
    (10, 7, "canonical", "norm", 1),
    (32, 6, "full", "component", 0),
    (17, 3, "full", "norm", 0),
    (5, 4, "canonical", "component", 1),
    (24, 5, "full", "component", 2),
    (64, 2, "canonical", "norm", 0),
    (130, 1, "full", "component", 0),
])
def test_table_driven_kernels_match_compiled_kernels(channels, m_max, parity, normalization,
                                                     layout):
    """For compiled plans, the table-driven entry points give the compiled
    kernels' results (within fp32 rounding: the two sum the terms in
    different orders), through the C ABI with the module's own tables."""
    from ictc_o2_hp import _native
    from ictc_o2_hp.native_o2 import _path_metadata
    from ictc_o2_hp.plan import TPPlan
    print(f"case tables vs compiled C{channels} m{m_max} {parity} {normalization} "
          f"layout {layout}", flush=True)
    native = _native.TPNativePlan(channels, m_max, parity, normalization, layout)
    assert native.compiled
    info, coef = (t.cuda() for t in _path_metadata(TPPlan(channels, m_max, parity,
                                                          normalization), layout))
    tables = _native.TablesCall(native, info.data_ptr(), coef.data_ptr(), info.shape[0])
    gen = torch.Generator(device="cuda").manual_seed(channels + m_max)
    n = 3001
    x, y, g = (torch.randn((n, native.width), device="cuda", generator=gen) for _ in range(3))
    w = torch.randn(native.weight_numel, device="cuda", generator=gen)
    stream = torch.cuda.current_stream().cuda_stream
    results = []
    for kernels in (native, tables):
        out, dx, dy = (torch.empty_like(x) for _ in range(3))
        dw = torch.empty_like(w)
        kernels.forward(x.data_ptr(), y.data_ptr(), w.data_ptr(), out.data_ptr(), n, stream)
        ws_bytes = kernels.workspace_bytes(n)
        ws = torch.empty(max(1, ws_bytes // 4), device="cuda")
        kernels.backward(x.data_ptr(), y.data_ptr(), w.data_ptr(), g.data_ptr(), dx.data_ptr(),
                         dy.data_ptr(), dw.data_ptr(), ws.data_ptr(), ws_bytes, n, 7, stream)
        results.append([t.double().cpu().numpy() for t in (out, dx, dy, dw)])
    torch.cuda.synchronize()
    for name, a, b in zip(("out", "dx", "dy", "dw"), *results):
        assert O.normalized_error(a, b) <= 1e-6, name


def test_table_driven_backward_roles_and_reproducible():
    """Role subsets of the table-driven backward and bitwise repeatable dw."""
    torch.manual_seed(3)
    from ictc_o2_hp import _native
    assert not _native.TPNativePlan(8, 9, "full", "component", 0).compiled
    module = _module(8, 9, "full")
    gen = torch.Generator(device="cuda").manual_seed(8)
    x = torch.randn((500, module.representation_dimension), device="cuda", generator=gen)
    y = torch.randn(x.shape, device="cuda", generator=gen)
    g = torch.randn(x.shape, device="cuda", generator=gen)
    xr, yr = x.clone().requires_grad_(), y.clone().requires_grad_()
    full = torch.autograd.grad(module(xr, yr), (xr, yr, module.weight), g)
    again = torch.autograd.grad(module(xr, yr), (xr, yr, module.weight), g)
    for a, b in zip(full, again):
        assert torch.equal(a, b)
    (dy_only,) = torch.autograd.grad(module(x, yr), (yr,), g)
    assert torch.equal(dy_only, full[1])
