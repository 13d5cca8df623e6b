"""GPU parity of the uvu kernels against the fp64 uvu oracle (gate 1e-5)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import uvu_oracle as U
from oracle.o2_oracle import normalized_error

TOL = 1e-5
pytestmark = pytest.mark.gpu


def _run(module, x, y, w, g, wrt=(True, True, True)):
    xt = torch.from_numpy(x).float().cuda().requires_grad_(wrt[0])
    yt = torch.from_numpy(y).float().cuda().requires_grad_(wrt[1])
    wt = torch.from_numpy(w).float().cuda().requires_grad_(wrt[2])
    out = module(xt, yt, wt)
    inputs = [t for t, want in zip((xt, yt, wt), wrt) if want]
    grads = torch.autograd.grad(out, inputs, torch.from_numpy(g).float().cuda())
    torch.cuda.synchronize()
    return out.detach().double().cpu().numpy(), [t.double().cpu().numpy() for t in grads]


def _case(c, v, m, kw, shared, n, seed, wrt=(True, True, True)):
    from ictc_o2_hp import UvuTensorProduct
    print(f"uvu case C={c} V={v} M={m} {kw} shared={shared} N={n} wrt={wrt}", flush=True)
    module = UvuTensorProduct(c, v, m, shared_weights=shared, internal_weights=False, **kw).cuda()
    plan = U.UvuOraclePlan(c, v, m, **kw)
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, plan.width1))
    y = rng.standard_normal((n, plan.width2))
    g = rng.standard_normal((n, plan.width1))
    w = rng.standard_normal((plan.weight_numel,) if shared else (n, plan.weight_numel))
    w /= np.sqrt(v)
    out, grads = _run(module, x, y, w, g, wrt)
    ref_out = U.forward(plan, x, y, w, shared)
    ref = U.backward(plan, x, y, w, g, shared)
    assert normalized_error(ref_out, out) <= TOL
    for r, a in zip([r for r, want in zip(ref, wrt) if want], grads):
        assert a.shape == r.shape
        assert normalized_error(r, a) <= TOL


CASES = [
    (64, 1, 4, {"parity": "canonical"}, False, 700),                 # configs[4] TP shape
    (128, 32, 4, {"parity": "full"}, False, 24),                     # configs[3] shape, few rows
    (16, 4, 2, {"parity": "full"}, True, 500),                       # shared weights
    (130, 3, 2, {"parity": "canonical", "parity_in2": "full"}, True, 40),
    (24, 1, 6, {"parity": "full", "parity_in2": "canonical"}, False, 50),
    (5, 2, 3, {"parity": "canonical", "m_max_in2": 1, "path_normalization": "path"}, False, 33),
    (7, 3, 1, {"parity": "full", "normalization": "norm", "path_normalization": "element"},
     True, 1),
    # Per-row weights with V = 4 G, G | 64: the row-streaming kernels.
    (7, 4, 4, {"parity": "full", "m_max_in2": 2}, False, 17),                  # G = 1
    (5, 8, 3, {"parity": "full"}, False, 30),                                  # G = 2
    (12, 16, 2, {"parity": "canonical", "parity_in2": "full"}, False, 20),     # G = 4
    (3, 64, 2, {"parity": "full", "path_normalization": "path"}, False, 10),   # G = 16
    (2, 256, 1, {"parity": "canonical"}, False, 5),                            # G = 64
]


@pytest.mark.parametrize("c,v,m,kw,shared,n", CASES)
def test_uvu_parity(c, v, m, kw, shared, n):
    _case(c, v, m, kw, shared, n, seed=c * 100 + v * 10 + m)


# Per-row weights with 3 <= V <= 7 not a multiple of 4: one wave per row (and
# V = 1, 2 through the generic kernels).
WAVE_ROWS = [
    (130, 3, 2, {"parity": "full"}, 40),                   # two channel passes per lane
    (64, 6, 4, {"parity": "canonical", "parity_in2": "full"}, 30),
    (16, 7, 6, {"parity": "full"}, 9),
    (96, 5, 3, {"parity": "full", "path_normalization": "path"}, 17),
    (24, 1, 4, {"parity": "canonical", "normalization": "norm"}, 65),
    (40, 2, 7, {"parity": "canonical"}, 12),
]


@pytest.mark.parametrize("c,v,m,kw,n", WAVE_ROWS)
def test_uvu_wave_rows(c, v, m, kw, n):
    _case(c, v, m, kw, False, n, seed=c * 7 + v + m)
    for wrt in ((True, False, False), (False, True, False), (False, False, True)):
        _case(c, v, m, kw, False, 5, seed=c + v, wrt=wrt)


# V = 1 with shared weights (the reference's default mode) and m_max_in2 ==
# m_max: the plan-specialised kernels shared with the radial product.
SHARED_V1 = [
    (16, 2, {"parity": "canonical"}, 300),
    (128, 4, {"parity": "full"}, 129),                                    # channels split
    (32, 6, {"parity": "full", "parity_in2": "canonical"}, 1000),
    (48, 3, {"parity": "canonical", "parity_in2": "full", "path_normalization": "path"}, 70),
    (16, 1, {"parity": "full", "normalization": "norm"}, 1),
    (64, 6, {"parity": "full"}, 40),                                      # 508 paths
]


@pytest.mark.parametrize("c,m,kw,n", SHARED_V1)
def test_uvu_shared_v1_kernels(c, m, kw, n):
    from ictc_o2_hp import UvuTensorProduct, uvu_ops
    _case(c, 1, m, kw, True, n, seed=c + m + n)
    module = UvuTensorProduct(c, 1, m, shared_weights=True, **kw)
    assert uvu_ops.shared_plan(module._kernel_metadata_id) is not None


def test_uvu_shared_v1_roles_and_reproducible():
    from ictc_o2_hp import UvuTensorProduct
    for wrt in ((True, False, False), (False, True, False), (False, False, True),
                (False, True, True)):
        _case(64, 1, 4, {"parity": "full"}, True, 90, seed=8, wrt=wrt)
    torch.manual_seed(9)
    module = UvuTensorProduct(32, 1, 5, parity="full", parity_in2="canonical").cuda()
    x = torch.randn(40000, module.input1_dimension, device="cuda")
    y = torch.randn(40000, module.input2_dimension, device="cuda")
    g = torch.randn_like(x)
    first = torch.autograd.grad(module(x, y), module.weight, g)[0]
    second = torch.autograd.grad(module(x, y), module.weight, g)[0]
    assert torch.equal(first, second)
    halves = sum(torch.autograd.grad(module(x[s:s + 20000], y[s:s + 20000]), module.weight,
                                     g[s:s + 20000])[0] for s in (0, 20000))
    assert normalized_error(first.double().cpu().numpy(), halves.double().cpu().numpy()) <= TOL


# 2 <= V <= 8 with shared weights: the v projection, dy and dw on the matrix
# cores (o2mi_uvu_vshared.hpp).
SHARED_V = [
    (16, 2, 2, {"parity": "canonical"}, 300),
    (32, 3, 4, {"parity": "full"}, 200),
    (128, 8, 4, {"parity": "full"}, 129),                                 # channels split
    (48, 5, 3, {"parity": "canonical", "parity_in2": "full", "path_normalization": "path"}, 70),
    (16, 7, 1, {"parity": "full", "normalization": "norm"}, 1),
    (32, 4, 6, {"parity": "full", "parity_in2": "canonical"}, 257),
    (64, 8, 6, {"parity": "full"}, 40),                                   # 508 paths
    (16, 6, 0, {"parity": "full"}, 33),
]


@pytest.mark.parametrize("c,v,m,kw,n", SHARED_V)
def test_uvu_shared_v_kernels(c, v, m, kw, n):
    from ictc_o2_hp import UvuTensorProduct, uvu_ops
    _case(c, v, m, kw, True, n, seed=c + v + m + n)
    module = UvuTensorProduct(c, v, m, shared_weights=True, **kw)
    assert uvu_ops.shared_plan(module._kernel_metadata_id) is not None


def test_uvu_shared_v_roles_and_reproducible():
    from ictc_o2_hp import UvuTensorProduct, uvu_ops
    for wrt in ((True, False, False), (False, True, False), (False, False, True),
                (False, True, True)):
        _case(64, 4, 4, {"parity": "full"}, True, 90, seed=11, wrt=wrt)
    torch.manual_seed(12)
    module = UvuTensorProduct(32, 8, 5, parity="full", parity_in2="canonical").cuda()
    assert uvu_ops.shared_plan(module._kernel_metadata_id) is not None
    x = torch.randn(40000, module.input1_dimension, device="cuda")
    y = torch.randn(40000, module.input2_dimension, device="cuda")
    g = torch.randn_like(x)
    first = torch.autograd.grad(module(x, y), module.weight, g)[0]
    second = torch.autograd.grad(module(x, y), module.weight, g)[0]
    assert torch.equal(first, second)
    halves = sum(torch.autograd.grad(module(x[s:s + 20000], y[s:s + 20000]), module.weight,
                                     g[s:s + 20000])[0] for s in (0, 20000))
    assert normalized_error(first.double().cpu().numpy(), halves.double().cpu().numpy()) <= TOL
    # V above the kernels' 8 copies keeps the generic kernels.
    wide = UvuTensorProduct(16, 9, 2, parity="full")
    assert uvu_ops.shared_plan(wide._kernel_metadata_id) is None


# V = 1 with per-row weights (external weights, as a radial product feeds
# them): the streamed radial kernels reading each row's weights from memory.
ROWS_V1 = [
    (64, 4, {"parity": "canonical"}, 700),                                # configs[4] TP shape
    (128, 4, {"parity": "full"}, 100),                                    # 4 pairs, one edge group
    (256, 2, {"parity": "full"}, 50),                                     # 128-channel spans over grid y
    (96, 2, {"parity": "canonical"}, 90),                                 # idle pair; 64 + 32 channel spans
    (32, 6, {"parity": "full", "parity_in2": "canonical"}, 300),
    (48, 3, {"parity": "canonical", "parity_in2": "full", "path_normalization": "path"}, 70),
    (16, 0, {"parity": "full", "normalization": "norm"}, 1),
    (16, 6, {"parity": "full"}, 40),                                      # 508 paths
]


@pytest.mark.parametrize("c,m,kw,n", ROWS_V1)
def test_uvu_rows_v1_kernels(c, m, kw, n):
    from ictc_o2_hp import UvuTensorProduct, uvu_ops
    _case(c, 1, m, kw, False, n, seed=c + m + n + 1)
    module = UvuTensorProduct(c, 1, m, shared_weights=False, internal_weights=False, **kw)
    assert uvu_ops._fused_plan(module._kernel_metadata_id, False) is not None


def test_uvu_rows_v1_roles():
    for wrt in ((True, False, False), (False, True, False), (False, False, True),
                (True, False, True), (False, True, True)):
        _case(64, 1, 3, {"parity": "full"}, False, 90, seed=13, wrt=wrt)


@pytest.mark.parametrize("wrt", [(True, False, False), (False, True, False), (False, False, True),
                                 (True, False, True)])
def test_uvu_gradient_roles(wrt):
    _case(12, 2, 3, {"parity": "full"}, False, 40, seed=5, wrt=wrt)
    _case(12, 2, 3, {"parity": "full"}, True, 40, seed=6, wrt=wrt)
    _case(16, 8, 2, {"parity": "full"}, False, 33, seed=7, wrt=wrt)     # row kernels


def test_uvu_golden_vectors(golden_uvu):
    from ictc_o2_hp import UvuTensorProduct
    cases = {
        "c3_v2_m2_full": (3, 2, 2, {"parity": "full"}, True),
        "c4_v1_m4_canonical": (4, 1, 4, {"parity": "canonical"}, False),
        "c3_v1_m6_full_in2canonical": (3, 1, 6, {"parity": "full", "parity_in2": "canonical"},
                                       False),
        "c2_v3_m3_canonical_in2full_m2_path": (2, 3, 3, {"parity": "canonical",
                                                         "parity_in2": "full", "m_max_in2": 2,
                                                         "path_normalization": "path"}, False),
        "c2_v2_m1_full_norm_element": (2, 2, 1, {"parity": "full", "normalization": "norm",
                                                 "path_normalization": "element"}, True),
    }
    for name, (c, v, m, kw, shared) in cases.items():
        module = UvuTensorProduct(c, v, m, shared_weights=shared, internal_weights=False,
                                  **kw).cuda()
        x, y, w, g = (golden_uvu[f"{name}/{k}"] for k in ("x", "y", "w", "g"))
        out, grads = _run(module, x, y, w, g)
        for key, value in zip(("out", "dx", "dy", "dw"), [out, *grads]):
            assert normalized_error(golden_uvu[f"{name}/{key}"], value) <= TOL, (name, key)


@pytest.mark.parametrize("c,v,shared", [(8, 2, True), (8, 2, False), (16, 1, True), (16, 2, True),
                                        (16, 1, False)])
def test_uvu_empty_rows(c, v, shared):
    from ictc_o2_hp import UvuTensorProduct
    module = UvuTensorProduct(c, v, 2, shared_weights=shared, internal_weights=False).cuda()
    x = torch.zeros(0, module.input1_dimension, device="cuda", requires_grad=True)
    y = torch.zeros(0, module.input2_dimension, device="cuda", requires_grad=True)
    w = torch.zeros((module.weight_numel,) if shared else (0, module.weight_numel),
                    device="cuda", requires_grad=True)
    out = module(x, y, w)
    dx, dy, dw = torch.autograd.grad(out, (x, y, w), torch.zeros_like(out))
    assert out.shape == x.shape and dx.shape == x.shape and dy.shape == y.shape
    assert dw.shape == w.shape and torch.count_nonzero(dw).item() == 0


def test_uvu_into_ops_and_internal_weights():
    from ictc_o2_hp import UvuTensorProduct, uvu_ops
    torch.manual_seed(0)
    module = UvuTensorProduct(16, 1, 4, parity="canonical").cuda()   # internal shared weights
    x = torch.randn(50, module.input1_dimension, device="cuda")
    y = torch.randn(50, module.input2_dimension, device="cuda")
    args = (module._path_info, module._coefficients, module._first_order, module._second_order,
            module._kernel_metadata_id, True)
    result = torch.empty_like(x)
    uvu_ops.uvu_forward_into(x, y, module.weight.detach(), *args, result)
    assert torch.equal(result, module(x, y))
    g = torch.randn_like(x)
    gx, gy, gw = torch.empty_like(x), torch.empty_like(y), torch.empty_like(module.weight)
    uvu_ops.uvu_backward_into(x, y, module.weight.detach(), g, *args, 7, gx, gy, gw)
    ref = uvu_ops.uvu_backward(x, y, module.weight.detach(), g, *args, 7)
    for a, b in zip((gx, gy, gw), ref):
        assert torch.equal(a, b)


def test_uvu_torch_compile():
    from ictc_o2_hp import UvuTensorProduct
    torch.manual_seed(1)
    module = UvuTensorProduct(32, 1, 3, parity="full", shared_weights=False).cuda()
    compiled = torch.compile(module, fullgraph=True, dynamic=False)
    x = torch.randn(64, module.input1_dimension, device="cuda", requires_grad=True)
    y = torch.randn(64, module.input2_dimension, device="cuda", requires_grad=True)
    w = torch.randn(64, module.weight_numel, device="cuda", requires_grad=True)
    g = torch.randn_like(x)
    eager = torch.autograd.grad(module(x, y, w), (x, y, w), g)
    comp = torch.autograd.grad(compiled(x, y, w), (x, y, w), g)
    for a, b in zip(eager, comp):
        assert torch.equal(a, b)


def test_uvu_double_backward():
    from ictc_o2_hp import UvuTensorProduct
    torch.manual_seed(2)
    module = UvuTensorProduct(4, 1, 2, parity="full", shared_weights=False).cuda()
    x = torch.randn(6, module.input1_dimension, device="cuda", requires_grad=True)
    y = torch.randn(6, module.input2_dimension, device="cuda", requires_grad=True)
    w = torch.randn(6, module.weight_numel, device="cuda", requires_grad=True)
    (gy,) = torch.autograd.grad(module(x, y, w).square().sum(), y, create_graph=True)
    (hw,) = torch.autograd.grad(gy.sum(), w)
    m64 = UvuTensorProduct(4, 1, 2, parity="full", shared_weights=False).double()
    x64, y64, w64 = (t.detach().double().cpu().requires_grad_() for t in (x, y, w))
    (gy64,) = torch.autograd.grad(m64(x64, y64, w64).square().sum(), y64, create_graph=True)
    (hw64,) = torch.autograd.grad(gy64.sum(), w64)
    assert normalized_error(hw64.numpy(), hw.double().cpu().numpy()) <= TOL


# C = 8: generic kernels; C = 16: the plan-specialised shared V = 1, V = 2 and
# per-row V = 1 kernels.
@pytest.mark.parametrize("c,v,shared", [(8, 2, False), (8, 2, True), (16, 1, True), (16, 2, True),
                                        (16, 1, False)])
def test_uvu_second_and_third_order(c, v, shared):
    """Cotangents on all three first-order results, the grad_output term, and
    third order, against the fp64 CPU module."""
    from ictc_o2_hp import UvuTensorProduct
    torch.manual_seed(3)
    module = UvuTensorProduct(c, v, 2, parity="full", shared_weights=shared).cuda()
    n = 21
    x = torch.randn(n, module.input1_dimension, device="cuda", requires_grad=True)
    y = torch.randn(n, module.input2_dimension, device="cuda", requires_grad=True)
    wshape = (module.weight_numel,) if shared else (n, module.weight_numel)
    w = torch.randn(wshape, device="cuda", requires_grad=True)

    def orders(mod, a, b, c):
        out = mod(a, b, c)
        e = (out * out.roll(1, 0)).sum()
        ga, gb, gc = torch.autograd.grad(e, (a, b, c), create_graph=True)
        s = ga.square().sum() + (gb * b).sum() + gc.square().sum()
        ha, hb, hc = torch.autograd.grad(s, (a, b, c), create_graph=True)
        t = ha.sum() + hb.square().sum() + hc.sum()
        return (ga, gb, gc, ha, hb, hc) + torch.autograd.grad(t, (a, b, c))

    print(f"case uvu orders 1-3 C={c} V={v} shared={shared}", flush=True)
    got = orders(module, x, y, w)
    m64 = UvuTensorProduct(c, v, 2, parity="full", shared_weights=shared).double()
    x64, y64, w64 = (t.detach().double().cpu().requires_grad_() for t in (x, y, w))
    want = orders(m64, x64, y64, w64)
    for r, a in zip(want, got):
        assert normalized_error(r.detach().numpy(), a.detach().double().cpu().numpy()) <= TOL
