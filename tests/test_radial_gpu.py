"""GPU parity of RadialUvuTensorProduct against the fp64 radial oracle (gate 1e-5).

Fused structures (m_max <= 6, C % 16 == 0, H <= 64, H % 4 == 0) run the gfx950
radial kernels (weights generated on the matrix cores); the others run the
composed GPU path (fp32 GEMM + uvu kernels).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import uvu_oracle as U
from oracle.o2_oracle import normalized_error

TOL = 1e-5
pytestmark = pytest.mark.gpu
ROLES = ("x", "y", "hidden", "alpha", "bias")


def _build(c, m, parity, parity_in2, hidden, bias, seed, **kw):
    from ictc_o2_hp import RadialUvuTensorProduct, UvuTensorProduct
    tp = UvuTensorProduct(c, 1, m, parity=parity, parity_in2=parity_in2, shared_weights=False,
                          **kw).cuda()
    linear = torch.nn.Linear(hidden, tp.weight_numel, bias=bias).cuda()
    rng = np.random.default_rng(seed + 1)
    with torch.no_grad():
        linear.weight.copy_(torch.from_numpy(rng.standard_normal(linear.weight.shape)
                                             / np.sqrt(hidden)))
        if bias:
            linear.bias.copy_(torch.from_numpy(rng.standard_normal(linear.bias.shape) * 0.5))
    plan = U.UvuOraclePlan(c, 1, m, parity=parity, parity_in2=parity_in2, **kw)
    return tp, linear, RadialUvuTensorProduct(tp, linear), plan


def _case(c, m, parity, parity_in2, hidden, n, bias=True, seed=0, roles=ROLES, **kw):
    print(f"radial case C={c} m={m} {parity}/{parity_in2} H={hidden} N={n} bias={bias} "
          f"roles={roles} {kw}", flush=True)
    tp, linear, module, plan = _build(c, m, parity, parity_in2, hidden, bias, seed, **kw)
    rng = np.random.default_rng(seed)
    arrays = [rng.standard_normal((n, plan.width1)), rng.standard_normal((n, plan.width2)),
              rng.standard_normal((n, hidden))]
    g = rng.standard_normal((n, plan.width1)).astype(np.float32)
    x, y, h = (torch.from_numpy(a.astype(np.float32)).cuda().requires_grad_(r in roles)
               for a, r in zip(arrays, ROLES))
    out = module(x, y, h)
    wrt = [t for t, r in zip((x, y, h, linear.weight, linear.bias), ROLES)
           if r in roles and t is not None]
    grads = torch.autograd.grad(out, wrt, torch.from_numpy(g).cuda()) if wrt else []
    torch.cuda.synchronize()
    alpha = linear.weight.detach().double().cpu().numpy()
    b = linear.bias.detach().double().cpu().numpy() if bias else None
    xs, ys, hs = (t.detach().double().cpu().numpy() for t in (x, y, h))
    ref_out = U.radial_forward(plan, xs, ys, hs, alpha, b)
    assert normalized_error(ref_out, out.detach().double().cpu().numpy()) <= TOL
    ref = U.radial_backward(plan, xs, ys, hs, alpha, b, g.astype(np.float64))
    expected = [r for r, name in zip(ref, ROLES) if name in roles and r is not None]
    assert len(expected) == len(grads)
    for r, a in zip(expected, grads):
        assert a.shape == r.shape
        assert normalized_error(r, a.double().cpu().numpy()) <= TOL
    return tp, module


def test_configs4_structure_runs_fused():
    from ictc_o2_hp import radial_ops
    tp, _ = _case(64, 4, "canonical", "canonical", 64, 1000, seed=4)
    assert radial_ops.fused_plan(tp._kernel_metadata_id, 64) is not None


@pytest.mark.parametrize("n", [1, 127, 129, 300])
def test_ragged_edge_counts(n):
    _case(16, 2, "canonical", "canonical", 64, n, seed=n)


FUSED = [
    (16, 0, "canonical", "canonical", 64, {}),
    (32, 1, "full", "full", 32, {}),
    (16, 1, "full", "canonical", 20, {"path_normalization": "path"}),
    (48, 2, "canonical", "full", 64, {"normalization": "norm"}),
    (16, 3, "canonical", "canonical", 8, {"path_normalization": "element"}),
    (32, 0, "full", "full", 12, {}),
    (16, 6, "canonical", "canonical", 64, {}),            # 64 paths
    (32, 5, "full", "canonical", 32, {"normalization": "norm"}),
    (16, 4, "canonical", "full", 40, {"path_normalization": "path"}),
    (16, 3, "full", "full", 64, {}),                      # 148 paths
    (16, 6, "full", "full", 16, {}),                      # 508 paths
]


@pytest.mark.parametrize("c,m,parity,parity_in2,hidden,kw", FUSED)
def test_fused_structures(c, m, parity, parity_in2, hidden, kw):
    from ictc_o2_hp import radial_ops
    tp, _ = _case(c, m, parity, parity_in2, hidden, 200, seed=c + m, **kw)
    assert radial_ops.fused_plan(tp._kernel_metadata_id, hidden) is not None


# The reference's radial benchmark structure (m_max 6, full first input,
# canonical angular input, 254 paths): streamed kernels, alpha staged in
# chunks; the affine adjoints run in 4 path groups.
STREAMED = [
    (16, 64, 300, True, {}),
    (32, 48, 129, False, {"path_normalization": "path"}),
    (64, 64, 65, True, {"normalization": "norm"}),
    (48, 20, 1, True, {}),
]


@pytest.mark.parametrize("c,hidden,n,bias,kw", STREAMED)
def test_streamed_structure(c, hidden, n, bias, kw):
    from ictc_o2_hp import radial_ops
    tp, _ = _case(c, 6, "full", "canonical", hidden, n, bias=bias, seed=c + n, **kw)
    assert radial_ops.fused_plan(tp._kernel_metadata_id, hidden) is not None


@pytest.mark.parametrize("roles", [("x",), ("y",), ("hidden",), ("alpha",), ("y", "bias")])
def test_streamed_gradient_roles(roles):
    _case(16, 6, "full", "canonical", 64, 70, seed=21, roles=roles)
    # C = 48 with 70 edges: the channel tiles are split over grid y, so dy and
    # dhidden come from the split partials (and are skipped when not requested).
    _case(48, 6, "full", "canonical", 64, 70, seed=22, roles=roles)


def test_streamed_affine_adjoints_reproducible():
    tp, linear, module, plan = _build(16, 6, "full", "canonical", 64, True, 22)
    torch.manual_seed(22)
    x = torch.randn(700, tp.input1_dimension, device="cuda")
    y = torch.randn(700, tp.input2_dimension, device="cuda")
    h = torch.randn(700, 64, device="cuda")
    g = torch.randn(700, tp.input1_dimension, device="cuda")
    first = torch.autograd.grad(module(x, y, h), (linear.weight, linear.bias), g)
    second = torch.autograd.grad(module(x, y, h), (linear.weight, linear.bias), g)
    for a, b in zip(first, second):
        assert torch.equal(a, b)


def test_streamed_channel_split_matches_unsplit():
    """Below one edge block per CU the streamed kernels split the channels
    over grid y (dy / dhidden as fixed-order sums of split partials).  A run
    of 33,024 edges (258 blocks: unsplit) must equal the two halves (129
    blocks each: channels split in two) row by row, and the oracle on a row
    subset."""
    tp, linear, module, plan = _build(32, 6, "full", "canonical", 64, True, 23)
    n = 33024
    torch.manual_seed(23)
    x = torch.randn(n, tp.input1_dimension, device="cuda", requires_grad=True)
    y = torch.randn(n, tp.input2_dimension, device="cuda", requires_grad=True)
    h = torch.randn(n, 64, device="cuda", requires_grad=True)
    g = torch.randn(n, tp.input1_dimension, device="cuda")
    params = (x, y, h, linear.weight, linear.bias)
    print("case streamed split n=33024 C=32", flush=True)
    out = module(x, y, h)
    whole = torch.autograd.grad(out, params, g)
    half = n // 2
    parts = []
    for lo, hi in ((0, half), (half, n)):
        xs, ys, hs = (t.detach()[lo:hi].clone().requires_grad_() for t in (x, y, h))
        o = module(xs, ys, hs)
        parts.append((o,) + torch.autograd.grad(o, (xs, ys, hs, linear.weight, linear.bias),
                                                g[lo:hi]))
    torch.cuda.synchronize()
    assert torch.equal(out.detach(), torch.cat([parts[0][0], parts[1][0]]))
    assert torch.equal(whole[0], torch.cat([parts[0][1], parts[1][1]]))
    for k in (1, 2):   # dy, dhidden: split partial sums, another summation order
        cat = torch.cat([parts[0][k + 1], parts[1][k + 1]]).double().cpu().numpy()
        assert normalized_error(whole[k].double().cpu().numpy(), cat) <= TOL
    for k in (3, 4):   # dalpha, dbias: linear in the rows
        both = (parts[0][k + 1] + parts[1][k + 1]).double().cpu().numpy()
        assert normalized_error(both, whole[k].double().cpu().numpy()) <= TOL
    rows = np.random.default_rng(23).choice(n, 48, replace=False)
    alpha = linear.weight.detach().double().cpu().numpy()
    b = linear.bias.detach().double().cpu().numpy()
    xs, ys, hs, gs = (t.detach()[rows].double().cpu().numpy() for t in (x, y, h, g))
    ref_out = U.radial_forward(plan, xs, ys, hs, alpha, b)
    assert normalized_error(ref_out, out.detach()[rows].double().cpu().numpy()) <= TOL
    ref = U.radial_backward(plan, xs, ys, hs, alpha, b, gs)
    for r, a in zip(ref[:3], whole[:3]):
        assert normalized_error(r, a[rows].double().cpu().numpy()) <= TOL


# The streamed kernels read the 16-channel tiles of a block in pairs (the
# one-component entries of the second tile carried from the first tile's
# loads).  40,000 edges (313 blocks) run unsplit: C / 32 pairs plus a single
# tile when C % 32 == 16.  The slices 20,000 and 18,000 (157 and 141 blocks)
# split the channels in two 32-channel spans (a pair each, or a pair and a
# single tile for C = 48); 2,000 edges (16 blocks) split them into single
# tiles.  The pairing changes loads only, so output and dx agree bitwise.
PAIRED = [
    (48, 4, "canonical", "canonical", 64, {}),            # configs[4] structure at C = 48
    (64, 3, "full", "full", 32, {}),                      # two one-component entries
    (48, 6, "full", "canonical", 64, {"normalization": "norm"}),   # 254 paths
    (32, 2, "canonical", "full", 16, {"path_normalization": "path"}),
]


@pytest.mark.parametrize("c,m,parity,parity_in2,hidden,kw", PAIRED)
def test_paired_tiles_match_split_launches(c, m, parity, parity_in2, hidden, kw):
    from ictc_o2_hp import radial_ops
    tp, linear, module, plan = _build(c, m, parity, parity_in2, hidden, True, c + m, **kw)
    assert radial_ops.fused_plan(tp._kernel_metadata_id, hidden) is not None
    n = 40000
    print(f"case paired tiles C={c} m={m} {parity}/{parity_in2} H={hidden} n={n}", flush=True)
    torch.manual_seed(c + m)
    x = torch.randn(n, tp.input1_dimension, device="cuda", requires_grad=True)
    y = torch.randn(n, tp.input2_dimension, device="cuda", requires_grad=True)
    h = torch.randn(n, hidden, device="cuda", requires_grad=True)
    g = torch.randn(n, tp.input1_dimension, device="cuda")
    params = (x, y, h, linear.weight, linear.bias)
    out = module(x, y, h)
    whole = torch.autograd.grad(out, params, g)
    parts = []
    for lo, hi in ((0, 20000), (20000, 22000), (22000, n)):
        xs, ys, hs = (t.detach()[lo:hi].clone().requires_grad_() for t in (x, y, h))
        o = module(xs, ys, hs)
        parts.append((o,) + torch.autograd.grad(o, (xs, ys, hs, linear.weight, linear.bias),
                                                g[lo:hi]))
    torch.cuda.synchronize()
    assert torch.equal(out.detach(), torch.cat([p[0] for p in parts]))
    assert torch.equal(whole[0], torch.cat([p[1] for p in parts]))
    for k in (1, 2):   # dy, dhidden: split partial sums, another summation order
        cat = torch.cat([p[k + 1] for p in parts]).double().cpu().numpy()
        assert normalized_error(whole[k].double().cpu().numpy(), cat) <= TOL
    for k in (3, 4):   # dalpha, dbias: linear in the rows
        total = sum(p[k + 1] for p in parts).double().cpu().numpy()
        assert normalized_error(total, whole[k].double().cpu().numpy()) <= TOL
    rows = np.random.default_rng(c + m).choice(n, 32, replace=False)
    alpha = linear.weight.detach().double().cpu().numpy()
    b = linear.bias.detach().double().cpu().numpy()
    xs, ys, hs, gs = (t.detach()[rows].double().cpu().numpy() for t in (x, y, h, g))
    ref_out = U.radial_forward(plan, xs, ys, hs, alpha, b)
    assert normalized_error(ref_out, out.detach()[rows].double().cpu().numpy()) <= TOL
    ref = U.radial_backward(plan, xs, ys, hs, alpha, b, gs)
    for r, a in zip(ref[:3], whole[:3]):
        assert normalized_error(r, a[rows].double().cpu().numpy()) <= TOL


COMPOSED = [
    (24, 2, "canonical", "canonical", 64, {}),      # C % 16 != 0
    (16, 2, "canonical", "canonical", 6, {}),       # H % 4 != 0
    (16, 7, "canonical", "canonical", 64, {}),      # m_max 7: no kernel compiled
    (16, 2, "canonical", "canonical", 96, {}),      # H > 64
]


@pytest.mark.parametrize("c,m,parity,parity_in2,hidden,kw", COMPOSED)
def test_composed_structures(c, m, parity, parity_in2, hidden, kw):
    from ictc_o2_hp import radial_ops
    tp, _ = _case(c, m, parity, parity_in2, hidden, 150, seed=7, **kw)
    assert radial_ops.fused_plan(tp._kernel_metadata_id, hidden) is None


def test_without_bias():
    _case(32, 4, "canonical", "canonical", 64, 257, bias=False, seed=9)
    _case(24, 2, "canonical", "canonical", 16, 40, bias=False, seed=10)


@pytest.mark.parametrize("roles", [("hidden", "alpha", "bias"), ("x",), ("y",),
                                   ("x", "alpha"), ("hidden",)])
def test_gradient_roles(roles):
    _case(16, 4, "canonical", "canonical", 64, 130, seed=11, roles=roles)
    _case(64, 4, "canonical", "canonical", 64, 130, seed=12, roles=roles)   # split channels


def test_empty_edges():
    tp, linear, module, _ = _build(16, 2, "canonical", "canonical", 64, True, 0)
    x = torch.zeros(0, tp.input1_dimension, device="cuda", requires_grad=True)
    y = torch.zeros(0, tp.input2_dimension, device="cuda", requires_grad=True)
    h = torch.zeros(0, 64, device="cuda", requires_grad=True)
    out = module(x, y, h)
    grads = torch.autograd.grad(out, (x, y, h, linear.weight, linear.bias), torch.zeros_like(out))
    assert out.shape == x.shape
    assert [tuple(t.shape) for t in grads] == [tuple(x.shape), tuple(y.shape), tuple(h.shape),
                                               tuple(linear.weight.shape),
                                               tuple(linear.bias.shape)]
    assert torch.count_nonzero(grads[3]).item() == 0 and torch.count_nonzero(grads[4]).item() == 0


def test_affine_adjoints_reproducible_and_batched():
    tp, linear, module, plan = _build(32, 3, "canonical", "canonical", 64, True, 12)
    torch.manual_seed(12)
    x = torch.randn(4, 300, tp.input1_dimension, device="cuda")
    y = torch.randn(4, 300, tp.input2_dimension, device="cuda")
    h = torch.randn(4, 300, 64, device="cuda")
    g = torch.randn(4, 300, tp.input1_dimension, device="cuda")
    first = torch.autograd.grad(module(x, y, h), (linear.weight, linear.bias), g)
    second = torch.autograd.grad(module(x, y, h), (linear.weight, linear.bias), g)
    for a, b in zip(first, second):
        assert torch.equal(a, b)
    flat = torch.autograd.grad(module(x.reshape(1200, -1), y.reshape(1200, -1),
                                      h.reshape(1200, -1)),
                               (linear.weight, linear.bias), g.reshape(1200, -1))
    for a, b in zip(first, flat):
        assert torch.equal(a, b)


def test_torch_compile_fullgraph():
    tp, linear, module, _ = _build(32, 2, "canonical", "canonical", 64, True, 13)
    compiled = torch.compile(module, fullgraph=True, dynamic=False)
    torch.manual_seed(13)
    x = torch.randn(96, tp.input1_dimension, device="cuda", requires_grad=True)
    y = torch.randn(96, tp.input2_dimension, device="cuda", requires_grad=True)
    h = torch.randn(96, 64, device="cuda", requires_grad=True)
    g = torch.randn(96, tp.input1_dimension, device="cuda")
    params = (x, y, h, linear.weight, linear.bias)
    eager = torch.autograd.grad(module(x, y, h), params, g)
    comp = torch.autograd.grad(compiled(x, y, h), params, g)
    for a, b in zip(eager, comp):
        assert torch.equal(a, b)


@pytest.mark.parametrize("c,hidden", [(16, 8), (24, 8)])   # fused, composed
def test_double_backward(c, hidden):
    from ictc_o2_hp import RadialUvuTensorProduct, UvuTensorProduct
    tp, linear, module, _ = _build(c, 2, "canonical", "canonical", hidden, True, 14)
    torch.manual_seed(14)
    x = torch.randn(20, tp.input1_dimension, device="cuda", requires_grad=True)
    y = torch.randn(20, tp.input2_dimension, device="cuda", requires_grad=True)
    h = torch.randn(20, hidden, device="cuda", requires_grad=True)

    def second_order(mod, lin, xx, yy, hh):
        loss = mod(xx, yy, hh).square().sum()
        gx, gh = torch.autograd.grad(loss, (xx, hh), create_graph=True)
        return torch.autograd.grad(gx.square().sum() + gh.sum(), (yy, lin.weight, lin.bias))

    got = second_order(module, linear, x, y, h)
    tp64 = UvuTensorProduct(c, 1, 2, parity="canonical", shared_weights=False).double()
    lin64 = torch.nn.Linear(hidden, tp64.weight_numel).double()
    with torch.no_grad():
        lin64.weight.copy_(linear.weight.double().cpu())
        lin64.bias.copy_(linear.bias.double().cpu())
    ref_module = RadialUvuTensorProduct(tp64, lin64)
    x64, y64, h64 = (t.detach().double().cpu().requires_grad_() for t in (x, y, h))
    want = second_order(ref_module, lin64, x64, y64, h64)
    for r, a in zip(want, got):
        assert normalized_error(r.detach().numpy(), a.double().cpu().numpy()) <= TOL
