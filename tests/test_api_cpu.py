"""Drop-in API of the modules on the CPU (PyTorch algebra path)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import o2_oracle as O

from conftest import GOLDEN


def test_public_names():
    import ictc_o2_hp
    # The reference's public names (__init__.py:4-25).
    names = ("TensorProduct", "TupleTensorProduct", "ComponentMajorTensorProduct",
             "ReferenceTensorProduct", "UvuTensorProduct", "ReferenceUvuTensorProduct",
             "RadialUvuTensorProduct")
    for name in names:
        assert getattr(ictc_o2_hp, name) is not None
    assert set(names) <= set(ictc_o2_hp.__all__)
    assert ictc_o2_hp.__version__ == "0.1.6.dev0"
    with pytest.raises(AttributeError):
        ictc_o2_hp.NotAnOperator


@pytest.mark.parametrize("args", [(0, 2), (1.5, 2), (4, -1), (4, 1.5)])
def test_constructor_validation(args):
    from ictc_o2_hp import TensorProduct, ReferenceTensorProduct
    for cls in (TensorProduct, ReferenceTensorProduct):
        with pytest.raises(ValueError):
            cls(*args)


def test_bad_parity():
    from ictc_o2_hp import TensorProduct
    with pytest.raises(ValueError):
        TensorProduct(4, 2, parity="odd")


def test_width_errors():
    from ictc_o2_hp import TensorProduct, ComponentMajorTensorProduct
    for cls in (TensorProduct, ComponentMajorTensorProduct):
        tp = cls(4, 2)
        x = torch.randn(3, tp.representation_dimension)
        with pytest.raises(ValueError):
            tp(x[:, :-1], x[:, :-1])
        with pytest.raises(ValueError):
            tp(x, x[:2])


def test_default_weights_match_reference_init():
    """torch.manual_seed(0) then the per-path randn(out_mul) * 0.02 sequence
    (native_o2.py:117), recorded from the reference."""
    from ictc_o2_hp import TensorProduct
    golden = np.load(GOLDEN / "default_weights.npz")
    for c, m, parity in ((32, 2, "canonical"), (17, 3, "full"), (128, 6, "full")):
        torch.manual_seed(0)
        tp = TensorProduct(c, m, parity=parity)
        assert np.array_equal(tp.weight.detach().numpy(), golden[f"C{c}_m{m}_{parity}"])


def test_state_dict_layout():
    """weight, cg_<p>, odd_to_even, even_to_odd persistent; routing not."""
    from ictc_o2_hp import TensorProduct, ReferenceTensorProduct
    tp = TensorProduct(8, 3, parity="full")
    keys = set(tp.state_dict())
    expected = {"weight", "odd_to_even", "even_to_odd"} | {f"cg_{p}" for p in range(len(tp.paths))}
    assert keys == expected
    assert tp.state_dict()["cg_0"].dtype == torch.float64
    assert tp.weight.shape == (tp.parameter_count,)
    ref = ReferenceTensorProduct(8, 3, parity="full")
    rkeys = set(ref.state_dict())
    assert rkeys == (expected - {"weight"}) | {f"weights.{p}" for p in range(len(ref.paths))}
    tp.copy_weights_to_r5(ref)
    other = TensorProduct(8, 3, parity="full")
    other.load_weights_from_r5(ref)
    assert torch.equal(other.weight, tp.weight)
    with pytest.raises(ValueError):
        TensorProduct(8, 2).copy_weights_to_r5(ref)


def test_attributes():
    from ictc_o2_hp import TensorProduct
    tp = TensorProduct(128, 6, parity="full")
    assert tp.representation_dimension == 3328
    assert tp.parameter_count == 19712
    assert len(tp.paths) == 85
    assert len(tp.blocks) == 8 and tp.keys[0] == ("scalar", 1)
    assert tp.representation_spec()[2]["labels"] == "1e+1o"


@pytest.mark.parametrize("parity", ["canonical", "full"])
def test_cpu_forward_and_vjp_match_oracle(parity):
    from ictc_o2_hp import TensorProduct
    torch.manual_seed(1)
    tp = TensorProduct(6, 4, parity=parity)
    plan = O.OraclePlan(6, 4, parity)
    x = torch.randn(9, tp.representation_dimension, requires_grad=True)
    y = torch.randn(9, tp.representation_dimension, requires_grad=True)
    g = torch.randn(9, tp.representation_dimension)
    out = tp(x, y)
    grads = torch.autograd.grad(out, (x, y, tp.weight), g)
    w = tp.weight.detach().double().numpy()
    ref = [O.forward(plan, x.detach().numpy(), y.detach().numpy(), w),
           *O.backward(plan, x.detach().numpy(), y.detach().numpy(), w, g.numpy())]
    for r, a in zip(ref, [out, *grads]):
        assert O.normalized_error(r, a.detach().double().numpy()) < 1e-6


def test_tuple_flat_component_major_and_reference_agree():
    from ictc_o2_hp import (ComponentMajorTensorProduct, ReferenceTensorProduct, TensorProduct,
                            TupleTensorProduct)
    torch.manual_seed(2)
    flat = TensorProduct(5, 3, parity="full")
    tup = TupleTensorProduct(5, 3, parity="full")
    cm = ComponentMajorTensorProduct(5, 3, parity="full")
    ref = ReferenceTensorProduct(5, 3, parity="full")
    for m in (tup, cm):
        m.weight.data.copy_(flat.weight.data)
    flat.copy_weights_to_r5(ref)
    x = torch.randn(4, flat.representation_dimension)
    y = torch.randn(4, flat.representation_dimension)
    out = flat(x, y)
    blocks = lambda v: tuple(v[:, s:s + b.multiplicity * b.irrep_dimension]
                             .reshape(4, b.multiplicity, b.irrep_dimension)
                             for s, b in zip(flat._plan.key_offsets, flat.blocks))
    tup_out = torch.cat([b.reshape(4, -1) for b in tup(blocks(x), blocks(y))], dim=-1)
    ref_out = torch.cat([b.reshape(4, -1) for b in ref(blocks(x), blocks(y))], dim=-1)
    cm_out = cm._unpack(cm(cm._pack(blocks(x)), cm._pack(blocks(y))))
    cm_out = torch.cat([b.reshape(4, -1) for b in cm_out], dim=-1)
    for other in (tup_out, ref_out, cm_out):
        assert torch.allclose(out, other, rtol=1e-5, atol=1e-6)


def test_double_module_uses_fp32_internal_compute_like_reference():
    """native_o2.py:82 / fast_o2.py:87-95: the compute dtype stays float32."""
    from ictc_o2_hp import TensorProduct
    tp = TensorProduct(3, 2, parity="full").double()
    x = torch.randn(2, tp.representation_dimension, dtype=torch.float64)
    out = tp(x, x)
    assert out.dtype == torch.float64
    tp.internal_compute_dtype = torch.float64
    out64 = tp(x, x)
    assert (out - out64).abs().max() > 0


def test_missing_library_raises(monkeypatch, tmp_path):
    from ictc_o2_hp import _native
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setenv("ICTC_O2_HP_AMD_LIBRARY", str(tmp_path / "absent.so"))
    with pytest.raises(_native.NativeLibraryError):
        _native.library()


def _monomial_values(L, pts):
    """x^a y^(L-a) at the points, a = 0..L (the monomial order of the projectors)."""
    return np.stack([pts[:, 0] ** a * pts[:, 1] ** (L - a) for a in range(L + 1)], axis=1)


@pytest.mark.parametrize("L", [0, 1, 2, 5, 8])
def test_harmonic_projectors_split_polynomials_by_frequency(L):
    """build_harmonic_projectors_2d (o2_math.py:140-157): P[(L, m)] has one
    row per frequency-m harmonic, reads back the frequency-m part of
    r^(L-m) * (Re, Im)(x + i y)^m exactly (up to the basis' sign and scale) and
    nothing of the other frequencies, and rotations of the plane act on each
    P[(L, m)] a as norm-preserving maps (checked by refitting rotated
    polynomials from point values)."""
    from ictc_o2_hp import o2_math
    proj = o2_math.build_harmonic_projectors_2d(L)
    ms = [L - 2 * k for k in range(L // 2 + 1)]
    assert proj.Lmax == L and set(proj.P) == {(l, l - 2 * k) for l in range(L + 1)
                                             for k in range(l // 2 + 1)}
    rng = np.random.default_rng(L)
    pts = rng.standard_normal((4 * (L + 1), 2))
    mono = _monomial_values(L, pts)
    r2 = (pts ** 2).sum(axis=1)
    z = pts[:, 0] + 1j * pts[:, 1]
    for m in ms:
        P = proj.P[(L, m)].numpy()
        assert P.shape == (o2_math.so2_irrep_dim(m), L + 1) and P.dtype == np.float64
        for m2 in ms:
            parts = [np.real(z ** m2)] + ([np.imag(z ** m2)] if m2 > 0 else [])
            for part in parts:
                values = r2 ** ((L - m2) // 2) * part
                coeffs = np.linalg.lstsq(mono, values, rcond=None)[0]
                got = P @ coeffs
                if m2 != m:
                    assert np.abs(got).max() < 1e-9 * max(1.0, np.abs(coeffs).max())
                else:
                    assert np.abs(got).max() > 1e-6
    # Rotation by t: p(R^-1 v) has the same frequency-m norm as p.
    a = rng.standard_normal(L + 1)
    t = 0.7
    rot = np.array([[np.cos(t), np.sin(t)], [-np.sin(t), np.cos(t)]])
    rotated = np.linalg.lstsq(mono, _monomial_values(L, pts @ rot.T) @ a, rcond=None)[0]
    for m in ms:
        P = proj.P[(L, m)].numpy()
        assert abs(np.linalg.norm(P @ rotated) - np.linalg.norm(P @ a)) < 1e-8 * (1 + np.linalg.norm(P @ a))


def test_harmonic_projectors_planted_mistake_is_caught():
    """A projector built with the identity instead of the Gaussian Gram matrix
    mixes frequencies: its frequency-0 row of degree 4 sees Re (x + i y)^4."""
    from ictc_o2_hp import o2_math
    L, m = 4, 0
    lifted = o2_math._radial_lift(m, 2) @ o2_math._harmonic_basis(m)
    wrong = np.linalg.solve(lifted.T @ lifted, lifted.T)
    pts = np.random.default_rng(1).standard_normal((20, 2))
    z = pts[:, 0] + 1j * pts[:, 1]
    coeffs = np.linalg.lstsq(_monomial_values(L, pts), np.real(z ** 4), rcond=None)[0]
    assert np.abs(o2_math.build_harmonic_projectors_2d(L).P[(L, m)].numpy() @ coeffs).max() < 1e-9
    assert np.abs(wrong @ coeffs).max() > 1e-3


def test_o2_math_public_functions():
    from ictc_o2_hp import o2_math
    assert o2_math.o2_valid_output_keys("2", "2") == [("scalar", 1), ("scalar", -1), ("freq", 4)]
    assert o2_math.o2_valid_output_keys("0o", "3") == [("freq", 3)]
    cg = o2_math.o2_cg_tensor("0o", "1", "1")
    assert torch.equal(cg[0], torch.tensor([[0.0, 1.0], [-1.0, 0.0]], dtype=torch.float64))
    g = torch.tensor([[0.0, -1.0], [1.0, 0.0]], dtype=torch.float64)
    rep = o2_math.o2_representation(g, "2")
    assert torch.allclose(rep, torch.tensor([[-1.0, 0.0], [0.0, -1.0]], dtype=torch.float64),
                          atol=1e-12)
    with pytest.raises(ValueError):
        o2_math.o2_cg_tensor("0x", "1", "1")


# The reference's op schemas, written out from its signatures
# (triton_o2.py:786-794, :878-887; uvu_triton.py:267-284, :391-414;
# radial_streamed.py:81-115).  Namespaces: triton_o2.py:22, uvu_triton.py:12.
_REFERENCE_SCHEMAS = {
    ("ictc_o2_hp_v0_1_6_dev0", "o2_forward"):
        "(Tensor left, Tensor right, Tensor weight, Tensor path_info, "
        "Tensor path_coefficients, SymInt metadata_id) -> Tensor",
    ("ictc_o2_hp_v0_1_6_dev0", "o2_backward"):
        "(Tensor left, Tensor right, Tensor weight, Tensor grad_output, Tensor path_info, "
        "Tensor path_coefficients, SymInt metadata_id) -> (Tensor, Tensor, Tensor)",
    ("ictc_o2_hp_v0_1_6_dev0_uvu", "forward"):
        "(Tensor left, Tensor right, Tensor weight, Tensor info, Tensor coefficients, "
        "Tensor first_order, Tensor second_order, SymInt metadata_id, bool shared) -> Tensor",
    ("ictc_o2_hp_v0_1_6_dev0_uvu", "forward_into"):
        "(Tensor left, Tensor right, Tensor weight, Tensor info, Tensor coefficients, "
        "Tensor first_order, Tensor second_order, SymInt metadata_id, bool shared, "
        "Tensor(a9!) result) -> ()",
    ("ictc_o2_hp_v0_1_6_dev0_uvu", "backward"):
        "(Tensor left, Tensor right, Tensor weight, Tensor grad_output, Tensor info, "
        "Tensor coefficients, Tensor first_order, Tensor second_order, SymInt metadata_id, "
        "bool shared, SymInt needed=7) -> (Tensor, Tensor, Tensor)",
    ("ictc_o2_hp_v0_1_6_dev0_uvu", "backward_into"):
        "(Tensor left, Tensor right, Tensor weight, Tensor grad_output, Tensor info, "
        "Tensor coefficients, Tensor first_order, Tensor second_order, SymInt metadata_id, "
        "bool shared, SymInt needed, Tensor(a11!) gx, Tensor(a12!) gy, Tensor(a13!) gw) -> ()",
    ("ictc_o2_hp_v0_1_6_dev0_uvu", "radial_stream_forward"):
        "(Tensor left, Tensor angular, Tensor radial, Tensor alpha, Tensor bias, Tensor info, "
        "Tensor coefficients, Tensor first_order, Tensor second_order, SymInt metadata_id, "
        "bool has_bias, bool save_first) -> (Tensor, Tensor)",
    ("ictc_o2_hp_v0_1_6_dev0_uvu", "radial_stream_backward"):
        "(Tensor left, Tensor angular, Tensor radial, Tensor alpha, Tensor bias, "
        "Tensor cached_weights, Tensor grad_output, Tensor info, Tensor coefficients, "
        "Tensor first_order, Tensor second_order, SymInt metadata_id, bool has_bias, "
        "SymInt needed=31) -> (Tensor, Tensor, Tensor, Tensor, Tensor)",
}


@pytest.mark.parametrize("namespace,name", sorted(_REFERENCE_SCHEMAS))
def test_ops_resolve_under_reference_namespaces(namespace, name):
    """Callers and compiled graphs name the reference's versioned ops."""
    import ictc_o2_hp
    from ictc_o2_hp import ops, radial_ops, uvu_ops  # noqa: F401  (registration)
    assert ictc_o2_hp.__version__.replace(".", "_") == "0_1_6_dev0"
    op = getattr(getattr(torch.ops, namespace), name).default
    schema = str(op._schema)
    assert schema == f"{namespace}::{name}{_REFERENCE_SCHEMAS[(namespace, name)]}"


@pytest.mark.parametrize("parity", ["canonical", "full"])
def test_apply_full_parity_o2_is_a_symmetry_of_the_product(parity):
    """f(g x, g y) = g f(x, y) for rotations and reflections, with g acting
    through apply_full_parity_o2 in the public copy bases.  A missing det(g)
    factor on copy 1 or a transposed representation matrix breaks it."""
    from ictc_o2_hp import ReferenceTensorProduct
    from ictc_o2_hp.native_o2 import apply_full_parity_o2
    torch.manual_seed(9)
    tp = ReferenceTensorProduct(3, 3, parity=parity).double()
    tp.internal_compute_dtype = torch.float64
    blocks = lambda: tuple(torch.randn(5, b.multiplicity, b.irrep_dimension, dtype=torch.float64)
                           for b in tp.blocks)
    x, y = blocks(), blocks()
    for angle, reflect in ((0.7, False), (2.1, True)):
        c, s = np.cos(angle), np.sin(angle)
        g = torch.tensor([[c, -s], [s, c]], dtype=torch.float64)
        if reflect:
            g = g @ torch.tensor([[1.0, 0.0], [0.0, -1.0]], dtype=torch.float64)
        lhs = tp(apply_full_parity_o2(tp, x, g), apply_full_parity_o2(tp, y, g))
        rhs = apply_full_parity_o2(tp, tp(x, y), g)
        for a, b in zip(lhs, rhs):
            assert torch.allclose(a, b, atol=1e-12)
    # The action of a reflection is not the identity on odd blocks.
    moved = apply_full_parity_o2(tp, x, torch.diag(torch.tensor([1.0, -1.0], dtype=torch.float64)))
    assert any(not torch.allclose(a, b) for a, b in zip(moved, x))


# ---- fixtures recorded from the reference (tests/golden/make_layouts_and_state.py)

def _layout_cases():
    data = np.load(GOLDEN / "layout_vectors.npz")
    for name in sorted({k.split("/")[0] for k in data.files}):
        c, m, parity, norm = name.split("_")
        yield name, int(c[1:]), int(m[1:]), parity, norm, {k.split("/")[1]: data[k]
                                                            for k in data.files
                                                            if k.startswith(name + "/")}


def test_oracle_component_major_layouts_match_reference_vectors():
    """oracle layouts 1 / 2 (component-major) against the reference's
    component-major product (triton_o2.py:1204-1278 CPU path, fp64)."""
    for name, c, m, parity, norm, v in _layout_cases():
        plan = O.OraclePlan(c, m, parity, norm)
        layout = 1 if parity == "canonical" else 2
        out = O.forward(plan, v["x"], v["y"], v["weight"], layout)
        dx, dy, dw = O.backward(plan, v["x"], v["y"], v["weight"], v["g"], layout)
        for ref, got in ((v["out"], out), (v["dx"], dx), (v["dy"], dy), (v["dw"], dw)):
            assert O.normalized_error(ref, got) < 1e-12, name


def test_component_major_module_matches_reference_vectors():
    """ComponentMajorTensorProduct's CPU path in fp64 against the same vectors;
    _unpack / _pack against the reference's storage order."""
    from ictc_o2_hp import ComponentMajorTensorProduct, TensorProduct
    for name, c, m, parity, norm, v in _layout_cases():
        module = ComponentMajorTensorProduct(c, m, parity=parity, normalization=norm).double()
        module.internal_compute_dtype = torch.float64
        with torch.no_grad():
            module.weight.copy_(torch.from_numpy(v["weight"]))
        x = torch.from_numpy(v["x"]).requires_grad_()
        y = torch.from_numpy(v["y"]).requires_grad_()
        out = module(x, y)
        grads = torch.autograd.grad(out, (x, y, module.weight), torch.from_numpy(v["g"]))
        for ref, got in zip((v["out"], v["dx"], v["dy"], v["dw"]), (out, *grads)):
            assert O.normalized_error(ref, got.detach().numpy()) < 1e-12, name
        # Tuple round trip: the channel-major product on unpacked blocks, packed back.
        flat = TensorProduct(c, m, parity=parity, normalization=norm).double()
        flat.internal_compute_dtype = torch.float64
        with torch.no_grad():
            flat.weight.copy_(module.weight)
        from ictc_o2_hp.native_o2 import _split_blocks
        xb, yb = module._unpack(x.detach()), module._unpack(y.detach())
        cat = lambda blocks: torch.cat([b.reshape(b.shape[0], -1) for b in blocks], dim=-1)
        with torch.no_grad():
            packed = module._pack(_split_blocks(flat(cat(xb), cat(yb)), flat._plan))
        assert O.normalized_error(v["out"], packed.numpy()) < 1e-12, name


_STATE_MODULES = {
    "TensorProduct_c3_m2_full": lambda I: I.TensorProduct(3, 2, parity="full"),
    "TensorProduct_c4_m3_canonical_norm": lambda I: I.TensorProduct(
        4, 3, parity="canonical", normalization="norm"),
    "TupleTensorProduct_c3_m2_full": lambda I: I.TupleTensorProduct(3, 2, parity="full"),
    "ComponentMajorTensorProduct_c3_m2_canonical": lambda I: I.ComponentMajorTensorProduct(
        3, 2, parity="canonical"),
    "ReferenceTensorProduct_c3_m2_full": lambda I: I.ReferenceTensorProduct(3, 2, parity="full"),
    "UvuTensorProduct_c3_v2_m2_full_shared": lambda I: I.UvuTensorProduct(3, 2, 2, parity="full"),
    "UvuTensorProduct_c4_v1_m2_canonical_external": lambda I: I.UvuTensorProduct(
        4, 1, 2, parity="canonical", shared_weights=False),
    "ReferenceUvuTensorProduct_c2_v3_m1_full": lambda I: I.ReferenceUvuTensorProduct(
        2, 3, 1, parity="full"),
    "RadialUvuTensorProduct_c4_m2_canonical_h8": lambda I: I.RadialUvuTensorProduct(
        I.UvuTensorProduct(4, 1, 2, parity="canonical", shared_weights=False),
        torch.nn.Linear(8, I.UvuTensorProduct(4, 1, 2, parity="canonical",
                                              shared_weights=False).weight_numel)),
}


@pytest.mark.parametrize("name", sorted(_STATE_MODULES))
def test_state_dict_matches_reference_record(name):
    """Keys, shapes and dtypes of every state-dict entry equal the reference's
    (recorded from its modules), so checkpoints load strictly both ways."""
    import json
    import ictc_o2_hp
    records = json.loads((GOLDEN / "state_dicts.json").read_text())
    module = _STATE_MODULES[name](ictc_o2_hp)
    mine = [[k, list(v.shape), str(v.dtype).replace("torch.", "")]
            for k, v in module.state_dict().items()]
    assert mine == records[name]


@pytest.mark.parametrize("name", ["TensorProduct_c3_m2_full",
                                  "ComponentMajorTensorProduct_c3_m2_canonical",
                                  "UvuTensorProduct_c3_v2_m2_full_shared"])
def test_reference_checkpoint_loads_and_reproduces_its_outputs(name):
    import ictc_o2_hp
    data = np.load(GOLDEN / "state_dict_values.npz")
    prefix = f"{name}/state/"
    state = {k[len(prefix):]: torch.from_numpy(data[k]) for k in data.files
             if k.startswith(prefix)}
    module = _STATE_MODULES[name](ictc_o2_hp)
    module.load_state_dict(state, strict=True)
    with torch.no_grad():
        out = module(torch.from_numpy(data[f"{name}/x"]), torch.from_numpy(data[f"{name}/y"]))
    assert O.normalized_error(data[f"{name}/out"].astype(np.float64),
                              out.double().numpy()) < 1e-6
