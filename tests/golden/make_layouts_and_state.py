"""Write the component-major layout vectors and the state-dict records under
tests/golden/ from the reference's own classes.

Run in the build container only (the reference is not present on GPU boxes):

    python tests/golden/make_layouts_and_state.py /root/reference

* ``layout_vectors.npz``: fp64 inputs with out, dx, dy, dw of the reference's
  component-major product (``triton_o2.XuLayoutTritonPathWeightedTensorProductO2``,
  the class behind ``api.ComponentMajorTensorProduct``), canonical (layout 1)
  and full parity (layout 2).  On the CPU that class evaluates its PyTorch
  path (``triton_o2.py:1260-1278``: ``_unpack`` -> tuple algebra -> ``_pack``);
  no Triton kernel runs.  It is built with ``internal_compute_dtype=float64``
  so the vectors are exact to fp64 rounding.
* ``state_dicts.json``: key, shape and dtype of every state-dict entry of the
  public modules, and ``state_dict_values.npz`` the values of a
  ``TensorProduct`` / ``ComponentMajorTensorProduct`` / ``UvuTensorProduct``
  checkpoint with the outputs those reference modules give on stored inputs.

The fixtures are data only; nothing of the reference's source is stored.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent

LAYOUT_CASES = (
    # name, C, m_max, parity, normalization, rows
    ("c3_m2_canonical_component", 3, 2, "canonical", "component", 5),
    ("c5_m3_canonical_norm", 5, 3, "canonical", "norm", 4),
    ("c3_m2_full_component", 3, 2, "full", "component", 5),
    ("c4_m3_full_norm", 4, 3, "full", "norm", 3),
)


def _import_reference(root: str):
    sys.path.insert(0, str(Path(root) / "src"))
    import ictc_o2_hp  # noqa: E402
    if "reference" not in str(Path(ictc_o2_hp.__file__).resolve()):
        raise SystemExit("refusing to run: ictc_o2_hp did not resolve to the reference tree")
    from ictc_o2_hp import api, o2_math, reference, triton_o2, uvu_o2  # noqa: E402
    from ictc_o2_hp import radial_uvu  # noqa: E402
    return api, o2_math, reference, triton_o2, uvu_o2, radial_uvu


def layout_vectors(o2_math, triton_o2):
    arrays = {}
    rng = np.random.default_rng(20261202)
    for name, channels, m_max, parity, normalization, rows in LAYOUT_CASES:
        module = triton_o2.XuLayoutTritonPathWeightedTensorProductO2(
            o2_math, channels, m_max, parity=parity, normalization=normalization,
            internal_compute_dtype=torch.float64).double()
        width = module.representation_dimension
        x, y, g = (rng.standard_normal((rows, width)) for _ in range(3))
        weight = rng.standard_normal(module.weight.numel())
        with torch.no_grad():
            module.weight.copy_(torch.from_numpy(weight))
        xt = torch.from_numpy(x).requires_grad_()
        yt = torch.from_numpy(y).requires_grad_()
        out = module(xt, yt)
        dx, dy, dw = torch.autograd.grad(out, (xt, yt, module.weight), torch.from_numpy(g))
        for key, value in (("x", x), ("y", y), ("g", g), ("weight", weight),
                           ("out", out.detach()), ("dx", dx), ("dy", dy), ("dw", dw)):
            arrays[f"{name}/{key}"] = np.asarray(value)
    np.savez_compressed(OUT / "layout_vectors.npz", **arrays)


def _describe(module):
    return [[key, list(value.shape), str(value.dtype).replace("torch.", "")]
            for key, value in module.state_dict().items()]


def state_dicts(api, reference, uvu_o2, radial_uvu):
    torch.manual_seed(0)
    modules = {
        "TensorProduct_c3_m2_full": api.TensorProduct(3, 2, parity="full"),
        "TensorProduct_c4_m3_canonical_norm": api.TensorProduct(
            4, 3, parity="canonical", normalization="norm"),
        "TupleTensorProduct_c3_m2_full": api.TupleTensorProduct(3, 2, parity="full"),
        "ComponentMajorTensorProduct_c3_m2_canonical": api.ComponentMajorTensorProduct(
            3, 2, parity="canonical"),
        "ReferenceTensorProduct_c3_m2_full": reference.ReferenceTensorProduct(3, 2, parity="full"),
        "UvuTensorProduct_c3_v2_m2_full_shared": uvu_o2.UvuTensorProduct(3, 2, 2, parity="full"),
        "UvuTensorProduct_c4_v1_m2_canonical_external": uvu_o2.UvuTensorProduct(
            4, 1, 2, parity="canonical", shared_weights=False),
        "ReferenceUvuTensorProduct_c2_v3_m1_full": uvu_o2.ReferenceUvuTensorProduct(
            2, 3, 1, parity="full"),
    }
    tp = uvu_o2.UvuTensorProduct(4, 1, 2, parity="canonical", shared_weights=False)
    modules["RadialUvuTensorProduct_c4_m2_canonical_h8"] = radial_uvu.RadialUvuTensorProduct(
        tp, torch.nn.Linear(8, tp.weight_numel))
    records = {name: _describe(module) for name, module in modules.items()}
    (OUT / "state_dicts.json").write_text(json.dumps(records, indent=1))

    # Checkpoint values and the outputs the reference modules give with them.
    arrays = {}
    rng = np.random.default_rng(20261203)
    for name in ("TensorProduct_c3_m2_full", "ComponentMajorTensorProduct_c3_m2_canonical",
                 "UvuTensorProduct_c3_v2_m2_full_shared"):
        module = modules[name]
        for key, value in module.state_dict().items():
            arrays[f"{name}/state/{key}"] = value.detach().numpy().copy()
        if name.startswith("Uvu"):
            x = rng.standard_normal((4, module.input1_dimension)).astype(np.float32)
            y = rng.standard_normal((4, module.input2_dimension)).astype(np.float32)
        else:
            x, y = (rng.standard_normal((4, module.representation_dimension)).astype(np.float32)
                    for _ in range(2))
        with torch.no_grad():
            out = module(torch.from_numpy(x), torch.from_numpy(y))
        arrays[f"{name}/x"], arrays[f"{name}/y"] = x, y
        arrays[f"{name}/out"] = out.numpy()
    np.savez_compressed(OUT / "state_dict_values.npz", **arrays)


def main():
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    torch.set_default_dtype(torch.float32)
    api, o2_math, reference, triton_o2, uvu_o2, radial_uvu = _import_reference(root)
    layout_vectors(o2_math, triton_o2)
    state_dicts(api, reference, uvu_o2, radial_uvu)
    print("layout vectors and state-dict records written to", OUT)


if __name__ == "__main__":
    main()
