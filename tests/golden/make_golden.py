"""Write the golden fixtures under tests/golden/ from the reference's own code.

Run in the build container only (the reference is not present on GPU boxes):

    python tests/golden/make_golden.py /root/reference

It imports the reference's pure-PyTorch modules (``o2_math``, ``native_o2``,
``fast_o2``, ``uvu_o2``) -- never its Triton modules -- and records what the
mathematical checks in tests/ cannot pin on their own:

* ``cg_tables.json``: per (m_max, parity, normalization) the path list, the
  sparse coupling terms and the packed weight offsets, exactly as
  ``fast_o2.FastPathWeightedTensorProductO2`` extracts them (the per-path sign
  conventions are only fixed by the reference's basis choices);
* ``default_weights.npz``: the default-initialised packed ``weight`` under
  ``torch.manual_seed(0)`` (pins the per-path randn order of ``native_o2.py:117``);
* ``tp_vectors.npz``: small fp64 inputs with out, dx, dy, dw from the
  reference's einsum algebra (``native_o2.py:183-221``) run in float64;
* ``uvu_tables.json`` / ``uvu_vectors.npz``: uvu plans (paths, padded
  coefficients) and small fp64 forward/VJP vectors from
  ``uvu_o2.ReferenceUvuTensorProduct``.

The fixtures are data only; nothing of the reference's source is stored.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent


def _import_reference(root: str):
    sys.path.insert(0, str(Path(root) / "src"))
    from ictc_o2_hp import o2_math, native_o2, fast_o2, uvu_o2  # noqa: E402
    if "reference" not in str(Path(o2_math.__file__).resolve()):
        raise SystemExit("refusing to run: ictc_o2_hp did not resolve to the reference tree")
    return o2_math, native_o2, fast_o2, uvu_o2


def _key_token(key):
    if key[0] == "scalar":
        return "0e" if key[1] == 1 else "0o"
    return str(key[1])


def cg_tables(o2_math, fast_o2):
    tables = {}
    for m_max in range(0, 9):
        for parity in ("canonical", "full"):
            for normalization in ("component", "norm"):
                module = fast_o2.PackedFastPathWeightedTensorProductO2(
                    o2_math, 1, m_max, parity=parity, normalization=normalization)
                tables[f"{m_max}/{parity}/{normalization}"] = {
                    "paths": [[_key_token(k) for k in path] for path in module.paths],
                    "terms": [[[list(t) for t in comp] for comp in path]
                              for path in module._sparse_cg],
                    "weight_offsets": [list(o) for o in module._weight_offsets],
                    "width": module.representation_dimension,
                }
    (OUT / "cg_tables.json").write_text(json.dumps(tables))


def default_weights(o2_math, fast_o2):
    arrays = {}
    for channels, m_max, parity in ((32, 2, "canonical"), (17, 3, "full"), (128, 6, "full")):
        torch.manual_seed(0)
        module = fast_o2.PackedFastPathWeightedTensorProductO2(
            o2_math, channels, m_max, parity=parity)
        arrays[f"C{channels}_m{m_max}_{parity}"] = module.weight.detach().numpy().copy()
    np.savez_compressed(OUT / "default_weights.npz", **arrays)


TP_CASES = (
    # name, C, m_max, parity, normalization, rows
    ("c32_m2_canonical_component", 32, 2, "canonical", "component", 8),
    ("c17_m3_full_component", 17, 3, "full", "component", 6),
    ("c4_m6_full_norm", 4, 6, "full", "norm", 5),
    ("c3_m1_canonical_norm", 3, 1, "canonical", "norm", 4),
    ("c2_m0_full_component", 2, 0, "full", "component", 3),
    ("c5_m4_canonical_component", 5, 4, "canonical", "component", 4),
)


def tp_vectors(o2_math, native_o2):
    arrays = {}
    rng = np.random.default_rng(20260601)
    for name, channels, m_max, parity, normalization, rows in TP_CASES:
        module = native_o2.FullParityPathWeightedTensorProductO2(
            o2_math, channels, m_max, parity=parity, normalization=normalization,
            internal_compute_dtype=torch.float64).double()
        width = module.representation_dimension
        x = rng.standard_normal((rows, width))
        y = rng.standard_normal((rows, width))
        g = rng.standard_normal((rows, width))
        weight = rng.standard_normal(sum(p.numel() for p in module.weights))
        with torch.no_grad():
            cursor = 0
            for parameter in module.weights:
                parameter.copy_(torch.from_numpy(weight[cursor:cursor + parameter.numel()]))
                cursor += parameter.numel()

        def split(flat):
            parts, start = [], 0
            for block in module.blocks:
                size = block.multiplicity * block.irrep_dimension
                parts.append(flat[:, start:start + size].reshape(
                    rows, block.multiplicity, block.irrep_dimension))
                start += size
            return tuple(parts)

        xt = torch.from_numpy(x).requires_grad_()
        yt = torch.from_numpy(y).requires_grad_()
        out_blocks = module(split(xt), split(yt))
        out = torch.cat([b.reshape(rows, -1) for b in out_blocks], dim=-1)
        grads = torch.autograd.grad(out, (xt, yt, *module.weights), torch.from_numpy(g))
        arrays[f"{name}/x"] = x
        arrays[f"{name}/y"] = y
        arrays[f"{name}/g"] = g
        arrays[f"{name}/weight"] = weight
        arrays[f"{name}/out"] = out.detach().numpy()
        arrays[f"{name}/dx"] = grads[0].numpy()
        arrays[f"{name}/dy"] = grads[1].numpy()
        arrays[f"{name}/dw"] = torch.cat([d.reshape(-1) for d in grads[2:]]).numpy()
    np.savez_compressed(OUT / "tp_vectors.npz", **arrays)


UVU_CASES = (
    # name, C, V, m_max, kwargs, shared, rows
    ("c3_v2_m2_full", 3, 2, 2, {"parity": "full"}, True, 4),
    ("c4_v1_m4_canonical", 4, 1, 4, {"parity": "canonical"}, False, 5),
    ("c3_v1_m6_full_in2canonical", 3, 1, 6,
     {"parity": "full", "parity_in2": "canonical"}, False, 3),
    ("c2_v3_m3_canonical_in2full_m2_path", 2, 3, 3,
     {"parity": "canonical", "parity_in2": "full", "m_max_in2": 2,
      "path_normalization": "path"}, False, 4),
    ("c2_v2_m1_full_norm_element", 2, 2, 1,
     {"parity": "full", "normalization": "norm", "path_normalization": "element"}, True, 3),
)

UVU_PLANS = (
    ("c128_v32_m4_full", 128, 32, 4, {"parity": "full"}),
    ("c64_v1_m4_canonical", 64, 1, 4, {"parity": "canonical"}),
    ("c128_v1_m6_full_in2canonical", 128, 1, 6, {"parity": "full", "parity_in2": "canonical"}),
)


def _uvu_entry(entry):
    return [_key_token(entry.key), entry.copy, entry.offset, entry.dim]


def uvu_tables_and_vectors(uvu_o2):
    tables = {}
    for name, channels, v, m_max, kwargs in UVU_PLANS + tuple(c[:5] for c in UVU_CASES):
        module = uvu_o2.ReferenceUvuTensorProduct(channels, v, m_max, shared_weights=True,
                                                  **kwargs)
        tables[name] = {
            "paths": [list(p) for p in module.paths],
            "coefficients": [list(row) for row in module._coefficient_values],
            "entries_in1": [_uvu_entry(e) for e in module.entries_in1],
            "entries_in2": [_uvu_entry(e) for e in module.entries_in2],
            "input1_dimension": module.input1_dimension,
            "input2_dimension": module.input2_dimension,
            "weight_numel": module.weight_numel,
        }
    (OUT / "uvu_tables.json").write_text(json.dumps(tables))

    arrays = {}
    rng = np.random.default_rng(20260602)
    for name, channels, v, m_max, kwargs, shared, rows in UVU_CASES:
        module = uvu_o2.ReferenceUvuTensorProduct(
            channels, v, m_max, shared_weights=shared, internal_weights=False,
            **kwargs).double()
        x = rng.standard_normal((rows, module.input1_dimension))
        y = rng.standard_normal((rows, module.input2_dimension))
        g = rng.standard_normal((rows, module.input1_dimension))
        wshape = (module.weight_numel,) if shared else (rows, module.weight_numel)
        w = rng.standard_normal(wshape)
        xt, yt, wt = (torch.from_numpy(a).requires_grad_() for a in (x, y, w))
        out = module(xt, yt, wt)
        dx, dy, dw = torch.autograd.grad(out, (xt, yt, wt), torch.from_numpy(g))
        for key, value in (("x", x), ("y", y), ("g", g), ("w", w), ("out", out.detach()),
                           ("dx", dx), ("dy", dy), ("dw", dw)):
            arrays[f"{name}/{key}"] = np.asarray(value)
    np.savez_compressed(OUT / "uvu_vectors.npz", **arrays)


def main():
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    torch.set_default_dtype(torch.float32)
    o2_math, native_o2, fast_o2, uvu_o2 = _import_reference(root)
    cg_tables(o2_math, fast_o2)
    default_weights(o2_math, fast_o2)
    tp_vectors(o2_math, native_o2)
    uvu_tables_and_vectors(uvu_o2)
    print("golden fixtures written to", OUT)


if __name__ == "__main__":
    main()
