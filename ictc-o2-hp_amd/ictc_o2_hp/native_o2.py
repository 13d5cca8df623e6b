"""Path-weighted O(2) tensor-product modules (tuple, packed, flat layouts).

Module surface of Parity-LRX/ICTC-O2-HP:

* ``FullParityPathWeightedTensorProductO2``: one parameter per path, the
  original einsum algebra (``native_o2.py:64-221``);
* ``PackedPathWeightedTensorProductO2``: the same paths with one flat
  ``weight`` and ``copy_weights_to_r5`` / ``load_weights_from_r5``
  (``fast_o2.py:152-186``);
* ``FlatPathWeightedTensorProductO2`` / ``ComponentMajorPathWeightedTensorProductO2``:
  flat channel-major / component-major rows (``triton_o2.py:1169-1278``).

State-dict keys and shapes match the reference: ``weight`` (or
``weights.<p>``), ``cg_<p>`` and ``odd_to_even`` / ``even_to_odd`` persistent;
routing and kernel metadata non-persistent.  CUDA float32 inputs on the
weight's device run the gfx950 kernels; other devices and dtypes run the
PyTorch algebra, as in the reference (``triton_o2.py:1134-1143``).
"""
from __future__ import annotations

from typing import Any, Iterable

import torch

from . import ops
from .plan import (RepresentationBlock, TPPlan, canonical_blocks,  # noqa: F401
                   full_parity_blocks)
from .torch_algebra import flat_forward

O2Key = tuple

_J = ((0.0, -1.0), (1.0, 0.0))


class FullParityPathWeightedTensorProductO2(torch.nn.Module):
    """Depthwise path-weighted O(2) product with cyclic channel/copy routing."""

    def __init__(self, o2_module: Any, channels: int, max_frequency: int, *,
                 parity: str = "full", normalization: str = "component",
                 internal_compute_dtype: torch.dtype = torch.float32) -> None:
        super().__init__()
        self.o2 = o2_module
        self.channels = int(channels)
        self.max_frequency = int(max_frequency)
        if parity not in ("canonical", "full"):
            raise ValueError(parity)
        self.parity = parity
        self.normalization = normalization
        self.internal_compute_dtype = internal_compute_dtype
        self._plan = TPPlan(self.channels, self.max_frequency, parity, normalization)
        self.blocks = self._plan.blocks
        self.keys = self._plan.keys
        self.block_by_key = self._plan.block_by_key
        self.paths = self._plan.paths

        self.weights = torch.nn.ParameterList()
        self._cg_names, self._index_names = [], []
        for p, (key1, key2, key3) in enumerate(self.paths):
            out_mul = self.block_by_key[key3].multiplicity
            in1 = self.block_by_key[key1].multiplicity
            in2 = self.block_by_key[key2].multiplicity
            # Same draw order as the reference: one randn(out_mul) per path.
            self.weights.append(torch.nn.Parameter(torch.randn(out_mul) * 0.02))
            self.register_buffer(f"cg_{p}", torch.from_numpy(self._plan.cg[p].copy()),
                                 persistent=True)
            self.register_buffer(f"input1_index_{p}", torch.arange(out_mul) % in1,
                                 persistent=False)
            self.register_buffer(f"input2_index_{p}", torch.arange(out_mul) % in2,
                                 persistent=False)
            self._cg_names.append(f"cg_{p}")
            self._index_names.append((f"input1_index_{p}", f"input2_index_{p}"))
        j = torch.tensor(_J, dtype=torch.float64)
        self.register_buffer("odd_to_even", j.transpose(0, 1).contiguous(), persistent=True)
        self.register_buffer("even_to_odd", j.contiguous(), persistent=True)

    @property
    def representation_dimension(self) -> int:
        return sum(b.multiplicity * b.irrep_dimension for b in self.blocks)

    @property
    def parameter_count(self) -> int:
        return sum(p.numel() for p in self.parameters())

    def representation_spec(self):
        rows = []
        for b in self.blocks:
            if b.frequency == 0:
                labels = b.token
            else:
                labels = str(b.frequency) if self.parity == "canonical" else \
                    f"{b.frequency}e+{b.frequency}o"
            rows.append({"labels": labels, "frequency": b.frequency,
                         "irrep_dimension": b.irrep_dimension,
                         "multiplicity": b.multiplicity, "parity_copies": b.parity_copies})
        return rows

    def _twist(self, key, value, matrix):
        if key[0] != "freq" or self.parity == "canonical":
            return value
        even, odd = value.split(self.channels, dim=-2)
        t = matrix.to(device=value.device, dtype=value.dtype)
        return torch.cat((even, torch.einsum("...ci,ij->...cj", odd, t)), dim=-2)

    def forward(self, left, right):
        """Original einsum algebra (``native_o2.py:183-221``)."""
        if len(left) != len(self.keys) or len(right) != len(self.keys):
            raise ValueError("one tensor per representation block is required")
        lhs = {k: self._twist(k, v, self.odd_to_even) for k, v in zip(self.keys, left)}
        rhs = {k: self._twist(k, v, self.odd_to_even) for k, v in zip(self.keys, right)}
        sample = left[0]
        out = {b.key: torch.zeros(*sample.shape[:-2], b.multiplicity, b.irrep_dimension,
                                  dtype=sample.dtype, device=sample.device)
               for b in self.blocks}
        dtype = self.internal_compute_dtype
        for p, (key1, key2, key3) in enumerate(self.paths):
            i1, i2 = (getattr(self, n) for n in self._index_names[p])
            a = lhs[key1].index_select(-2, i1).to(dtype)
            b = rhs[key2].index_select(-2, i2).to(dtype)
            cg = getattr(self, self._cg_names[p]).to(device=sample.device, dtype=dtype)
            value = torch.einsum("...om,...on,mnk,o->...ok", a, b, cg,
                                 self._path_weight(p).to(dtype))
            out[key3] = out[key3] + value.to(sample.dtype)
        return tuple(self._twist(k, out[k], self.even_to_odd) for k in self.keys)

    def _path_weight(self, p: int) -> torch.Tensor:
        return self.weights[p]


def _path_metadata(plan: TPPlan, layout: int):
    """int32 [P, 25] / f32 [P, 4] path metadata of ``runtime_weight.py:14-29``."""
    keys = plan.key_spec(layout)
    rows, coefficients = [], []
    for path in plan.table:
        row = []
        for key in (path.key1, path.key2, path.key3):
            row.extend(keys[key][:4])
        row.append(path.weight_start)
        terms = list(path.terms) + [None] * (4 - len(path.terms))
        for term in terms:
            row.extend((term.i, term.j, term.k) if term else (0, 0, 0))
        rows.append(row)
        coefficients.append([term.coefficient if term else 0.0 for term in terms])
    return (torch.tensor(rows, dtype=torch.int32),
            torch.tensor(coefficients, dtype=torch.float32))


class PackedPathWeightedTensorProductO2(FullParityPathWeightedTensorProductO2):
    """Same paths with all weights in one flat parameter ``weight``."""

    _layout = 0

    def __init__(self, *args, **kwargs) -> None:
        super().__init__(*args, **kwargs)
        self._weight_offsets = self._plan.weight_offsets
        initial = [p.detach() for p in self.weights]
        del self.weights
        self.weight = torch.nn.Parameter(torch.cat(initial))
        info, coefficients = _path_metadata(self._plan, self._layout)
        self.register_buffer("_weight_path_info", info, persistent=False)
        self.register_buffer("_weight_path_coefficients", coefficients, persistent=False)
        self._metadata_id = ops.register(self._plan, self._layout)

    def _path_weight(self, p: int) -> torch.Tensor:
        start, end = self._weight_offsets[p]
        return self.weight[start:end]

    def copy_weights_to_r5(self, reference: FullParityPathWeightedTensorProductO2) -> None:
        """Copy the packed weight into a per-path reference module (``fast_o2.py:173-178``)."""
        if len(reference.weights) != len(self._weight_offsets):
            raise ValueError("r5 path count differs")
        with torch.no_grad():
            for parameter, (start, end) in zip(reference.weights, self._weight_offsets):
                parameter.copy_(self.weight[start:end])

    def load_weights_from_r5(self, reference: FullParityPathWeightedTensorProductO2) -> None:
        """Copy per-path reference weights into ``weight`` (``fast_o2.py:180-186``)."""
        if len(reference.weights) != len(self._weight_offsets):
            raise ValueError("r5 path count differs")
        with torch.no_grad():
            for parameter, (start, end) in zip(reference.weights, self._weight_offsets):
                self.weight[start:end].copy_(parameter)

    # ---- dispatch -------------------------------------------------------------
    def _on_kernels(self, *tensors: torch.Tensor) -> bool:
        """CUDA float32 operands on the weight's device use the HIP kernels."""
        device = tensors[0].device
        return (device.type == "cuda" and self.weight.dtype == torch.float32
                and self.weight.device == device
                and all(t.device == device and t.dtype == torch.float32 for t in tensors))

    def _flat(self, left: torch.Tensor, right: torch.Tensor) -> torch.Tensor:
        width = self.representation_dimension
        if self._on_kernels(left, right):
            out = ops.o2_forward(left.reshape(-1, width).contiguous(),
                                 right.reshape(-1, width).contiguous(), self.weight,
                                 self._weight_path_info, self._weight_path_coefficients,
                                 self._metadata_id)
            return out.reshape(left.shape)
        dtype = self.internal_compute_dtype
        out = flat_forward(left.reshape(-1, width).to(dtype), right.reshape(-1, width).to(dtype),
                           self.weight.to(dtype), self._plan, self._layout)
        return out.to(left.dtype).reshape(left.shape)

    def _block_slices(self):
        for start, block in zip(self._plan.key_offsets, self.blocks):
            yield start, block.multiplicity * block.irrep_dimension, block

    def forward(self, left, right):
        """Tuple API: one (*batch, multiplicity, irrep_dimension) tensor per block."""
        if len(left) != len(self.keys) or len(right) != len(self.keys):
            raise ValueError("one tensor per representation block is required")
        batch = left[0].shape[:-2]
        lf = torch.cat([v.reshape(*batch, -1) for v in left], dim=-1)
        rf = torch.cat([v.reshape(*batch, -1) for v in right], dim=-1)
        out = self._flat(lf, rf)
        return tuple(out[..., s:s + n].reshape(*batch, b.multiplicity, b.irrep_dimension)
                     for s, n, b in self._block_slices())


class FlatPathWeightedTensorProductO2(PackedPathWeightedTensorProductO2):
    """Flat channel-major rows (*batch, W) in and out (``triton_o2.py:1169-1201``)."""

    def forward(self, left: torch.Tensor, right: torch.Tensor) -> torch.Tensor:
        if (left.ndim < 1 or left.shape[-1] != self.representation_dimension
                or right.shape != left.shape):
            raise ValueError("flat O(2) inputs must have the configured width")
        return self._flat(left, right)


class ComponentMajorPathWeightedTensorProductO2(PackedPathWeightedTensorProductO2):
    """Flat rows with [component, channel] (canonical) or [copy, component,
    channel] (full) frequency blocks (``triton_o2.py:1204-1278``)."""

    def __init__(self, *args, **kwargs) -> None:
        parity = kwargs.get("parity", "full")
        self._layout = 1 if parity == "canonical" else 2
        super().__init__(*args, **kwargs)

    def _unpack(self, value: torch.Tensor):
        batch = value.shape[:-1]
        pieces = []
        for start, width, block in self._block_slices():
            part = value[..., start:start + width]
            mul, dim = block.multiplicity, block.irrep_dimension
            if dim == 1:
                part = part.reshape(*batch, mul, 1)
            elif self.parity == "full":
                part = part.reshape(*batch, mul // self.channels, dim, self.channels) \
                    .transpose(-1, -2).reshape(*batch, mul, dim)
            else:
                part = part.reshape(*batch, dim, mul).transpose(-1, -2)
            pieces.append(part)
        return tuple(pieces)

    def _pack(self, blocks) -> torch.Tensor:
        pieces = []
        for value, block in zip(blocks, self.blocks):
            batch = value.shape[:-2]
            width = block.multiplicity * block.irrep_dimension
            if block.irrep_dimension == 1:
                part = value.reshape(*batch, width)
            elif self.parity == "full":
                part = value.reshape(*batch, block.parity_copies, self.channels,
                                     block.irrep_dimension).transpose(-1, -2).reshape(*batch, width)
            else:
                part = value.transpose(-1, -2).reshape(*batch, width)
            pieces.append(part)
        return torch.cat(pieces, dim=-1)

    def forward(self, left: torch.Tensor, right: torch.Tensor) -> torch.Tensor:
        if (left.ndim < 1 or left.shape[-1] != self.representation_dimension
                or right.shape != left.shape):
            raise ValueError("flat O(2) inputs must have the configured width")
        return self._flat(left, right)


def apply_full_parity_o2(module, tensors: Iterable[torch.Tensor],
                         group_element: torch.Tensor):
    """Act with an O(2) element on per-block tensors in the public copy bases
    (``native_o2.py:224-247``): the second copy transforms with det(g) * R_m(g)."""
    outputs = []
    det = torch.linalg.det(group_element)
    for block, value in zip(module.blocks, tensors):
        matrix = module.o2.o2_representation(group_element, block.key).to(
            device=value.device, dtype=value.dtype)
        if block.frequency == 0 or module.parity == "canonical":
            outputs.append(torch.einsum("...ab,...cb->...ca", matrix, value))
            continue
        even, odd = value.split(module.channels, dim=-2)
        odd_matrix = det[..., None, None] * matrix
        outputs.append(torch.cat((torch.einsum("...ab,...cb->...ca", matrix, even),
                                  torch.einsum("...ab,...cb->...ca", odd_matrix, odd)), dim=-2))
    return tuple(outputs)
