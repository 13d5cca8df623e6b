"""Path-weighted O(2) tensor-product modules (tuple, packed, flat layouts).

Module surface of Parity-LRX/ICTC-O2-HP:

* ``FullParityPathWeightedTensorProductO2``: one parameter per path
  (``native_o2.py:64-221``), evaluated with the flat-row PyTorch algebra;
* ``PackedPathWeightedTensorProductO2``: the same paths with one flat
  ``weight`` and ``copy_weights_to_r5`` / ``load_weights_from_r5``
  (``fast_o2.py:152-186``);
* ``FlatPathWeightedTensorProductO2`` / ``ComponentMajorPathWeightedTensorProductO2``:
  flat channel-major / component-major rows (``triton_o2.py:1169-1278``).

State-dict keys and shapes match the reference: ``weight`` (or
``weights.<p>``), ``cg_<p>`` and ``odd_to_even`` / ``even_to_odd`` persistent;
kernel metadata non-persistent.  CUDA float32 inputs on the
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
        for p, path in enumerate(self._plan.table):
            # Same draw order as the reference: one randn(out_mul) per path.
            self.weights.append(torch.nn.Parameter(torch.randn(path.weight_count) * 0.02))
            self.register_buffer(f"cg_{p}", torch.from_numpy(self._plan.cg[p].copy()),
                                 persistent=True)
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
        """One dict per block (``native_o2.py:145-165``): its label ("0e", "0o",
        "m" canonical, "me+mo" full), frequency, irrep dimension, multiplicity
        and parity copies."""
        fields = ("frequency", "irrep_dimension", "multiplicity", "parity_copies")
        spec = []
        for block in self.blocks:
            m = block.frequency
            label = block.token if m == 0 else (f"{m}e+{m}o" if self.parity == "full" else str(m))
            spec.append({"labels": label, **{name: getattr(block, name) for name in fields}})
        return spec

    def _packed_weight(self) -> torch.Tensor:
        """All path weights in path order, as one differentiable vector."""
        return torch.cat(list(self.weights))

    def forward(self, left, right):
        """Tuple API: one (*batch, multiplicity, irrep_dimension) tensor per
        block in and out (``native_o2.py:183-221``), evaluated as the flat-row
        algebra on the concatenated blocks in ``internal_compute_dtype``."""
        if len(left) != len(self.keys) or len(right) != len(self.keys):
            raise ValueError("one tensor per representation block is required")
        batch = left[0].shape[:-2]
        dtype = self.internal_compute_dtype
        width = self.representation_dimension
        x = torch.cat([v.reshape(*batch, -1) for v in left], dim=-1).reshape(-1, width)
        y = torch.cat([v.reshape(*batch, -1) for v in right], dim=-1).reshape(-1, width)
        out = flat_forward(x.to(dtype), y.to(dtype), self._packed_weight().to(dtype), self._plan)
        out = out.to(left[0].dtype).reshape(*batch, width)
        return _split_blocks(out, self._plan)


def _split_blocks(flat: torch.Tensor, plan: TPPlan):
    """Channel-major flat rows [..., W] -> one [..., multiplicity, dim] view per block."""
    sizes = [b.multiplicity * b.irrep_dimension for b in plan.blocks]
    return tuple(part.unflatten(-1, (b.multiplicity, b.irrep_dimension))
                 for part, b in zip(flat.split(sizes, dim=-1), plan.blocks))


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

    def _packed_weight(self) -> torch.Tensor:
        return self.weight

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

    def forward(self, left, right):
        """Tuple API: one (*batch, multiplicity, irrep_dimension) tensor per block."""
        if len(left) != len(self.keys) or len(right) != len(self.keys):
            raise ValueError("one tensor per representation block is required")
        batch = left[0].shape[:-2]
        lf = torch.cat([v.reshape(*batch, -1) for v in left], dim=-1)
        rf = torch.cat([v.reshape(*batch, -1) for v in right], dim=-1)
        return _split_blocks(self._flat(lf, rf), self._plan)


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

    def _channel_major_columns(self, device) -> torch.Tensor:
        """Column of this layout's row that holds each channel-major element:
        channel_major_row = row[..., columns] (``triton_o2.py:110-121``)."""
        columns = getattr(self, "_columns", None)
        if columns is None:
            plan = self._plan
            order = [plan.element_offset(key, channel, component, self._layout)
                     for key, block in enumerate(plan.blocks)
                     for channel in range(block.multiplicity)
                     for component in range(block.irrep_dimension)]
            columns = torch.tensor(order, dtype=torch.long)
            self._columns = columns
            self._inverse_columns = torch.argsort(columns)
        return columns.to(device)

    def _unpack(self, value: torch.Tensor):
        """Component-major rows [..., W] -> one [..., multiplicity, dim] tensor per block."""
        columns = self._channel_major_columns(value.device)
        return _split_blocks(value.index_select(-1, columns), self._plan)

    def _pack(self, blocks) -> torch.Tensor:
        """Inverse of ``_unpack``."""
        batch = blocks[0].shape[:-2]
        flat = torch.cat([b.reshape(*batch, -1) for b in blocks], dim=-1)
        self._channel_major_columns(flat.device)
        return flat.index_select(-1, self._inverse_columns.to(flat.device))

    def forward(self, left: torch.Tensor, right: torch.Tensor) -> torch.Tensor:
        if (left.ndim < 1 or left.shape[-1] != self.representation_dimension
                or right.shape != left.shape):
            raise ValueError("flat O(2) inputs must have the configured width")
        return self._flat(left, right)


def apply_full_parity_o2(module, tensors: Iterable[torch.Tensor],
                         group_element: torch.Tensor):
    """Act with the O(2) element ``group_element`` [..., 2, 2] on per-block
    tensors [..., multiplicity, dim] in the public copy bases
    (``native_o2.py:224-247``): every row of a block transforms with the key's
    representation matrix, and in full parity the second copy of each frequency
    block (its last C rows) carries an extra factor det(g)."""
    det = torch.linalg.det(group_element)
    outputs = []
    for block, value in zip(module.blocks, tensors):
        matrix = module.o2.o2_representation(group_element, block.key).to(
            device=value.device, dtype=value.dtype)
        moved = torch.matmul(value, matrix.transpose(-1, -2))
        if module.parity == "full" and block.frequency > 0:
            second_copy = torch.arange(block.multiplicity, device=value.device) >= module.channels
            scale = torch.where(second_copy, det.to(value.dtype)[..., None],
                                torch.ones((), dtype=value.dtype, device=value.device))
            moved = moved * scale[..., None]
        outputs.append(moved)
    return tuple(outputs)
