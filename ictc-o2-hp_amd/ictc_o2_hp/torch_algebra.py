"""Differentiable PyTorch form of the O(2) tensor product on flat rows.

Used where the reference uses PyTorch: inputs that are not CUDA float32
(``triton_o2.py:1176-1193``: CPU or other dtypes take the PyTorch algebra) and
second derivatives, which the reference also recomputes in PyTorch
(``triton_o2.py:969-1064``).  First-order CUDA float32 work never comes here.

The map is the one of ``fast_o2.py:80-149``: canonicalise copy 1, accumulate
every path's weighted coupling with cyclic channel routing, restore copy 1.
"""
from __future__ import annotations

from typing import List

import torch

from .plan import TPPlan


def split_canonical(flat: torch.Tensor, plan: TPPlan, layout: int = 0) -> List[torch.Tensor]:
    """Flat rows [N, W] -> per key [N, mul, dim] in the canonical copy basis."""
    n = flat.shape[0]
    c = plan.channels
    blocks = []
    for start, block in zip(plan.key_offsets, plan.blocks):
        mul, dim = block.multiplicity, block.irrep_dimension
        part = flat[:, start:start + mul * dim]
        if dim == 1 or layout == 0:
            part = part.reshape(n, mul, dim)
        elif layout == 1:
            part = part.reshape(n, dim, mul).transpose(1, 2)
        else:
            part = part.reshape(n, mul // c, dim, c).permute(0, 1, 3, 2).reshape(n, mul, dim)
        if plan.full and dim == 2:
            even, odd = part[:, :c], part[:, c:]
            part = torch.cat((even, torch.stack((-odd[..., 1], odd[..., 0]), dim=-1)), dim=1)
        blocks.append(part)
    return blocks


def join_restored(blocks: List[torch.Tensor], plan: TPPlan, layout: int = 0) -> torch.Tensor:
    """Inverse of ``split_canonical``."""
    n = blocks[0].shape[0]
    c = plan.channels
    parts = []
    for value, block in zip(blocks, plan.blocks):
        mul, dim = block.multiplicity, block.irrep_dimension
        if plan.full and dim == 2:
            even, odd = value[:, :c], value[:, c:]
            value = torch.cat((even, torch.stack((odd[..., 1], -odd[..., 0]), dim=-1)), dim=1)
        if dim == 2 and layout == 1:
            value = value.transpose(1, 2)
        elif dim == 2 and layout == 2:
            value = value.reshape(n, mul // c, c, dim).permute(0, 1, 3, 2)
        parts.append(value.reshape(n, -1))
    return torch.cat(parts, dim=-1)


def flat_forward(left: torch.Tensor, right: torch.Tensor, weight: torch.Tensor,
                 plan: TPPlan, layout: int = 0) -> torch.Tensor:
    """out[N, W] for flat x, y [N, W] and the packed weight [P_w]."""
    first = split_canonical(left, plan, layout)
    second = split_canonical(right, plan, layout)
    outputs: List[torch.Tensor | None] = [None] * len(plan.keys)
    for path in plan.table:
        mul = plan.blocks[path.key3].multiplicity
        a = _route(first[path.key1], mul)
        b = _route(second[path.key2], mul)
        components: List[torch.Tensor | None] = [None] * plan.blocks[path.key3].irrep_dimension
        for term in path.terms:
            value = a[..., term.i] * b[..., term.j]
            if term.coefficient != 1.0:
                value = value * term.coefficient
            components[term.k] = value if components[term.k] is None else components[term.k] + value
        value = torch.stack(components, dim=-1)
        value = value * weight[path.weight_start:path.weight_start + mul].view(1, mul, 1)
        outputs[path.key3] = value if outputs[path.key3] is None else outputs[path.key3] + value
    return join_restored(outputs, plan, layout)


def _route(value: torch.Tensor, mul: int) -> torch.Tensor:
    """Channel routing o -> o mod in_mul for an output multiplicity ``mul``."""
    in_mul = value.shape[1]
    if in_mul == mul:
        return value
    if in_mul > mul:
        return value[:, :mul]
    return value.repeat(1, mul // in_mul, 1)
