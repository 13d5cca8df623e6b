"""CPU PyTorch port of the reference's CPU algebra, timed as bench.py's CPU baseline.

TEST INFRASTRUCTURE ONLY (see o2_oracle.py): imported by tests/ and by the
``cpu_baseline`` leg of bench.py, never by the product.

Restates ``FastPathWeightedTensorProductO2.forward`` (``fast_o2.py:80-149``)
in float32 with PyTorch autograd for dx, dy and dw: the same per-path op
sequence (slice the copies, product of components scaled by the sparse
coupling coefficient, multiply by the path weight, accumulate, restore the
copy basis).  Couplings come from ``o2_oracle.coupling``.
"""
from __future__ import annotations

from typing import List

import numpy as np
import torch

from .o2_oracle import OraclePlan


class CPUPort:
    def __init__(self, channels: int, m_max: int, parity: str = "full",
                 normalization: str = "component"):
        self.plan = OraclePlan(channels, m_max, parity, normalization)
        self.sparse = []
        for cg in self.plan.cgs:
            comps = []
            for k in range(cg.shape[2]):
                comps.append(tuple((i, j, float(cg[i, j, k])) for i in range(cg.shape[0])
                                   for j in range(cg.shape[1]) if abs(cg[i, j, k]) > 1e-12))
            self.sparse.append(tuple(comps))

    def _split(self, flat: torch.Tensor) -> List[torch.Tensor]:
        plan, n = self.plan, flat.shape[0]
        out = []
        for off, b in zip(plan.offsets, plan.blocks):
            v = flat[:, off:off + b.mul * b.dim].reshape(n, b.mul, b.dim)
            if plan.full and b.dim == 2:    # fast_o2.py:61-66
                even, odd = v.split(plan.C, dim=-2)
                v = torch.cat((even, torch.stack((-odd[..., 1], odd[..., 0]), dim=-1)), dim=-2)
            out.append(v)
        return out

    def forward(self, x: torch.Tensor, y: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
        plan, n = self.plan, x.shape[0]
        first, second = self._split(x), self._split(y)
        outputs = [None] * len(plan.keys)
        for p, (k1, k2, k3) in enumerate(plan.path_index):
            copies = plan.blocks[k3].copies
            a = first[k1].reshape(n, plan.blocks[k1].copies, plan.C, plan.blocks[k1].dim)
            b = second[k2].reshape(n, plan.blocks[k2].copies, plan.C, plan.blocks[k2].dim)
            if a.shape[1] > copies:
                a = a[:, :copies]
            if b.shape[1] > copies:
                b = b[:, :copies]
            comps = []
            for terms in self.sparse[p]:       # fast_o2.py:41-59
                acc = None
                for i, j, coef in terms:
                    t = a[..., i] * b[..., j]
                    if coef != 1.0:
                        t = t * coef
                    acc = t if acc is None else acc + t
                comps.append(acc)
            value = torch.stack(comps, dim=-1)
            s0, s1 = plan.weight_slices[p]
            value = value * weight[s0:s1].reshape(1, copies, plan.C, 1)
            outputs[k3] = value if outputs[k3] is None else outputs[k3] + value
        parts = []
        for value, b in zip(outputs, plan.blocks):
            value = value.reshape(n, b.mul, b.dim)
            if plan.full and b.dim == 2:       # fast_o2.py:68-73
                even, odd = value.split(plan.C, dim=-2)
                value = torch.cat((even, torch.stack((odd[..., 1], -odd[..., 0]), dim=-1)), dim=-2)
            parts.append(value.reshape(n, -1))
        return torch.cat(parts, dim=-1)

    def forward_vjp(self, x: np.ndarray, y: np.ndarray, weight: np.ndarray, grad: np.ndarray):
        """out, dx, dy, dw in float32 through PyTorch autograd."""
        xt = torch.as_tensor(x, dtype=torch.float32).requires_grad_()
        yt = torch.as_tensor(y, dtype=torch.float32).requires_grad_()
        wt = torch.as_tensor(weight, dtype=torch.float32).requires_grad_()
        out = self.forward(xt, yt, wt)
        dx, dy, dw = torch.autograd.grad(out, (xt, yt, wt), torch.as_tensor(grad, dtype=torch.float32))
        return out.detach(), dx, dy, dw
