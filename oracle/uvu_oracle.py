"""CPU oracle of the O(2) uvu product and the radial composition (float64, numpy).

TEST INFRASTRUCTURE ONLY (see o2_oracle.py).

Restates ``uvu_o2.py`` of Parity-LRX/ICTC-O2-HP:

* entries (key, copy) with [copy, channel, component] layout (``uvu_o2.py:27-41``);
* paths (out k, first i, second j) in that order, couplings = normalised O(2)
  CG (``o2_oracle.coupling``) in the copy bases (J for copy 1), padded to
  [out][in1][in2], optional 1/sqrt(V * paths into k) (``uvu_o2.py:121-145``);
* forward out[k][n,u,:] += sum_ij x[n,u,i] (sum_v w[p,u,v] y[n,v,j]) cg[:,i,j]
  (``uvu_o2.py:50-73``); weights shared [P*C*V] or per row [N, P*C*V];
* backward: the exact transpose (dx, dy, dw), written out;
* radial: ``tp(left, angular, hidden @ alpha^T + bias)`` (``radial_uvu.py:52``) and
  its chain rule to hidden, alpha, bias;
* gathered radial: ``left = table[index]``, the node -> edge gather a model does
  before the reference's radial chain (docs/RADIAL.md:97-99), whose adjoint adds
  each edge's row adjoint onto its table row (``np.add.at``); an index outside
  the table reads a zero row and receives nothing.

Pinned by tests/golden/uvu_tables.json and uvu_vectors.npz (recorded from the
reference), finite differences and the bilinear adjoint identity.
"""
from __future__ import annotations

import math
from typing import List, NamedTuple

import numpy as np

from .o2_oracle import coupling, valid_outputs

_J = np.array([[0.0, -1.0], [1.0, 0.0]])


class Entry(NamedTuple):
    key: tuple
    copy: int
    offset: int
    dim: int


def entries(channels: int, order: int, parity: str):
    keys = [("scalar", 1)] + ([("scalar", -1)] if parity == "full" else [])
    keys += [("freq", m) for m in range(1, order + 1)]
    out, cursor = [], 0
    for key in keys:
        dim = 1 if key[0] == "scalar" else 2
        copies = 2 if (parity == "full" and dim == 2) else 1
        for copy in range(copies):
            out.append(Entry(key, copy, cursor + copy * channels * dim, dim))
        cursor += copies * channels * dim
    return out, cursor


def _basis(e: Entry) -> np.ndarray:
    return _J if e.copy else np.eye(e.dim)


class UvuOraclePlan:
    def __init__(self, channels, channels_in2, m_max, parity="full", parity_in2=None,
                 m_max_in2=None, normalization="component", path_normalization="none"):
        self.C, self.V = channels, channels_in2
        parity_in2 = parity if parity_in2 is None else parity_in2
        m_max_in2 = m_max if m_max_in2 is None else m_max_in2
        self.first, self.width1 = entries(channels, m_max, parity)
        self.second, self.width2 = entries(channels_in2, m_max_in2, parity_in2)
        self.paths: List[tuple] = []
        cgs = []
        for k, out in enumerate(self.first):
            start = len(self.paths)
            for i, a in enumerate(self.first):
                for j, b in enumerate(self.second):
                    if out.key not in valid_outputs(a.key, b.key):
                        continue
                    cg = coupling(a.key, b.key, out.key, normalization)
                    cg = np.einsum("abk,ai,bj,kl->ijl", cg, _basis(a), _basis(b), _basis(out))
                    self.paths.append((i, j, k))
                    cgs.append(cg.transpose(2, 0, 1))        # [out][in1][in2]
            if path_normalization != "none":
                scale = math.sqrt(channels_in2 * (len(self.paths) - start))
                for p in range(start, len(self.paths)):
                    cgs[p] = cgs[p] / scale
        self.cgs = cgs
        self.weight_numel = len(self.paths) * channels * channels_in2

    def padded(self) -> np.ndarray:
        out = np.zeros((len(self.cgs), 2, 2, 2))
        for p, cg in enumerate(self.cgs):
            out[p, :cg.shape[0], :cg.shape[1], :cg.shape[2]] = cg
        return out

    def _views(self, x, y, n):
        xs = [x[:, e.offset:e.offset + self.C * e.dim].reshape(n, self.C, e.dim) for e in self.first]
        ys = [y[:, e.offset:e.offset + self.V * e.dim].reshape(n, self.V, e.dim) for e in self.second]
        return xs, ys

    def _w(self, weight, p, n, shared):
        s = p * self.C * self.V
        if shared:
            return np.broadcast_to(weight[s:s + self.C * self.V].reshape(1, self.C, self.V),
                                   (n, self.C, self.V))
        return weight[:, s:s + self.C * self.V].reshape(n, self.C, self.V)


def forward(plan: UvuOraclePlan, x, y, weight, shared: bool) -> np.ndarray:
    x, y, weight = (np.asarray(a, dtype=np.float64) for a in (x, y, weight))
    n = x.shape[0]
    xs, ys = plan._views(x, y, n)
    outs = [np.zeros((n, plan.C, e.dim)) for e in plan.first]
    for p, (i, j, k) in enumerate(plan.paths):
        proj = np.einsum("nuv,nvj->nuj", plan._w(weight, p, n, shared), ys[j])
        outs[k] += np.einsum("nui,nuj,kij->nuk", xs[i], proj, plan.cgs[p])
    return np.concatenate([o.reshape(n, -1) for o in outs], axis=1)


def backward(plan: UvuOraclePlan, x, y, weight, grad, shared: bool):
    """(dx, dy, dw) for cotangent ``grad``; dw has the weight's shape."""
    x, y, weight, grad = (np.asarray(a, dtype=np.float64) for a in (x, y, weight, grad))
    n = x.shape[0]
    xs, ys = plan._views(x, y, n)
    gs = [grad[:, e.offset:e.offset + plan.C * e.dim].reshape(n, plan.C, e.dim) for e in plan.first]
    dxs = [np.zeros_like(v) for v in xs]
    dys = [np.zeros_like(v) for v in ys]
    dw = np.zeros_like(weight)
    for p, (i, j, k) in enumerate(plan.paths):
        w = plan._w(weight, p, n, shared)
        cg = plan.cgs[p]
        proj = np.einsum("nuv,nvj->nuj", w, ys[j])
        dxs[i] += np.einsum("nuk,kij,nuj->nui", gs[k], cg, proj)
        r = np.einsum("nui,nuk,kij->nuj", xs[i], gs[k], cg)          # d out / d proj
        dys[j] += np.einsum("nuv,nuj->nvj", w, r)
        s = p * plan.C * plan.V
        if shared:
            dw[s:s + plan.C * plan.V] += np.einsum("nuj,nvj->uv", r, ys[j]).reshape(-1)
        else:
            dw[:, s:s + plan.C * plan.V] += np.einsum("nuj,nvj->nuv", r, ys[j]).reshape(n, -1)
    dx = np.concatenate([d.reshape(n, -1) for d in dxs], axis=1)
    dy = np.concatenate([d.reshape(n, -1) for d in dys], axis=1)
    return dx, dy, dw


def radial_forward(plan: UvuOraclePlan, x, y, hidden, alpha, bias):
    """tp(x, y, hidden @ alpha^T + bias) with per-row weights (``radial_uvu.py:52``)."""
    w = np.asarray(hidden, np.float64) @ np.asarray(alpha, np.float64).T
    if bias is not None:
        w = w + np.asarray(bias, np.float64)
    return forward(plan, x, y, w, shared=False)


def radial_backward(plan: UvuOraclePlan, x, y, hidden, alpha, bias, grad):
    """(dx, dy, dhidden, dalpha, dbias) of ``radial_forward``."""
    hidden = np.asarray(hidden, np.float64)
    alpha = np.asarray(alpha, np.float64)
    w = hidden @ alpha.T
    if bias is not None:
        w = w + np.asarray(bias, np.float64)
    dx, dy, dw = backward(plan, x, y, w, grad, shared=False)
    return dx, dy, dw @ alpha, dw.T @ hidden, (dw.sum(axis=0) if bias is not None else None)


def gather(table, index):
    """table[index] with a zero row for an index outside [0, len(table))."""
    table = np.asarray(table)
    index = np.asarray(index, dtype=np.int64)
    valid = (index >= 0) & (index < table.shape[0])
    out = np.zeros((index.shape[0], table.shape[1]), dtype=table.dtype)
    out[valid] = table[index[valid]]
    return out


def scatter_add(rows, index, n):
    """Adjoint of ``gather``: sum rows[e] into row index[e] of an [n, width] array."""
    rows = np.asarray(rows)
    index = np.asarray(index, dtype=np.int64)
    valid = (index >= 0) & (index < n)
    out = np.zeros((n, rows.shape[1]), dtype=rows.dtype)
    np.add.at(out, index[valid], rows[valid])
    return out


def radial_gather_forward(plan: UvuOraclePlan, table, index, y, hidden, alpha, bias):
    """radial_forward on the gathered rows table[index]."""
    return radial_forward(plan, gather(table, index), y, hidden, alpha, bias)


def radial_gather_backward(plan: UvuOraclePlan, table, index, y, hidden, alpha, bias, grad):
    """(dtable, dy, dhidden, dalpha, dbias): radial_backward on the gathered
    rows, with the row adjoints added onto the table."""
    dx, dy, dh, da, db = radial_backward(plan, gather(table, index), y, hidden, alpha, bias, grad)
    return scatter_add(dx, index, np.asarray(table).shape[0]), dy, dh, da, db
