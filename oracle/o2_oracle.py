"""CPU oracle for the O(2) tensor-product hot path (float64, numpy).

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module; only
tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of bench.py
may use it, and only as the checker.

What it restates (Parity-LRX/ICTC-O2-HP, ``src/ictc_o2_hp/``):

* ``coupling``: the normalised O(2) coupling tensors of ``o2_math.py:295-346``
  with ``native_o2.py:118-123``, written in closed form.  The reference builds
  its frequency-m harmonics as s_m * (cos m t, sin m t) with s_m = +1 for
  m = 1, 2 (mod 4) and -1 for m = 0, 3 (mod 4) (the sign fix and the even-m
  negation of ``o2_math.py:76-84, :130-133``); products of two harmonics then
  follow from the angle-sum identities.  Pinned by tests/golden/cg_tables.json.
* ``blocks`` / ``paths``: ``native_o2.py:35-61``, ``:101-108``.
* ``forward``: the einsum algebra of ``native_o2.py:183-221`` on the flat
  layouts of ``triton_o2.py:110-121`` (layout 0 = channel-major,
  1 = canonical component-major, 2 = full component-major), including the
  copy-1 reflection twist (``native_o2.py:167-181``; ``fast_o2.py:61-73``) and
  the cyclic channel routing ``arange(out_mul) % in_mul`` (``native_o2.py:128-129``).
* ``backward``: the exact transpose of ``forward`` (dx, dy, dw), written out
  rather than taken from autograd, following ``triton_o2.py:452-501`` for the
  input adjoint (scatter over the routing) and ``:571-607`` for dw.
  Pinned by finite differences, the bilinear adjoint identity and
  tests/golden/tp_vectors.npz.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Tuple

import numpy as np

Key = Tuple[str, int]
_ROOT2 = math.sqrt(2.0)


def _basis_sign(m: int) -> float:
    return 1.0 if m % 4 in (1, 2) else -1.0


def _dim(key: Key) -> int:
    return 1 if key[0] == "scalar" else 2


def valid_outputs(k1: Key, k2: Key) -> List[Key]:
    """``o2_math.py:348-372``."""
    if k1[0] == "scalar" and k2[0] == "scalar":
        return [("scalar", k1[1] * k2[1])]
    if k1[0] == "scalar":
        return [k2]
    if k2[0] == "scalar":
        return [k1]
    if k1[1] == k2[1]:
        return [("scalar", 1), ("scalar", -1), ("freq", 2 * k1[1])]
    return [("freq", abs(k1[1] - k2[1])), ("freq", k1[1] + k2[1])]


def raw_coupling(k1: Key, k2: Key, k3: Key) -> np.ndarray:
    """Unnormalised coupling C[i, j, k] up to a positive factor per path."""
    c = np.zeros((_dim(k1), _dim(k2), _dim(k3)))
    if k1[0] == "scalar" and k2[0] == "scalar":
        if k3 == ("scalar", k1[1] * k2[1]):
            c[0, 0, 0] = 1.0
        return c
    if k1[0] == "scalar" or k2[0] == "scalar":
        freq, scalar = (k2, k1) if k1[0] == "scalar" else (k1, k2)
        if k3 != freq:
            return c
        # out = v for the even scalar, out = J v = (-v1, v0) for the odd one.
        table = {(0, 0): 1.0, (1, 1): 1.0} if scalar[1] == 1 else {(1, 0): -1.0, (0, 1): 1.0}
        for (src, dst), value in table.items():
            if k1[0] == "scalar":
                c[0, src, dst] = value
            else:
                c[src, 0, dst] = value
        return c
    m1, m2 = k1[1], k2[1]
    s = _basis_sign(m1) * _basis_sign(m2)
    if k3[0] == "scalar":
        if m1 != m2:
            return c
        if k3[1] == 1:      # cos(0) part: a0 b0 + a1 b1 (s_m1 s_m2 = 1)
            c[0, 0, 0] = c[1, 1, 0] = 1.0
        else:               # antisymmetric form a0 b1 - a1 b0
            c[0, 1, 0], c[1, 0, 0] = 1.0, -1.0
        return c
    m3 = k3[1]
    s *= _basis_sign(m3)
    if m3 == m1 + m2:       # alpha * beta
        c[0, 0, 0], c[1, 1, 0] = s, -s
        c[0, 1, 1], c[1, 0, 1] = s, s
    elif m3 == m1 - m2:     # alpha * conj(beta)
        c[0, 0, 0], c[1, 1, 0] = s, s
        c[1, 0, 1], c[0, 1, 1] = s, -s
    elif m3 == m2 - m1:     # conj(alpha) * beta
        c[0, 0, 0], c[1, 1, 0] = s, s
        c[0, 1, 1], c[1, 0, 1] = s, -s
    return c


def coupling(k1: Key, k2: Key, k3: Key, normalization: str = "component") -> np.ndarray:
    c = raw_coupling(k1, k2, k3)
    norm = np.linalg.norm(c)
    if norm > 1e-30:
        c = c * ((math.sqrt(c.shape[2]) if normalization == "component" else 1.0) / norm)
    return c


@dataclass(frozen=True)
class Block:
    key: Key
    mul: int
    dim: int
    copies: int


class OraclePlan:
    """Keys, paths, couplings and packed weight offsets of one TensorProduct."""

    def __init__(self, channels: int, m_max: int, parity: str = "full",
                 normalization: str = "component"):
        if parity not in ("canonical", "full"):
            raise ValueError(parity)
        self.C, self.M, self.parity, self.normalization = channels, m_max, parity, normalization
        self.full = parity == "full"
        keys: List[Key] = [("scalar", 1)] + ([("scalar", -1)] if self.full else [])
        keys += [("freq", m) for m in range(1, m_max + 1)]
        self.keys = keys
        copies = 2 if self.full else 1
        self.blocks = [Block(k, channels if k[0] == "scalar" else copies * channels,
                             _dim(k), 1 if k[0] == "scalar" else copies) for k in keys]
        self.offsets, cursor = [], 0
        for b in self.blocks:
            self.offsets.append(cursor)
            cursor += b.mul * b.dim
        self.width = cursor
        present = set(keys)
        self.paths = [(a, b, c) for a in keys for b in keys
                      for c in valid_outputs(a, b) if c in present]
        idx = {k: n for n, k in enumerate(keys)}
        self.path_index = [(idx[a], idx[b], idx[c]) for a, b, c in self.paths]
        self.cgs = [coupling(a, b, c, normalization) for a, b, c in self.paths]
        self.weight_slices, start = [], 0
        for _, _, k3 in self.path_index:
            self.weight_slices.append((start, start + self.blocks[k3].mul))
            start += self.blocks[k3].mul
        self.weight_numel = start

    # ---- storage ------------------------------------------------------------
    def unpack(self, flat: np.ndarray, layout: int = 0) -> List[np.ndarray]:
        """Flat rows -> one (N, mul, dim) array per key, public bases."""
        n = flat.shape[0]
        out = []
        for off, b in zip(self.offsets, self.blocks):
            part = flat[:, off:off + b.mul * b.dim]
            if b.dim == 1:
                out.append(part.reshape(n, b.mul, 1))
            elif layout == 0:
                out.append(part.reshape(n, b.mul, 2))
            elif layout == 1:
                out.append(part.reshape(n, 2, b.mul).transpose(0, 2, 1))
            else:
                out.append(part.reshape(n, b.copies, 2, self.C).transpose(0, 1, 3, 2)
                           .reshape(n, b.mul, 2))
        return out

    def pack(self, blocks: List[np.ndarray], layout: int = 0) -> np.ndarray:
        n = blocks[0].shape[0]
        parts = []
        for value, b in zip(blocks, self.blocks):
            if b.dim == 1 or layout == 0:
                parts.append(value.reshape(n, -1))
            elif layout == 1:
                parts.append(value.transpose(0, 2, 1).reshape(n, -1))
            else:
                parts.append(value.reshape(n, b.copies, self.C, 2).transpose(0, 1, 3, 2)
                             .reshape(n, -1))
        return np.concatenate(parts, axis=1)

    def twist(self, blocks: List[np.ndarray], inverse: bool = False) -> List[np.ndarray]:
        """Copy-1 basis change: (v0, v1) -> (-v1, v0), or its inverse."""
        if not self.full:
            return [v.copy() for v in blocks]
        out = []
        for v, b in zip(blocks, self.blocks):
            v = v.copy()
            if b.dim == 2:
                odd = v[:, self.C:, :].copy()
                if inverse:
                    v[:, self.C:, 0], v[:, self.C:, 1] = odd[..., 1], -odd[..., 0]
                else:
                    v[:, self.C:, 0], v[:, self.C:, 1] = -odd[..., 1], odd[..., 0]
            out.append(v)
        return out

    def routing(self, path: int):
        k1, k2, k3 = self.path_index[path]
        o = np.arange(self.blocks[k3].mul)
        return o % self.blocks[k1].mul, o % self.blocks[k2].mul


def _components(blocks: List[np.ndarray]) -> List[np.ndarray]:
    """(N, mul, dim) blocks -> contiguous (dim, N, mul) arrays (fast row-wise math)."""
    return [np.ascontiguousarray(v.transpose(2, 0, 1)) for v in blocks]


def _blocks(components: List[np.ndarray]) -> List[np.ndarray]:
    return [c.transpose(1, 2, 0) for c in components]


def _route(value: np.ndarray, index: np.ndarray) -> np.ndarray:
    """value[:, :, index] without a gather when the routing is the identity."""
    if index.shape[0] == value.shape[2] and index[-1] == value.shape[2] - 1:
        return value
    return value[:, :, index]


def forward(plan: OraclePlan, x: np.ndarray, y: np.ndarray, weight: np.ndarray,
            layout: int = 0) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    w = np.asarray(weight, dtype=np.float64)
    xs = _components(plan.twist(plan.unpack(x, layout)))
    ys = _components(plan.twist(plan.unpack(y, layout)))
    n = x.shape[0]
    outs = [np.zeros((b.dim, n, b.mul)) for b in plan.blocks]
    for p, (k1, k2, k3) in enumerate(plan.path_index):
        r1, r2 = plan.routing(p)
        s0, s1 = plan.weight_slices[p]
        a, b, cg, wp = _route(xs[k1], r1), _route(ys[k2], r2), plan.cgs[p], w[s0:s1]
        # out[k, n, o] += w[o] * sum_ij cg[i, j, k] a[i, n, o] b[j, n, o]
        for i, j, k in _entries(cg):
            outs[k3][k] += (cg[i, j, k] * wp) * (a[i] * b[j])
    return plan.pack(plan.twist(_blocks(outs), inverse=True), layout)


def _entries(cg: np.ndarray):
    """Index triples of the coupling tensor's entries (zeros contribute nothing)."""
    return [idx for idx in np.ndindex(*cg.shape) if cg[idx] != 0.0]


def backward(plan: OraclePlan, x: np.ndarray, y: np.ndarray, weight: np.ndarray,
             grad: np.ndarray, layout: int = 0):
    """Returns (dx, dy, dw) for cotangent ``grad``."""
    x = np.asarray(x, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    w = np.asarray(weight, dtype=np.float64)
    xs = _components(plan.twist(plan.unpack(x, layout)))
    ys = _components(plan.twist(plan.unpack(y, layout)))
    gs = _components(plan.twist(plan.unpack(np.asarray(grad, dtype=np.float64), layout)))
    n = x.shape[0]
    dxs = [np.zeros((b.dim, n, b.mul)) for b in plan.blocks]
    dys = [np.zeros((b.dim, n, b.mul)) for b in plan.blocks]
    dw = np.zeros(plan.weight_numel)
    for p, (k1, k2, k3) in enumerate(plan.path_index):
        r1, r2 = plan.routing(p)
        s0, s1 = plan.weight_slices[p]
        a, b, g, cg = _route(xs[k1], r1), _route(ys[k2], r2), gs[k3], plan.cgs[p]
        wp = w[s0:s1]
        da = np.zeros_like(a)
        db = np.zeros_like(b)
        for i, j, k in _entries(cg):
            gk = cg[i, j, k] * g[k]
            da[i] += wp * gk * b[j]
            db[j] += wp * gk * a[i]
            dw[s0:s1] += (gk * a[i] * b[j]).sum(axis=0)
        # Several output channels can route to one input channel: scatter-add.
        _scatter_channels(dxs[k1], da)
        _scatter_channels(dys[k2], db)
    # The twist is orthogonal, so its transpose is its inverse.
    dx = plan.pack(plan.twist(_blocks(dxs), inverse=True), layout)
    dy = plan.pack(plan.twist(_blocks(dys), inverse=True), layout)
    return dx, dy, dw


def _scatter_channels(dst: np.ndarray, src: np.ndarray) -> None:
    """dst[..., o % mul_in] += src[..., o] for o < mul_out (the transpose of the
    routing ``arange(mul_out) % mul_in``; mul_out is mul_in/2, mul_in or 2*mul_in)."""
    mul_in, mul_out = dst.shape[2], src.shape[2]
    if mul_out == mul_in:
        dst += src
    elif mul_out < mul_in:
        dst[:, :, :mul_out] += src
    else:
        dst += src.reshape(src.shape[0], src.shape[1], mul_out // mul_in, mul_in).sum(axis=2)


def backward_chunked(plan: OraclePlan, x, y, weight, grad, chunk: int = 2048, layout: int = 0):
    """``backward`` over row chunks (bounded memory), dw summed over chunks."""
    n = x.shape[0]
    dx = np.empty((n, plan.width))
    dy = np.empty((n, plan.width))
    dw = np.zeros(plan.weight_numel)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        a, b, c = backward(plan, x[s:e], y[s:e], weight, grad[s:e], layout)
        dx[s:e], dy[s:e] = a, b
        dw += c
    return dx, dy, dw


def normalized_error(reference: np.ndarray, actual: np.ndarray) -> float:
    """max|ref - act| / max(1e-7, max|ref|, max|act|) (``benchmarks/eqx/scripts/support.py:33-35``)."""
    reference = np.asarray(reference, dtype=np.float64)
    actual = np.asarray(actual, dtype=np.float64)
    if reference.size == 0:
        return 0.0
    scale = max(1e-7, float(np.abs(reference).max()), float(np.abs(actual).max()))
    return float(np.abs(reference - actual).max()) / scale
