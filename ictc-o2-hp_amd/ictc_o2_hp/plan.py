"""Immutable path plans for the O(2) tensor products.

A plan is everything the kernels need that depends only on the representation
(channels C, m_max, parity, normalization): the blocks and their offsets in a
flat row, the ordered path list, each path's sparse coupling terms and the
offset of its weights in the packed weight vector.  It is built once per
module on the host, in fp64, from ``o2_math``.

Semantics follow Parity-LRX/ICTC-O2-HP:

* blocks and key order: ``native_o2.py:25-61``;
* path enumeration (k1, then k2, then each admissible k3 that is present):
  ``native_o2.py:101-108``;
* per-path normalisation: ``native_o2.py:118-123``;
* sparse terms (output component, then first, then second component, kept when
  |coef| > 1e-12): ``fast_o2.py:19-36``;
* packed weight offsets in path order: ``fast_o2.py:155-167``;
* flat layouts 0/1/2 addressing: ``triton_o2.py:99-121``.
"""
from __future__ import annotations

from dataclasses import dataclass
from functools import lru_cache
from typing import Tuple

import numpy as np

from . import o2_math

O2Key = Tuple[str, int]

PARITIES = ("canonical", "full")
NORMALIZATIONS = ("component", "norm")


@dataclass(frozen=True)
class RepresentationBlock:
    """One irrep block of a flat row (mirrors ``native_o2.py:25-32``)."""
    token: str
    key: O2Key
    frequency: int
    irrep_dimension: int
    multiplicity: int
    parity_copies: int


def full_parity_blocks(max_frequency: int, channels: int) -> Tuple[RepresentationBlock, ...]:
    """0e, 0o, then frequencies 1..M with two copies each (``native_o2.py:35-48``)."""
    if max_frequency < 0:
        raise ValueError("max_frequency must be non-negative")
    if channels <= 0:
        raise ValueError("channels must be positive")
    return (
        RepresentationBlock("0e", ("scalar", 1), 0, 1, channels, 1),
        RepresentationBlock("0o", ("scalar", -1), 0, 1, channels, 1),
        *(RepresentationBlock(str(m), ("freq", m), m, 2, 2 * channels, 2)
          for m in range(1, max_frequency + 1)),
    )


def canonical_blocks(max_frequency: int, channels: int) -> Tuple[RepresentationBlock, ...]:
    """0e, then frequencies 1..M with one copy each (``native_o2.py:51-61``)."""
    if max_frequency < 0 or channels <= 0:
        raise ValueError("invalid frequency or channels")
    return (
        RepresentationBlock("0e", ("scalar", 1), 0, 1, channels, 1),
        *(RepresentationBlock(str(m), ("freq", m), m, 2, channels, 1)
          for m in range(1, max_frequency + 1)),
    )


@dataclass(frozen=True)
class PathTerm:
    i: int          # first-input component
    j: int          # second-input component
    k: int          # output component
    coefficient: float


@dataclass(frozen=True)
class TPPath:
    key1: int       # index into plan.keys
    key2: int
    key3: int
    weight_start: int
    weight_count: int   # multiplicity of key3: C or 2C weights
    terms: Tuple[PathTerm, ...]

    @property
    def magnitude(self) -> float:
        """Common |coefficient| of the path's terms (checked at build time)."""
        return max(abs(t.coefficient) for t in self.terms)


class TPPlan:
    """Paths, coefficients and flat-row geometry of ``TensorProduct``."""

    def __init__(self, channels: int, m_max: int, parity: str = "full",
                 normalization: str = "component") -> None:
        if parity not in PARITIES:
            raise ValueError(parity)
        self.channels = int(channels)
        self.m_max = int(m_max)
        self.parity = parity
        self.full = parity == "full"
        self.normalization = normalization
        self.blocks = (full_parity_blocks if self.full else canonical_blocks)(
            self.m_max, self.channels)
        self.keys = tuple(b.key for b in self.blocks)
        self.block_by_key = {b.key: b for b in self.blocks}
        index = {key: n for n, key in enumerate(self.keys)}

        offsets, cursor = [], 0
        for block in self.blocks:
            offsets.append(cursor)
            cursor += block.multiplicity * block.irrep_dimension
        self.key_offsets = tuple(offsets)
        self.width = cursor

        key_paths = []
        for key1 in self.keys:
            for key2 in self.keys:
                for key3 in o2_math.valid_output_keys(key1, key2):
                    if key3 in index:
                        key_paths.append((key1, key2, key3))
        self.paths = tuple(key_paths)

        cgs, table, start = [], [], 0
        for key1, key2, key3 in self.paths:
            cg = o2_math.normalized_cg(key1, key2, key3, normalization)
            cgs.append(cg)
            terms = tuple(
                PathTerm(i, j, k, float(cg[i, j, k]))
                for k in range(cg.shape[2]) for i in range(cg.shape[0])
                for j in range(cg.shape[1]) if abs(cg[i, j, k]) > 1.0e-12)
            mul3 = self.block_by_key[key3].multiplicity
            table.append(TPPath(index[key1], index[key2], index[key3], start, mul3, terms))
            start += mul3
        self.cg = tuple(cgs)
        self.table = tuple(table)
        self.weight_numel = start
        self.weight_offsets = tuple((p.weight_start, p.weight_start + p.weight_count)
                                    for p in self.table)

    # ---- geometry -----------------------------------------------------------
    @property
    def representation_dimension(self) -> int:
        return self.width

    def key_spec(self, layout: int = 0):
        """(start, multiplicity, dim, is_frequency, layout) per key, the tuple
        form of ``triton_o2.py:1100-1109``."""
        return tuple((off, b.multiplicity, b.irrep_dimension, int(b.frequency > 0), layout)
                     for off, b in zip(self.key_offsets, self.blocks))

    def element_offset(self, key: int, channel: int, component: int, layout: int = 0) -> int:
        """Position of (key, channel, component) in a flat row (``triton_o2.py:110-121``)."""
        start = self.key_offsets[key]
        block = self.blocks[key]
        if block.irrep_dimension == 1:
            return start + channel
        if layout == 0:
            return start + channel * 2 + component
        if layout == 1:
            return start + channel + component * block.multiplicity
        c = self.channels
        return start + (channel // c) * 2 * c + component * c + channel % c

    def dense_cg(self, path: int) -> np.ndarray:
        return self.cg[path]

    def signature(self) -> tuple:
        return (self.m_max, self.parity, self.normalization)


@lru_cache(maxsize=None)
def tp_plan(channels: int, m_max: int, parity: str, normalization: str) -> TPPlan:
    return TPPlan(channels, m_max, parity, normalization)


@lru_cache(maxsize=None)
def kernel_table(m_max: int, parity: str, normalization: str):
    """Channel-independent description used to generate the HIP tables.

    Returns (keys, paths) where keys[k] = (offset_units, dim) with the offset
    in units of C, and paths[p] = (k1, k2, k3, weight_start_units, magnitude,
    ((i, j, k, sign), ...)); offsets are in units of C because the table is
    built with C = 1.  Every term of a path has the same |coef|, so a
    path's coupling is sign * magnitude with the magnitude folded into the
    weight inside the kernels.
    """
    plan = TPPlan(1, m_max, parity, normalization)
    keys = tuple((off, b.irrep_dimension) for off, b in zip(plan.key_offsets, plan.blocks))
    paths = []
    for path in plan.table:
        mag = path.magnitude
        for term in path.terms:
            if abs(abs(term.coefficient) - mag) > 1e-12 * mag:
                raise ValueError("path coefficients do not share one magnitude")
        paths.append((path.key1, path.key2, path.key3, path.weight_start, mag,
                      tuple((t.i, t.j, t.k, 1 if t.coefficient > 0 else -1)
                            for t in path.terms)))
    return keys, tuple(paths)
