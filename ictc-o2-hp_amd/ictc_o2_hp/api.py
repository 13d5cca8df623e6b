"""Public operators with the internal Cartesian O(2) coefficient source
(``api.py`` of Parity-LRX/ICTC-O2-HP: same names, arguments and errors)."""
from __future__ import annotations

from . import o2_math
from .native_o2 import (ComponentMajorPathWeightedTensorProductO2,
                        FlatPathWeightedTensorProductO2, PackedPathWeightedTensorProductO2)


def _validate(channels, m_max):
    if int(channels) != channels or channels < 1:
        raise ValueError("channels must be a positive integer")
    if int(m_max) != m_max or m_max < 0:
        raise ValueError("m_max must be a nonnegative integer")


class TensorProduct(FlatPathWeightedTensorProductO2):
    """Flat channel-major O(2) product with all path weights trainable.

    Inputs/outputs: ``(*batch, representation_dimension)``.  Positive-frequency
    blocks use ``[copy, channel, component]`` in full parity and
    ``[channel, component]`` in canonical parity; the second copy keeps its
    reflection-twisted Cartesian basis.
    """

    def __init__(self, channels, m_max, *, parity="full", normalization="component"):
        _validate(channels, m_max)
        super().__init__(o2_math, int(channels), int(m_max), parity=parity,
                         normalization=normalization)


class TupleTensorProduct(PackedPathWeightedTensorProductO2):
    """One ``(*batch, multiplicity, irrep_dimension)`` tensor per block."""

    def __init__(self, channels, m_max, *, parity="full", normalization="component"):
        _validate(channels, m_max)
        super().__init__(o2_math, int(channels), int(m_max), parity=parity,
                         normalization=normalization)


class ComponentMajorTensorProduct(ComponentMajorPathWeightedTensorProductO2):
    """Flat product with ``[copy, component, channel]`` frequency blocks; the
    bases are the same as TensorProduct's."""

    def __init__(self, channels, m_max, *, parity="full", normalization="component"):
        _validate(channels, m_max)
        super().__init__(o2_math, int(channels), int(m_max), parity=parity,
                         normalization=normalization)
