"""The public TensorProduct classes, with the package's own O(2) coupling
tables (``api.py`` of Parity-LRX/ICTC-O2-HP: same names, arguments and
errors)."""
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
    """O(2) tensor product on flat rows ``(*batch, representation_dimension)``,
    one trainable weight per (path, output channel) in ``weight``.

    Row layout: the scalar blocks, then per frequency m a block stored
    channel-major, ``[copy, channel, component]`` (full parity, two copies)
    or ``[channel, component]`` (canonical).  Copy 1 is stored in its own
    Cartesian basis, a quarter turn J away from copy 0's.
    """

    def __init__(self, channels, m_max, *, parity="full", normalization="component"):
        _validate(channels, m_max)
        super().__init__(o2_math, int(channels), int(m_max), parity=parity,
                         normalization=normalization)


class TupleTensorProduct(PackedPathWeightedTensorProductO2):
    """Tuple form: inputs and output are one tensor per block, shaped
    ``(*batch, multiplicity, irrep_dimension)``; same weights as TensorProduct."""

    def __init__(self, channels, m_max, *, parity="full", normalization="component"):
        _validate(channels, m_max)
        super().__init__(o2_math, int(channels), int(m_max), parity=parity,
                         normalization=normalization)


class ComponentMajorTensorProduct(ComponentMajorPathWeightedTensorProductO2):
    """TensorProduct with component-major frequency blocks:
    ``[copy, component, channel]`` (full) or ``[component, channel]``
    (canonical).  Only the storage order differs; values and copy bases are
    TensorProduct's."""

    def __init__(self, channels, m_max, *, parity="full", normalization="component"):
        _validate(channels, m_max)
        super().__init__(o2_math, int(channels), int(m_max), parity=parity,
                         normalization=normalization)
