"""``ReferenceTensorProduct``: the tuple-API product with a separate
parameter per path, evaluated in PyTorch only (``reference.py`` of
Parity-LRX/ICTC-O2-HP); it never loads the HIP library."""
from __future__ import annotations

from . import o2_math
from .native_o2 import FullParityPathWeightedTensorProductO2


class ReferenceTensorProduct(FullParityPathWeightedTensorProductO2):
    """Tuple-API O(2) product, weights ``weights.<p>`` per path, PyTorch only."""

    def __init__(self, channels, m_max, *, parity="full", normalization="component"):
        if int(channels) != channels or channels < 1:
            raise ValueError("channels must be a positive integer")
        if int(m_max) != m_max or m_max < 0:
            raise ValueError("m_max must be a nonnegative integer")
        super().__init__(o2_math, int(channels), int(m_max), parity=parity,
                         normalization=normalization)
