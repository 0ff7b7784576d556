"""Jakal-Net operator API, MI355X build of the native hot path.

Public names of the reference's ``src/jakal_net/__init__.py:1-70`` that belong
to the hot path: layers, the propagation / transition operators, the low-rank
score modules and the native-backend status calls.
"""

from jakal_net.core import Layer, LayerDelta
from jakal_net.modules import (
    LowRankBilinearPairwise,
    LowRankBilinearRoute,
    MultiHeadPairwise,
    MultiHeadRoute,
    TemperatureScaledRoute,
)
from jakal_net.native_backend import native_available, native_status
from jakal_net.propagation import Propagation, SparsePropagation
from jakal_net.transition import SparseTransition, Transition

__all__ = [
    "Layer",
    "LayerDelta",
    "LowRankBilinearPairwise",
    "LowRankBilinearRoute",
    "MultiHeadPairwise",
    "MultiHeadRoute",
    "Propagation",
    "SparsePropagation",
    "SparseTransition",
    "TemperatureScaledRoute",
    "Transition",
    "native_available",
    "native_status",
]
