"""MI355X-native fused EGNN/MPNN message-passing layer.

The hot path (fused forward, recompute backward, per-graph schedule) is
hand-written HIP for gfx950 behind the C-ABI of ``include/egnn.h``; this
package is its host side: the ctypes binding, the autograd wrapper, and the
reference's Python surface (``models/EGNN``, ``datasets_loaders``).
"""
from . import graphs  # noqa: F401  (numpy only)

__version__ = "0.1.0"
