"""MI355X-native (gfx950 HIP) implementation of AutoSAGE's sparse hot path.

Public names are those of the reference package (``autosage/__init__.py:1-17``).
"""

from ._auto import calibrate_full, csr_attention_forward, sddmm_csr_auto, spmm_csr_auto
from ._version import __version__
from .conv import AutoSAGEConv
from .ops import load_native, native_available, spmm_csr, validate_csr

__all__ = [
    "AutoSAGEConv",
    "__version__",
    "calibrate_full",
    "csr_attention_forward",
    "load_native",
    "native_available",
    "sddmm_csr_auto",
    "spmm_csr",
    "spmm_csr_auto",
    "validate_csr",
]
