"""GPU kernels of the spectral decode path (HIP for gfx950).

Same names as unsloth_spectral/kernels/__init__.py:37-67.  There is no
Triton here and no optional import: the entry points always run the HIP
kernels of libspectral_hip.so.  ``TRITON_AVAILABLE`` stays False (no Triton
kernel exists); ``HIP_AVAILABLE`` reports whether the library loads.
"""
from .. import _lib
from .spectral_attention import (  # noqa: F401
    TritonSpectralConfig,
    spectral_attention_decode,
    spectral_score_forward,
    spectral_value_forward,
)

TRITON_AVAILABLE = False
TRITON_VERSION = None

try:
    _lib.load()
    HIP_AVAILABLE = True
except ImportError:
    HIP_AVAILABLE = False

__all__ = [
    "spectral_attention_decode",
    "spectral_score_forward",
    "spectral_value_forward",
    "TritonSpectralConfig",
    "TRITON_AVAILABLE",
    "TRITON_VERSION",
    "HIP_AVAILABLE",
]
