"""unsloth_spectral -- spectral KV-cache compression on MI355X (gfx950).

Drop-in for the API of unsloth_spectral/__init__.py:76-108: the cache stores
cold 512-token blocks as K ~ C @ B (C: INT8 coefficients [T, k] with FP32
scales, B: FP16 basis [k, D]) plus an FP16 tail, and decode attention runs
directly on (C, B) in a fused HIP kernel.  All compute runs through
libspectral_hip.so (built in-tree by unsloth-spectral_amd/build.py); there is
no CPU fallback.
"""
import os

__version__ = "0.1.0"

from .spectral_cache import SpectralBlock, SpectralCache  # noqa: E402
from .spectral_attention import (  # noqa: E402
    apply_rope,
    repeat_kv,
    repeat_kv_spectral,
    spectral_attention_forward,
    validate_spectral_attention,
)
from .rsvd import batched_randomized_svd, compress_matrices  # noqa: E402
from .kernels import (  # noqa: E402
    HIP_AVAILABLE,
    TRITON_AVAILABLE,
    TRITON_VERSION,
    TritonSpectralConfig,
    spectral_attention_decode,
    spectral_score_forward,
    spectral_value_forward,
)
from .integration import CapturedDecode, get_cache_stats, patch_unsloth_attention  # noqa: E402

__all__ = [
    "CapturedDecode",
    "SpectralCache",
    "SpectralBlock",
    "spectral_attention_forward",
    "spectral_attention_decode",
    "spectral_score_forward",
    "spectral_value_forward",
    "validate_spectral_attention",
    "batched_randomized_svd",
    "patch_unsloth_attention",
    "get_cache_stats",
    "TritonSpectralConfig",
    "TRITON_AVAILABLE",
    "TRITON_VERSION",
    "HIP_AVAILABLE",
]


def print_banner():
    print("=" * 70)
    print(f"  UNSLOTH SPECTRAL v{__version__} (HIP / gfx950)")
    print("  Spectral KV-cache compression: INT8 C [T,k] + FP16 B [k,D]")
    print("  Fused decode attention: " + ("HIP kernels loaded" if HIP_AVAILABLE else "HIP library MISSING"))
    print("=" * 70)


if not os.environ.get("UNSLOTH_SPECTRAL_QUIET"):
    print_banner()
