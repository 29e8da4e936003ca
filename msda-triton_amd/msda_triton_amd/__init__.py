"""MI355X-native multi-scale deformable attention.

Drop-in for ``msda_triton`` (reference: src/msda_triton/__init__.py:9-12):
exports the same operator name and signature, computed by hand-written HIP
kernels for gfx950 (libmsda_hip.so).
"""

from .ops import multi_scale_deformable_attention

__all__ = ["multi_scale_deformable_attention"]
__version__ = "0.1.0"
