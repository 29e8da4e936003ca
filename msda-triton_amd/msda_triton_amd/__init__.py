"""MI355X-native multi-scale deformable attention.

Drop-in for ``msda_triton`` (reference: src/msda_triton/__init__.py:9-12):
exports the same operator name and signature, computed by hand-written HIP
kernels for gfx950 (libmsda_hip.so).
"""

from .ops import multi_scale_deformable_attention

__all__ = ["multi_scale_deformable_attention", "msda_op", "MultiScaleDeformableAttnFunction",
           "MSDeformAttnFunction", "multi_scale_deformable_attention_fused", "MSDACrossAttention",
           "msda_fused_op"]


def __getattr__(name):
    # torch.library registration, the mmcv / Deformable-DETR shims and the
    # fused front-end load on first use, keeping `import msda_triton_amd` as
    # light as the reference's.
    if name in ("msda_op", "msda_fused_op"):
        from . import library

        return getattr(library, name)
    if name in ("MultiScaleDeformableAttnFunction", "MSDeformAttnFunction"):
        from . import compat

        return getattr(compat, name)
    if name in ("multi_scale_deformable_attention_fused", "MSDACrossAttention"):
        from . import fused

        return getattr(fused, name)
    raise AttributeError(name)


__version__ = "0.1.0"
