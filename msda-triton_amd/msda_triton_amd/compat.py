"""Call-site shims for code written against mmcv / Deformable-DETR.

Deformable-DETR, DINO and mmcv-based models call
``MultiScaleDeformableAttnFunction.apply(value, value_spatial_shapes,
value_level_start_index, sampling_locations, attention_weights,
im2col_step)`` (Deformable-DETR names it ``MSDeformAttnFunction``); the
reference benchmarks exactly that call shape against its own operator
(benchmarks/modal_benchmark.py:231-233) and describes its operator as that
function minus ``im2col_step`` (README.md:72).  These classes keep that
signature and route to the MI355X operator.  ``im2col_step`` only chunked the
batch in mmcv's CUDA kernel launch; the HIP kernels process the whole batch
(slicing it themselves when 32-bit addressing requires), so it is accepted
and ignored.
"""

from __future__ import annotations

from .ops import multi_scale_deformable_attention


class MultiScaleDeformableAttnFunction:
    """``MultiScaleDeformableAttnFunction.apply(value, spatial_shapes,
    level_start_index, sampling_locations, attention_weights, im2col_step)``
    -> ``(B, Q, M*D)``, differentiable in value, sampling_locations and
    attention_weights."""

    @staticmethod
    def apply(value, value_spatial_shapes, value_level_start_index, sampling_locations,
              attention_weights, im2col_step=None):
        del im2col_step
        return multi_scale_deformable_attention(value, value_spatial_shapes,
                                                value_level_start_index, sampling_locations,
                                                attention_weights)


# Deformable-DETR's name for the same function.
MSDeformAttnFunction = MultiScaleDeformableAttnFunction
