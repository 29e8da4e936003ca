"""The operator as `torch.library` custom ops: ``torch.ops.msda_amd.forward``
and ``torch.ops.msda_amd.backward``, with fake (shape) implementations and a
registered autograd formula.

`multi_scale_deformable_attention` in ops.py mirrors the reference's
`torch.autograd.Function` (src/msda_triton/ops.py:36-93), which
`torch.compile` cannot trace into: it graph-breaks around the opaque ctypes
calls.  Registered custom ops are traceable as single nodes
(`torch.compile(fullgraph=True)` works), so `msda_op` below is the entry for
compiled models.  Both entries call the same C ABI (include/msda_hip.h).
"""

from __future__ import annotations

import torch

from . import _native
from .ops import _DTYPE_CODE, _on_device, _prepare, _stream, backward_raw


@torch.library.custom_op("msda_amd::forward", mutates_args=(), device_types="cuda")
def _forward(value: torch.Tensor, spatial_shapes: torch.Tensor, level_start_index: torch.Tensor,
             sampling_locations: torch.Tensor, attention_weights: torch.Tensor,
             fp32_grad_accum: bool, deterministic: bool) -> torch.Tensor:
    B, S, M, D = value.shape
    _, Q, _, L, K, _ = sampling_locations.shape
    out = value.new_empty(B, Q, M * D)
    lib = _native.load()
    with _on_device(value):
        rc = lib.msda_forward(
            value.data_ptr(), spatial_shapes.data_ptr(), level_start_index.data_ptr(),
            sampling_locations.data_ptr(), attention_weights.data_ptr(), out.data_ptr(),
            B, S, M, D, Q, L, K, _DTYPE_CODE[value.dtype], _stream(value))
    _native.check(rc, "msda_forward")
    return out


@_forward.register_fake
def _forward_fake(value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
                  fp32_grad_accum, deterministic):
    B, S, M, D = value.shape
    return value.new_empty(B, sampling_locations.shape[1], M * D)


@torch.library.custom_op("msda_amd::backward", mutates_args=(), device_types="cuda")
def _backward(value: torch.Tensor, spatial_shapes: torch.Tensor, level_start_index: torch.Tensor,
              sampling_locations: torch.Tensor, attention_weights: torch.Tensor,
              grad_output: torch.Tensor, fp32_grad_accum: bool, deterministic: bool
              ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return backward_raw(value, spatial_shapes, level_start_index, sampling_locations,
                        attention_weights, grad_output, fp32_grad_accum, deterministic)


@_backward.register_fake
def _backward_fake(value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
                   grad_output, fp32_grad_accum, deterministic):
    return (torch.empty_like(value), torch.empty_like(sampling_locations),
            torch.empty_like(attention_weights))


def _setup_context(ctx, inputs, output):
    (value, spatial_shapes, level_start_index, sampling_locations, attention_weights, fp32,
     det) = inputs
    ctx.save_for_backward(value, spatial_shapes, level_start_index, sampling_locations,
                          attention_weights)
    ctx.fp32_grad_accum = fp32
    ctx.deterministic = det


def _autograd_backward(ctx, grad_out):
    value, spatial_shapes, level_start_index, sampling_locations, attention_weights = (
        ctx.saved_tensors)
    gv, gl, ga = torch.ops.msda_amd.backward(value, spatial_shapes, level_start_index,
                                             sampling_locations, attention_weights, grad_out,
                                             ctx.fp32_grad_accum, ctx.deterministic)
    return gv, None, None, gl, ga, None, None


torch.library.register_autograd("msda_amd::forward", _autograd_backward,
                                setup_context=_setup_context)


def msda_op(value, spatial_shapes, level_start_index, sampling_locations, attention_weights, *,
            fp32_grad_accum: bool | None = None, deterministic: bool | None = None):
    """Same contract as `multi_scale_deformable_attention` (validation,
    defaults, empty-input early return), computed through the registered
    custom ops so that `torch.compile` captures it as one node."""
    prep = _prepare(value, spatial_shapes, level_start_index, sampling_locations,
                    attention_weights, fp32_grad_accum, deterministic)
    if isinstance(prep, torch.Tensor):  # B == 0 or Q == 0
        return prep
    return torch.ops.msda_amd.forward(*prep)


# ---------------------------------------------------------------------------
# Fused front-end (fused.py) as custom ops: forward returns (out, lse).
# ---------------------------------------------------------------------------

@torch.library.custom_op("msda_amd::fused_forward", mutates_args=(), device_types="cuda")
def _fused_forward(value: torch.Tensor, spatial_shapes: torch.Tensor,
                   level_start_index: torch.Tensor, reference_points: torch.Tensor,
                   sampling_offsets: torch.Tensor, attention_logits: torch.Tensor,
                   fp32_grad_accum: bool, ref_levels: int, deterministic: bool
                   ) -> tuple[torch.Tensor, torch.Tensor]:
    from .fused import fused_forward_raw

    out, lse = fused_forward_raw(value, spatial_shapes, level_start_index, reference_points,
                                 sampling_offsets, attention_logits, ref_levels)
    B, Q, M, D = out.shape
    return out.view(B, Q, M * D), lse


@_fused_forward.register_fake
def _fused_forward_fake(value, spatial_shapes, level_start_index, reference_points,
                        sampling_offsets, attention_logits, fp32_grad_accum, ref_levels,
                        deterministic):
    B, S, M, D = value.shape
    Q = sampling_offsets.shape[1]
    return (value.new_empty(B, Q, M * D),
            value.new_empty(B, Q, M, dtype=torch.float32))


@torch.library.custom_op("msda_amd::fused_backward", mutates_args=(), device_types="cuda")
def _fused_backward(value: torch.Tensor, spatial_shapes: torch.Tensor,
                    level_start_index: torch.Tensor, reference_points: torch.Tensor,
                    sampling_offsets: torch.Tensor, attention_logits: torch.Tensor,
                    lse: torch.Tensor, out: torch.Tensor, grad_output: torch.Tensor,
                    fp32_grad_accum: bool, ref_levels: int, deterministic: bool
                    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    from .fused import fused_backward_raw

    B, S, M, D = value.shape
    Q = sampling_offsets.shape[1]
    return fused_backward_raw(value, spatial_shapes, level_start_index, reference_points,
                              sampling_offsets, attention_logits, lse, out.view(B, Q, M, D),
                              grad_output, ref_levels, fp32_grad_accum, need_ref_grad=True,
                              deterministic=deterministic)


@_fused_backward.register_fake
def _fused_backward_fake(value, spatial_shapes, level_start_index, reference_points,
                         sampling_offsets, attention_logits, lse, out, grad_output,
                         fp32_grad_accum, ref_levels, deterministic):
    return (torch.empty_like(value), torch.empty_like(reference_points),
            torch.empty_like(sampling_offsets), torch.empty_like(attention_logits))


def _fused_setup_context(ctx, inputs, output):
    (value, spatial_shapes, level_start_index, reference_points, sampling_offsets,
     attention_logits, fp32, ref_levels, det) = inputs
    out, lse = output
    ctx.save_for_backward(value, spatial_shapes, level_start_index, reference_points,
                          sampling_offsets, attention_logits, lse, out)
    ctx.fp32_grad_accum = fp32
    ctx.ref_levels = ref_levels
    ctx.deterministic = det


def _fused_autograd_backward(ctx, grad_out, grad_lse):
    del grad_lse  # the log-sum-exp is an auxiliary output
    (value, spatial_shapes, level_start_index, reference_points, sampling_offsets,
     attention_logits, lse, out) = ctx.saved_tensors
    gv, gref, goff, glog = torch.ops.msda_amd.fused_backward(
        value, spatial_shapes, level_start_index, reference_points, sampling_offsets,
        attention_logits, lse, out, grad_out, ctx.fp32_grad_accum, ctx.ref_levels,
        ctx.deterministic)
    return gv, None, None, gref, goff, glog, None, None, None


torch.library.register_autograd("msda_amd::fused_forward", _fused_autograd_backward,
                                setup_context=_fused_setup_context)


def msda_fused_op(value, spatial_shapes, level_start_index, reference_points, sampling_offsets,
                  attention_logits, *, fp32_grad_accum: bool | None = None,
                  deterministic: bool | None = None):
    """Same contract as `multi_scale_deformable_attention_fused`, through the
    registered custom ops (one graph node under `torch.compile`)."""
    from .fused import _prepare_fused

    prep = _prepare_fused(value, spatial_shapes, level_start_index, reference_points,
                          sampling_offsets, attention_logits, fp32_grad_accum, deterministic)
    if isinstance(prep, torch.Tensor):
        return prep
    out, _ = torch.ops.msda_amd.fused_forward(*prep)
    return out
