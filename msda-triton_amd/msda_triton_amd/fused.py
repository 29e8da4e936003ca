"""Fused MSDeformAttn front-end: softmax of the attention logits and
reference point + offset / (W_l, H_l) computed inside the HIP kernels.

The reference's attention layer (labs/solutions/lab00.py:194-208,
``MSDACrossAttention.forward``) builds the operator's inputs with three
PyTorch ops

    weights   = weight_proj(query).reshape(B, Q, M, L*K).softmax(-1)
    locations = reference_points[:, :, None, None, None, :]
                + offsets / spatial_shapes.flip(-1)[None, None, None, :, None, :]

and then calls ``multi_scale_deformable_attention``.  Here the kernels take
the reference points, offsets and logits directly (C ABI
``msda_fused_forward`` / ``msda_fused_backward``), so the (B, Q, M, L, K)
locations and weights are never written to or read back from memory, and
their backward (softmax backward, division, broadcast sum) happens in the
same kernels.  The forward also returns each (b, q, m)'s log-sum-exp of the
logits, which the backward reuses.
"""

from __future__ import annotations

import torch
from torch import nn
from torch.autograd.function import once_differentiable

from . import _native
from .ops import (_DTYPE_CODE, _FLOAT_DTYPES, _as_index_tensor, _on_device, _ptr, _stream,
                  _use_deterministic, _use_fp32_grad_accum, aligned_rows,
                  deterministic_workspace)


def fused_forward_raw(value, spatial_shapes, level_start_index, reference_points,
                      sampling_offsets, attention_logits, ref_levels: int, need_lse: bool = True):
    """One call of ``msda_fused_forward`` on prepared (contiguous, validated)
    tensors.  Returns ``(out (B, Q, M, D), lse (B, Q, M) fp32 or None)``."""
    B, S, M, D = value.shape
    _, Q, _, L, K, _ = sampling_offsets.shape
    out = value.new_empty(B, Q, M, D)
    lse = (torch.empty(B, Q, M, dtype=torch.float32, device=value.device)
           if need_lse else None)
    lib = _native.load()
    with _on_device(value):
        rc = lib.msda_fused_forward(
            _ptr(value), _ptr(spatial_shapes), _ptr(level_start_index), _ptr(reference_points),
            _ptr(sampling_offsets), _ptr(attention_logits), _ptr(out), _ptr(lse),
            B, S, M, D, Q, L, K, ref_levels, _DTYPE_CODE[value.dtype], _stream(value))
    _native.check(rc, "msda_fused_forward")
    return out, lse


def fused_backward_raw(value, spatial_shapes, level_start_index, reference_points,
                       sampling_offsets, attention_logits, lse, out, grad_out, ref_levels: int,
                       fp32_grad_accum: bool, need_ref_grad: bool = True,
                       deterministic: bool = False):
    """One call of ``msda_fused_backward`` (``_deterministic``).  Returns
    ``(grad_value, grad_reference_points or None, grad_offsets, grad_logits)``."""
    B, S, M, D = value.shape
    _, Q, _, L, K, _ = sampling_offsets.shape
    grad_out = aligned_rows(grad_out.reshape(B, Q, M, D))
    grad_value = torch.empty_like(value)  # written in full by the library
    grad_ref = torch.empty_like(reference_points) if need_ref_grad else None
    grad_off = torch.empty_like(sampling_offsets)
    grad_logits = torch.empty_like(attention_logits)
    lib = _native.load()
    if deterministic:
        fn, name, scratch = (lib.msda_fused_backward_deterministic,
                             "msda_fused_backward_deterministic",
                             deterministic_workspace(value, sampling_offsets))
    else:
        fn, name, scratch = lib.msda_fused_backward, "msda_fused_backward", None
        if fp32_grad_accum and value.dtype != torch.float32:
            scratch = torch.empty(value.shape, dtype=torch.float32, device=value.device)
    with _on_device(value):
        rc = fn(_ptr(value), _ptr(spatial_shapes), _ptr(level_start_index), _ptr(reference_points),
                _ptr(sampling_offsets), _ptr(attention_logits), _ptr(lse), _ptr(out),
                _ptr(grad_out), _ptr(grad_value), _ptr(scratch), _ptr(grad_ref), _ptr(grad_off),
                _ptr(grad_logits), B, S, M, D, Q, L, K, ref_levels, _DTYPE_CODE[value.dtype],
                _stream(value))
    _native.check(rc, name)
    return grad_value, grad_ref, grad_off, grad_logits


class _FusedMSDAFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, value, spatial_shapes, level_start_index, reference_points,
                sampling_offsets, attention_logits, fp32_grad_accum, ref_levels,
                deterministic=False):
        out, lse = fused_forward_raw(value, spatial_shapes, level_start_index, reference_points,
                                     sampling_offsets, attention_logits, ref_levels)
        ctx.save_for_backward(value, spatial_shapes, level_start_index, reference_points,
                              sampling_offsets, attention_logits, lse, out)
        ctx.fp32_grad_accum = fp32_grad_accum
        ctx.ref_levels = ref_levels
        ctx.deterministic = deterministic
        B, Q, M, D = out.shape
        return out.view(B, Q, M * D)

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_out):
        (value, spatial_shapes, level_start_index, reference_points, sampling_offsets,
         attention_logits, lse, out) = ctx.saved_tensors
        gv, gref, goff, glog = fused_backward_raw(
            value, spatial_shapes, level_start_index, reference_points, sampling_offsets,
            attention_logits, lse, out, grad_out, ctx.ref_levels, ctx.fp32_grad_accum,
            need_ref_grad=ctx.needs_input_grad[3], deterministic=ctx.deterministic)
        return gv, None, None, gref, goff, glog, None, None, None


def _prepare_fused(value, spatial_shapes, level_start_index, reference_points, sampling_offsets,
                   attention_logits, fp32_grad_accum, deterministic=None):
    """Validation and defaults.  Returns the empty output for B == 0 or Q == 0,
    else the argument tuple of the device computation (logits viewed as
    (B, Q, M, L, K))."""
    if value.dim() != 4:
        raise ValueError(f"value must be (B, S, M, D), got {tuple(value.shape)}")
    if sampling_offsets.dim() != 6 or sampling_offsets.shape[-1] != 2:
        raise ValueError(
            f"sampling_offsets must be (B, Q, M, L, K, 2), got {tuple(sampling_offsets.shape)}")
    B, S, M, D = value.shape
    _, Q, _, L, K, _ = sampling_offsets.shape
    if sampling_offsets.shape[0] != B or sampling_offsets.shape[2] != M:
        raise ValueError(f"sampling_offsets {tuple(sampling_offsets.shape)} inconsistent with "
                         f"value {tuple(value.shape)}")
    if attention_logits.shape == (B, Q, M, L * K):
        attention_logits = attention_logits.reshape(B, Q, M, L, K)
    if attention_logits.shape != (B, Q, M, L, K):
        raise ValueError(f"attention_logits must be {(B, Q, M, L, K)} or {(B, Q, M, L * K)}, "
                         f"got {tuple(attention_logits.shape)}")
    if reference_points.shape == (B, Q, 2):
        ref_levels = 0
    elif reference_points.shape == (B, Q, L, 2):
        ref_levels = 1
    else:
        raise ValueError(f"reference_points must be {(B, Q, 2)} or {(B, Q, L, 2)}, got "
                         f"{tuple(reference_points.shape)}")
    if spatial_shapes.shape != (L, 2):
        raise ValueError(f"spatial_shapes must be ({L}, 2), got {tuple(spatial_shapes.shape)}")
    dtypes = {value.dtype, sampling_offsets.dtype, attention_logits.dtype, reference_points.dtype}
    if len(dtypes) != 1:
        raise ValueError(
            f"value/reference_points/sampling_offsets/attention_logits dtypes must match, got "
            f"{value.dtype}/{reference_points.dtype}/{sampling_offsets.dtype}/"
            f"{attention_logits.dtype}")
    if value.dtype not in _FLOAT_DTYPES:
        raise ValueError(f"unsupported dtype {value.dtype}; use fp32, fp16 or bf16")
    if value.device.type != "cuda":
        raise ValueError("the operator requires CUDA-API (ROCm/HIP) device tensors")
    devices = {value.device, reference_points.device, sampling_offsets.device,
               attention_logits.device}
    if len(devices) != 1:
        raise ValueError("value, reference_points, sampling_offsets and attention_logits must "
                         "share a device")

    spatial_shapes = _as_index_tensor(spatial_shapes, value.device)
    if level_start_index is None:
        hw = spatial_shapes.prod(-1)
        level_start_index = torch.cat([hw.new_zeros(1), hw.cumsum(0)[:-1]])
    else:
        if level_start_index.shape != (L,):
            raise ValueError(
                f"level_start_index must be ({L},), got {tuple(level_start_index.shape)}")
        level_start_index = _as_index_tensor(level_start_index, value.device)

    if B == 0 or Q == 0:
        return value.new_zeros(B, Q, M * D)
    if fp32_grad_accum is None:
        fp32_grad_accum = _use_fp32_grad_accum(value)
    return (value.contiguous(), spatial_shapes, level_start_index, reference_points.contiguous(),
            sampling_offsets.contiguous(), attention_logits.contiguous(), bool(fp32_grad_accum),
            ref_levels, _use_deterministic(deterministic))


def multi_scale_deformable_attention_fused(
    value: torch.Tensor,
    spatial_shapes: torch.Tensor,
    level_start_index: torch.Tensor | None,
    reference_points: torch.Tensor,
    sampling_offsets: torch.Tensor,
    attention_logits: torch.Tensor,
    *,
    fp32_grad_accum: bool | None = None,
    deterministic: bool | None = None,
) -> torch.Tensor:
    """``multi_scale_deformable_attention(value, spatial_shapes,
    level_start_index, ref + offsets / (W_l, H_l), softmax(logits))`` in one
    fused operator (math of labs/solutions/lab00.py:201-208).

    Args:
        value: ``(B, S, M, D)``.
        spatial_shapes: ``(L, 2)`` integer ``(H_l, W_l)``.
        level_start_index: ``(L,)`` or ``None``.
        reference_points: ``(B, Q, 2)`` (shared by all levels) or
            ``(B, Q, L, 2)`` (per level), normalised ``(x, y)``.
        sampling_offsets: ``(B, Q, M, L, K, 2)`` in level-l pixel units.
        attention_logits: ``(B, Q, M, L, K)`` or ``(B, Q, M, L*K)``; the
            softmax runs over the L*K points of each (b, q, m).
        fp32_grad_accum, deterministic: as in ``multi_scale_deformable_attention``.

    Returns:
        ``(B, Q, M * D)`` in the value dtype.  Differentiable in value,
        reference_points, sampling_offsets and attention_logits.
    """
    prep = _prepare_fused(value, spatial_shapes, level_start_index, reference_points,
                          sampling_offsets, attention_logits, fp32_grad_accum, deterministic)
    if isinstance(prep, torch.Tensor):
        return prep
    return _FusedMSDAFunction.apply(*prep)


class MSDACrossAttention(nn.Module):
    """Deformable-DETR style multi-scale deformable attention layer on the
    fused operator.  Same constructor, parameters and forward contract as the
    reference's layer (labs/solutions/lab00.py:169-208): value/offset/weight/
    output projections; offsets in each level's pixel units; softmax over all
    L*K points; ``reference_points`` ``(B, Q, 2)`` (or ``(B, Q, L, 2)``) in
    [0, 1].  Returns ``(B, Q, C)``.

    The four projections run on the library's MFMA projection kernels
    (``projection.projection``): the value projection zeroes the rows flagged
    in ``input_padding_mask`` (``(B, S)`` bool, Deformable-DETR's padded
    pixels) in its epilogue, and the offset and logit projections share one
    pass over the query rows.  Those kernels need ``embed_dim`` and
    ``num_heads * num_levels * num_points`` to be multiples of 8; other
    configurations keep the ``nn.Linear`` modules' own GEMMs (padded rows are
    then zeroed with ``masked_fill``)."""

    def __init__(self, embed_dim: int, num_heads: int, num_levels: int, num_points: int):
        super().__init__()
        if embed_dim % num_heads != 0:
            raise ValueError("embed_dim must be divisible by num_heads")
        self.num_heads = num_heads
        self.num_levels = num_levels
        self.num_points = num_points
        self.head_dim = embed_dim // num_heads
        M, L, K = num_heads, num_levels, num_points
        self.value_proj = nn.Linear(embed_dim, embed_dim)
        self.offset_proj = nn.Linear(embed_dim, M * L * K * 2)
        self.weight_proj = nn.Linear(embed_dim, M * L * K)
        self.out_proj = nn.Linear(embed_dim, embed_dim)
        self.native_projections = embed_dim % 8 == 0 and (M * L * K) % 8 == 0

    def forward(self, query, reference_points, value, spatial_shapes, level_start_index=None,
                *, input_padding_mask=None, fp32_grad_accum=None, deterministic=None):
        B, Q, _ = query.shape
        _, S, _ = value.shape
        M, L, K, D = self.num_heads, self.num_levels, self.num_points, self.head_dim
        if self.native_projections:
            from .projection import projection

            v = projection(value, self.value_proj.weight, self.value_proj.bias,
                           row_mask=input_padding_mask)
            offsets, logits = projection(query, self.offset_proj.weight, self.offset_proj.bias,
                                         weight2=self.weight_proj.weight,
                                         bias2=self.weight_proj.bias)
        else:
            v = self.value_proj(value)
            if input_padding_mask is not None:
                v = v.masked_fill(input_padding_mask[..., None], 0.0)
            offsets = self.offset_proj(query)
            logits = self.weight_proj(query)
        out = multi_scale_deformable_attention_fused(
            v.reshape(B, S, M, D), spatial_shapes, level_start_index, reference_points,
            offsets.reshape(B, Q, M, L, K, 2), logits.reshape(B, Q, M, L, K),
            fp32_grad_accum=fp32_grad_accum, deterministic=deterministic)
        if self.native_projections:
            return projection(out, self.out_proj.weight, self.out_proj.bias)
        return self.out_proj(out)
