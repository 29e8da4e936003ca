"""Projections either side of the operator on the HIP MFMA kernels.

The reference's attention layer (labs/solutions/lab00.py:187-208) wraps the
operator in four ``nn.Linear`` projections: ``value_proj`` feeding ``value``
(B, S, M, D), ``offset_proj`` and ``weight_proj`` of the query rows, and
``out_proj`` of the operator's output.  ``projection`` computes them with the
library's ``msda_projection_forward`` / ``msda_projection_backward``:

* ``y = input @ weight.T + bias`` with fp32 accumulation and one rounding,
  rows flagged in ``row_mask`` set to zero (Deformable-DETR's
  ``value.masked_fill(padding_mask[..., None], 0)`` fused into the epilogue);
* ``weight2`` / ``bias2`` add a second output from the same input rows in the
  same pass (the offset and logit projections of the query);
* the backward computes ``grad_input`` with the same kernel (masked rows get
  zero gradient) and ``grad_weight`` / ``grad_bias`` from per-chunk partials
  reduced in a fixed order -- bitwise reproducible run to run.

There is no fallback: CPU tensors raise, a missing library raises.
"""

from __future__ import annotations

import torch

from . import _native
from .ops import _DTYPE_CODE, _on_device, _ptr, _stream


def _check(input, weight, bias, weight2, bias2, row_mask):
    if input.device.type != "cuda":
        raise ValueError("projection requires CUDA (HIP) tensors")
    if input.dtype not in _DTYPE_CODE:
        raise ValueError(f"unsupported dtype {input.dtype}")
    for name, t in (("weight", weight), ("bias", bias), ("weight2", weight2), ("bias2", bias2)):
        if t is None:
            continue
        if t.dtype != input.dtype or t.device != input.device:
            raise ValueError(f"{name} must match input's dtype and device")
    if input.dim() < 1 or weight.dim() != 2 or weight.shape[1] != input.shape[-1]:
        raise ValueError("weight must be (out_features, in_features) with in_features == "
                         "input.shape[-1]")
    if bias is not None and bias.shape != (weight.shape[0],):
        raise ValueError("bias must be (out_features,)")
    if weight2 is not None:
        if weight2.dim() != 2 or weight2.shape[1] != input.shape[-1]:
            raise ValueError("weight2 must be (out_features2, in_features)")
        if bias2 is not None and bias2.shape != (weight2.shape[0],):
            raise ValueError("bias2 must be (out_features2,)")
    elif bias2 is not None:
        raise ValueError("bias2 given without weight2")
    if row_mask is not None:
        if row_mask.shape != input.shape[:-1]:
            raise ValueError("row_mask must have shape input.shape[:-1]")
        if row_mask.dtype not in (torch.bool, torch.uint8):
            raise ValueError("row_mask must be bool or uint8")


def _mask_bytes(row_mask, dev):
    if row_mask is None:
        return None
    m = row_mask.to(device=dev)
    if m.dtype == torch.bool:
        m = m.view(torch.uint8)
    return m.contiguous()


class _ProjectionFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, input, weight, bias, weight2, bias2, mask):
        lead = input.shape[:-1]
        x = input.contiguous()
        w = weight.contiguous()
        w2 = None if weight2 is None else weight2.contiguous()
        b = None if bias is None else bias.contiguous()
        b2 = None if bias2 is None else bias2.contiguous()
        rows = x.numel() // x.shape[-1] if x.shape[-1] else 0
        n1 = w.shape[0]
        n2 = 0 if w2 is None else w2.shape[0]
        y = torch.empty(*lead, n1, dtype=x.dtype, device=x.device)
        y2 = None if w2 is None else torch.empty(*lead, n2, dtype=x.dtype, device=x.device)
        with _on_device(x):
            rc = _native.load().msda_projection_forward(
                _ptr(x), _ptr(w), _ptr(b), _ptr(w2), _ptr(b2), _ptr(mask), _ptr(y), _ptr(y2),
                rows, x.shape[-1], n1 + n2, n1, _DTYPE_CODE[x.dtype], _stream(x))
        _native.check(rc, "msda_projection_forward")
        ctx.save_for_backward(x, w, w2, mask)
        ctx.has_bias = (bias is not None, bias2 is not None)
        return (y,) if y2 is None else (y, y2)

    @staticmethod
    def backward(ctx, gy, gy2=None):
        x, w, w2, mask = ctx.saved_tensors
        need_x, need_w, need_b, need_w2, need_b2, _ = ctx.needs_input_grad
        need_b = need_b and ctx.has_bias[0]
        need_b2 = need_b2 and ctx.has_bias[1]
        rows = x.numel() // x.shape[-1] if x.shape[-1] else 0
        n1 = w.shape[0]
        n2 = 0 if w2 is None else w2.shape[0]
        dt = _DTYPE_CODE[x.dtype]
        gy = gy.contiguous()
        if w2 is not None:
            gy2 = (torch.zeros(*x.shape[:-1], n2, dtype=x.dtype, device=x.device)
                   if gy2 is None else gy2.contiguous())
        gx = torch.empty_like(x) if need_x else None
        gw = torch.empty_like(w) if need_w else None
        gb = torch.empty(n1, dtype=x.dtype, device=x.device) if need_b else None
        gw2 = torch.empty_like(w2) if need_w2 else None
        gb2 = torch.empty(n2, dtype=x.dtype, device=x.device) if need_b2 else None
        lib = _native.load()
        ws = None
        # grad_input needs the workspace too (it holds the transposed weights).
        if (need_x and rows > 0) or need_w or need_b or need_w2 or need_b2:
            nbytes = lib.msda_projection_workspace_bytes(rows, x.shape[-1], n1 + n2, dt)
            if nbytes < 0:
                raise RuntimeError("msda_projection_workspace_bytes rejected the shape")
            ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=x.device)
        with _on_device(x):
            rc = lib.msda_projection_backward(
                _ptr(x), _ptr(w), _ptr(w2), _ptr(mask), _ptr(gy), _ptr(gy2), _ptr(gx), _ptr(gw),
                _ptr(gb), _ptr(gw2), _ptr(gb2), _ptr(ws), rows, x.shape[-1], n1 + n2, n1, dt,
                _stream(x))
        _native.check(rc, "msda_projection_backward")
        return gx, gw, gb, gw2, gb2, None


def projection(input: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None, *,
               row_mask: torch.Tensor | None = None, weight2: torch.Tensor | None = None,
               bias2: torch.Tensor | None = None):
    """``input @ weight.T + bias`` (``torch.nn.functional.linear``) on the HIP
    projection kernels, differentiable in input, weights and biases.

    Args:
        input: ``(..., in_features)`` fp32 / fp16 / bf16 on a HIP device;
            ``in_features`` a multiple of 16 bytes (8 half or 4 fp32 elements),
            at most 512 for half precision.
        weight: ``(out_features, in_features)``, bias ``(out_features,)`` or None.
        row_mask: bool / uint8 of shape ``input.shape[:-1]``; flagged rows of
            the output are zero (and receive zero gradient).
        weight2, bias2: a second projection of the same rows, computed in the
            same pass; then ``(y, y2)`` is returned.
    """
    _check(input, weight, bias, weight2, bias2, row_mask)
    mask = _mask_bytes(row_mask, input.device)
    out = _ProjectionFunction.apply(input, weight, bias, weight2, bias2, mask)
    return out[0] if weight2 is None else out
