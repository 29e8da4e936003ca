"""Public MSDA operator on MI355X: HIP kernels (libmsda_hip.so) behind a
torch.autograd.Function.

Mirrors the reference's operator boundary, src/msda_triton/ops.py:96-199
(validation, defaults, early return) and its autograd Function,
src/msda_triton/ops.py:36-93, with the Triton launches replaced by calls into
the C ABI of include/msda_hip.h.
"""

from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from . import _native

_FLOAT_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
_DTYPE_CODE = {
    torch.float32: _native.DTYPE_F32,
    torch.float16: _native.DTYPE_F16,
    torch.bfloat16: _native.DTYPE_BF16,
}


def _use_fp32_grad_accum(value: torch.Tensor) -> bool:
    """Default accumulator for grad_value (reference: src/msda_triton/ops.py:
    21-33, which picks fp32 only where the dtype's atomic add would be an
    emulated compare-and-swap loop).  gfx950 has native fp32, packed-fp16 and
    packed-bf16 global atomics, so the native-dtype path is used for every
    dtype, as the reference does on SM >= 9.0.  The default (row-dedup)
    backward sums every row's contributions inside a workgroup in fp32 before
    its one rounded atomic, which keeps native half-precision accumulation
    within tolerance even when many samples share corners.  ``True`` still
    gives a full fp32 accumulation, rounded once."""
    del value
    return False


def _use_deterministic(deterministic: bool | None) -> bool:
    """``None`` follows ``torch.use_deterministic_algorithms``: grad_value is
    then bitwise reproducible (the other gradients always are)."""
    if deterministic is None:
        return torch.are_deterministic_algorithms_enabled()
    return bool(deterministic)


def deterministic_workspace(value: torch.Tensor,
                            sampling_locations: torch.Tensor) -> torch.Tensor | None:
    """Scratch of the deterministic backward (the int64 accumulator), sized
    by the library for this shape; None when the call takes the owner path,
    which is reproducible without one."""
    B, S, M, D = value.shape
    _, Q, _, L, K, _ = sampling_locations.shape
    nbytes = _native.load().msda_deterministic_workspace_bytes(B, S, M, D, Q, L, K,
                                                               _DTYPE_CODE[value.dtype])
    if nbytes < 0:
        raise ValueError("unsupported shape or dtype for the deterministic backward")
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=value.device)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> int:
    """torch's current HIP stream on t's device, as the raw handle the C ABI
    takes (without building a Stream object per call)."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


class _on_device:
    """The C ABI launches on the current HIP device; make t's device current
    for the call (restoring it after), at no cost when it already is."""

    __slots__ = ("idx", "prev")

    def __init__(self, t: torch.Tensor):
        self.idx = t.device.index
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if cur != self.idx:
            self.prev = cur
            torch.cuda.set_device(self.idx)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False


def _as_index_tensor(t: torch.Tensor, dev: torch.device) -> torch.Tensor:
    """int64, on dev, contiguous -- without a copy (or a call) when it is."""
    if t.device != dev or t.dtype != torch.int64:
        t = t.to(device=dev, dtype=torch.int64)
    return t if t.is_contiguous() else t.contiguous()


class _MSDAFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, value, spatial_shapes, level_start_index, sampling_locations,
                attention_weights, fp32_grad_accum, deterministic=False):
        B, S, M, D = value.shape
        _, Q, _, L, K, _ = sampling_locations.shape
        lib = _native.load()
        out = value.new_empty(B, Q, M, D)
        with _on_device(value):
            rc = lib.msda_forward(
                _ptr(value), _ptr(spatial_shapes), _ptr(level_start_index),
                _ptr(sampling_locations), _ptr(attention_weights), _ptr(out),
                B, S, M, D, Q, L, K, _DTYPE_CODE[value.dtype], _stream(value),
            )
        _native.check(rc, "msda_forward")
        ctx.save_for_backward(value, spatial_shapes, level_start_index,
                              sampling_locations, attention_weights)
        ctx.fp32_grad_accum = fp32_grad_accum
        ctx.deterministic = deterministic
        return out.view(B, Q, M * D)

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_out):
        value, spatial_shapes, level_start_index, sampling_locations, attention_weights = (
            ctx.saved_tensors
        )
        grad_value, grad_loc, grad_attn = backward_raw(
            value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
            grad_out, ctx.fp32_grad_accum, ctx.deterministic)
        return grad_value, None, None, grad_loc, grad_attn, None, None


def aligned_rows(t: torch.Tensor) -> torch.Tensor:
    """t contiguous and 16-byte aligned.  A contiguous view can start at any
    element offset; the owner-computes backward reads grad_output in 16-byte
    chunks and is taken only for aligned pointers -- it is also the
    deterministic backward that needs no workspace, so a misaligned view
    would otherwise be refused there."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone(memory_format=torch.contiguous_format)


def backward_raw(value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
                 grad_out, fp32_grad_accum: bool, deterministic: bool):
    """One call of ``msda_backward`` (or ``msda_backward_deterministic``) on
    prepared tensors; returns (grad_value, grad_loc, grad_attn)."""
    B, S, M, D = value.shape
    _, Q, _, L, K, _ = sampling_locations.shape
    grad_out = aligned_rows(grad_out.reshape(B, Q, M, D))
    lib = _native.load()
    grad_value = torch.empty_like(value)  # written in full by the library
    grad_loc = torch.empty_like(sampling_locations)
    grad_attn = torch.empty_like(attention_weights)
    with _on_device(value):
        if deterministic:
            ws = deterministic_workspace(value, sampling_locations)
            rc = lib.msda_backward_deterministic(
                _ptr(value), _ptr(spatial_shapes), _ptr(level_start_index),
                _ptr(sampling_locations), _ptr(attention_weights), _ptr(grad_out),
                _ptr(grad_value), _ptr(ws), _ptr(grad_loc), _ptr(grad_attn),
                B, S, M, D, Q, L, K, _DTYPE_CODE[value.dtype], _stream(value))
            _native.check(rc, "msda_backward_deterministic")
        else:
            accum = None
            if fp32_grad_accum and value.dtype != torch.float32:
                accum = torch.empty(value.shape, dtype=torch.float32, device=value.device)
            rc = lib.msda_backward(
                _ptr(value), _ptr(spatial_shapes), _ptr(level_start_index),
                _ptr(sampling_locations), _ptr(attention_weights), _ptr(grad_out),
                _ptr(grad_value), _ptr(accum), _ptr(grad_loc), _ptr(grad_attn),
                B, S, M, D, Q, L, K, _DTYPE_CODE[value.dtype], _stream(value))
            _native.check(rc, "msda_backward")
    return grad_value, grad_loc, grad_attn


def multi_scale_deformable_attention(
    value: torch.Tensor,
    spatial_shapes: torch.Tensor,
    level_start_index: torch.Tensor | None,
    sampling_locations: torch.Tensor,
    attention_weights: torch.Tensor,
    *,
    fp32_grad_accum: bool | None = None,
    deterministic: bool | None = None,
) -> torch.Tensor:
    """Multi-scale deformable attention (Zhu et al. 2021, Eq. 1) on MI355X.

    For each query, head, feature level l and sampling point k, bilinearly
    samples ``value`` at ``sampling_locations`` and aggregates the samples
    weighted by ``attention_weights``.  Sampling uses ``x_im = x * W_l - 0.5``
    (== ``grid_sample`` with ``align_corners=False, padding_mode="zeros"``).
    Same signature and semantics as the reference,
    src/msda_triton/ops.py:96-138.

    Args:
        value: ``(B, S, M, D)`` flattened multi-scale feature maps,
            ``S = sum_l H_l * W_l``, ``M`` heads, head dim ``D``.
        spatial_shapes: ``(L, 2)`` integer ``(H_l, W_l)`` per level.
        level_start_index: ``(L,)`` integer offset of each level along ``S``,
            or ``None`` to compute it from ``spatial_shapes``.
        sampling_locations: ``(B, Q, M, L, K, 2)`` normalized ``(x, y)``;
            locations outside ``[0, 1]`` sample zeros.
        attention_weights: ``(B, Q, M, L, K)``.
        fp32_grad_accum: accumulate ``grad_value`` in an fp32 scratch buffer
            (rounded once to the value dtype) instead of native-dtype atomics.
            ``None`` selects the native atomics (see ``_use_fp32_grad_accum``).
        deterministic: make ``grad_value`` bitwise reproducible (decoder-style
            calls are on their default path; others accumulate in int64
            fixed point, exact sums, slower).  ``None`` follows
            ``torch.are_deterministic_algorithms_enabled()``.  Overrides
            ``fp32_grad_accum``.  Not in the reference's signature (keyword
            only, so calls written for the reference are unaffected).

    Returns:
        ``(B, Q, M * D)`` output, same dtype as ``value``.

    Note:
        By default ``grad_value`` of encoder-style calls (many samples per
        batch, head and level) is accumulated with floating-point atomics,
        so it is not bitwise deterministic (as in the reference); see
        ``deterministic``.  Decoder-style calls are reproducible either way.
    """
    prep = _prepare(value, spatial_shapes, level_start_index, sampling_locations,
                    attention_weights, fp32_grad_accum, deterministic)
    if isinstance(prep, torch.Tensor):  # B == 0 or Q == 0: no autograd link
        return prep
    return _MSDAFunction.apply(*prep)


def _prepare(value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
             fp32_grad_accum, deterministic=None):
    """Validation and defaults of the operator boundary
    (src/msda_triton/ops.py:140-199).  Returns the empty output for B == 0 or
    Q == 0, else the argument tuple of the device computation."""
    if value.dim() != 4:
        raise ValueError(f"value must be (B, S, M, D), got {tuple(value.shape)}")
    if sampling_locations.dim() != 6 or sampling_locations.shape[-1] != 2:
        raise ValueError(
            f"sampling_locations must be (B, Q, M, L, K, 2), got {tuple(sampling_locations.shape)}"
        )
    B, S, M, D = value.shape
    _, Q, _, L, K, _ = sampling_locations.shape
    if sampling_locations.shape[0] != B or sampling_locations.shape[2] != M:
        raise ValueError(
            f"sampling_locations {tuple(sampling_locations.shape)} inconsistent with value "
            f"{tuple(value.shape)}"
        )
    if attention_weights.shape != (B, Q, M, L, K):
        raise ValueError(
            f"attention_weights must be {(B, Q, M, L, K)}, got {tuple(attention_weights.shape)}"
        )
    if spatial_shapes.shape != (L, 2):
        raise ValueError(f"spatial_shapes must be ({L}, 2), got {tuple(spatial_shapes.shape)}")
    if not (value.dtype == sampling_locations.dtype == attention_weights.dtype):
        raise ValueError(
            f"value/sampling_locations/attention_weights dtypes must match, got "
            f"{value.dtype}/{sampling_locations.dtype}/{attention_weights.dtype}"
        )
    if value.dtype not in _FLOAT_DTYPES:
        raise ValueError(f"unsupported dtype {value.dtype}; use fp32, fp16 or bf16")
    if value.device.type != "cuda":
        raise ValueError(
            "the operator requires CUDA-API (ROCm/HIP) device tensors; for CPU use a "
            "grid_sample-based reference implementation"
        )
    if not (value.device == sampling_locations.device == attention_weights.device):
        raise ValueError("value, sampling_locations and attention_weights must share a device")

    spatial_shapes = _as_index_tensor(spatial_shapes, value.device)
    if level_start_index is None:
        hw = spatial_shapes.prod(-1)
        level_start_index = torch.cat([hw.new_zeros(1), hw.cumsum(0)[:-1]])
    else:
        if level_start_index.shape != (L,):
            raise ValueError(
                f"level_start_index must be ({L},), got {tuple(level_start_index.shape)}"
            )
        level_start_index = _as_index_tensor(level_start_index, value.device)

    if B == 0 or Q == 0:
        return value.new_zeros(B, Q, M * D)

    if fp32_grad_accum is None:
        fp32_grad_accum = _use_fp32_grad_accum(value)

    return (
        value.contiguous(),
        spatial_shapes,
        level_start_index,
        sampling_locations.contiguous(),
        attention_weights.contiguous(),
        bool(fp32_grad_accum),
        _use_deterministic(deterministic),
    )
