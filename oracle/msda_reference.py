"""CPU restatement of the reference's MSDA oracle -- TEST INFRASTRUCTURE ONLY
(see oracle/__init__.py for who may import it).

The reference validates its kernels against a per-level
``torch.nn.functional.grid_sample`` implementation (tests/reference_impls.py:
12-45) whose own correctness is pinned by a pure-loop version
(tests/reference_impls.py:48-87, tests/test_msda.py:101-120).  Both are
restated here from their published algorithm, together with the hand-derived
flat-index backward of labs/solutions/lab07.py:12-104, which gives gradients
that do not go through grid_sample's autograd.

Conventions (src/msda_triton/kernels.py:29-34): normalised location x in
[0, 1] maps to image coordinate x * W_l - 0.5, i.e. grid_sample with
align_corners=False and padding_mode="zeros" on the grid 2x - 1.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def level_start_index_of(spatial_shapes: torch.Tensor) -> torch.Tensor:
    """Exclusive cumulative sum of H_l * W_l (src/msda_triton/ops.py:174-176)."""
    hw = spatial_shapes.prod(-1)
    return torch.cat([hw.new_zeros(1), hw.cumsum(0)[:-1]])


def msda_reference(
    value: torch.Tensor,
    spatial_shapes: torch.Tensor,
    sampling_locations: torch.Tensor,
    attention_weights: torch.Tensor,
) -> torch.Tensor:
    """MSDA through one ``F.grid_sample`` call per level.

    Follows tests/reference_impls.py:12-45: split value by level, view each
    level as a (B*M, D, H, W) image, sample it at the (B*M, Q, K) grid
    ``2 * loc - 1``, weight the L*K samples by the attention weights and sum.
    Differentiable through torch autograd.  Returns (B, Q, M*D).
    """
    B, S, M, D = value.shape
    _, Q, _, L, K, _ = sampling_locations.shape
    sizes = [(int(h), int(w)) for h, w in spatial_shapes.tolist()]
    per_level = value.split([h * w for h, w in sizes], dim=1)
    grid = 2 * sampling_locations - 1  # [0,1] -> [-1,1]
    samples = []
    for lvl, (h, w) in enumerate(sizes):
        # (B, h*w, M, D) -> (B, M, D, h*w) -> (B*M, D, h, w)
        img = per_level[lvl].permute(0, 2, 3, 1).reshape(B * M, D, h, w)
        # (B, Q, M, K, 2) -> (B, M, Q, K, 2) -> (B*M, Q, K, 2)
        g = grid[:, :, :, lvl].permute(0, 2, 1, 3, 4).reshape(B * M, Q, K, 2)
        samples.append(
            F.grid_sample(img, g, mode="bilinear", padding_mode="zeros", align_corners=False)
        )  # (B*M, D, Q, K)
    stacked = torch.cat(samples, dim=-1)  # (B*M, D, Q, L*K), level-major
    attn = attention_weights.permute(0, 2, 1, 3, 4).reshape(B * M, 1, Q, L * K)
    out = (stacked * attn).sum(-1)  # (B*M, D, Q)
    return out.reshape(B, M * D, Q).transpose(1, 2).contiguous()


def msda_naive(
    value: torch.Tensor,
    spatial_shapes: torch.Tensor,
    sampling_locations: torch.Tensor,
    attention_weights: torch.Tensor,
) -> torch.Tensor:
    """Pure-loop MSDA with hand-rolled bilinear interpolation (tiny inputs
    only), following tests/reference_impls.py:48-87.  Returns (B, Q, M*D)."""
    B, S, M, D = value.shape
    _, Q, _, L, K, _ = sampling_locations.shape
    sizes = [(int(h), int(w)) for h, w in spatial_shapes.tolist()]
    starts = [0]
    for h, w in sizes[:-1]:
        starts.append(starts[-1] + h * w)
    out = value.new_zeros(B, Q, M, D)
    for b in range(B):
        for q in range(Q):
            for m in range(M):
                for lvl, (h, w) in enumerate(sizes):
                    for k in range(K):
                        x = float(sampling_locations[b, q, m, lvl, k, 0]) * w - 0.5
                        y = float(sampling_locations[b, q, m, lvl, k, 1]) * h - 0.5
                        a = attention_weights[b, q, m, lvl, k]
                        x0, y0 = math.floor(x), math.floor(y)
                        fx, fy = x - x0, y - y0
                        for yy, xx, wt in (
                            (y0, x0, (1 - fx) * (1 - fy)),
                            (y0, x0 + 1, fx * (1 - fy)),
                            (y0 + 1, x0, (1 - fx) * fy),
                            (y0 + 1, x0 + 1, fx * fy),
                        ):
                            if 0 <= xx < w and 0 <= yy < h:
                                out[b, q, m] += a * wt * value[b, starts[lvl] + yy * w + xx, m]
    return out.view(B, Q, M * D)


def msda_backward_analytic(
    value: torch.Tensor,
    spatial_shapes: torch.Tensor,
    level_start_index: torch.Tensor,
    sampling_locations: torch.Tensor,
    attention_weights: torch.Tensor,
    grad_out: torch.Tensor,
    dtype: torch.dtype = torch.float32,
):
    """Hand-derived gradients, vectorised over (B, Q, M), looping over (l, k),
    following the derivation of labs/solutions/lab07.py:12-104 and
    src/msda_triton/kernels.py:248-291:

      grad_attn     = <g, sum_c w_c v_c>
      grad_loc[x]   = A W <g, (v01 - v00)(1 - ly) + (v11 - v10) ly>
      grad_loc[y]   = A H <g, (v10 - v00)(1 - lx) + (v11 - v01) lx>
      grad_value[c] += A w_c g      (index_add_ scatter)

    Returns (grad_value (B,S,M,D), grad_loc (B,Q,M,L,K,2), grad_attn
    (B,Q,M,L,K)) in `dtype`.
    """
    B, S, M, D = value.shape
    _, Q, _, L, K, _ = sampling_locations.shape
    flat = value.reshape(-1).to(dtype)
    loc = sampling_locations.to(dtype)
    attn = attention_weights.to(dtype)
    g = grad_out.reshape(B, Q, M, D).to(dtype)
    grad_value = torch.zeros(flat.numel(), dtype=dtype)
    grad_loc = torch.zeros(B, Q, M, L, K, 2, dtype=dtype)
    grad_attn = torch.zeros(B, Q, M, L, K, dtype=dtype)
    b_idx = torch.arange(B)[:, None, None]
    m_idx = torch.arange(M)[None, None, :]
    chan = torch.arange(D)
    row_base = (b_idx * S) * M + m_idx  # + pixel * M selects the (b, pixel, m) row

    for lvl in range(L):
        H = int(spatial_shapes[lvl, 0])
        W = int(spatial_shapes[lvl, 1])
        start = int(level_start_index[lvl])
        for k in range(K):
            x = loc[:, :, :, lvl, k, 0] * W - 0.5
            y = loc[:, :, :, lvl, k, 1] * H - 0.5
            a = attn[:, :, :, lvl, k]
            x0f, y0f = torch.floor(x), torch.floor(y)
            lx, ly = x - x0f, y - y0f
            x0, y0 = x0f.long(), y0f.long()
            corners = []
            for dy, dx in ((0, 0), (0, 1), (1, 0), (1, 1)):
                xc, yc = x0 + dx, y0 + dy
                valid = (xc >= 0) & (xc < W) & (yc >= 0) & (yc < H)
                idx = ((row_base + (start + yc * W + xc) * M) * D)[..., None] + chan
                idx = torch.where(valid[..., None], idx, torch.zeros_like(idx))
                v = flat[idx] * valid[..., None].to(dtype)
                corners.append((idx, valid, v))
            (i00, m00, v00), (i01, m01, v01), (i10, m10, v10), (i11, m11, v11) = corners
            w00, w01 = (1 - lx) * (1 - ly), lx * (1 - ly)
            w10, w11 = (1 - lx) * ly, lx * ly
            sampled = (v00 * w00[..., None] + v01 * w01[..., None]
                       + v10 * w10[..., None] + v11 * w11[..., None])
            grad_attn[:, :, :, lvl, k] = (g * sampled).sum(-1)
            ddx = (v01 - v00) * (1 - ly)[..., None] + (v11 - v10) * ly[..., None]
            ddy = (v10 - v00) * (1 - lx)[..., None] + (v11 - v01) * lx[..., None]
            grad_loc[:, :, :, lvl, k, 0] = a * W * (g * ddx).sum(-1)
            grad_loc[:, :, :, lvl, k, 1] = a * H * (g * ddy).sum(-1)
            ga = g * a[..., None]
            for (idx, valid, _), wc in zip(corners, (w00, w01, w10, w11)):
                contrib = ga * (wc * valid.to(dtype))[..., None]
                grad_value.index_add_(0, idx.reshape(-1), contrib.reshape(-1))
    return grad_value.view(B, S, M, D), grad_loc, grad_attn


def run_reference(value, spatial_shapes, loc, attn, grad_out=None, dtype=torch.float32):
    """Oracle forward (and backward when grad_out is given) on CPU leaf copies
    of the given (already dtype-rounded) inputs, upcast to `dtype`.  With
    dtype=float32 this is the reference's test protocol (tests/test_msda.py:
    80-93).  Returns (out, grads or None) on CPU in `dtype`.

    float64 is the exact-arithmetic variant: grid_sample works on the grid
    2*loc - 1, and in float32 that rounding moves the image coordinate by up
    to W * 2^-25 pixels, which at W = 128 already shifts grad_loc by ~3e-4
    and can flip the bilinear cell at a knot.  Large fp32 inputs are checked
    against float64."""
    shapes = spatial_shapes.cpu()
    grad = grad_out is not None
    v = value.detach().to(dtype).cpu().requires_grad_(grad)
    lo = loc.detach().to(dtype).cpu().requires_grad_(grad)
    a = attn.detach().to(dtype).cpu().requires_grad_(grad)
    if not grad:
        with torch.no_grad():
            return msda_reference(v, shapes, lo, a), None
    out = msda_reference(v, shapes, lo, a)
    out.backward(grad_out.detach().to(dtype).cpu())
    return out.detach(), (v.grad, lo.grad, a.grad)


def run_reference_fp32(value, spatial_shapes, loc, attn, grad_out=None):
    """The reference's fp32 CPU protocol (tests/test_msda.py:80-93)."""
    return run_reference(value, spatial_shapes, loc, attn, grad_out, dtype=torch.float32)


def msda_fused_reference(value, spatial_shapes, reference_points, sampling_offsets,
                         attention_logits):
    """The attention layer's front-end composed with the operator, as the
    reference's MSDACrossAttention.forward does it (labs/solutions/lab00.py:
    201-208): softmax of the logits over the L*K points of each (b, q, m),
    locations = reference point + offset / (W_l, H_l), then
    ``msda_reference``.  ``reference_points`` is (B, Q, 2) as there, or
    (B, Q, L, 2) (one point per level, the Deformable-DETR layout).
    Differentiable in all four tensors through torch autograd."""
    B, Q, M, L, K, _ = sampling_offsets.shape
    weights = attention_logits.reshape(B, Q, M, L * K).softmax(-1).reshape(B, Q, M, L, K)
    scale = spatial_shapes.flip(-1).to(sampling_offsets.dtype)  # (L, 2) as (W_l, H_l)
    if reference_points.dim() == 3:
        ref = reference_points[:, :, None, None, None, :]
    else:
        ref = reference_points[:, :, None, :, None, :]
    locs = ref + sampling_offsets / scale[None, None, None, :, None, :]
    return msda_reference(value, spatial_shapes, locs, weights)


def run_fused_reference(value, spatial_shapes, reference_points, sampling_offsets,
                        attention_logits, grad_out=None, dtype=torch.float64):
    """``msda_fused_reference`` on CPU leaf copies upcast to `dtype`, with the
    four gradients when grad_out is given.  Returns (out, grads or None), grads
    ordered (value, reference_points, sampling_offsets, attention_logits)."""
    shapes = spatial_shapes.cpu()
    grad = grad_out is not None
    leaves = [t.detach().to(dtype).cpu().requires_grad_(grad)
              for t in (value, reference_points, sampling_offsets, attention_logits)]
    if not grad:
        with torch.no_grad():
            return msda_fused_reference(leaves[0], shapes, *leaves[1:]), None
    out = msda_fused_reference(leaves[0], shapes, *leaves[1:])
    out.backward(grad_out.detach().to(dtype).cpu())
    return out.detach(), tuple(t.grad for t in leaves)
