"""Shared test inputs and tolerances.

`make_inputs` restates the reference's seeded generator
(tests/test_msda.py:65-77: value randn -> loc rand -> attn rand + softmax over
L*K, CPU torch.Generator), so the same seeds give the same bits.  Tolerances
are the reference's assert_close values (tests/test_msda.py:43-55) plus the
norm-relative bounds of the operator's accuracy target.
"""

import torch

DTYPES = [torch.float32, torch.float16, torch.bfloat16]

FWD_TOL = {
    torch.float64: dict(rtol=1e-9, atol=1e-10),
    torch.float32: dict(rtol=1e-5, atol=1e-5),
    torch.float16: dict(rtol=5e-3, atol=5e-3),
    torch.bfloat16: dict(rtol=3e-2, atol=3e-2),
}
BWD_TOL = {
    torch.float32: dict(rtol=1e-4, atol=1e-4),
    torch.float16: dict(rtol=3e-2, atol=3e-2),
    torch.bfloat16: dict(rtol=8e-2, atol=8e-2),
}
# Norm-relative error bounds, rel_err(x, ref) = ||x - ref||_2 / ||ref||_2:
# forward 1e-5 (fp32) / 1e-2 (fp16, bf16); each gradient 1e-4 / 2e-2.
FWD_RELERR = {torch.float32: 1e-5, torch.float16: 1e-2, torch.bfloat16: 1e-2}
BWD_RELERR = {torch.float32: 1e-4, torch.float16: 2e-2, torch.bfloat16: 2e-2}

CASES = [
    dict(id="decoder", B=2, Q=100, M=4, D=32, K=4, shapes=[(24, 32), (12, 16), (6, 8)]),
    dict(id="single_level_point", B=1, Q=17, M=1, D=16, K=1, shapes=[(13, 9)]),
    dict(id="nonpow2_D", B=2, Q=33, M=2, D=24, K=3, shapes=[(10, 14), (5, 7)]),
    dict(id="wide", B=1, Q=64, M=8, D=64, K=4, shapes=[(16, 16), (8, 8)]),
]


def case_kwargs(case):
    return {k: v for k, v in case.items() if k != "id"}


def make_inputs(B, Q, M, D, shapes, K, dtype, device, loc_lo=0.0, loc_hi=1.0, seed=0):
    gen = torch.Generator().manual_seed(seed)
    L = len(shapes)
    S = sum(h * w for h, w in shapes)
    value = torch.randn(B, S, M, D, generator=gen).to(device, dtype)
    loc = loc_lo + (loc_hi - loc_lo) * torch.rand(B, Q, M, L, K, 2, generator=gen)
    loc = loc.to(device, dtype)
    attn = torch.rand(B, Q, M, L, K, generator=gen)
    attn = attn.flatten(3).softmax(-1).view(B, Q, M, L, K).to(device, dtype)
    spatial_shapes = torch.tensor(shapes, dtype=torch.long, device=device)
    hw = spatial_shapes.prod(-1)
    starts = torch.cat([hw.new_zeros(1), hw.cumsum(0)[:-1]])
    return value, spatial_shapes, starts, loc, attn


def per_pixel(grad_loc: torch.Tensor, shapes: torch.Tensor) -> torch.Tensor:
    """grad_loc (B, Q, M, L, K, 2) divided by each level's (W, H): the
    gradient with respect to the pixel coordinate.  In fp32 it carries the
    dot products' rounding (~32 channels, then corner differences) without
    the factor W that the normalised location adds (up to 167 at the
    decoder's finest level), so the reference's elementwise 1e-4 applies to
    it at any map size."""
    hw = shapes.detach().cpu().double().clamp_min(1.0)  # empty levels: grad_loc is 0
    wh = torch.stack([hw[:, 1], hw[:, 0]], -1).view(1, 1, 1, -1, 1, 2)
    return grad_loc.detach().cpu().double() / wh


def rel_err(x: torch.Tensor, ref: torch.Tensor) -> float:
    x = x.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = ref.norm().item()
    num = (x - ref).norm().item()
    return num / den if den > 0 else num


def make_fused_inputs(B, Q, M, D, shapes, K, dtype, device, per_level=False, offset_sigma=2.0,
                      logit_sigma=1.0, seed=0):
    """Inputs of the fused front-end: value N(0,1); reference points U[0,1)
    ((B,Q,2), or (B,Q,L,2) when per_level); offsets N(0, offset_sigma) in
    level pixels (so points near a border fall outside); logits
    N(0, logit_sigma).  Drawn on a CPU generator, then cast and moved."""
    gen = torch.Generator().manual_seed(seed)
    L = len(shapes)
    S = sum(h * w for h, w in shapes)
    value = torch.randn(B, S, M, D, generator=gen)
    ref = torch.rand(*((B, Q, L, 2) if per_level else (B, Q, 2)), generator=gen)
    off = offset_sigma * torch.randn(B, Q, M, L, K, 2, generator=gen)
    logits = logit_sigma * torch.randn(B, Q, M, L, K, generator=gen)
    ref = ref.to(dtype)
    off = _off_knots(off.to(dtype), ref, shapes, per_level)
    spatial_shapes = torch.tensor(shapes, dtype=torch.long, device=device)
    hw = spatial_shapes.prod(-1)
    starts = torch.cat([hw.new_zeros(1), hw.cumsum(0)[:-1]])
    cast = lambda t: t.to(device, dtype)  # noqa: E731
    return cast(value), spatial_shapes, starts, cast(ref), cast(off), cast(logits)


def _off_knots(off, ref, shapes, per_level, margin=1e-3):
    """Nudge (in the storage dtype) every offset whose image coordinate
    ref * W + offset - 0.5 lies within `margin` px of an integer.  At such a
    bilinear knot d(out)/d(location) jumps, and which side an implementation
    lands on depends on its last rounding (the float64 oracle's included), so
    gradients there are not comparable.  Half-precision inputs hit knots
    exactly with noticeable probability."""
    dtype = off.dtype
    sizes = torch.tensor([[w, h] for h, w in shapes], dtype=torch.float64)  # (L, 2) as (W, H)
    r = ref.double()[:, :, None, :, None, :] if per_level else ref.double()[:, :, None, None, None, :]
    for step in (0.05, 0.1, 0.2, 0.4):
        o = off.double()
        x = r * sizes[None, None, None, :, None, :] + o - 0.5
        near = (x - x.round()).abs() < margin
        if not near.any():
            break
        off = torch.where(near, (o + step).to(dtype), off)
    return off
