"""Pinning the CPU oracle (CPU only).

The oracle's arithmetic is torch's grid_sample (and its autograd), restated
the way the reference uses it.  These checks pin it independently of that
restatement:
  * float64 agreement with the pure-loop version (the reference's own check,
    tests/test_msda.py:101-120), including out-of-bounds and exact corners;
  * closed forms: constant field, pixel-centre gathers, fields linear in
    (x, y), all-out-of-bounds, the half-out-of-bounds known answer of
    tests/test_labs.py:86-91;
  * backward: float64 gradcheck, a hand-derived flat-index backward
    (labs/solutions/lab07.py:12-104), the adjoint identity of a map linear in
    value, grad_attn as one-hot forwards, the linear-field location gradient,
    mass conservation of the value gradient;
  * planted mistakes: wrong-convention variants of the oracle (align_corners,
    a dropped -0.5, swapped x/y, border padding, a transposed level layout)
    must each fail at least one of the closed forms above.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from msda_cases import make_inputs
from oracle import (level_start_index_of, msda_backward_analytic, msda_naive, msda_reference,
                    run_reference, run_reference_fp32)

F64 = torch.float64


def _interior_loc(shapes, B, Q, M, K, gen, margin=1.0):
    """Locations whose four bilinear corners are all inside every level:
    image coordinate in [margin, W - 1 - margin]."""
    L = len(shapes)
    loc = torch.empty(B, Q, M, L, K, 2, dtype=F64)
    for lvl, (h, w) in enumerate(shapes):
        ux = torch.rand(B, Q, M, K, generator=gen, dtype=F64)
        uy = torch.rand(B, Q, M, K, generator=gen, dtype=F64)
        x = margin + ux * (w - 1 - 2 * margin)
        y = margin + uy * (h - 1 - 2 * margin)
        loc[:, :, :, lvl, :, 0] = (x + 0.5) / w
        loc[:, :, :, lvl, :, 1] = (y + 0.5) / h
    return loc


# ---------------------------------------------------------------------------
# grid_sample restatement vs pure loops (float64)
# ---------------------------------------------------------------------------

def test_reference_matches_naive_cpu():
    value, shapes, _, loc, attn = make_inputs(
        B=2, Q=5, M=2, D=4, shapes=[(5, 7), (3, 4)], K=3, dtype=F64, device="cpu",
        loc_lo=-0.3, loc_hi=1.3)
    torch.testing.assert_close(msda_reference(value, shapes, loc, attn),
                               msda_naive(value, shapes, loc, attn), rtol=1e-10, atol=1e-12)


def test_reference_matches_naive_cpu_exact_corners():
    value, shapes, _, loc, attn = make_inputs(
        B=1, Q=4, M=1, D=3, shapes=[(4, 6)], K=2, dtype=F64, device="cpu")
    grid_vals = torch.tensor([0.0, 0.5, 1.0], dtype=F64)
    loc = grid_vals[torch.randint(0, 3, loc.shape, generator=torch.Generator().manual_seed(1))]
    torch.testing.assert_close(msda_reference(value, shapes, loc, attn),
                               msda_naive(value, shapes, loc, attn), rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("case", [
    dict(B=1, Q=7, M=1, D=3, shapes=[(4, 6)], K=1),
    dict(B=1, Q=4, M=2, D=5, shapes=[(6, 5), (3, 3)], K=2, loc_lo=-0.4, loc_hi=1.4),
    dict(B=2, Q=3, M=3, D=2, shapes=[(2, 9), (1, 1), (5, 2)], K=4, loc_lo=-1.0, loc_hi=2.0),
])
def test_reference_matches_naive_more_cases(case):
    value, shapes, _, loc, attn = make_inputs(**case, dtype=F64, device="cpu")
    torch.testing.assert_close(msda_reference(value, shapes, loc, attn),
                               msda_naive(value, shapes, loc, attn), rtol=1e-10, atol=1e-12)


# ---------------------------------------------------------------------------
# Closed forms (forward)
# ---------------------------------------------------------------------------

SHAPES = [(6, 9), (3, 5), (2, 2)]


def _check_constant_field(fn):
    B, Q, M, D, K = 2, 6, 3, 4, 3
    S = sum(h * w for h, w in SHAPES)
    gen = torch.Generator().manual_seed(11)
    c = torch.randn(M, D, generator=gen, dtype=F64)
    value = c.expand(B, S, M, D).contiguous()
    loc = _interior_loc(SHAPES, B, Q, M, K, gen, margin=0.0)
    attn = torch.rand(B, Q, M, len(SHAPES), K, generator=gen, dtype=F64)
    out = fn(value, torch.tensor(SHAPES), loc, attn).view(B, Q, M, D)
    expect = attn.sum((-1, -2))[..., None] * c
    torch.testing.assert_close(out, expect, rtol=1e-12, atol=1e-12)


def _check_pixel_centres(fn):
    B, Q, M, D, K = 2, 5, 2, 3, 2
    S = sum(h * w for h, w in SHAPES)
    starts = level_start_index_of(torch.tensor(SHAPES)).tolist()
    gen = torch.Generator().manual_seed(12)
    value = torch.randn(B, S, M, D, generator=gen, dtype=F64)
    attn = torch.rand(B, Q, M, len(SHAPES), K, generator=gen, dtype=F64)
    loc = torch.empty(B, Q, M, len(SHAPES), K, 2, dtype=F64)
    expect = torch.zeros(B, Q, M, D, dtype=F64)
    for lvl, (h, w) in enumerate(SHAPES):
        ii = torch.randint(0, h, (B, Q, M, K), generator=gen)
        jj = torch.randint(0, w, (B, Q, M, K), generator=gen)
        loc[:, :, :, lvl, :, 0] = (jj.to(F64) + 0.5) / w
        loc[:, :, :, lvl, :, 1] = (ii.to(F64) + 0.5) / h
        for b in range(B):
            for q in range(Q):
                for m in range(M):
                    for k in range(K):
                        s = starts[lvl] + int(ii[b, q, m, k]) * w + int(jj[b, q, m, k])
                        expect[b, q, m] += attn[b, q, m, lvl, k] * value[b, s, m]
    torch.testing.assert_close(fn(value, torch.tensor(SHAPES), loc, attn).view(B, Q, M, D),
                               expect, rtol=1e-12, atol=1e-12)


def _linear_field(B, M, D, gen):
    """value[b, pixel (i, j) of level l, m, :] = alpha_l j + beta_l i + gamma_l."""
    S = sum(h * w for h, w in SHAPES)
    value = torch.empty(B, S, M, D, dtype=F64)
    coef = []
    s0 = 0
    for h, w in SHAPES:
        a, bt, g = (torch.randn(M, D, generator=gen, dtype=F64) for _ in range(3))
        ii, jj = torch.meshgrid(torch.arange(h, dtype=F64), torch.arange(w, dtype=F64),
                                indexing="ij")
        field = a * jj.reshape(-1, 1, 1) + bt * ii.reshape(-1, 1, 1) + g  # (h*w, M, D)
        value[:, s0:s0 + h * w] = field
        coef.append((a, bt, g))
        s0 += h * w
    return value, coef


def _check_linear_field(fn):
    B, Q, M, D, K = 2, 5, 2, 3, 3
    gen = torch.Generator().manual_seed(13)
    value, coef = _linear_field(B, M, D, gen)
    loc = _interior_loc(SHAPES, B, Q, M, K, gen, margin=0.0)
    attn = torch.rand(B, Q, M, len(SHAPES), K, generator=gen, dtype=F64)
    expect = torch.zeros(B, Q, M, D, dtype=F64)
    for lvl, (h, w) in enumerate(SHAPES):
        a, bt, g = coef[lvl]
        x = loc[:, :, :, lvl, :, 0] * w - 0.5
        y = loc[:, :, :, lvl, :, 1] * h - 0.5
        A = attn[:, :, :, lvl, :]
        expect += (A * x).sum(-1)[..., None] * a + (A * y).sum(-1)[..., None] * bt \
            + A.sum(-1)[..., None] * g
    torch.testing.assert_close(fn(value, torch.tensor(SHAPES), loc, attn).view(B, Q, M, D),
                               expect, rtol=1e-11, atol=1e-11)


def _check_all_out_of_bounds(fn):
    B, Q, M, D, K = 1, 6, 2, 3, 2
    S = sum(h * w for h, w in SHAPES)
    gen = torch.Generator().manual_seed(14)
    value = torch.randn(B, S, M, D, generator=gen, dtype=F64)
    attn = torch.rand(B, Q, M, len(SHAPES), K, generator=gen, dtype=F64)
    # Image coordinates <= -1 or >= W: both bilinear corners of that axis outside.
    loc = torch.rand(B, Q, M, len(SHAPES), K, 2, generator=gen, dtype=F64)
    side = torch.rand(loc.shape, generator=gen) < 0.5
    loc = torch.where(side, -0.6 - loc, 1.6 + loc)
    out = fn(value, torch.tensor(SHAPES), loc, attn)
    torch.testing.assert_close(out, torch.zeros_like(out), rtol=0, atol=1e-15)


def _check_half_out_kat(fn):
    """tests/test_labs.py:86-91: on an all-ones 3x3 image, pixel (x, y) =
    (-0.5, 1.0) is half outside (-> 0.5), (-1.0, 1.0) fully outside (-> 0)."""
    value = torch.ones(1, 9, 1, 2, dtype=F64)
    shapes = torch.tensor([[3, 3]])
    attn = torch.ones(1, 2, 1, 1, 1, dtype=F64)
    # x_im = loc_x * 3 - 0.5  ->  loc_x = (x_im + 0.5) / 3
    loc = torch.tensor([[(-0.5 + 0.5) / 3, (1.0 + 0.5) / 3],
                        [(-1.0 + 0.5) / 3, (1.0 + 0.5) / 3]], dtype=F64).view(1, 2, 1, 1, 1, 2)
    out = fn(value, shapes, loc, attn).view(2, 2)
    torch.testing.assert_close(out, torch.tensor([[0.5, 0.5], [0.0, 0.0]], dtype=F64))


def _check_level_layout(fn):
    """A level sampled at a pixel centre returns that level's own pixel:
    starts are the exclusive cumsum of H*W, rows are row-major (i*W + j)."""
    shapes = [(2, 3), (3, 2)]
    S = 12
    value = torch.arange(S, dtype=F64).view(1, S, 1, 1).contiguous()
    attn = torch.zeros(1, 2, 1, 2, 1, dtype=F64)
    attn[0, 0, 0, 0, 0] = 1.0  # query 0 reads level 0 at (i=1, j=2) -> row 5
    attn[0, 1, 0, 1, 0] = 1.0  # query 1 reads level 1 at (i=2, j=0) -> row 6 + 4 = 10
    loc = torch.zeros(1, 2, 1, 2, 1, 2, dtype=F64)
    loc[0, 0, 0, 0, 0] = torch.tensor([(2 + 0.5) / 3, (1 + 0.5) / 2])
    loc[0, 1, 0, 1, 0] = torch.tensor([(0 + 0.5) / 2, (2 + 0.5) / 3])
    out = fn(value, torch.tensor(shapes), loc, attn).view(2)
    torch.testing.assert_close(out, torch.tensor([5.0, 10.0], dtype=F64))


FORWARD_CHECKS = [_check_constant_field, _check_pixel_centres, _check_linear_field,
                  _check_all_out_of_bounds, _check_half_out_kat, _check_level_layout]


@pytest.mark.parametrize("fn", [msda_reference, msda_naive], ids=["grid_sample", "naive"])
@pytest.mark.parametrize("check", FORWARD_CHECKS, ids=lambda c: c.__name__[7:])
def test_forward_closed_forms(check, fn):
    check(fn)


# ---------------------------------------------------------------------------
# Planted mistakes: each wrong variant fails at least one closed form.
# ---------------------------------------------------------------------------

def _variant(mode="bilinear", padding="zeros", align=False, shift=0.0, swap_xy=False,
             level_major=True):
    def fn(value, spatial_shapes, loc, attn):
        B, S, M, D = value.shape
        _, Q, _, L, K, _ = loc.shape
        sizes = [(int(h), int(w)) for h, w in spatial_shapes.tolist()]
        per = value.split([h * w for h, w in sizes], dim=1)
        lc = loc.flip(-1) if swap_xy else loc
        outs = []
        for lvl, (h, w) in enumerate(sizes):
            img = per[lvl].permute(0, 2, 3, 1).reshape(B * M, D, h, w)
            if not level_major:
                img = per[lvl].permute(0, 2, 3, 1).reshape(B * M, D, w, h).transpose(-1, -2)
            size = torch.tensor([w, h], dtype=loc.dtype)
            g = 2 * (lc[:, :, :, lvl] + shift / size) - 1
            g = g.permute(0, 2, 1, 3, 4).reshape(B * M, Q, K, 2)
            outs.append(F.grid_sample(img, g, mode=mode, padding_mode=padding,
                                      align_corners=align))
        st = torch.cat(outs, -1)
        a = attn.permute(0, 2, 1, 3, 4).reshape(B * M, 1, Q, L * K)
        return (st * a).sum(-1).reshape(B, M * D, Q).transpose(1, 2)
    return fn


def _fails_some_check(fn):
    for check in FORWARD_CHECKS:
        try:
            check(fn)
        except AssertionError:
            return True
    return False


def test_planted_variant_matches_when_correct():
    assert not _fails_some_check(_variant())


@pytest.mark.parametrize("kwargs", [
    dict(align=True), dict(shift=0.5), dict(shift=-0.5), dict(swap_xy=True),
    dict(padding="border"), dict(level_major=False), dict(mode="nearest"),
], ids=["align_corners", "no_half_shift", "double_half_shift", "swapped_xy", "border_padding",
        "transposed_level", "nearest"])
def test_planted_mistakes_are_caught(kwargs):
    assert _fails_some_check(_variant(**kwargs))


# ---------------------------------------------------------------------------
# Backward
# ---------------------------------------------------------------------------

def _away_from_knots(loc, shapes, eps=1e-3):
    """Nudge image coordinates off integers (grid_sample's derivative is
    discontinuous there, which finite differences cannot handle)."""
    loc = loc.clone()
    for lvl, (h, w) in enumerate(shapes):
        for c, n in ((0, w), (1, h)):
            x = loc[:, :, :, lvl, :, c] * n - 0.5
            frac = x - torch.floor(x)
            x = torch.where(frac < eps, x + 2 * eps, torch.where(frac > 1 - eps, x - 2 * eps, x))
            loc[:, :, :, lvl, :, c] = (x + 0.5) / n
    return loc


def test_gradcheck_float64():
    shapes = [(4, 5), (2, 3)]
    value, sh, _, loc, attn = make_inputs(B=1, Q=3, M=2, D=3, shapes=shapes, K=2, dtype=F64,
                                          device="cpu", loc_lo=-0.2, loc_hi=1.2)
    loc = _away_from_knots(loc, shapes)
    inputs = (value.requires_grad_(True), loc.requires_grad_(True), attn.requires_grad_(True))
    assert torch.autograd.gradcheck(lambda v, l, a: msda_reference(v, sh, l, a), inputs,
                                    eps=1e-6, atol=1e-7)


@pytest.mark.parametrize("lo,hi", [(0.0, 1.0), (-0.5, 1.5)])
def test_analytic_backward_matches_autograd(lo, hi):
    shapes = [(7, 9), (4, 5), (2, 3)]
    value, sh, starts, loc, attn = make_inputs(B=2, Q=6, M=3, D=5, shapes=shapes, K=3,
                                               dtype=F64, device="cpu", loc_lo=lo, loc_hi=hi)
    g = torch.randn(2, 6, 15, generator=torch.Generator().manual_seed(7), dtype=F64)
    v, lc, a = (t.clone().requires_grad_(True) for t in (value, loc, attn))
    msda_reference(v, sh, lc, a).backward(g)
    gv, gl, ga = msda_backward_analytic(value, sh, starts, loc, attn, g, dtype=F64)
    torch.testing.assert_close(gv, v.grad, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(gl, lc.grad, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(ga, a.grad, rtol=1e-10, atol=1e-12)


def test_value_gradient_is_the_adjoint():
    """out is linear in value, so <grad_value, V'> = <g, out(V')> for any V'."""
    shapes = [(6, 7), (3, 4)]
    value, sh, _, loc, attn = make_inputs(B=2, Q=8, M=2, D=4, shapes=shapes, K=3, dtype=F64,
                                          device="cpu", loc_lo=-0.3, loc_hi=1.3)
    gen = torch.Generator().manual_seed(5)
    g = torch.randn(2, 8, 8, generator=gen, dtype=F64)
    v = value.clone().requires_grad_(True)
    msda_reference(v, sh, loc, attn).backward(g)
    for _ in range(3):
        vp = torch.randn(value.shape, generator=gen, dtype=F64)
        lhs = (v.grad * vp).sum()
        rhs = (g * msda_reference(vp, sh, loc, attn)).sum()
        torch.testing.assert_close(lhs, rhs, rtol=1e-12, atol=1e-12)


def test_attention_gradient_is_the_sample():
    """out is linear in attn: grad_attn[p] = <g, out with attn = one-hot(p)>."""
    shapes = [(5, 6), (2, 3)]
    value, sh, _, loc, attn = make_inputs(B=1, Q=2, M=2, D=3, shapes=shapes, K=2, dtype=F64,
                                          device="cpu", loc_lo=-0.2, loc_hi=1.2)
    g = torch.randn(1, 2, 6, generator=torch.Generator().manual_seed(6), dtype=F64)
    a = attn.clone().requires_grad_(True)
    msda_reference(value, sh, loc, a).backward(g)
    for idx in np.ndindex(*attn.shape):
        onehot = torch.zeros_like(attn)
        onehot[idx] = 1.0
        expect = (g * msda_reference(value, sh, loc, onehot)).sum()
        torch.testing.assert_close(a.grad[idx], expect, rtol=1e-12, atol=1e-12)


def test_location_gradient_on_linear_field():
    """On value = alpha j + beta i + gamma, bilinear sampling is exactly linear
    in the image coordinate, so d out / d loc_x = A * W_l * alpha_l."""
    B, Q, M, D, K = 2, 4, 2, 3, 2
    gen = torch.Generator().manual_seed(15)
    value, coef = _linear_field(B, M, D, gen)
    loc = _interior_loc(SHAPES, B, Q, M, K, gen, margin=0.1)
    attn = torch.rand(B, Q, M, len(SHAPES), K, generator=gen, dtype=F64)
    g = torch.randn(B, Q, M * D, generator=gen, dtype=F64)
    lc = loc.clone().requires_grad_(True)
    msda_reference(value, torch.tensor(SHAPES), lc, attn).backward(g)
    gm = g.view(B, Q, M, D)
    for lvl, (h, w) in enumerate(SHAPES):
        a, bt, _ = coef[lvl]
        A = attn[:, :, :, lvl, :]
        ex = A * w * (gm * a).sum(-1)[..., None]
        ey = A * h * (gm * bt).sum(-1)[..., None]
        torch.testing.assert_close(lc.grad[:, :, :, lvl, :, 0], ex, rtol=1e-10, atol=1e-11)
        torch.testing.assert_close(lc.grad[:, :, :, lvl, :, 1], ey, rtol=1e-10, atol=1e-11)


def test_value_gradient_mass_conservation():
    """With every corner inside, the bilinear weights of a sample sum to 1, so
    sum_s grad_value[b, s, m, :] = sum_{q,l,k} A g[b, q, m, :]."""
    B, Q, M, D, K = 2, 7, 3, 4, 3
    gen = torch.Generator().manual_seed(16)
    S = sum(h * w for h, w in SHAPES)
    value = torch.randn(B, S, M, D, generator=gen, dtype=F64).requires_grad_(True)
    loc = _interior_loc(SHAPES, B, Q, M, K, gen, margin=0.0)
    attn = torch.rand(B, Q, M, len(SHAPES), K, generator=gen, dtype=F64)
    g = torch.randn(B, Q, M * D, generator=gen, dtype=F64)
    msda_reference(value, torch.tensor(SHAPES), loc, attn).backward(g)
    expect = (attn.sum((-1, -2))[..., None] * g.view(B, Q, M, D)).sum(1)
    torch.testing.assert_close(value.grad.sum(1), expect, rtol=1e-12, atol=1e-12)


def test_run_reference_fp32_protocol():
    """fp32 CPU leaf copies of dtype-rounded inputs (tests/test_msda.py:80-93)."""
    value, sh, _, loc, attn = make_inputs(B=1, Q=4, M=2, D=4, shapes=[(5, 6)], K=2,
                                          dtype=torch.bfloat16, device="cpu")
    g = torch.randn(1, 4, 8).to(torch.bfloat16)
    out, (gv, gl, ga) = run_reference_fp32(value, sh, loc, attn, g)
    assert out.dtype == gv.dtype == gl.dtype == ga.dtype == torch.float32
    ref = msda_reference(value.double(), sh, loc.double(), attn.double())
    torch.testing.assert_close(out.double(), ref, rtol=1e-6, atol=1e-6)
    assert math.isfinite(gv.sum().item())


def test_fp32_formula_matches_float64_where_fp32_grid_sample_drifts():
    """At W = 128 the fp32 grid_sample oracle's grid 2*loc - 1 rounds the
    image coordinate enough to move grad_loc beyond 1e-4; the kernels' fp32
    formula x = loc*W - 0.5 (exact for power-of-two W) stays within 1e-4 of
    the float64 oracle.  This is why fp32 inputs at full size are checked
    against float64."""
    gen = torch.Generator().manual_seed(21)
    shapes = [(128, 128)]
    B, Q, M, D, K = 1, 512, 2, 32, 4
    value = torch.randn(B, 128 * 128, M, D, generator=gen)
    loc = torch.rand(B, Q, M, 1, K, 2, generator=gen) * 0.3  # small locs: 2*loc - 1 rounds
    attn = torch.rand(B, Q, M, 1, K, generator=gen)
    g = torch.randn(B, Q, M * D, generator=gen)
    sh = torch.tensor(shapes)
    starts = level_start_index_of(sh)
    _, (_, gl64, _) = run_reference(value, sh, loc, attn, g, dtype=F64)
    _, (_, gl32, _) = run_reference(value, sh, loc, attn, g, dtype=torch.float32)
    _, gl_formula, _ = msda_backward_analytic(value, sh, starts, loc, attn, g, dtype=torch.float32)
    torch.testing.assert_close(gl_formula.double(), gl64, rtol=1e-4, atol=1e-4)
    drift = (gl32.double() - gl64).abs() / (1 + gl64.abs())
    assert drift.max() > 1e-4  # the fp32 oracle itself exceeds the fp32 tolerance here
