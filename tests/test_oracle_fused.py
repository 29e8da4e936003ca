"""Pinning of the fused front-end oracle (oracle.msda_fused_reference), the
composition of labs/solutions/lab00.py:201-208 (softmax over L*K; reference
point + offset / (W_l, H_l); the operator).

Each check is a property the composition must have independently of how it
is written -- weights that sum to one, an exact landing on chosen pixel
centres, invariance to a per-pair logit shift, chain-rule identities between
its gradients and the operator's -- and each plausible mistake (softmax over
K instead of L*K, offsets divided by (H, W) instead of (W, H), a reference
point broadcast to the wrong axis) is planted in a variant and shown to fail
one of them.
"""

import pytest
import torch

from oracle import msda_fused_reference, msda_reference, run_fused_reference, run_reference

F64 = torch.float64
SHAPES = [(6, 9), (4, 7), (3, 5)]  # W != H on every level


def _inputs(B=2, Q=5, M=3, D=4, K=2, per_level=False, seed=0, sigma=1.0):
    g = torch.Generator().manual_seed(seed)
    L = len(SHAPES)
    S = sum(h * w for h, w in SHAPES)
    value = torch.randn(B, S, M, D, generator=g, dtype=F64)
    ref = torch.rand(*((B, Q, L, 2) if per_level else (B, Q, 2)), generator=g, dtype=F64)
    ref = 0.25 + 0.5 * ref  # keep ref +- a pixel inside the map
    off = sigma * torch.randn(B, Q, M, L, K, 2, generator=g, dtype=F64)
    logits = torch.randn(B, Q, M, L, K, generator=g, dtype=F64)
    shapes = torch.tensor(SHAPES, dtype=torch.long)
    return value, shapes, ref, off, logits


def _variant(mistake):
    """msda_fused_reference with one planted mistake."""

    def fn(value, shapes, ref, off, logits):
        B, Q, M, L, K, _ = off.shape
        if mistake == "softmax_over_K":
            w = logits.softmax(-1)
        else:
            w = logits.reshape(B, Q, M, L * K).softmax(-1).reshape(B, Q, M, L, K)
        scale = shapes.flip(-1).to(off.dtype)
        if mistake == "scale_HW":
            scale = shapes.to(off.dtype)
        if ref.dim() == 3:
            r = ref[:, :, None, None, None, :]
        elif mistake == "ref_level_axis":
            r = ref[:, :, None, None, :, :][..., :1, :] if K == 1 else ref[:, :, :1, None, None, :]
        else:
            r = ref[:, :, None, :, None, :]
        return msda_reference(value, shapes, r + off / scale[None, None, None, :, None, :], w)

    return fn


MISTAKES = ["softmax_over_K", "scale_HW", "ref_level_axis"]


def _constant_field_check(fn, per_level):
    """A per-(b, m, channel) constant value field with every corner inside
    the map gives out = that constant: the weights sum to one."""
    value, shapes, ref, off, logits = _inputs(per_level=per_level)
    # ref in [0.4, 0.6] and |offset| <= 0.6 px keep all corners inside maps >= 3 px
    ref = 0.4 + 0.2 * (ref - 0.25) / 0.5
    off = (0.3 * off).clamp(-0.6, 0.6)
    B, S, M, D = value.shape
    c = torch.randn(B, 1, M, D, dtype=F64)
    value = c.expand(B, S, M, D).contiguous()
    out = fn(value, shapes, ref, off, logits)
    expect = c.reshape(B, 1, M * D).expand_as(out)
    return torch.allclose(out, expect, rtol=1e-12, atol=1e-12)


def _pixel_landing_check(fn, per_level):
    """Offsets chosen so that every location is the centre of a chosen pixel
    (i, j) of its level: loc = ((j + 0.5) / W, (i + 0.5) / H).  Bilinear
    sampling there is an exact gather, so out = sum_s A_s value[pixel_s]."""
    value, shapes, ref, off, logits = _inputs(per_level=per_level, seed=3)
    B, Q, M, L, K, _ = off.shape
    g = torch.Generator().manual_seed(11)
    starts = [0]
    for h, w in SHAPES[:-1]:
        starts.append(starts[-1] + h * w)
    off = torch.empty_like(off)
    expect = torch.zeros(B, Q, M, value.shape[-1], dtype=F64)
    weights = logits.reshape(B, Q, M, L * K).softmax(-1).reshape(B, Q, M, L, K)
    for lvl, (h, w) in enumerate(SHAPES):
        ii = torch.randint(0, h, (B, Q, M, K), generator=g)
        jj = torch.randint(0, w, (B, Q, M, K), generator=g)
        rl = ref[:, :, None, None, :] if ref.dim() == 3 else ref[:, :, lvl, None, None, :]
        off[:, :, :, lvl, :, 0] = (jj.to(F64) + 0.5) - rl[..., 0] * w
        off[:, :, :, lvl, :, 1] = (ii.to(F64) + 0.5) - rl[..., 1] * h
        rows = starts[lvl] + ii * w + jj  # (B, Q, M, K)
        for b in range(B):
            for m in range(M):
                picked = value[b, rows[b, :, m, :], m, :]  # (Q, K, D)
                expect[b, :, m] += (weights[b, :, m, lvl, :, None] * picked).sum(1)
    out = fn(value, shapes, ref, off, logits)
    return torch.allclose(out, expect.reshape(B, Q, -1), rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize("per_level", [False, True])
def test_constant_field_weights_sum_to_one(per_level):
    assert _constant_field_check(msda_fused_reference, per_level)


@pytest.mark.parametrize("per_level", [False, True])
def test_offsets_landing_on_pixel_centres_gather_exactly(per_level):
    assert _pixel_landing_check(msda_fused_reference, per_level)


@pytest.mark.parametrize("mistake", MISTAKES)
def test_planted_mistakes_fail_a_check(mistake):
    fn = _variant(mistake)
    per_level = mistake == "ref_level_axis"
    ok = _constant_field_check(fn, per_level) and _pixel_landing_check(fn, per_level)
    assert not ok, f"planted mistake {mistake!r} passed every check"


def test_per_level_reference_equal_across_levels_matches_shared():
    value, shapes, ref, off, logits = _inputs()
    L = len(SHAPES)
    ref_l = ref[:, :, None, :].expand(-1, -1, L, -1).contiguous()
    a = msda_fused_reference(value, shapes, ref, off, logits)
    b = msda_fused_reference(value, shapes, ref_l, off, logits)
    torch.testing.assert_close(a, b, rtol=0, atol=0)


def test_logit_shift_invariance():
    """softmax is invariant to adding a constant per (b, q, m): the output
    does not change, so the logit gradient sums to zero over each pair's
    L*K points."""
    value, shapes, ref, off, logits = _inputs()
    shift = torch.randn(logits.shape[:3], dtype=F64)[..., None, None]
    a = msda_fused_reference(value, shapes, ref, off, logits)
    b = msda_fused_reference(value, shapes, ref, off, logits + shift)
    torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)
    g = torch.randn(a.shape, dtype=F64)
    _, grads = run_fused_reference(value, shapes, ref, off, logits, g)
    torch.testing.assert_close(grads[3].sum((-1, -2)), torch.zeros(logits.shape[:3], dtype=F64),
                               rtol=0, atol=1e-12)


@pytest.mark.parametrize("per_level", [False, True])
def test_gradients_follow_the_chain_rule_through_the_operator(per_level):
    """With loc = ref + off / (W, H) and A = softmax(logits):
    d/d(off) = d/d(loc) / (W, H); d/d(ref) = sum over the points built on it
    of d/d(loc); d/d(logit) = A (d/dA - <A, d/dA>) and <A, d/dA> =
    <grad_out, out> per pair; d/d(value) is the operator's."""
    value, shapes, ref, off, logits = _inputs(per_level=per_level, seed=5)
    B, Q, M, L, K, _ = off.shape
    D = value.shape[-1]
    gout = torch.randn(B, Q, M * D, dtype=F64)
    out, (gv, gref, goff, glog) = run_fused_reference(value, shapes, ref, off, logits, gout)

    scale = shapes.flip(-1).to(F64)[None, None, None, :, None, :]
    r = ref[:, :, None, None, None, :] if not per_level else ref[:, :, None, :, None, :]
    loc = r + off / scale
    A = logits.reshape(B, Q, M, L * K).softmax(-1).reshape(B, Q, M, L, K)
    out2, (gv2, gloc, gattn) = run_reference(value, shapes, loc, A, gout, dtype=F64)
    torch.testing.assert_close(out, out2, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(gv, gv2, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(goff, gloc / scale, rtol=1e-10, atol=1e-12)
    gref2 = gloc.sum((2, 3, 4)) if not per_level else gloc.sum((2, 4))
    torch.testing.assert_close(gref, gref2, rtol=1e-10, atol=1e-12)
    delta = (gout.view(B, Q, M, D) * out.view(B, Q, M, D)).sum(-1)
    torch.testing.assert_close((A * gattn).sum((-1, -2)), delta, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(glog, A * (gattn - delta[..., None, None]), rtol=1e-10,
                               atol=1e-12)


def test_gradcheck_float64():
    value, shapes, ref, off, logits = _inputs(B=1, Q=2, M=2, D=2, K=2, seed=9, sigma=0.7)
    leaves = [t.clone().requires_grad_(True) for t in (value, ref, off, logits)]
    assert torch.autograd.gradcheck(
        lambda v, r, o, lg: msda_fused_reference(v, shapes, r, o, lg), leaves, eps=1e-6,
        atol=1e-6, rtol=1e-4)
