"""GPU parity: the HIP kernels (through the C ABI, via the autograd
operator) against the CPU oracle on identical seeded inputs.

Restates the reference's GPU contract (tests/test_msda.py:128-245) and adds
edge cases of this implementation's launch shapes: odd head dims (padded
lanes), many levels, L*K beyond one LDS pass, exact bilinear knots, empty
inputs, and the benchmark presets at full size.
"""

import pytest
import torch

from msda_cases import (BWD_RELERR, BWD_TOL, CASES, DTYPES, FWD_RELERR, FWD_TOL, case_kwargs,
                        make_inputs, rel_err)
from msda_triton_amd import multi_scale_deformable_attention as msda
from oracle import run_reference_fp32

pytestmark = pytest.mark.gpu
DEVICE = "cuda"


def check_fwd(out, ref, dtype):
    torch.testing.assert_close(out.float().cpu(), ref, **FWD_TOL[dtype])
    assert rel_err(out, ref) <= FWD_RELERR[dtype]


def check_bwd(grads, refs, dtype, names=("grad_value", "grad_loc", "grad_attn")):
    for name, g, r in zip(names, grads, refs):
        torch.testing.assert_close(g.float().cpu(), r, **BWD_TOL[dtype], msg=lambda m: f"{name}: {m}")
        e = rel_err(g, r)
        assert e <= BWD_RELERR[dtype], f"{name}: rel_err {e:.3e} > {BWD_RELERR[dtype]}"


def run_fwd_bwd(value, shapes, starts, loc, attn, grad_seed=7, **kw):
    v = value.clone().requires_grad_(True)
    lo = loc.clone().requires_grad_(True)
    a = attn.clone().requires_grad_(True)
    out = msda(v, shapes, starts, lo, a, **kw)
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(grad_seed))
    g = g.to(out.device, out.dtype)
    out.backward(g)
    return out.detach(), g, (v.grad, lo.grad, a.grad)


# ---------------------------------------------------------------------------
# Forward
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("case", CASES, ids=[c["id"] for c in CASES])
def test_forward_matches_reference(case, dtype):
    value, shapes, starts, loc, attn = make_inputs(**case_kwargs(case), dtype=dtype, device=DEVICE)
    out = msda(value, shapes, starts, loc, attn)
    assert out.dtype == dtype and out.shape == (case["B"], case["Q"], case["M"] * case["D"])
    ref, _ = run_reference_fp32(value, shapes, loc, attn)
    check_fwd(out, ref, dtype)


def test_forward_out_of_bounds_locations():
    value, shapes, starts, loc, attn = make_inputs(
        B=2, Q=64, M=4, D=32, shapes=[(14, 20), (7, 10)], K=4,
        dtype=torch.float32, device=DEVICE, loc_lo=-0.5, loc_hi=1.5)
    out = msda(value, shapes, starts, loc, attn)
    ref, _ = run_reference_fp32(value, shapes, loc, attn)
    check_fwd(out, ref, torch.float32)


def test_forward_level_start_index_optional_and_noncontiguous():
    value, shapes, starts, loc, attn = make_inputs(
        B=2, Q=50, M=4, D=32, shapes=[(12, 16), (6, 8)], K=4, dtype=torch.float32, device=DEVICE)
    out = msda(value, shapes, starts, loc, attn)
    torch.testing.assert_close(out, msda(value, shapes, None, loc, attn))
    value_nc = value.transpose(1, 2).contiguous().transpose(1, 2)
    assert not value_nc.is_contiguous()
    torch.testing.assert_close(out, msda(value_nc, shapes, starts, loc, attn))
    # Host-side (CPU) shapes/starts are moved to the device by the operator.
    torch.testing.assert_close(out, msda(value, shapes.cpu(), starts.cpu(), loc, attn))


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("D", [1, 3, 5, 8, 12, 48, 100, 128])
def test_forward_head_dims(D, dtype):
    """Head dims whose rows do not fill 16-byte lane chunks or a power of two
    of lanes (narrow chunks, padded lanes)."""
    value, shapes, starts, loc, attn = make_inputs(
        B=2, Q=19, M=3, D=D, shapes=[(7, 9), (4, 5)], K=3, dtype=dtype, device=DEVICE,
        loc_lo=-0.2, loc_hi=1.2)
    out = msda(value, shapes, starts, loc, attn)
    ref, _ = run_reference_fp32(value, shapes, loc, attn)
    check_fwd(out, ref, dtype)


@pytest.mark.parametrize("L,K", [(1, 1), (1, 2), (2, 8), (5, 3), (4, 16), (3, 60), (12, 2)])
def test_forward_level_point_counts(L, K):
    """L*K from 1 to 180: one slot per pair, partial slots, several LDS passes."""
    shapes = [(max(2, 17 >> i), max(2, 23 >> i)) for i in range(L)]
    value, shapes, starts, loc, attn = make_inputs(
        B=2, Q=21, M=2, D=32, shapes=shapes, K=K, dtype=torch.float32, device=DEVICE,
        loc_lo=-0.1, loc_hi=1.1)
    out = msda(value, shapes, starts, loc, attn)
    ref, _ = run_reference_fp32(value, shapes, loc, attn)
    check_fwd(out, ref, torch.float32)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_forward_exact_knots(dtype):
    """Locations on {0, 1/4, 1/2, 3/4, 1}: integer and half-integer image
    coordinates, the floor / zero-padding boundary cases."""
    value, shapes, starts, loc, attn = make_inputs(
        B=1, Q=40, M=2, D=16, shapes=[(4, 6), (3, 5)], K=4, dtype=dtype, device=DEVICE)
    knots = torch.tensor([0.0, 0.25, 0.5, 0.75, 1.0])
    idx = torch.randint(0, 5, loc.shape, generator=torch.Generator().manual_seed(3))
    loc = knots[idx].to(DEVICE, dtype)
    out = msda(value, shapes, starts, loc, attn)
    ref, _ = run_reference_fp32(value, shapes, loc, attn)
    check_fwd(out, ref, dtype)


def test_empty_batch_and_queries():
    value, shapes, starts, loc, attn = make_inputs(
        B=2, Q=5, M=2, D=8, shapes=[(4, 4)], K=2, dtype=torch.float32, device=DEVICE)
    out = msda(value[:0], shapes, starts, loc[:0], attn[:0])
    assert out.shape == (0, 5, 16)
    out = msda(value, shapes, starts, loc[:, :0], attn[:, :0])
    assert out.shape == (2, 0, 16)


# ---------------------------------------------------------------------------
# Backward
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("fp32_grad_accum", [False, True], ids=["native_acc", "fp32_acc"])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("case", CASES, ids=[c["id"] for c in CASES])
def test_backward_matches_reference(case, dtype, fp32_grad_accum):
    value, shapes, starts, loc, attn = make_inputs(**case_kwargs(case), dtype=dtype, device=DEVICE)
    _, g, grads = run_fwd_bwd(value, shapes, starts, loc, attn, fp32_grad_accum=fp32_grad_accum)
    for t, ref_t in zip(grads, (value, loc, attn)):
        assert t.dtype == dtype and t.shape == ref_t.shape
    _, refs = run_reference_fp32(value, shapes, loc, attn, g)
    check_bwd(grads, refs, dtype)


def test_backward_out_of_bounds_locations():
    value, shapes, starts, loc, attn = make_inputs(
        B=2, Q=64, M=4, D=32, shapes=[(14, 20), (7, 10)], K=4,
        dtype=torch.float32, device=DEVICE, loc_lo=-0.5, loc_hi=1.5)
    _, g, grads = run_fwd_bwd(value, shapes, starts, loc, attn)
    _, refs = run_reference_fp32(value, shapes, loc, attn, g)
    check_bwd(grads, refs, torch.float32)


def test_fp32_accum_paths_agree_at_fp32():
    value, shapes, starts, loc, attn = make_inputs(
        B=2, Q=100, M=4, D=32, shapes=[(24, 32), (12, 16)], K=4,
        dtype=torch.float32, device=DEVICE)
    grads = []
    for fp32_acc in (False, True):
        v = value.clone().requires_grad_(True)
        out = msda(v, shapes, starts, loc, attn, fp32_grad_accum=fp32_acc)
        out.backward(torch.ones_like(out))
        grads.append(v.grad)
    torch.testing.assert_close(grads[0], grads[1], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("D", [1, 3, 5, 12, 100])
def test_backward_head_dims(D, dtype):
    value, shapes, starts, loc, attn = make_inputs(
        B=2, Q=19, M=3, D=D, shapes=[(7, 9), (4, 5)], K=3, dtype=dtype, device=DEVICE,
        loc_lo=-0.2, loc_hi=1.2)
    _, g, grads = run_fwd_bwd(value, shapes, starts, loc, attn, fp32_grad_accum=True)
    _, refs = run_reference_fp32(value, shapes, loc, attn, g)
    check_bwd(grads, refs, dtype)


@pytest.mark.parametrize("L,K", [(1, 1), (2, 8), (5, 3), (3, 60)])
def test_backward_level_point_counts(L, K):
    shapes = [(max(2, 17 >> i), max(2, 23 >> i)) for i in range(L)]
    value, shapes, starts, loc, attn = make_inputs(
        B=2, Q=21, M=2, D=32, shapes=shapes, K=K, dtype=torch.float32, device=DEVICE,
        loc_lo=-0.1, loc_hi=1.1)
    _, g, grads = run_fwd_bwd(value, shapes, starts, loc, attn)
    _, refs = run_reference_fp32(value, shapes, loc, attn, g)
    check_bwd(grads, refs, torch.float32)


def test_backward_loc_and_attn_grads_are_deterministic():
    value, shapes, starts, loc, attn = make_inputs(
        B=2, Q=100, M=4, D=32, shapes=[(24, 32), (12, 16)], K=4,
        dtype=torch.bfloat16, device=DEVICE)
    _, _, g1 = run_fwd_bwd(value, shapes, starts, loc, attn)
    _, _, g2 = run_fwd_bwd(value, shapes, starts, loc, attn)
    assert torch.equal(g1[1], g2[1]) and torch.equal(g1[2], g2[2])


# ---------------------------------------------------------------------------
# Every kernel variant: launch-shape overrides (msda_set_launch_override)
# ---------------------------------------------------------------------------

OVERRIDES = [
    dict(),                                          # defaults: owner backward
    dict(BWD_OWNER=0),                               # binned owner backward (where it fits)
    dict(BWD_OWNER=0, BWD_BIN=0),                    # atomic row-dedup backward
    dict(BWD_OWNER=0, BWD_BIN=0, BWD_PRIV=0),        # direct, 16 lanes/row
    dict(BWD_OWNER=0, BWD_BIN=0, BWD_PRIV=0, BWD_CB=16, BWD_TS=4),
    dict(BWD_OWNER=0, BWD_BIN=0, BWD_PRIV=0, BWD_CB=8, BWD_TS=16),
    dict(OWN_MIX=0),                                 # owner path, gradient workgroups last
    dict(OWN_MIX=1),                                 # owner path, gradient workgroups first
    dict(OWN_MIX=-1),                                # owner path, gradient kernel launched apart
    dict(FWD_TS=1, FWD_CB=8),                        # owner path, other dot-kernel shapes
    dict(FWD_TS=1), dict(FWD_TS=16),
    dict(FWD_CB=8, FWD_TS=4), dict(FWD_CB=4, FWD_TS=2),
]


@pytest.fixture
def launch_knobs(request, overrides):
    overrides(**request.param)
    return request.param


@pytest.mark.parametrize("launch_knobs", OVERRIDES, indirect=True,
                         ids=lambda d: ",".join(f"{k}={v}" for k, v in d.items()) or "default")
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("case", [CASES[0], CASES[3]], ids=[CASES[0]["id"], CASES[3]["id"]])
def test_kernel_variants_match_reference(case, dtype, launch_knobs):
    value, shapes, starts, loc, attn = make_inputs(**case_kwargs(case), dtype=dtype, device=DEVICE,
                                                   loc_lo=-0.1, loc_hi=1.1)
    out, g, grads = run_fwd_bwd(value, shapes, starts, loc, attn, fp32_grad_accum=True)
    ref, refs = run_reference_fp32(value, shapes, loc, attn, g)
    check_fwd(out, ref, dtype)
    check_bwd(grads, refs, dtype)
