"""GPU parity of the binned owner backward (grad_value for calls with many
samples per (batch, head, level): samples binned by band of value rows, each
band summed in LDS and stored once, or added with atomics when its entries
are split over several workgroups).

The cases stress what the binning can get wrong: levels wider than a band
(a sample's corners then span three bands), samples piled onto a few bands
(split bands, atomic adds), corners outside the maps, an empty level, fp32
accumulation, and the fused front-end -- each against the oracle.
"""

import pytest
import torch

from msda_cases import DTYPES, _off_knots, make_fused_inputs, make_inputs
from oracle import run_fused_reference
from test_gpu_fused import check as check_fused
from test_gpu_fused import run_fused
from test_gpu_owner import BINNED, _analytic, check_grads, fwd_bwd, plan, reference_grads

pytestmark = pytest.mark.gpu
DEVICE = "cuda"

BIN_CASES = [
    # Q*K = 2400 per level: beyond the owner path's 2048.
    dict(id="encoder_like", B=2, Q=600, M=4, D=32, K=4, shapes=[(24, 40), (12, 20), (6, 10)]),
    # 300 px rows: wider than a 256-row band.
    dict(id="wide_level", B=1, Q=800, M=2, D=32, K=4, shapes=[(6, 300), (3, 150)]),
    # D = 64 and D = 16 heads (128- and 32-byte half rows).
    dict(id="d64", B=1, Q=700, M=2, D=64, K=4, shapes=[(20, 30), (10, 15)]),
    dict(id="d16", B=1, Q=700, M=4, D=16, K=4, shapes=[(30, 40), (15, 20)]),
    # an empty level between two others
    dict(id="empty_level", B=1, Q=700, M=2, D=32, K=4, shapes=[(20, 30), (0, 7), (5, 8)]),
]


def _inputs(case, dtype, **kw):
    args = {k: v for k, v in case.items() if k != "id"}
    return make_inputs(**args, dtype=dtype, device=DEVICE, **kw)


@pytest.mark.parametrize("fp32_grad_accum", [False, True], ids=["native", "fp32acc"])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("case", BIN_CASES, ids=[c["id"] for c in BIN_CASES])
def test_binned_matches_reference(case, dtype, fp32_grad_accum):
    value, shapes, starts, loc, attn = _inputs(case, dtype, loc_lo=-0.1, loc_hi=1.1)
    if value.dtype == torch.float32 and case["D"] == 64:
        pytest.skip("256-byte fp32 rows: not on the binned path")
    assert plan(value, loc) == BINNED
    print(f"binned {case['id']} {dtype} fp32acc={fp32_grad_accum}", flush=True)
    g, grads = fwd_bwd(value, shapes, starts, loc, attn, fp32_grad_accum=fp32_grad_accum)
    if case["id"] == "empty_level":  # grid_sample rejects empty maps: hand-derived float64
        refs = [r.float() for r in _analytic(value, shapes, starts, loc, attn, g)]
    else:
        _, refs = reference_grads(value, shapes, loc, attn, g)
    check_grads(grads, refs, dtype, shapes)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_binned_split_bands(dtype):
    """Locations N(0.5, 0.01): each (b, m, level)'s 6000 samples land in one
    or two bands, whose entries are split over several workgroups that add
    their sums with atomics."""
    B, Q, M, D, K = 1, 1500, 2, 32, 4
    shapes = [(40, 60), (20, 30)]
    value, sh, starts, loc, attn = make_inputs(B=B, Q=Q, M=M, D=D, shapes=shapes, K=K,
                                               dtype=dtype, device=DEVICE)
    gen = torch.Generator().manual_seed(5)
    loc = (0.5 + 0.01 * torch.randn(loc.shape, generator=gen)).to(DEVICE, dtype)
    assert plan(value, loc) == BINNED
    g, grads = fwd_bwd(value, sh, starts, loc, attn)
    _, refs = reference_grads(value, sh, loc, attn, g)
    check_grads(grads, refs, dtype, sh)


def test_binned_against_atomic_path(overrides):
    """Encoder-like call: the binned path and the row-dedup atomic path with
    fp32 accumulation agree (same fp32 sums, another order)."""
    case = BIN_CASES[0]
    value, shapes, starts, loc, attn = _inputs(case, torch.float32)
    g1, grads1 = fwd_bwd(value, shapes, starts, loc, attn)
    overrides(BWD_BIN=0)
    g2, grads2 = fwd_bwd(value, shapes, starts, loc, attn, fp32_grad_accum=True)
    assert torch.equal(g1, g2)
    torch.testing.assert_close(grads1[0], grads2[0], rtol=1e-5, atol=1e-5)
    for a, b in zip(grads1[1:], grads2[1:]):  # same dot products, other lane split
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)


def test_binned_batch_slices_of_at_most_1024_groups():
    """B*M*L = 1280 (b, m, level) groups: more than one binned launch holds,
    so the batch runs in slices of 4 + 1 elements (256 groups each), every
    slice on the binned path with its own bookkeeping.  Tiny maps: the
    2080 samples of a group pile onto <= 64 pixels (split bands)."""
    B, Q, M, D, K = 5, 520, 64, 8, 4
    shapes = [(8, 8), (4, 4), (2, 2), (1, 1)]
    value, sh, starts, loc, attn = make_inputs(B=B, Q=Q, M=M, D=D, shapes=shapes, K=K,
                                               dtype=torch.float32, device=DEVICE,
                                               loc_lo=-0.1, loc_hi=1.1)
    assert plan(value, loc) == BINNED
    g, grads = fwd_bwd(value, sh, starts, loc, attn)
    _, refs = reference_grads(value, sh, loc, attn, g)
    check_grads(grads, refs, torch.float32, sh)


FUSED_BIN_CASE = dict(B=2, Q=600, M=4, D=32, K=4, shapes=[(24, 40), (12, 20), (6, 10)])


@pytest.mark.parametrize("per_level", [False, True], ids=["shared_ref", "per_level_ref"])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_fused_binned_matches_reference(dtype, per_level):
    """The fused front-end's binned kernels (offsets from reference points,
    softmax weights formed from the saved log-sum-exp) against the float64
    oracle of the composition."""
    value, shapes, starts, ref, off, logits = make_fused_inputs(
        **FUSED_BIN_CASE, dtype=dtype, device=DEVICE, per_level=per_level)
    assert plan(value, off) == BINNED
    print(f"fused binned {dtype} per_level={per_level}", flush=True)
    out, g, grads = run_fused(value, shapes, starts, ref, off, logits)
    ref_out, ref_grads = run_fused_reference(value, shapes, ref, off, logits, g)
    check_fused(out, grads, ref_out, ref_grads, dtype)


@pytest.mark.parametrize("per_level", [False, True], ids=["shared_ref", "per_level_ref"])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_fused_binned_split_bands(dtype, per_level):
    """Reference points N(0.5, 0.01) and offsets N(0, 0.5) px: each (b, m,
    level)'s 6000 samples land in one or two bands, whose entries are split
    over several workgroups that add their sums with atomics."""
    B, Q, M, D, K = 1, 1500, 2, 32, 4
    shapes = [(40, 60), (20, 30)]
    value, sh, starts, ref, off, logits = make_fused_inputs(
        B=B, Q=Q, M=M, D=D, K=K, shapes=shapes, dtype=torch.float32, device="cpu",
        per_level=per_level, offset_sigma=0.5)
    gen = torch.Generator().manual_seed(11)
    ref = (0.5 + 0.01 * torch.randn(ref.shape, generator=gen)).to(dtype)
    off = _off_knots(off.to(dtype), ref, shapes, per_level)
    value, ref, off, logits = (t.to(DEVICE, dtype) for t in (value, ref, off, logits))
    sh, starts = sh.to(DEVICE), starts.to(DEVICE)
    assert plan(value, off) == BINNED
    out, g, grads = run_fused(value, sh, starts, ref, off, logits)
    ref_out, ref_grads = run_fused_reference(value, sh, ref, off, logits, g)
    check_fused(out, grads, ref_out, ref_grads, dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("case", BIN_CASES[:3], ids=[c["id"] for c in BIN_CASES[:3]])
def test_deterministic_binned_matches_reference(case, dtype):
    """deterministic=True on the binned path (int64 fixed-point band sums):
    identical bits on two calls, oracle parity."""
    value, shapes, starts, loc, attn = _inputs(case, dtype, loc_lo=-0.1, loc_hi=1.1)
    if value.dtype == torch.float32 and case["D"] == 64:
        pytest.skip("256-byte fp32 rows: not on the binned path")
    B, S, M, D = value.shape
    _, Q, _, L, K, _ = loc.shape
    from msda_triton_amd import _native
    code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[dtype]
    assert _native.load().msda_backward_plan(B, S, M, D, Q, L, K, code, 1) == BINNED
    g1, grads1 = fwd_bwd(value, shapes, starts, loc, attn, deterministic=True)
    g2, grads2 = fwd_bwd(value, shapes, starts, loc, attn, deterministic=True)
    for a, b in zip(grads1, grads2):
        assert torch.equal(a, b)
    _, refs = reference_grads(value, shapes, loc, attn, g1)
    check_grads(grads1, refs, dtype, shapes)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_deterministic_binned_split_bands(dtype):
    """Split bands (several work items per band) in deterministic mode: the
    items' int64 partial sums add exactly, so two calls agree bit for bit."""
    B, Q, M, D, K = 1, 1500, 2, 32, 4
    shapes = [(40, 60), (20, 30)]
    value, sh, starts, loc, attn = make_inputs(B=B, Q=Q, M=M, D=D, shapes=shapes, K=K,
                                               dtype=dtype, device=DEVICE)
    gen = torch.Generator().manual_seed(5)
    loc = (0.5 + 0.01 * torch.randn(loc.shape, generator=gen)).to(DEVICE, dtype)
    g1, grads1 = fwd_bwd(value, sh, starts, loc, attn, deterministic=True)
    g2, grads2 = fwd_bwd(value, sh, starts, loc, attn, deterministic=True)
    for a, b in zip(grads1, grads2):
        assert torch.equal(a, b)
    _, refs = reference_grads(value, sh, loc, attn, g1)
    check_grads(grads1, refs, dtype, sh)
