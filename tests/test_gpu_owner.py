"""GPU parity of the owner-computes grad_value backward.

Calls with few samples per (batch, head, level) (Q * K <= 2048, rows of a
multiple of 16 bytes) take a backward without atomics: workgroups that own
bands of value rows write every grad_value element once, and the direct
kernel computes grad_loc / grad_attn without its scatter.  These tests check
that path against the oracle on the cases that stress it -- bands that
split coarse levels, padded lanes, many samples piled onto one band (more
CSR entries than one pass holds), level tables other than the cumulative
one (gaps, overlaps, reordered levels) -- and against the atomic kernels it
replaces (override BWD_OWNER=0).
"""

import pytest
import torch

from msda_cases import BWD_RELERR, BWD_TOL, DTYPES, make_inputs, per_pixel, rel_err
from msda_triton_amd import _native
from msda_triton_amd import multi_scale_deformable_attention as msda
from oracle import msda_backward_analytic, run_reference, run_reference_fp32


def reference_grads(value, shapes, loc, attn, g):
    """The reference's fp32 CPU protocol for half inputs; float64 for fp32
    inputs, whose maps here are wide enough (W up to 84) that the fp32
    grid_sample grid's own rounding (~W * 2^-25 px) shows in grad_loc next to
    the kernels' (compensated) coordinates."""
    if value.dtype == torch.float32:
        return run_reference(value, shapes, loc, attn, g, dtype=torch.float64)
    return run_reference_fp32(value, shapes, loc, attn, g)

pytestmark = pytest.mark.gpu
DEVICE = "cuda"
OWNER, DEDUP, BINNED = 2, 1, 3
DCODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def plan(value, loc):
    """grad_value path the library takes for these inputs (msda_backward_plan)."""
    B, S, M, D = value.shape
    _, Q, _, L, K, _ = loc.shape
    return _native.load().msda_backward_plan(B, S, M, D, Q, L, K, DCODE[value.dtype], 0)


def check_grads(grads, refs, dtype, shapes=None):
    for name, g, r in zip(("grad_value", "grad_loc", "grad_attn"), grads, refs):
        e = rel_err(g, r)
        assert e <= BWD_RELERR[dtype], f"{name}: rel_err {e:.3e} > {BWD_RELERR[dtype]}"
        if name == "grad_loc" and dtype == torch.float32 and shapes is not None:
            g, r = per_pixel(g, shapes), per_pixel(r, shapes)  # elementwise per pixel
        torch.testing.assert_close(g.float().cpu(), r.float(), **BWD_TOL[dtype],
                                   msg=lambda m: f"{name}: {m}")


def fwd_bwd(value, shapes, starts, loc, attn, seed=7, **kw):
    v = value.clone().requires_grad_(True)
    lo = loc.clone().requires_grad_(True)
    a = attn.clone().requires_grad_(True)
    out = msda(v, shapes, starts, lo, a, **kw)
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(seed)).to(out.device,
                                                                                  out.dtype)
    out.backward(g)
    torch.cuda.synchronize()
    return g, (v.grad, lo.grad, a.grad)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("owner", ["1", "0", "bin"])
def test_decoder_shapes_both_paths(dtype, owner, overrides):
    """Decoder-style call (Q*K = 1200 per level, coarse levels split into
    several bands) on the owner path, the atomic one and the binned one."""
    overrides(BWD_OWNER=1 if owner == "1" else 0, BWD_BIN=1 if owner == "bin" else 0)
    value, shapes, starts, loc, attn = make_inputs(
        B=2, Q=300, M=4, D=32, shapes=[(50, 84), (25, 42), (13, 21), (7, 11)], K=4,
        dtype=dtype, device=DEVICE, loc_lo=-0.1, loc_hi=1.1)
    # fp32: 38 KB of grad_out, the 40 KB build
    expect = {"1": OWNER, "0": DEDUP, "bin": BINNED}[owner]
    assert plan(value, loc) == expect
    g, grads = fwd_bwd(value, shapes, starts, loc, attn)
    _, refs = reference_grads(value, shapes, loc, attn, g)
    check_grads(grads, refs, dtype, shapes)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("Q", [304, 305, 640])
def test_grad_out_staging_builds(Q, dtype):
    """grad_out rows of (b, m) up to 19456 bytes take the four-per-CU build,
    up to 40960 bytes the two-per-CU one (Q * D * elem at the edges of both)."""
    value, shapes, starts, loc, attn = make_inputs(
        B=1, Q=Q, M=2, D=32, shapes=[(30, 40), (15, 20), (8, 10)], K=2, dtype=dtype,
        device=DEVICE, loc_lo=-0.1, loc_hi=1.1)
    fits = Q * 32 * value.element_size() <= 40960
    assert (plan(value, loc) == OWNER) == fits  # beyond: the binned path
    g, grads = fwd_bwd(value, shapes, starts, loc, attn)
    _, refs = reference_grads(value, shapes, loc, attn, g)
    check_grads(grads, refs, dtype, shapes)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("D", [8, 16, 24, 48, 64, 128])
def test_row_widths(D, dtype):
    """Rows of 16 to 512 bytes: 1 to 16 lanes per row (padded lanes when
    the chunk count is not a power of two); rows wider than 16 chunks and
    rows not a multiple of 16 bytes take the atomic path."""
    value, shapes, starts, loc, attn = make_inputs(
        B=2, Q=40, M=3, D=D, shapes=[(9, 13), (5, 7)], K=3, dtype=dtype, device=DEVICE,
        loc_lo=-0.2, loc_hi=1.2)
    row = D * value.element_size()
    assert (plan(value, loc) == OWNER) == (row % 16 == 0 and row <= 256)
    g, grads = fwd_bwd(value, shapes, starts, loc, attn)
    _, refs = reference_grads(value, shapes, loc, attn, g)
    check_grads(grads, refs, dtype, shapes)


@pytest.mark.parametrize("QK", [(128, 16), (128, 17)], ids=["QK2048_owner", "QK2176_other"])
def test_sample_count_boundary(QK):
    """Q*K = 2048 (8 samples per lane, the owner path's limit) and beyond."""
    Q, K = QK
    value, shapes, starts, loc, attn = make_inputs(
        B=1, Q=Q, M=2, D=32, shapes=[(20, 30), (10, 15)], K=K, dtype=torch.float32,
        device=DEVICE)
    assert (plan(value, loc) == OWNER) == (Q * K <= 2048)
    g, grads = fwd_bwd(value, shapes, starts, loc, attn)
    _, refs = reference_grads(value, shapes, loc, attn, g)
    check_grads(grads, refs, torch.float32, shapes)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
@pytest.mark.parametrize("D", [8, 32])
def test_samples_piled_on_one_band(dtype, D):
    """All 2048 samples of a (b, m, level) within a pixel or two: 8192 corner
    entries on a handful of rows of one band, more than one CSR pass holds,
    so the band is processed in several sub-bands, and single rows span
    dozens of the entry slices (their pieces summed in groups).  D = 8 gives
    rows of one or two lanes (256 or 128 slices per pass), D = 32 of four
    or eight.  The sums' order is fixed by the inputs: two runs agree
    bitwise."""
    value, shapes, starts, loc, attn = make_inputs(
        B=1, Q=128, M=2, D=D, shapes=[(16, 16), (8, 8)], K=16, dtype=torch.float32,
        device="cpu")
    gen = torch.Generator().manual_seed(11)
    loc = 0.5 + 0.02 * torch.rand(loc.shape, generator=gen)
    value, loc, attn = (t.to(DEVICE, dtype) for t in (value, loc, attn))
    shapes = shapes.to(DEVICE)
    assert plan(value, loc) == OWNER
    g, grads = fwd_bwd(value, shapes, starts.to(DEVICE), loc, attn)
    _, refs = reference_grads(value, shapes, loc, attn, g)
    check_grads(grads, refs, dtype, shapes)
    _, again = fwd_bwd(value, shapes, starts.to(DEVICE), loc, attn)
    assert torch.equal(grads[0], again[0])


def _analytic(value, shapes, starts, loc, attn, g):
    return msda_backward_analytic(value.double().cpu(), shapes.cpu(), starts.cpu(),
                                  loc.double().cpu(), attn.double().cpu(), g.double().cpu(),
                                  dtype=torch.float64)


@pytest.mark.parametrize("path", ["owner", "binned"])
@pytest.mark.parametrize("layout", ["trailing_rows", "gap_between_levels", "overlapping_levels",
                                    "reversed_levels"])
def test_nonstandard_level_tables(layout, path):
    """level_start_index other than the cumulative sum of H*W: value rows no
    level covers must get zero gradient, rows two levels share get both
    levels' contributions.  Checked against the float64 hand backward, which
    indexes rows through the given starts.  Q = 60 takes the owner path,
    Q = 600 (Q*K = 2400) the binned one."""
    hw = [(12, 10), (6, 5), (3, 4)]
    sizes = [h * w for h, w in hw]
    if layout == "trailing_rows":
        starts, S = [0, 120, 150], 150 + 12 + 1500
    elif layout == "gap_between_levels":
        starts, S = [0, 1300, 1400], 1500
    elif layout == "overlapping_levels":
        starts, S = [0, 100, 110], 130
    else:
        starts, S = [42, 12, 0], 162
    assert all(s + n <= S for s, n in zip(starts, sizes))
    B, Q, M, D, K = 2, 60 if path == "owner" else 600, 2, 32, 4
    gen = torch.Generator().manual_seed(5)
    want = OWNER if path == "owner" else BINNED
    assert plan(torch.empty(B, S, M, D), torch.empty(B, Q, M, 3, K, 2)) == want
    value = torch.randn(B, S, M, D, generator=gen)
    loc = -0.1 + 1.2 * torch.rand(B, Q, M, 3, K, 2, generator=gen)
    attn = torch.rand(B, Q, M, 3, K, generator=gen).flatten(3).softmax(-1).view(B, Q, M, 3, K)
    shapes_t = torch.tensor(hw, dtype=torch.long)
    starts_t = torch.tensor(starts, dtype=torch.long)
    g, grads = fwd_bwd(value.to(DEVICE), shapes_t.to(DEVICE), starts_t.to(DEVICE),
                       loc.to(DEVICE), attn.to(DEVICE))
    refs = _analytic(value, shapes_t, starts_t, loc, attn, g)
    check_grads(grads, refs, torch.float32, shapes_t)
    if layout in ("trailing_rows", "gap_between_levels"):
        covered = torch.zeros(S, dtype=torch.bool)
        for s, n in zip(starts, sizes):
            covered[s:s + n] = True
        assert torch.count_nonzero(grads[0][:, ~covered.to(DEVICE)]) == 0


def test_degenerate_levels():
    """Levels of one row or one column (corners 01 and 10 on the same pixel
    index never both in the map) and an empty level."""
    hw = [(1, 37), (29, 1), (0, 5), (4, 4)]
    B, Q, M, D, K = 1, 50, 2, 16, 4
    S = sum(h * w for h, w in hw)
    gen = torch.Generator().manual_seed(9)
    value = torch.randn(B, S, M, D, generator=gen)
    loc = -0.1 + 1.2 * torch.rand(B, Q, M, len(hw), K, 2, generator=gen)
    attn = torch.rand(B, Q, M, len(hw), K, generator=gen)
    shapes_t = torch.tensor(hw, dtype=torch.long)
    sizes = shapes_t.prod(-1)
    starts_t = torch.cat([sizes.new_zeros(1), sizes.cumsum(0)[:-1]])
    g, grads = fwd_bwd(value.to(DEVICE), shapes_t.to(DEVICE), None, loc.to(DEVICE),
                       attn.to(DEVICE))
    refs = _analytic(value, shapes_t, starts_t, loc, attn, g)
    check_grads(grads, refs, torch.float32, shapes_t)


def test_owner_and_atomic_paths_agree_on_decoder_preset(overrides):
    """Full decoder preset (bf16): the owner path (fp32 sums, one rounding)
    against the atomic path with fp32 accumulation -- same fp32 sums up to
    summation order, so they agree to a few bf16 ulps."""
    from msda_triton_amd.presets import make_preset_inputs

    value, shapes, starts, loc, attn = make_preset_inputs("decoder", device=DEVICE)
    assert plan(value, loc) == OWNER
    g1, grads1 = fwd_bwd(value, shapes, starts, loc, attn)
    overrides(BWD_OWNER=0, BWD_BIN=0)
    g2, grads2 = fwd_bwd(value, shapes, starts, loc, attn, fp32_grad_accum=True)
    assert torch.equal(g1, g2)
    for a, b in zip(grads1[1:], grads2[1:]):  # other kernels: same sums, other order
        assert rel_err(a, b) <= 1e-2
    d = (grads1[0].float() - grads2[0].float()).abs()
    scale = grads2[0].float().abs().clamp_min(2.0 ** -10)
    assert (d / scale).max().item() <= 2.0 ** -6
    assert rel_err(grads1[0], grads2[0]) <= 1e-3


@pytest.mark.parametrize("preset", ["decoder", "high_contention"])
def test_owner_path_is_bitwise_reproducible(preset):
    """The owner path sums every grad_value element in an order fixed by the
    inputs (per-wave rank counters, fixed slices): repeated calls give the
    same bits -- also where many samples pile onto a few rows."""
    from msda_triton_amd.presets import make_grad_out, make_preset_inputs

    value, shapes, starts, loc, attn = make_preset_inputs(preset, device=DEVICE)
    assert plan(value, loc) == OWNER
    g = make_grad_out(preset, device=DEVICE).view(value.shape[0], loc.shape[1], -1)
    runs = []
    for _ in range(3):
        v, lo, a = (t.clone().requires_grad_(True) for t in (value, loc, attn))
        msda(v, shapes, starts, lo, a).backward(g)
        runs.append((v.grad, lo.grad, a.grad))
    torch.cuda.synchronize()
    for r in runs[1:]:
        for x, y in zip(runs[0], r):
            assert torch.equal(x, y)
