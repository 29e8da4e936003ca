"""Deterministic backward (msda_backward_deterministic and its fused
variant): grad_value -- from the owner path where it applies, accumulated in
int64 fixed point otherwise -- must match the oracle
within the operator's tolerances and be bitwise identical from run to run --
also where float atomics are most order-sensitive (the high-contention
preset) -- through both backward kernels, every dtype, odd head dims, the
torch deterministic-algorithms switch, and gradient scales far from 1.
"""

import pytest
import torch

from msda_cases import (BWD_RELERR, CASES, DTYPES, case_kwargs, make_fused_inputs, make_inputs,
                        rel_err)
from msda_triton_amd import msda_op, multi_scale_deformable_attention as msda, presets
from msda_triton_amd.fused import multi_scale_deformable_attention_fused as msda_fused
from oracle import run_fused_reference, run_reference

pytestmark = pytest.mark.gpu
DEVICE = "cuda"


def grads_of(value, shapes, starts, loc, attn, g, **kw):
    v, lo, a = (t.clone().requires_grad_(True) for t in (value, loc, attn))
    out = msda(v, shapes, starts, lo, a, **kw)
    out.backward(g)
    return out.detach(), (v.grad, lo.grad, a.grad)


def seeded_grad(shape, dtype, scale=1.0, seed=7):
    g = torch.randn(shape, generator=torch.Generator().manual_seed(seed)) * scale
    return g.to(DEVICE, dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("case", CASES, ids=[c["id"] for c in CASES])
def test_deterministic_matches_reference(case, dtype):
    value, shapes, starts, loc, attn = make_inputs(**case_kwargs(case), dtype=dtype, device=DEVICE)
    B, Q, M, D = case["B"], case["Q"], case["M"], case["D"]
    g = seeded_grad((B, Q, M * D), dtype)
    _, grads = grads_of(value, shapes, starts, loc, attn, g, deterministic=True)
    _, refs = run_reference(value, shapes, loc, attn, g, dtype=torch.float64)
    for name, x, r in zip(("grad_value", "grad_loc", "grad_attn"), grads, refs):
        e = rel_err(x, r)
        assert e <= BWD_RELERR[dtype], f"{name}: rel_err {e:.3e}"


@pytest.mark.parametrize("path", ["owner", "row_dedup", "direct"])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_deterministic_is_bitwise_reproducible_under_contention(dtype, path, overrides):
    """High-contention locations (most samples share a few corners): two
    runs give identical bits; the fp32 result matches float64 closely --
    on the owner path and on the int64 fixed-point atomic paths."""
    overrides(BWD_OWNER=1 if path == "owner" else 0, BWD_PRIV=0 if path == "direct" else 1)
    value, shapes, starts, _, attn = make_inputs(B=2, Q=120, M=4, D=32, K=4,
                                                 shapes=[(40, 50), (20, 25)], dtype=dtype,
                                                 device=DEVICE)
    gen = torch.Generator().manual_seed(3)
    loc = (0.5 + 0.004 * torch.randn(2, 120, 4, 2, 4, 2, generator=gen)).to(DEVICE, dtype)
    g = seeded_grad((2, 120, 128), dtype)
    _, g1 = grads_of(value, shapes, starts, loc, attn, g, deterministic=True)
    _, g2 = grads_of(value, shapes, starts, loc, attn, g, deterministic=True)
    for name, a, b in zip(("grad_value", "grad_loc", "grad_attn"), g1, g2):
        assert torch.equal(a, b), name
    _, refs = run_reference(value, shapes, loc, attn, g, dtype=torch.float64)
    bound = 1e-6 if dtype == torch.float32 else BWD_RELERR[dtype]
    e = rel_err(g1[0], refs[0])
    assert e <= bound, f"grad_value rel_err {e:.3e}"


def test_deterministic_odd_half_head_dim():
    """Odd D in half precision takes the direct kernel with 2-byte chunks."""
    value, shapes, starts, loc, attn = make_inputs(B=1, Q=30, M=3, D=5, K=3,
                                                   shapes=[(9, 7), (4, 5)], dtype=torch.bfloat16,
                                                   device=DEVICE)
    g = seeded_grad((1, 30, 15), torch.bfloat16)
    _, grads = grads_of(value, shapes, starts, loc, attn, g, deterministic=True)
    _, refs = run_reference(value, shapes, loc, attn, g, dtype=torch.float64)
    for x, r in zip(grads, refs):
        assert rel_err(x, r) <= BWD_RELERR[torch.bfloat16]


@pytest.mark.parametrize("scale", [1e-6, 1e4])
def test_deterministic_scale_follows_gradient_magnitude(scale):
    value, shapes, starts, loc, attn = make_inputs(**case_kwargs(CASES[0]), dtype=torch.float32,
                                                   device=DEVICE)
    B, Q, M, D = 2, 100, 4, 32
    g = seeded_grad((B, Q, M * D), torch.float32, scale=scale)
    _, grads = grads_of(value, shapes, starts, loc, attn, g, deterministic=True)
    _, refs = run_reference(value, shapes, loc, attn, g, dtype=torch.float64)
    assert rel_err(grads[0], refs[0]) <= 1e-6


def test_torch_deterministic_switch_selects_it():
    value, shapes, starts, loc, attn = make_inputs(**case_kwargs(CASES[0]), dtype=torch.bfloat16,
                                                   device=DEVICE)
    g = seeded_grad((2, 100, 128), torch.bfloat16)
    _, explicit = grads_of(value, shapes, starts, loc, attn, g, deterministic=True)
    prev = torch.are_deterministic_algorithms_enabled()
    try:
        torch.use_deterministic_algorithms(True)
        _, implicit = grads_of(value, shapes, starts, loc, attn, g)
    finally:
        torch.use_deterministic_algorithms(prev)
    assert torch.equal(explicit[0], implicit[0])


def test_custom_op_deterministic():
    value, shapes, starts, loc, attn = make_inputs(**case_kwargs(CASES[2]), dtype=torch.float16,
                                                   device=DEVICE)
    v = value.clone().requires_grad_(True)
    out = msda_op(v, shapes, starts, loc, attn, deterministic=True)
    g = seeded_grad(out.shape, torch.float16)
    out.backward(g)
    _, refs = run_reference(value, shapes, loc, attn, g, dtype=torch.float64)
    assert rel_err(v.grad, refs[0]) <= BWD_RELERR[torch.float16]


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_fused_deterministic(dtype):
    value, shapes, starts, ref, off, logits = make_fused_inputs(
        B=2, Q=50, M=4, D=32, K=4, shapes=[(24, 32), (12, 16), (6, 8)], dtype=dtype,
        device=DEVICE, per_level=True)
    runs = []
    for _ in range(2):
        leaves = [t.clone().requires_grad_(True) for t in (value, ref, off, logits)]
        out = msda_fused(leaves[0], shapes, starts, *leaves[1:], deterministic=True)
        g = seeded_grad(out.shape, dtype)
        out.backward(g)
        runs.append(tuple(t.grad for t in leaves))
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    _, refs = run_fused_reference(value, shapes, ref, off, logits, g)
    for x, r in zip(runs[0], refs):
        assert rel_err(x, r) <= BWD_RELERR[dtype]


def test_deterministic_high_contention_preset_full_size():
    value, shapes, starts, loc, attn = presets.make_preset_inputs("high_contention", device=DEVICE)
    g = presets.make_grad_out("high_contention", device=DEVICE)
    _, g1 = grads_of(value, shapes, starts, loc, attn, g, deterministic=True)
    _, g2 = grads_of(value, shapes, starts, loc, attn, g, deterministic=True)
    assert torch.equal(g1[0], g2[0])
    _, refs = run_reference(value, shapes, loc, attn, g, dtype=torch.float64)
    for x, r in zip(g1, refs):
        assert rel_err(x, r) <= BWD_RELERR[torch.bfloat16]


@pytest.mark.parametrize("fused", [False, True], ids=["operator", "fused"])
def test_deterministic_misaligned_grad_out(fused):
    """grad_output as a contiguous view at an odd element offset (not 16-byte
    aligned): the deterministic backward of an owner-path call needs no
    workspace, and the host hands the library an aligned copy, so the call
    runs and matches the oracle, bit for bit on a second run."""
    dtype = torch.bfloat16
    B, Q, M, D, K, shapes_l = 2, 50, 4, 32, 4, [(24, 32), (12, 16), (6, 8)]
    flat = torch.randn(B * Q * M * D + 1, generator=torch.Generator().manual_seed(7))
    flat = flat.to(DEVICE, dtype)
    g = flat[1:].view(B, Q, M * D)
    assert g.is_contiguous() and g.data_ptr() % 16 != 0
    runs = []
    if fused:
        value, shapes, starts, ref, off, logits = make_fused_inputs(
            B=B, Q=Q, M=M, D=D, K=K, shapes=shapes_l, dtype=dtype, device=DEVICE, per_level=True)
        for _ in range(2):
            leaves = [t.clone().requires_grad_(True) for t in (value, ref, off, logits)]
            msda_fused(leaves[0], shapes, starts, *leaves[1:], deterministic=True).backward(g)
            runs.append(tuple(t.grad for t in leaves))
        _, refs = run_fused_reference(value, shapes, ref, off, logits, g)
    else:
        value, shapes, starts, loc, attn = make_inputs(B=B, Q=Q, M=M, D=D, K=K, shapes=shapes_l,
                                                       dtype=dtype, device=DEVICE)
        for _ in range(2):
            runs.append(grads_of(value, shapes, starts, loc, attn, g, deterministic=True)[1])
        _, refs = run_reference(value, shapes, loc, attn, g, dtype=torch.float64)
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    for x, r in zip(runs[0], refs):
        assert rel_err(x, r) <= BWD_RELERR[dtype]


def test_deterministic_c_abi_misaligned_grad_out_contract():
    """At the C ABI, a misaligned grad_output rules the owner path out, and
    the workspace query (0 bytes here) assumes aligned buffers: with no
    workspace the call is refused before any launch, buffers untouched.
    (The host operator hands the library aligned copies, see
    test_deterministic_misaligned_grad_out.)"""
    from msda_triton_amd import _native

    lib = _native.load()
    dtype = torch.bfloat16
    B, Q, M, D, K = 2, 50, 4, 32, 4
    value, shapes, starts, loc, attn = make_inputs(B=B, Q=Q, M=M, D=D, K=K,
                                                   shapes=[(24, 32), (12, 16)], dtype=dtype,
                                                   device=DEVICE)
    S, L = value.shape[1], 2
    flat = torch.randn(B * Q * M * D + 1, generator=torch.Generator().manual_seed(3))
    g_bad = flat.to(DEVICE, dtype)[1:]
    assert lib.msda_deterministic_workspace_bytes(B, S, M, D, Q, L, K, 2) == 0
    gv = torch.full_like(value, 3.0)
    gl, ga = torch.full_like(loc, 3.0), torch.full_like(attn, 3.0)
    st = torch.cuda.current_stream().cuda_stream
    rc = lib.msda_backward_deterministic(
        value.data_ptr(), shapes.data_ptr(), starts.data_ptr(), loc.data_ptr(), attn.data_ptr(),
        g_bad.data_ptr(), gv.data_ptr(), None, gl.data_ptr(), ga.data_ptr(), B, S, M, D, Q, L, K,
        2, st)
    assert rc == 1  # MSDA_ERR_INVALID_ARGUMENT
    torch.cuda.synchronize()
    assert bool((gv == 3.0).all()) and bool((gl == 3.0).all()) and bool((ga == 3.0).all())
