"""GPU parity of the fused MSDeformAttn front-end (C ABI msda_fused_forward /
msda_fused_backward) against the float64 CPU oracle of the composition
labs/solutions/lab00.py:201-208 (oracle.run_fused_reference), plus its
consistency with the plain operator, the saved log-sum-exp, determinism,
both backward kernels, and the attention layer built on it.

Tolerances are the operator's: forward rel-err <= 1e-5 (fp32) / 1e-2 (half),
each gradient <= 1e-4 / 2e-2.
"""

import pytest
import torch

from msda_cases import BWD_RELERR, DTYPES, FWD_RELERR, make_fused_inputs, rel_err
from msda_triton_amd import multi_scale_deformable_attention as msda
from msda_triton_amd.fused import (MSDACrossAttention, fused_forward_raw,
                                   multi_scale_deformable_attention_fused as msda_fused)
from oracle import msda_fused_reference, run_fused_reference

pytestmark = pytest.mark.gpu
DEVICE = "cuda"
NAMES = ("grad_value", "grad_reference_points", "grad_sampling_offsets", "grad_attention_logits")

FUSED_CASES = [
    dict(id="decoder_small", B=2, Q=50, M=4, D=32, K=4, shapes=[(24, 32), (12, 16), (6, 8)]),
    dict(id="single_point", B=1, Q=17, M=1, D=16, K=1, shapes=[(13, 9)]),
    dict(id="nonpow2", B=2, Q=33, M=2, D=24, K=3, shapes=[(10, 14), (5, 7)]),
    dict(id="wide_head", B=1, Q=40, M=8, D=64, K=4, shapes=[(16, 16), (8, 8)]),
    dict(id="many_points", B=1, Q=9, M=2, D=8, K=45, shapes=[(9, 11), (5, 6), (3, 3), (2, 2)]),
    dict(id="odd_D", B=1, Q=21, M=3, D=5, K=2, shapes=[(7, 6), (4, 3)]),
]


def kw(case):
    return {k: v for k, v in case.items() if k != "id"}


def run_fused(value, shapes, starts, ref, off, logits, grad_seed=7, **kwargs):
    leaves = [t.clone().requires_grad_(True) for t in (value, ref, off, logits)]
    out = msda_fused(leaves[0], shapes, starts, *leaves[1:], **kwargs)
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(grad_seed))
    g = g.to(out.device, out.dtype)
    out.backward(g)
    return out.detach(), g, tuple(t.grad for t in leaves)


def check(out, grads, ref_out, ref_grads, dtype):
    e = rel_err(out, ref_out)
    assert e <= FWD_RELERR[dtype], f"forward rel_err {e:.3e}"
    for name, g, r in zip(NAMES, grads, ref_grads):
        assert g.shape == r.shape, name
        e = rel_err(g, r)
        assert e <= BWD_RELERR[dtype], f"{name}: rel_err {e:.3e} > {BWD_RELERR[dtype]}"


@pytest.mark.parametrize("per_level", [False, True], ids=["shared_ref", "per_level_ref"])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("case", FUSED_CASES, ids=[c["id"] for c in FUSED_CASES])
def test_fused_matches_float64_oracle(case, dtype, per_level):
    value, shapes, starts, ref, off, logits = make_fused_inputs(
        **kw(case), dtype=dtype, device=DEVICE, per_level=per_level)
    out, g, grads = run_fused(value, shapes, starts, ref, off, logits)
    assert out.dtype == dtype and out.shape == (case["B"], case["Q"], case["M"] * case["D"])
    ref_out, ref_grads = run_fused_reference(value, shapes, ref, off, logits, g)
    check(out, grads, ref_out, ref_grads, dtype)


@pytest.mark.parametrize("priv", ["1", "0", "bin"], ids=["dedup", "direct", "binned"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
def test_fused_atomic_backward_kernels(dtype, priv, overrides):
    """The other backward kernels (row-dedup and direct atomics, binned
    owner) in their fused variants; the default for these sizes is the
    owner-computes backward.  The binned case uses Q = 400 so that its
    bookkeeping fits grad_attention_weights in every dtype."""
    from test_gpu_owner import plan

    overrides(BWD_OWNER=0, BWD_BIN=1 if priv == "bin" else 0, BWD_PRIV=0 if priv == "0" else 1)
    case = dict(FUSED_CASES[0], Q=400) if priv == "bin" else FUSED_CASES[0]
    value, shapes, starts, ref, off, logits = make_fused_inputs(
        **kw(case), dtype=dtype, device=DEVICE, per_level=True)
    assert plan(value, off) == {"1": 1, "0": 0, "bin": 3}[priv]
    out, g, grads = run_fused(value, shapes, starts, ref, off, logits)
    ref_out, ref_grads = run_fused_reference(value, shapes, ref, off, logits, g)
    check(out, grads, ref_out, ref_grads, dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_fused_fp32_accumulation(dtype):
    case = FUSED_CASES[0]
    value, shapes, starts, ref, off, logits = make_fused_inputs(
        **kw(case), dtype=dtype, device=DEVICE)
    out, g, grads = run_fused(value, shapes, starts, ref, off, logits, fp32_grad_accum=True)
    ref_out, ref_grads = run_fused_reference(value, shapes, ref, off, logits, g)
    check(out, grads, ref_out, ref_grads, dtype)


def test_fused_out_of_bounds_offsets():
    """Large offsets put many corners outside the maps (zeros padding)."""
    case = FUSED_CASES[0]
    value, shapes, starts, ref, off, logits = make_fused_inputs(
        **kw(case), dtype=torch.float32, device=DEVICE, offset_sigma=12.0)
    out, g, grads = run_fused(value, shapes, starts, ref, off, logits)
    ref_out, ref_grads = run_fused_reference(value, shapes, ref, off, logits, g)
    check(out, grads, ref_out, ref_grads, torch.float32)


def test_lse_is_the_log_sum_exp_of_the_logits():
    case = FUSED_CASES[0]
    value, shapes, starts, ref, off, logits = make_fused_inputs(
        **kw(case), dtype=torch.float32, device=DEVICE, logit_sigma=4.0)
    _, lse = fused_forward_raw(value, shapes, starts, ref, off, logits, 0)
    expect = torch.logsumexp(logits.double().flatten(3), -1)
    torch.testing.assert_close(lse.double(), expect, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("per_level", [False, True])
def test_fused_equals_operator_on_composed_inputs(per_level):
    """fp32: the fused kernels agree with the plain operator run on the
    locations and weights composed by PyTorch on the GPU."""
    case = FUSED_CASES[3]
    value, shapes, starts, ref, off, logits = make_fused_inputs(
        **kw(case), dtype=torch.float32, device=DEVICE, per_level=per_level)
    B, Q, M, L, K, _ = off.shape
    scale = shapes.flip(-1).float()[None, None, None, :, None, :]
    r = ref[:, :, None, None, None, :] if not per_level else ref[:, :, None, :, None, :]
    loc = r + off / scale
    attn = logits.flatten(3).softmax(-1).view(B, Q, M, L, K)
    a = msda(value, shapes, starts, loc, attn)
    b = msda_fused(value, shapes, starts, ref, off, logits)
    torch.testing.assert_close(b, a, rtol=2e-5, atol=2e-5)


def test_fused_gradients_are_deterministic():
    """Only grad_value uses atomics; the other three gradients are written
    once (grad_reference_points by a fixed-order reduction)."""
    case = FUSED_CASES[0]
    value, shapes, starts, ref, off, logits = make_fused_inputs(
        **kw(case), dtype=torch.bfloat16, device=DEVICE, per_level=True)
    _, _, g1 = run_fused(value, shapes, starts, ref, off, logits)
    _, _, g2 = run_fused(value, shapes, starts, ref, off, logits)
    for name, a, b in zip(NAMES[1:], g1[1:], g2[1:]):
        assert torch.equal(a, b), name


def test_fused_logits_in_flat_layout_and_no_reference_grad():
    """Logits given as (B, Q, M, L*K) get their gradient in that shape; a
    reference point that does not require grad is skipped."""
    case = FUSED_CASES[0]
    value, shapes, starts, ref, off, logits = make_fused_inputs(
        **kw(case), dtype=torch.float32, device=DEVICE)
    B, Q, M, L, K, _ = off.shape
    flat = logits.reshape(B, Q, M, L * K).clone().requires_grad_(True)
    o = off.clone().requires_grad_(True)
    out = msda_fused(value, shapes, None, ref, o, flat)
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(7)).to(DEVICE)
    out.backward(g)
    assert flat.grad.shape == (B, Q, M, L * K)
    _, ref_grads = run_fused_reference(value, shapes, ref, off, logits, g)
    assert rel_err(flat.grad.view(B, Q, M, L, K), ref_grads[3]) <= 1e-4
    assert rel_err(o.grad, ref_grads[2]) <= 1e-4


def test_fused_empty_inputs():
    value, shapes, starts, ref, off, logits = make_fused_inputs(
        B=1, Q=0, M=2, D=8, K=2, shapes=[(4, 4)], dtype=torch.float32, device=DEVICE)
    out = msda_fused(value, shapes, starts, ref, off, logits)
    assert out.shape == (1, 0, 16)


def test_fused_validation_messages():
    value, shapes, starts, ref, off, logits = make_fused_inputs(
        B=1, Q=4, M=2, D=8, K=2, shapes=[(4, 4)], dtype=torch.float32, device=DEVICE)
    with pytest.raises(ValueError, match="reference_points"):
        msda_fused(value, shapes, starts, ref[:, :, :1], off, logits)
    with pytest.raises(ValueError, match="attention_logits"):
        msda_fused(value, shapes, starts, ref, off, logits[..., :1])
    with pytest.raises(ValueError, match="dtypes"):
        msda_fused(value, shapes, starts, ref, off, logits.double())


def test_fused_decoder_preset_full_size():
    """The decoder preset's shapes (B4 Q300 M8 D32 L4 K4, 800x1333 pyramid)
    in bf16, per-level reference points."""
    value, shapes, starts, ref, off, logits = make_fused_inputs(
        B=4, Q=300, M=8, D=32, K=4, shapes=[(100, 167), (50, 84), (25, 42), (13, 21)],
        dtype=torch.bfloat16, device=DEVICE, per_level=True)
    out, g, grads = run_fused(value, shapes, starts, ref, off, logits)
    ref_out, ref_grads = run_fused_reference(value, shapes, ref, off, logits, g)
    check(out, grads, ref_out, ref_grads, torch.bfloat16)


@pytest.mark.parametrize("C,M,L,K,native", [(64, 4, 3, 4, True), (48, 2, 2, 3, False)],
                         ids=["projection_kernels", "linear_modules"])
@pytest.mark.parametrize("padded", [False, True], ids=["nomask", "padding_mask"])
def test_cross_attention_layer_matches_composed_reference(C, M, L, K, native, padded):
    """The layer (projections + fused operator) against the same weights run
    in float64 on the CPU through the oracle composition, every parameter's
    gradient included; with a padding mask the value rows of padded pixels
    are zeroed after the value projection (Deformable-DETR's masked_fill)."""
    torch.manual_seed(0)
    shapes_l = [(12, 16), (6, 8), (3, 4)][:L]
    layer = MSDACrossAttention(C, M, L, K).to(DEVICE)
    assert layer.native_projections == native
    with torch.no_grad():  # offsets of a few pixels, logits O(1)
        layer.offset_proj.weight.mul_(20.0)
    B, Q = 2, 30
    S = sum(h * w for h, w in shapes_l)
    g = torch.Generator().manual_seed(1)
    query = torch.randn(B, Q, C, generator=g).to(DEVICE).requires_grad_(True)
    value = torch.randn(B, S, C, generator=g).to(DEVICE).requires_grad_(True)
    refp = torch.rand(B, Q, 2, generator=g).to(DEVICE).requires_grad_(True)
    mask = None
    if padded:
        mask = torch.rand(B, S, generator=g) < 0.3
        mask[1, S // 2:] = True
        mask = mask.to(DEVICE)
    shapes = torch.tensor(shapes_l, device=DEVICE)
    out = layer(query, refp, value, shapes, input_padding_mask=mask)
    gout = torch.randn(out.shape, generator=g).to(DEVICE)
    out.backward(gout)

    cpu = MSDACrossAttention(C, M, L, K).double()
    cpu.load_state_dict({k: v.detach().double().cpu() for k, v in layer.state_dict().items()})
    q64 = query.detach().double().cpu().requires_grad_(True)
    v64 = value.detach().double().cpu().requires_grad_(True)
    r64 = refp.detach().double().cpu().requires_grad_(True)
    D = C // M
    vv = cpu.value_proj(v64)
    if padded:
        vv = vv.masked_fill(mask.cpu()[..., None], 0.0)
    vv = vv.reshape(B, S, M, D)
    offs = cpu.offset_proj(q64).reshape(B, Q, M, L, K, 2)
    logits = cpu.weight_proj(q64).reshape(B, Q, M, L, K)
    ref_out = cpu.out_proj(msda_fused_reference(vv, shapes.cpu(), r64, offs, logits))
    ref_out.backward(gout.double().cpu())
    assert rel_err(out, ref_out) <= 1e-5
    checks = [("query", query.grad, q64.grad), ("value", value.grad, v64.grad),
              ("reference_points", refp.grad, r64.grad)]
    for mod in ("value_proj", "offset_proj", "weight_proj", "out_proj"):
        for par in ("weight", "bias"):
            checks.append((f"{mod}.{par}", getattr(getattr(layer, mod), par).grad,
                           getattr(getattr(cpu, mod), par).grad))
    for name, a, b in checks:
        e = rel_err(a, b)
        assert e <= 1e-4, f"{name}: rel_err {e:.3e}"
