"""GPU parity at the benchmark presets' full sizes.

Each preset's seeded inputs go through the HIP operator and through the CPU
oracle on the same bits (fp32 upcast); forward and all three gradients are
compared with the reference's assert_close tolerances and the norm-relative
bounds (forward 1e-5 fp32 / 1e-2 half, gradients 1e-4 / 2e-2).  Size-free
properties are checked as well: the value gradient is the adjoint of the
forward (out is linear in value), and the output is linear in the attention
weights.
"""

import pytest
import torch

from msda_cases import BWD_RELERR, BWD_TOL, FWD_RELERR, FWD_TOL, per_pixel, rel_err
from msda_triton_amd import multi_scale_deformable_attention as msda
from msda_triton_amd import presets
from oracle import run_reference

pytestmark = pytest.mark.gpu
DEVICE = "cuda"


def _fwd_bwd(name, fp32_grad_accum, **kw):
    value, shapes, starts, loc, attn = presets.make_preset_inputs(name, device=DEVICE)
    g = presets.make_grad_out(name, device=DEVICE)
    v, lo, a = (t.clone().requires_grad_(True) for t in (value, loc, attn))
    out = msda(v, shapes, starts, lo, a, fp32_grad_accum=fp32_grad_accum, **kw)
    out.backward(g)
    torch.cuda.synchronize()
    return (value, shapes, loc, attn, g), out.detach(), (v.grad, lo.grad, a.grad)


@pytest.mark.parametrize("name,fp32_grad_accum", [
    ("tiny", False),
    ("decoder", False),
    ("decoder", True),
    ("decoder_fp16", False),
    ("decoder_fp32", False),
    ("high_contention", False),
    ("high_contention", True),
    ("encoder", False),
    ("encoder", True),
    ("mask2former_fp32", False),
    ("mask2former_bf16", False),
    ("mask2former_bf16", True),
])
def test_preset_matches_oracle(name, fp32_grad_accum):
    """Native-dtype accumulation is part of the contract here, also for the
    high-contention preset: the backward sums every row's contributions
    within a workgroup in fp32 and rounds once per (workgroup, row)."""
    dtype = presets.PRESETS[name]["dtype"]
    (value, shapes, loc, attn, g), out, grads = _fwd_bwd(name, fp32_grad_accum)
    # float64 oracle: the fp32 grid_sample grid (2*loc - 1) rounds the image
    # coordinate by up to W * 2^-25 px, visible in grad_loc at these sizes.
    ref, refs = run_reference(value, shapes, loc, attn, g, dtype=torch.float64)
    ref, refs = ref.float(), [r.float() for r in refs]
    torch.testing.assert_close(out.float().cpu(), ref, **FWD_TOL[dtype])
    assert rel_err(out, ref) <= FWD_RELERR[dtype]
    for nm, x, r in zip(("grad_value", "grad_loc", "grad_attn"), grads, refs):
        e = rel_err(x, r)
        assert e <= BWD_RELERR[dtype], f"{name} {nm}: rel_err {e:.3e}"
        if nm == "grad_loc" and dtype == torch.float32:  # elementwise per pixel (per_pixel)
            x, r = per_pixel(x, shapes).float(), per_pixel(r, shapes).float()
        torch.testing.assert_close(x.float().cpu(), r, **BWD_TOL[dtype], msg=lambda m: f"{nm}: {m}")


@pytest.mark.parametrize("name", ["encoder", "mask2former_fp32", "mask2former_bf16"])
def test_deterministic_binned_preset(name):
    """The deterministic backward of the encoder-style presets takes the
    binned path (int64 fixed-point band sums): two calls give identical bits,
    and the result matches the float64 oracle."""
    from msda_triton_amd import _native

    c = presets.preset_dims(name)
    dtype = presets.PRESETS[name]["dtype"]
    code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[dtype]
    plan = _native.load().msda_backward_plan(c["B"], c["S"], c["M"], c["D"], c["Q"], c["L"],
                                             c["K"], code, 1)
    assert plan == 3  # MSDA_BACKWARD_BINNED
    (value, shapes, loc, attn, g), _, grads1 = _fwd_bwd(name, False, deterministic=True)
    _, _, grads2 = _fwd_bwd(name, False, deterministic=True)
    for x, y in zip(grads1, grads2):
        assert torch.equal(x, y)
    _, refs = run_reference(value, shapes, loc, attn, g, dtype=torch.float64)
    for nm, x, r in zip(("grad_value", "grad_loc", "grad_attn"), grads1, refs):
        e = rel_err(x, r)
        assert e <= BWD_RELERR[dtype], f"{name} {nm}: rel_err {e:.3e}"


@pytest.mark.parametrize("name", ["decoder", "encoder", "mask2former_fp32"])
def test_value_gradient_is_adjoint_of_forward(name):
    """<grad_value, V'> == <g, out(V')> for a random V' (out is linear in
    value); evaluated in float64 from the kernels' outputs."""
    value, shapes, starts, loc, attn = presets.make_preset_inputs(name, device=DEVICE)
    g = presets.make_grad_out(name, device=DEVICE)
    v = value.clone().requires_grad_(True)
    msda(v, shapes, starts, loc, attn, fp32_grad_accum=True).backward(g)
    vp = torch.randn(value.shape, generator=torch.Generator().manual_seed(3)).to(DEVICE, value.dtype)
    out_p = msda(vp, shapes, starts, loc, attn)
    lhs = (v.grad.double() * vp.double()).sum().item()
    rhs = (g.double() * out_p.double()).sum().item()
    scale = ((v.grad.double().abs() * vp.double().abs()).sum()
             + (g.double().abs() * out_p.double().abs()).sum()).item()
    tol = 1e-6 if value.dtype == torch.float32 else 4e-3
    assert abs(lhs - rhs) <= tol * scale, (lhs, rhs, scale)


@pytest.mark.parametrize("name", ["decoder", "encoder"])
def test_output_is_linear_in_attention(name):
    value, shapes, starts, loc, attn = presets.make_preset_inputs(name, device=DEVICE)
    a2 = attn.flip(-1).contiguous()
    o1 = msda(value, shapes, starts, loc, attn).double()
    o2 = msda(value, shapes, starts, loc, a2).double()
    o12 = msda(value, shapes, starts, loc, (attn.float() + a2.float()).to(attn.dtype)).double()
    err = ((o12 - o1 - o2).norm() / (o1 + o2).norm()).item()
    assert err <= (1e-6 if value.dtype == torch.float32 else 1e-2), err
