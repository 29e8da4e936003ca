"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py): the CPU oracle must reproduce them, and the HIP
kernels must match them (fp32 inputs, float64 expected values)."""

from pathlib import Path

import numpy as np
import pytest
import torch

from msda_cases import BWD_TOL, FWD_TOL
from oracle import level_start_index_of, msda_backward_analytic, msda_naive, msda_reference

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = ["small_oob", "single_level", "three_levels", "wide_head"]


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: torch.from_numpy(z[k]) for k in z.files}


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_golden(name):
    f = load(name)
    v, sh, lo, a, g = (f[k] for k in ("value", "spatial_shapes", "sampling_locations",
                                      "attention_weights", "grad_out"))
    v64, l64, a64, g64 = (t.double() for t in (v, lo, a, g))
    torch.testing.assert_close(msda_naive(v64, sh, l64, a64), f["out"], rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(msda_reference(v64, sh, l64, a64), f["out"], rtol=1e-10, atol=1e-12)
    gv, gl, ga = msda_backward_analytic(v64, sh, level_start_index_of(sh), l64, a64, g64,
                                        dtype=torch.float64)
    torch.testing.assert_close(gv, f["grad_value"], rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(gl, f["grad_sampling_locations"], rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(ga, f["grad_attention_weights"], rtol=1e-12, atol=1e-12)


def test_oracle_reproduces_half_out_kat():
    f = load("kat_half_out")
    out = msda_reference(f["value"].double(), f["spatial_shapes"], f["sampling_locations"].double(),
                         f["attention_weights"].double())
    torch.testing.assert_close(out, f["out"], rtol=0, atol=1e-7)


@pytest.mark.gpu
@pytest.mark.parametrize("fp32_grad_accum", [False, True])
@pytest.mark.parametrize("name", CASES)
def test_kernels_match_golden(name, fp32_grad_accum):
    from msda_triton_amd import multi_scale_deformable_attention as msda

    f = load(name)
    dev = "cuda"
    v, lo, a = (f[k].to(dev).requires_grad_(True)
                for k in ("value", "sampling_locations", "attention_weights"))
    out = msda(v, f["spatial_shapes"].to(dev), None, lo, a, fp32_grad_accum=fp32_grad_accum)
    out.backward(f["grad_out"].to(dev))
    torch.testing.assert_close(out.detach().cpu().double(), f["out"], **FWD_TOL[torch.float32])
    for got, key in ((v.grad, "grad_value"), (lo.grad, "grad_sampling_locations"),
                     (a.grad, "grad_attention_weights")):
        torch.testing.assert_close(got.cpu().double(), f[key], **BWD_TOL[torch.float32])


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_kernels_match_half_out_kat(dtype):
    from msda_triton_amd import multi_scale_deformable_attention as msda

    f = load("kat_half_out")
    out = msda(f["value"].to("cuda", dtype), f["spatial_shapes"].to("cuda"), None,
               f["sampling_locations"].to("cuda", dtype), f["attention_weights"].to("cuda", dtype))
    # 0.5 and 0 are exact in every dtype; the locations (1/6, 1/2, -1/6)
    # round in half precision, which moves the half-out sample by < 1e-2.
    tol = 0 if dtype == torch.float32 else 1e-2
    torch.testing.assert_close(out.cpu().double().view(1, 2, 2), f["out"], rtol=0, atol=tol + 1e-7)
