"""Writes the golden fixtures in this folder (run from the repo root):

    python tests/golden/make_golden.py

Each fixture holds fp32 inputs (exactly representable, so a GPU fp32 run sees
the same numbers) and float64 expected outputs:
  out        from the pure-loop oracle  msda_naive          (tests/reference_impls.py:48-87)
  grad_*     from the hand-derived backward msda_backward_analytic
             (labs/solutions/lab07.py:12-104), float64
The known-answer fixture is the half-out-of-bounds check of
tests/test_labs.py:86-91 (expected 0.5 and 0.0 exactly).
The reference ships no golden files; these freeze the oracle's answers so a
regression in it, or a kernel, shows up against fixed data.
"""

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "tests")]

from msda_cases import make_inputs  # noqa: E402
from oracle import level_start_index_of, msda_backward_analytic, msda_naive  # noqa: E402

HERE = Path(__file__).resolve().parent

CASES = {
    "small_oob": dict(B=2, Q=5, M=2, D=4, shapes=[(5, 7), (3, 4)], K=3, loc_lo=-0.3, loc_hi=1.3),
    "single_level": dict(B=1, Q=7, M=1, D=3, shapes=[(4, 6)], K=1),
    "three_levels": dict(B=2, Q=3, M=3, D=8, shapes=[(2, 9), (1, 1), (5, 2)], K=4,
                         loc_lo=-1.0, loc_hi=2.0),
    "wide_head": dict(B=1, Q=6, M=2, D=64, shapes=[(6, 5), (3, 3)], K=2, loc_lo=-0.2,
                      loc_hi=1.2),
}


def make_case(name, kw, seed=0):
    value, shapes, _, loc, attn = make_inputs(**kw, dtype=torch.float32, device="cpu", seed=seed)
    if name == "small_oob":
        # also exercise exact knots: a third of the coordinates on {0, 1/2, 1}
        knots = torch.tensor([0.0, 0.5, 1.0])
        pick = torch.rand(loc.shape, generator=torch.Generator().manual_seed(9)) < 0.33
        idx = torch.randint(0, 3, loc.shape, generator=torch.Generator().manual_seed(10))
        loc = torch.where(pick, knots[idx], loc)
    B, Q, M, D = kw["B"], kw["Q"], kw["M"], kw["D"]
    g = torch.randn(B, Q, M * D, generator=torch.Generator().manual_seed(7))
    v64, l64, a64, g64 = (t.double() for t in (value, loc, attn, g))
    out = msda_naive(v64, shapes, l64, a64)
    gv, gl, ga = msda_backward_analytic(v64, shapes, level_start_index_of(shapes), l64, a64,
                                        g64, dtype=torch.float64)
    return dict(value=value.numpy(), spatial_shapes=shapes.numpy(), sampling_locations=loc.numpy(),
                attention_weights=attn.numpy(), grad_out=g.numpy(), out=out.numpy(),
                grad_value=gv.numpy(), grad_sampling_locations=gl.numpy(),
                grad_attention_weights=ga.numpy())


def make_kat():
    value = np.ones((1, 9, 1, 2), np.float32)
    shapes = np.array([[3, 3]], np.int64)
    attn = np.ones((1, 2, 1, 1, 1), np.float32)
    loc = np.array([[(-0.5 + 0.5) / 3, (1.0 + 0.5) / 3],
                    [(-1.0 + 0.5) / 3, (1.0 + 0.5) / 3]], np.float32).reshape(1, 2, 1, 1, 1, 2)
    out = np.array([[[0.5, 0.5], [0.0, 0.0]]], np.float64)
    return dict(value=value, spatial_shapes=shapes, sampling_locations=loc, attention_weights=attn,
                out=out)


def main():
    for name, kw in CASES.items():
        np.savez_compressed(HERE / f"{name}.npz", **make_case(name, kw))
    np.savez_compressed(HERE / "kat_half_out.npz", **make_kat())
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
