"""CPU oracle for the projections either side of the operator -- TEST
INFRASTRUCTURE ONLY (imported by tests/ and bench.py's CPU leg, never by the
product path).

The reference's attention layer applies four ``nn.Linear`` projections
(labs/solutions/lab00.py:187-190 constructs them; :199-201 value / offset /
weight projections, :208 the output projection): ``y = x W^T + b``.
Deformable-DETR-style callers additionally zero padded value rows after the
value projection (``value.masked_fill(padding_mask[..., None], 0)``); the
reference layer has no padding mask, so the mask is this build's extension
and is restated here as that masked_fill.

Everything is float64 numpy.  Pinned by tests/test_oracle_projection.py
against torch.nn.functional.linear + masked_fill + autograd in float64 (an
independent library routine), closed forms (identity and zero weights, zero
input, masked rows) and planted mistakes (a transposed weight, a dropped bias,
a mask applied to the input instead of the output rows' gradient).
"""

from __future__ import annotations

import numpy as np


def _f64(a):
    return None if a is None else np.asarray(a, dtype=np.float64)


def projection_reference(x, w, b=None, mask=None, w2=None, b2=None):
    """``y = x w^T + b`` over the last axis, rows with ``mask`` set to zero.

    x (..., in), w (out, in), b (out,), mask (...) bool.  With ``w2`` the
    second projection of the same rows is returned too: ``(y, y2)``.
    """
    x = _f64(x)
    outs = []
    for wi, bi in ((w, b), (w2, b2)):
        if wi is None:
            continue
        y = x @ _f64(wi).T
        if bi is not None:
            y = y + _f64(bi)
        if mask is not None:
            y = np.where(np.asarray(mask, dtype=bool)[..., None], 0.0, y)
        outs.append(y)
    return outs[0] if len(outs) == 1 else tuple(outs)


def projection_backward_reference(x, w, gy, mask=None, w2=None, gy2=None):
    """Gradients of ``projection_reference`` for output gradients gy (, gy2).

    Returns ``(gx, gw, gb, gw2, gb2)`` (the last two None without w2): masked
    rows pass no gradient, so gy is zeroed there first; then gx = gy w (+ gy2
    w2), gw = gy^T x, gb = column sums of gy, summed over every leading axis.
    """
    x = _f64(x)
    keep = None if mask is None else ~np.asarray(mask, dtype=bool)[..., None]
    xin = x.reshape(-1, x.shape[-1])
    res = []
    gx = np.zeros_like(x)
    for wi, gi in ((w, gy), (w2, gy2)):
        if wi is None:
            res.extend([None, None])
            continue
        g = _f64(gi)
        if keep is not None:
            g = np.where(keep, g, 0.0)
        gx = gx + g @ _f64(wi)
        g2 = g.reshape(-1, g.shape[-1])
        res.extend([g2.T @ xin, g2.sum(axis=0)])
    return (gx, *res)
