"""Pins the projection oracle (oracle/projection_reference.py) on the CPU:
against torch.nn.functional.linear + masked_fill + autograd in float64 (an
independent library routine; the reference layer's projections are
nn.Linear, labs/solutions/lab00.py:187-208), closed forms, and planted
mistakes that a plausible slip would make."""

import numpy as np
import pytest
import torch

from oracle import projection_backward_reference, projection_reference


def _case(seed, lead=(3, 7), cin=16, n1=12, n2=8, masked=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*lead, cin, generator=g, dtype=torch.float64)
    w = torch.randn(n1, cin, generator=g, dtype=torch.float64)
    b = torch.randn(n1, generator=g, dtype=torch.float64)
    w2 = torch.randn(n2, cin, generator=g, dtype=torch.float64) if n2 else None
    b2 = torch.randn(n2, generator=g, dtype=torch.float64) if n2 else None
    mask = (torch.rand(*lead, generator=g) < 0.3) if masked else None
    return x, w, b, w2, b2, mask


def _torch_layer(x, w, b, w2, b2, mask):
    outs = []
    for wi, bi in ((w, b), (w2, b2)):
        if wi is None:
            continue
        y = torch.nn.functional.linear(x, wi, bi)
        if mask is not None:
            y = y.masked_fill(mask[..., None], 0.0)
        outs.append(y)
    return outs


@pytest.mark.parametrize("seed,n2,masked", [(0, 8, True), (1, 0, True), (2, 8, False), (3, 0, False)])
def test_forward_matches_torch_linear(seed, n2, masked):
    x, w, b, w2, b2, mask = _case(seed, n2=n2, masked=masked)
    got = projection_reference(x.numpy(), w.numpy(), b.numpy(), None if mask is None else mask.numpy(),
                               None if w2 is None else w2.numpy(), None if b2 is None else b2.numpy())
    want = _torch_layer(x, w, b, w2, b2, mask)
    got = got if isinstance(got, tuple) else (got,)
    assert len(got) == len(want)
    for g_, w_ in zip(got, want):
        np.testing.assert_allclose(g_, w_.numpy(), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("seed,n2,masked", [(4, 8, True), (5, 0, True), (6, 8, False)])
def test_backward_matches_torch_autograd(seed, n2, masked):
    x, w, b, w2, b2, mask = _case(seed, n2=n2, masked=masked)
    params = [t.requires_grad_() for t in (x, w, b, w2, b2) if t is not None]
    outs = _torch_layer(x, w, b, w2, b2, mask)
    g = torch.Generator().manual_seed(seed + 100)
    gys = [torch.randn(o.shape, generator=g, dtype=torch.float64) for o in outs]
    grads = torch.autograd.grad(outs, params, gys)
    gx, gw, gb, gw2, gb2 = projection_backward_reference(
        x.detach().numpy(), w.detach().numpy(), gys[0].numpy(),
        None if mask is None else mask.numpy(), None if w2 is None else w2.detach().numpy(),
        gys[1].numpy() if n2 else None)
    mine = [gx, gw, gb] + ([gw2, gb2] if n2 else [])
    assert gw2 is None or n2
    for m_, t_ in zip(mine, grads):
        np.testing.assert_allclose(m_, t_.numpy(), rtol=1e-12, atol=1e-12)


def test_closed_forms():
    x, w, b, _, _, mask = _case(7, n1=16, n2=0)
    eye = np.eye(16)
    # identity weight: y = x + b on kept rows, 0 on masked rows
    y = projection_reference(x.numpy(), eye, b.numpy(), mask.numpy())
    want = np.where(mask.numpy()[..., None], 0.0, x.numpy() + b.numpy())
    np.testing.assert_array_equal(y, want)
    # zero input: y = b everywhere (no mask)
    y0 = projection_reference(np.zeros_like(x.numpy()), w.numpy(), b.numpy())
    np.testing.assert_array_equal(y0, np.broadcast_to(b.numpy(), y0.shape))
    # zero weight: gradients of x vanish, gw = gy^T x, gb = column sums
    gy = np.ones(x.shape[:-1] + (16,))
    gx, gw, gb, _, _ = projection_backward_reference(x.numpy(), np.zeros((16, 16)), gy)
    np.testing.assert_array_equal(gx, np.zeros_like(gx))
    np.testing.assert_allclose(gb, np.full(16, gy[..., 0].size))
    np.testing.assert_allclose(gw, np.broadcast_to(x.numpy().reshape(-1, 16).sum(0), (16, 16)))
    # every row masked: all gradients zero
    gx, gw, gb, _, _ = projection_backward_reference(x.numpy(), w.numpy(), gy,
                                                     np.ones(x.shape[:-1], bool))
    assert not gx.any() and not gw.any() and not gb.any()


def test_planted_mistakes_are_caught():
    x, w, b, _, _, mask = _case(8, cin=16, n1=16, n2=0)
    want = _torch_layer(x, w, b, None, None, mask)[0].numpy()
    ok = projection_reference(x.numpy(), w.numpy(), b.numpy(), mask.numpy())
    np.testing.assert_allclose(ok, want, rtol=1e-12, atol=1e-12)
    transposed = projection_reference(x.numpy(), w.numpy().T, b.numpy(), mask.numpy())
    no_bias = projection_reference(x.numpy(), w.numpy(), None, mask.numpy())
    for bad in (transposed, no_bias):
        assert np.abs(bad - want).max() > 1e-3
    # mask applied to the input instead of the output: masked rows would keep b
    bad_mask = projection_reference(np.where(mask.numpy()[..., None], 0, x.numpy()), w.numpy(),
                                    b.numpy())
    assert np.abs(bad_mask - want).max() > 1e-3
