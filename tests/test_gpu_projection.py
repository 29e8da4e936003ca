"""GPU parity of the projections either side of the operator (C ABI
msda_projection_forward / msda_projection_backward, the layer's nn.Linear
calls of labs/solutions/lab00.py:199-208 plus padded-row masking) against the
float64 CPU oracle (oracle/projection_reference.py) on the same rounded
inputs, and, at the decoder preset's full value size, against torch's fp32
linear on the GPU.

Tolerances (norm-relative): forward 1e-5 (fp32) / 1e-2 (half), gradients
1e-4 / 2e-2 -- the operator's bars.  Masked rows must be exactly zero, and
every gradient bitwise reproducible (no atomics anywhere on this path).
"""

import numpy as np
import pytest
import torch

from msda_cases import BWD_RELERR, DTYPES, FWD_RELERR, rel_err
from msda_triton_amd import _native
from msda_triton_amd.projection import projection
from oracle import projection_backward_reference, projection_reference

pytestmark = pytest.mark.gpu
DEVICE = "cuda"

# (leading shape, in_features, out_features of weight, of weight2 or 0)
CASES = [
    dict(id="one_row", lead=(1,), cin=256, n1=256, n2=0),
    dict(id="ragged_rows", lead=(2, 33), cin=256, n1=256, n2=0),
    dict(id="decoder_query", lead=(4, 300), cin=256, n1=256, n2=128),
    dict(id="m2f_query", lead=(2, 517), cin=256, n1=192, n2=96),
    dict(id="narrow", lead=(3, 100), cin=64, n1=32, n2=0),
    dict(id="tiny_split", lead=(5, 61), cin=32, n1=48, n2=16),
    dict(id="odd_cols", lead=(7, 19), cin=24, n1=40, n2=0),
    dict(id="wide_in", lead=(1, 1000), cin=512, n1=256, n2=0),
    dict(id="wide_out", lead=(2, 77), cin=128, n1=512, n2=0),
]


def make(case, dtype, seed=0, masked=True):
    g = torch.Generator().manual_seed(seed)
    lead, cin, n1, n2 = case["lead"], case["cin"], case["n1"], case["n2"]
    x = torch.randn(*lead, cin, generator=g)
    w = torch.randn(n1, cin, generator=g) / cin ** 0.5
    b = torch.randn(n1, generator=g)
    w2 = torch.randn(n2, cin, generator=g) / cin ** 0.5 if n2 else None
    b2 = torch.randn(n2, generator=g) if n2 else None
    mask = (torch.rand(*lead, generator=g) < 0.25) if masked else None
    cast = lambda t: None if t is None else t.to(DEVICE, dtype)  # noqa: E731
    return cast(x), cast(w), cast(b), cast(w2), cast(b2), (None if mask is None else mask.to(DEVICE))


def np64(t):
    return None if t is None else t.detach().double().cpu().numpy()


def run(x, w, b, w2, b2, mask, seed=7):
    leaves = [t.clone().requires_grad_(True) if t is not None else None for t in (x, w, b, w2, b2)]
    out = projection(leaves[0], leaves[1], leaves[2], row_mask=mask, weight2=leaves[3],
                     bias2=leaves[4])
    outs = out if isinstance(out, tuple) else (out,)
    g = torch.Generator().manual_seed(seed)
    gys = [torch.randn(o.shape, generator=g).to(DEVICE, o.dtype) for o in outs]
    torch.autograd.backward(outs, gys)
    return [o.detach() for o in outs], gys, [None if t is None else t.grad for t in leaves]


@pytest.mark.parametrize("masked", [True, False], ids=["mask", "nomask"])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("case", CASES, ids=lambda c: c["id"])
def test_projection_matches_oracle(case, dtype, masked):
    if dtype != torch.float32 and case["cin"] > 512:
        pytest.skip("half precision takes reductions up to 512")
    x, w, b, w2, b2, mask = make(case, dtype, masked=masked)
    outs, gys, grads = run(x, w, b, w2, b2, mask)
    m = np64(mask)
    ref = projection_reference(np64(x), np64(w), np64(b), None if m is None else m.astype(bool),
                               np64(w2), np64(b2))
    ref = ref if isinstance(ref, tuple) else (ref,)
    for o, r in zip(outs, ref):
        e = rel_err(o, torch.from_numpy(r))
        assert e <= FWD_RELERR[dtype], f"forward rel_err {e:.3e}"
        if mask is not None:
            assert not o[mask].any(), "masked rows must be exactly zero"
    rg = projection_backward_reference(np64(x), np64(w), np64(gys[0]),
                                       None if m is None else m.astype(bool), np64(w2),
                                       np64(gys[1]) if len(gys) > 1 else None)
    names = ("grad_input", "grad_weight", "grad_bias", "grad_weight2", "grad_bias2")
    for name, got, want in zip(names, grads, rg):
        if want is None:
            assert got is None, name
            continue
        e = rel_err(got, torch.from_numpy(want))
        assert e <= BWD_RELERR[dtype], f"{name}: rel_err {e:.3e}"
    if mask is not None:
        assert not grads[0][mask].any(), "masked rows get zero input gradient"


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_projection_backward_is_bitwise_reproducible(dtype):
    case = CASES[2]
    x, w, b, w2, b2, mask = make(case, dtype, seed=3)
    _, _, g1 = run(x, w, b, w2, b2, mask)
    _, _, g2 = run(x, w, b, w2, b2, mask)
    for a, c in zip(g1, g2):
        assert torch.equal(a, c)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_projection_empty_rows(dtype):
    x = torch.empty(0, 5, 64, device=DEVICE, dtype=dtype, requires_grad=True)
    w = torch.randn(32, 64, device=DEVICE, dtype=dtype, requires_grad=True)
    b = torch.randn(32, device=DEVICE, dtype=dtype, requires_grad=True)
    y = projection(x, w, b)
    assert y.shape == (0, 5, 32)
    y.sum().backward()
    assert x.grad.shape == x.shape
    assert not w.grad.any() and not b.grad.any()


def test_projection_without_bias_and_partial_grads():
    x, w, _, w2, _, mask = make(CASES[2], torch.bfloat16, seed=4)
    w.requires_grad_(True)
    y, y2 = projection(x, w, None, row_mask=mask, weight2=w2)  # only w needs a gradient
    gy = torch.randn_like(y)
    (y * gy).sum().backward()
    ref = projection_backward_reference(np64(x), np64(w), np64(gy), np64(mask).astype(bool),
                                        np64(w2), np.zeros(tuple(y2.shape)))
    assert rel_err(w.grad, torch.from_numpy(ref[1])) <= BWD_RELERR[torch.bfloat16]
    r1, r2 = projection_reference(np64(x), np64(w), None, np64(mask).astype(bool), np64(w2))
    assert rel_err(y, torch.from_numpy(r1)) <= 1e-2 and rel_err(y2, torch.from_numpy(r2)) <= 1e-2


def test_projection_rejects_unsupported_shapes():
    x = torch.randn(4, 20, device=DEVICE, dtype=torch.bfloat16)  # 40 bytes per row
    w = torch.randn(8, 20, device=DEVICE, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="unsupported shape"):
        projection(x, w)
    x = torch.randn(4, 520, device=DEVICE, dtype=torch.float16)
    w = torch.randn(8, 520, device=DEVICE, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="unsupported shape"):
        projection(x, w)


def test_value_projection_at_decoder_size():
    """Decoder preset's value rows (B=4, S=22223, C=256, bf16) with a padding
    mask, against torch's fp32 linear on the GPU (same rounded inputs)."""
    g = torch.Generator().manual_seed(11)
    B, S, C = 4, 22223, 256
    x = torch.randn(B, S, C, generator=g).to(DEVICE, torch.bfloat16)
    w = (torch.randn(C, C, generator=g) / 16).to(DEVICE, torch.bfloat16)
    b = torch.randn(C, generator=g).to(DEVICE, torch.bfloat16)
    mask = torch.zeros(B, S, dtype=torch.bool)
    mask[1, 20000:] = True  # a padded image: the tail of batch 1
    mask[3, ::7] = True
    mask = mask.to(DEVICE)
    outs, gys, grads = run(x, w, b, None, None, mask)
    xf, wf, bf = x.float().requires_grad_(), w.float().requires_grad_(), b.float().requires_grad_()
    ref = torch.nn.functional.linear(xf, wf, bf).masked_fill(mask[..., None], 0)
    ref.backward(gys[0].float())
    assert rel_err(outs[0], ref) <= 1e-2
    assert not outs[0][mask].any()
    for name, got, want in (("input", grads[0], xf.grad), ("weight", grads[1], wf.grad),
                            ("bias", grads[2], bf.grad)):
        e = rel_err(got, want)
        assert e <= 2e-2, f"{name}: rel_err {e:.3e}"


def test_workspace_size_is_positive_and_bounded():
    lib = _native.load()
    n = lib.msda_projection_workspace_bytes(88892, 256, 256, 2)
    # the transposed weight + at most ~one fp32 partial (dW, db) per CU
    assert 256 * 256 * 2 < n <= 256 * 256 * 2 + 2 * 256 * (256 * 256 + 256) * 4


def _c_backward(lib, x, w, w2, mask, gy, gy2, stream):
    """One msda_projection_backward call through the C ABI (every gradient
    asked for, so the weight half runs on the library's second stream);
    returns the gradients and the buffers the call used."""
    rows, cin = x.shape
    n1, n2 = w.shape[0], (w2.shape[0] if w2 is not None else 0)
    dcode = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[x.dtype]
    lib_ws = lib.msda_projection_workspace_bytes(rows, cin, n1 + n2, dcode)
    outs = dict(gx=torch.empty_like(x), gw=torch.empty_like(w), gb=torch.empty(n1, **_like(x)),
                gw2=torch.empty_like(w2) if n2 else None,
                gb2=torch.empty(n2, **_like(x)) if n2 else None,
                ws=torch.empty(lib_ws, dtype=torch.uint8, device=DEVICE))
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731

    def call():
        _native.check(lib.msda_projection_backward(
            p(x), p(w), p(w2), p(mask), p(gy), p(gy2), p(outs["gx"]), p(outs["gw"]),
            p(outs["gb"]), p(outs["gw2"]), p(outs["gb2"]), p(outs["ws"]), rows, cin, n1 + n2, n1,
            dcode, stream.cuda_stream), "projection backward")
    return outs, call


def _like(t):
    return dict(dtype=t.dtype, device=t.device)


@pytest.mark.parametrize("case", [CASES[2], CASES[7]], ids=lambda c: c["id"])
def test_projection_backward_second_stream_graph_replays(case):
    """The weight / bias half of the backward runs on a second stream forked
    from and joined into the caller's: on a non-default caller stream the
    gradients match the oracle, and a captured HIP graph of the call,
    replayed three times with eager work in between (outputs overwritten
    with NaN, the inputs' neighbours touched), reproduces the eager call's
    outputs bit for bit each time."""
    lib = _native.load()
    x, w, b, w2, b2, mask = make(case, torch.bfloat16, seed=9)
    x = x.reshape(-1, x.shape[-1])
    mask = mask.reshape(-1).to(torch.uint8)
    g = torch.Generator().manual_seed(12)
    gy = torch.randn(x.shape[0], w.shape[0], generator=g).to(DEVICE, x.dtype)
    gy2 = torch.randn(x.shape[0], w2.shape[0], generator=g).to(DEVICE, x.dtype) if w2 is not None else None
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        outs, call = _c_backward(lib, x, w, w2, mask, gy, gy2, side)
        call()
    side.synchronize()
    eager = {k: v.clone() for k, v in outs.items() if v is not None and k != "ws"}
    ref = projection_backward_reference(np64(x), np64(w), np64(gy), np64(mask).astype(bool),
                                        np64(w2), np64(gy2) if gy2 is not None else None)
    assert rel_err(eager["gx"], torch.from_numpy(ref[0])) <= BWD_RELERR[torch.bfloat16]
    assert rel_err(eager["gw"], torch.from_numpy(ref[1])) <= BWD_RELERR[torch.bfloat16]
    assert rel_err(eager["gb"], torch.from_numpy(ref[2])) <= BWD_RELERR[torch.bfloat16]

    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        outs_g, call_g = _c_backward(lib, x, w, w2, mask, gy, gy2, cap)
    cap.synchronize()
    with torch.cuda.graph(graph, stream=cap):
        call_g()
    for rep in range(3):
        for k, v in outs_g.items():
            if v is not None and k != "ws":
                v.fill_(float("nan"))
        (x.float().sum() + gy.float().sum()).item()  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        for k, v in eager.items():
            assert torch.equal(outs_g[k], v), f"replay {rep}: {k} differs from the eager call"


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_projection_weight_paths_agree_bitwise(dtype):
    """Launches with at most two 32-row blocks per workgroup load the weights
    straight into registers, larger ones through LDS; both feed the same MFMA
    operands, and each output row depends on its input row alone.  So the
    first 1,200 rows of a 30,000-row call (LDS path) equal a 1,200-row call
    on those rows (direct path) bit for bit, with the weight split in two and
    masked rows."""
    g = torch.Generator().manual_seed(21)
    x = torch.randn(30000, 256, generator=g).to(DEVICE, dtype)
    w = (torch.randn(256, 256, generator=g) / 16).to(DEVICE, dtype)
    b = torch.randn(256, generator=g).to(DEVICE, dtype)
    w2 = (torch.randn(128, 256, generator=g) / 16).to(DEVICE, dtype)
    b2 = torch.randn(128, generator=g).to(DEVICE, dtype)
    mask = (torch.rand(30000, generator=g) < 0.1).to(DEVICE)
    big = projection(x, w, b, row_mask=mask, weight2=w2, bias2=b2)
    small = projection(x[:1200], w, b, row_mask=mask[:1200], weight2=w2, bias2=b2)
    for yb, ys in zip(big, small):
        assert torch.equal(yb[:1200], ys)
    ref = projection_reference(np64(x[:1200]), np64(w), np64(b), np64(mask[:1200]).astype(bool),
                               np64(w2), np64(b2))
    for ys, r in zip(small, ref):
        assert rel_err(ys, torch.from_numpy(r)) <= FWD_RELERR[dtype]


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_projection_split_input_paths_agree_bitwise(dtype):
    """grad_input of a split call reads its reduction from two tensors
    (grad_output and grad_output2), picked per 16-byte piece.  Row r of it
    depends on row r of those alone, so the first 1,200 rows of a 30,000-row
    backward (weights through LDS) equal a 1,200-row backward on those rows
    (weights straight into registers) bit for bit, and the small call meets
    the oracle; masked rows get zeros."""
    g = torch.Generator().manual_seed(22)
    x = torch.randn(30000, 256, generator=g).to(DEVICE, dtype)
    w = (torch.randn(256, 256, generator=g) / 16).to(DEVICE, dtype)
    b = torch.randn(256, generator=g).to(DEVICE, dtype)
    w2 = (torch.randn(128, 256, generator=g) / 16).to(DEVICE, dtype)
    b2 = torch.randn(128, generator=g).to(DEVICE, dtype)
    mask = (torch.rand(30000, generator=g) < 0.1).to(DEVICE)
    gy = torch.randn(30000, 256, generator=g).to(DEVICE, dtype)
    gy2 = torch.randn(30000, 128, generator=g).to(DEVICE, dtype)

    def grad_input(n):
        xi = x[:n].clone().requires_grad_(True)
        outs = projection(xi, w, b, row_mask=mask[:n], weight2=w2, bias2=b2)
        torch.autograd.backward(outs, [gy[:n], gy2[:n]])
        return xi.grad

    big, small = grad_input(30000), grad_input(1200)
    assert torch.equal(big[:1200], small)
    assert not big[mask].any(), "masked rows get zero input gradient"
    ref = projection_backward_reference(np64(x[:1200]), np64(w), np64(gy[:1200]),
                                        np64(mask[:1200]).astype(bool), np64(w2),
                                        np64(gy2[:1200]))
    assert rel_err(small, torch.from_numpy(ref[0])) <= BWD_RELERR[dtype]
