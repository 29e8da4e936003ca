"""The allocation-free projection backward (C ABI
msda_projection_backward_noalloc): its workspace is the library's own device
array, so it must give msda_projection_backward's outputs bit for bit (same
kernels, fixed-order sums, no atomics) on two calls in a row -- the second
smaller, over the scratch contents the first left behind -- in every dtype;
shapes whose workspace exceeds the array are refused before any launch."""

import pytest
import torch

from msda_triton_amd import _native

pytestmark = pytest.mark.gpu
DEVICE = "cuda"
DCODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
SCRATCH_BYTES = 64 << 20


def _inputs(rows, cin, n1, n2, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cin, generator=g)
    w1 = torch.randn(n1, cin, generator=g) / cin ** 0.5
    w2 = torch.randn(n2, cin, generator=g) / cin ** 0.5 if n2 else None
    mask = (torch.rand(rows, generator=g) < 0.1).to(torch.uint8)
    gy1 = torch.randn(rows, n1, generator=g)
    gy2 = torch.randn(rows, n2, generator=g) if n2 else None
    cast = lambda t: None if t is None else t.to(DEVICE, dtype)  # noqa: E731
    return dict(rows=rows, cin=cin, n1=n1, n2=n2, dtype=dtype, x=cast(x), w1=cast(w1),
                w2=cast(w2), mask=mask.to(DEVICE), gy1=cast(gy1), gy2=cast(gy2))


def _call(lib, a, noalloc):
    """grad_input, grad_weight, grad_bias (and the second weight's) of one
    call; outputs start as NaN so that an unwritten element shows."""
    dtype, rows, cin, n1, n2 = a["dtype"], a["rows"], a["cin"], a["n1"], a["n2"]
    nan = lambda *s: torch.full(s, float("nan"), dtype=dtype, device=DEVICE)  # noqa: E731
    gx, gw1, gb1 = nan(rows, cin), nan(n1, cin), nan(n1)
    gw2, gb2 = (nan(n2, cin), nan(n2)) if n2 else (None, None)
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    st = torch.cuda.current_stream().cuda_stream
    args = (p(a["x"]), p(a["w1"]), p(a["w2"]), p(a["mask"]), p(a["gy1"]), p(a["gy2"]), p(gx),
            p(gw1), p(gb1), p(gw2), p(gb2))
    dims = (rows, cin, n1 + n2, n1, DCODE[dtype], st)
    if noalloc:
        rc = lib.msda_projection_backward_noalloc(*args, *dims)
    else:
        nbytes = lib.msda_projection_workspace_bytes(rows, cin, n1 + n2, DCODE[dtype])
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEVICE)
        rc = lib.msda_projection_backward(*args, p(ws), *dims)
    _native.check(rc, "projection backward")
    return [t for t in (gx, gw1, gb1, gw2, gb2) if t is not None]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=str)
def test_noalloc_projection_backward_matches_workspace_variant(dtype):
    lib = _native.load()
    print(f"no-alloc projection backward {dtype}", flush=True)
    # the decoder preset's value projection (88,892 rows), then the smaller
    # offset + logit projection of its 1,200 query rows
    big = _inputs(88892, 256, 256, 0, dtype, seed=1)
    small = _inputs(1200, 256, 256, 128, dtype, seed=2)
    for a in (big, small):
        need = lib.msda_projection_workspace_bytes(a["rows"], a["cin"], a["n1"] + a["n2"],
                                                   DCODE[dtype])
        assert 0 < need <= SCRATCH_BYTES
    got = [_call(lib, big, noalloc=True), _call(lib, small, noalloc=True)]
    torch.cuda.synchronize()
    want = [_call(lib, big, noalloc=False), _call(lib, small, noalloc=False)]
    torch.cuda.synchronize()
    for g_list, w_list in zip(got, want):
        assert len(g_list) == len(w_list)
        for g, w in zip(g_list, w_list):
            assert not torch.isnan(g).any()
            assert torch.equal(g, w)


def test_noalloc_projection_backward_refuses_beyond_its_scratch():
    """fp32 2048 x 2048: a workspace over 64 MiB -> MSDA_ERR_UNSUPPORTED_SHAPE,
    returned before any launch (outputs untouched)."""
    lib = _native.load()
    a = _inputs(10, 2048, 2048, 0, torch.float32, seed=3)
    assert lib.msda_projection_workspace_bytes(10, 2048, 2048, 0) > SCRATCH_BYTES
    gx = torch.full((10, 2048), 5.0, device=DEVICE)
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    rc = lib.msda_projection_backward_noalloc(
        p(a["x"]), p(a["w1"]), None, p(a["mask"]), p(a["gy1"]), None, p(gx), None, None, None,
        None, 10, 2048, 2048, 2048, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == 3
    torch.cuda.synchronize()
    assert bool((gx == 5.0).all())
