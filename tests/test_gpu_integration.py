"""GPU checks of the integration surfaces: the torch.library custom ops
(plain and fused front-end) under torch.compile(fullgraph=True), CUDA-graph
capture and replay of a full forward+backward (also of the deterministic
backward, bit for bit), the mmcv / Deformable-DETR call shim, and batches
whose value tensor exceeds 2^28 elements (split into slices by the library),
for the plain and the fused operator.

Every surface is checked against the CPU oracle on the same inputs, with the
reference's protocol and tolerances (tests/test_msda.py:43-55,80-93): a
wrong argument order inside a wrapper that the eager operator shares would
otherwise go unseen.
"""

import pytest
import torch

from msda_cases import (BWD_RELERR, BWD_TOL, FWD_RELERR, FWD_TOL, make_fused_inputs,
                        make_inputs, rel_err)
from msda_triton_amd import MultiScaleDeformableAttnFunction, msda_fused_op, msda_op
from msda_triton_amd import multi_scale_deformable_attention as msda
from msda_triton_amd.fused import multi_scale_deformable_attention_fused as msda_fused
from oracle import run_fused_reference, run_reference_fp32

pytestmark = pytest.mark.gpu
DEVICE = "cuda"
TWO_DTYPES = [torch.float32, torch.bfloat16]


def _case(dtype=torch.float32, **kw):
    args = dict(B=2, Q=40, M=4, D=32, shapes=[(12, 16), (6, 8)], K=4, dtype=dtype, device=DEVICE,
                loc_lo=-0.1, loc_hi=1.1)
    args.update(kw)
    return make_inputs(**args)


def _grad_out(shape, dtype):
    g = torch.randn(shape, generator=torch.Generator().manual_seed(5))
    return g.to(DEVICE, dtype)


def _fwd_bwd(fn, value, shapes, starts, loc, attn):
    v, lo, a = (t.clone().requires_grad_(True) for t in (value, loc, attn))
    out = fn(v, shapes, starts, lo, a)
    g = _grad_out(out.shape, out.dtype)
    out.backward(g)
    return [out.detach(), v.grad, lo.grad, a.grad], g


def check_oracle(got, value, shapes, loc, attn, g, dtype, out_scale=1.0):
    """got = [out, grad_value, grad_loc, grad_attn] against the fp32 CPU
    oracle (half inputs upcast, as the reference's tests do); `out_scale`
    multiplies the oracle's output (a wrapper that scales it)."""
    ref, refs = run_reference_fp32(value, shapes, loc, attn, g)
    if got[0] is not None:
        torch.testing.assert_close(got[0].float().cpu(), ref * out_scale, **FWD_TOL[dtype])
        assert rel_err(got[0], ref * out_scale) <= FWD_RELERR[dtype]
    for name, x, r in zip(("grad_value", "grad_loc", "grad_attn"), got[1:], refs):
        torch.testing.assert_close(x.float().cpu(), r, **BWD_TOL[dtype],
                                   msg=lambda m: f"{name}: {m}")
        e = rel_err(x, r)
        assert e <= BWD_RELERR[dtype], f"{name}: rel_err {e:.3e}"


@pytest.mark.parametrize("dtype", TWO_DTYPES, ids=str)
def test_custom_op_matches_oracle(dtype):
    """torch.ops.msda_amd via msda_op, eager: oracle parity, and the same
    results as the autograd Function."""
    args = _case(dtype)
    got, g = _fwd_bwd(msda_op, *args)
    value, shapes, _, loc, attn = args
    check_oracle(got, value, shapes, loc, attn, g, dtype)
    ref, _ = _fwd_bwd(msda, *args)
    for r, x in zip(ref, got):
        torch.testing.assert_close(x, r, rtol=0, atol=0)


@pytest.mark.parametrize("dtype", TWO_DTYPES, ids=str)
def test_custom_op_compiles_fullgraph(dtype):
    """torch.compile(fullgraph=True) of a layer around the custom op: its
    output and the three gradients against the oracle (grad_out of the sum
    of 2 * out is 2 everywhere)."""
    value, shapes, starts, loc, attn = _case(dtype)

    def layer(v, lo, a):
        return msda_op(v, shapes, starts, lo, a) * 2.0

    compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
    v, lo, a = (t.clone().requires_grad_(True) for t in (value, loc, attn))
    y = compiled(v, lo, a)
    g = _grad_out(y.shape, y.dtype)
    y.backward(g)
    # d(2 out)/d(.) . g = d(out)/d(.) . (2 g)
    check_oracle([y.detach(), v.grad, lo.grad, a.grad], value, shapes, loc, attn, 2 * g, dtype,
                 out_scale=2.0)


@pytest.mark.parametrize("dtype", TWO_DTYPES, ids=str)
def test_mmcv_shim_matches_oracle(dtype):
    """MultiScaleDeformableAttnFunction.apply(value, shapes, starts, loc,
    attn, im2col_step), the mmcv / Deformable-DETR call form."""
    args = _case(dtype)
    got, g = _fwd_bwd(
        lambda v, s, st, lo, a: MultiScaleDeformableAttnFunction.apply(v, s, st, lo, a, 64), *args)
    value, shapes, _, loc, attn = args
    check_oracle(got, value, shapes, loc, attn, g, dtype)


def test_cuda_graph_replays_forward_backward():
    """A captured fwd+bwd (library zero-fill is a kernel, not a memset)
    replays correctly several times, with eager work between the replays;
    every replay's output and gradients against the oracle."""
    dtype = torch.bfloat16
    value, shapes, starts, loc, attn = _case(dtype)
    v, lo, a = (t.clone().requires_grad_(True) for t in (value, loc, attn))
    g = _grad_out((2, 40, 128), dtype)
    msda(v, shapes, starts, lo, a, fp32_grad_accum=True).backward(g)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            v.grad = lo.grad = a.grad = None
            msda(v, shapes, starts, lo, a, fp32_grad_accum=True).backward(g)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    v.grad = lo.grad = a.grad = None
    with torch.cuda.graph(graph):
        out = msda(v, shapes, starts, lo, a, fp32_grad_accum=True)
        out.backward(g)
    eager = msda(value, shapes, starts, loc, attn)
    for _ in range(3):
        v.grad.fill_(7.0)  # stale contents: each replay must rewrite them
        lo.grad.fill_(7.0)
        a.grad.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(out.detach().float(), eager.float(), rtol=0, atol=0)
        check_oracle([out.detach(), v.grad, lo.grad, a.grad], value, shapes, loc, attn, g, dtype)
        _ = torch.randn(1000, device=DEVICE).sum().item()  # eager work between replays


def test_cuda_graph_deterministic_backward_is_bitwise_stable():
    """The deterministic backward (zero-fill, max, int64 scatter and cast are
    all kernels) captured in a graph gives the eager bits on every replay."""
    value, shapes, starts, loc, attn = _case(torch.bfloat16)
    g = torch.randn(2, 40, 128, generator=torch.Generator().manual_seed(6)).to(DEVICE, torch.bfloat16)

    def run():
        out = msda(v, shapes, starts, lo, a, deterministic=True)
        out.backward(g)
        return out

    v, lo, a = (t.clone().requires_grad_(True) for t in (value, loc, attn))
    run()
    eager = [t.grad.clone() for t in (v, lo, a)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            v.grad = lo.grad = a.grad = None
            run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    v.grad = lo.grad = a.grad = None
    with torch.cuda.graph(graph):
        run()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for r, x in zip(eager, (v.grad, lo.grad, a.grad)):
            assert torch.equal(x, r)
        _ = torch.randn(1000, device=DEVICE).sum().item()


def _fused_case(dtype=torch.float32):
    return make_fused_inputs(B=2, Q=40, M=4, D=32, K=4, shapes=[(12, 16), (6, 8)], dtype=dtype,
                             device=DEVICE, per_level=True)


def _fused_fwd_bwd(fn, value, shapes, starts, ref, off, logits):
    leaves = [t.clone().requires_grad_(True) for t in (value, ref, off, logits)]
    out = fn(leaves[0], shapes, starts, *leaves[1:])
    g = _grad_out(out.shape, out.dtype)
    out.backward(g)
    return [out.detach()] + [t.grad for t in leaves]


def test_fused_custom_op_matches_oracle_and_compiles():
    """The fused custom op, eager and under torch.compile(fullgraph=True),
    against the float64 oracle of the composition
    labs/solutions/lab00.py:201-208."""
    args = _fused_case()
    value, shapes, starts, ref, off, logits = args
    got = _fused_fwd_bwd(msda_fused_op, *args)
    g = _grad_out(got[0].shape, got[0].dtype)
    ref_out, ref_grads = run_fused_reference(value, shapes, ref, off, logits, g)
    for name, x, r in zip(("out", "grad_value", "grad_reference_points",
                           "grad_sampling_offsets", "grad_attention_logits"),
                          got, [ref_out] + list(ref_grads)):
        e = rel_err(x, r)
        tol = FWD_RELERR[torch.float32] if name == "out" else BWD_RELERR[torch.float32]
        assert e <= tol, f"{name}: rel_err {e:.3e}"
    want = _fused_fwd_bwd(msda_fused, *args)
    for r, x in zip(want, got):
        torch.testing.assert_close(x, r, rtol=0, atol=0)

    def layer(v, rp, o, lg):
        return msda_fused_op(v, shapes, starts, rp, o, lg) * 2.0

    compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
    leaves = [t.clone().requires_grad_(True) for t in (value, ref, off, logits)]
    y = compiled(*leaves)
    y.backward(g)
    ref_out2, ref_grads2 = run_fused_reference(value, shapes, ref, off, logits, 2 * g)
    assert rel_err(y.detach(), 2 * ref_out2) <= FWD_RELERR[torch.float32]
    for t, r in zip(leaves, ref_grads2):
        assert rel_err(t.grad, r) <= BWD_RELERR[torch.float32]


def test_batch_slicing_beyond_32bit_offsets():
    """3 batch elements of 2^27 + 64 value elements each: the library splits
    the batch into slices with 32-bit offsets.  Per-batch runs (one slice
    each) must give the same forward bits and the same gradients."""
    torch.manual_seed(0)
    B, M, D = 3, 1, 64
    h, w = 2048, 1025            # S*M*D = 134,348,800 > 2^27: two batches exceed 2^28
    S = h * w
    gen = torch.Generator(device=DEVICE).manual_seed(1)
    value = torch.randn(B, S, M, D, device=DEVICE, dtype=torch.bfloat16, generator=gen)
    Q, K = 16, 4
    loc = torch.rand(B, Q, M, 1, K, 2, device=DEVICE, generator=gen).to(torch.bfloat16)
    attn = torch.rand(B, Q, M, 1, K, device=DEVICE, generator=gen).to(torch.bfloat16)
    shapes = torch.tensor([[h, w]], device=DEVICE)
    out = msda(value, shapes, None, loc, attn)
    for b in range(B):
        ob = msda(value[b:b + 1], shapes, None, loc[b:b + 1], attn[b:b + 1])
        assert torch.equal(ob, out[b:b + 1])
    g = torch.randn(out.shape, device=DEVICE, generator=gen).to(torch.bfloat16)
    v = value.requires_grad_(True)
    msda(v, shapes, None, loc, attn, fp32_grad_accum=True).backward(g)
    for b in (0, B - 1):
        vb = value[b:b + 1].detach().clone().requires_grad_(True)
        msda(vb, shapes, None, loc[b:b + 1], attn[b:b + 1], fp32_grad_accum=True).backward(g[b:b + 1])
        torch.testing.assert_close(v.grad[b:b + 1].float(), vb.grad.float(), rtol=1e-2, atol=1e-2)


def test_fused_batch_slicing_beyond_32bit_offsets():
    """The fused path over the same 2^27-element batch elements: per-slice
    pointers of reference points, offsets, logits, log-sum-exp and output."""
    B, M, D, h, w, Q, K = 3, 1, 64, 2048, 1025, 16, 4
    S = h * w
    gen = torch.Generator(device=DEVICE).manual_seed(2)
    value = torch.randn(B, S, M, D, device=DEVICE, dtype=torch.bfloat16, generator=gen)
    ref = torch.rand(B, Q, 1, 2, device=DEVICE, generator=gen).to(torch.bfloat16)
    off = (4 * torch.randn(B, Q, M, 1, K, 2, device=DEVICE, generator=gen)).to(torch.bfloat16)
    logits = torch.randn(B, Q, M, 1, K, device=DEVICE, generator=gen).to(torch.bfloat16)
    shapes = torch.tensor([[h, w]], device=DEVICE)
    out = msda_fused(value, shapes, None, ref, off, logits)
    g = torch.randn(out.shape, device=DEVICE, generator=gen).to(torch.bfloat16)
    leaves = [t.clone().requires_grad_(True) for t in (ref, off, logits)]
    msda_fused(value, shapes, None, *leaves).backward(g)
    for b in range(B):
        ob = msda_fused(value[b:b + 1], shapes, None, ref[b:b + 1], off[b:b + 1], logits[b:b + 1])
        assert torch.equal(ob, out[b:b + 1])
        lb = [t[b:b + 1].clone().requires_grad_(True) for t in (ref, off, logits)]
        msda_fused(value[b:b + 1], shapes, None, *lb).backward(g[b:b + 1])
        for full, part in zip(leaves, lb):
            assert torch.equal(full.grad[b:b + 1], part.grad)
