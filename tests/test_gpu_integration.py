"""GPU checks of the integration surfaces: the torch.library custom ops
(plain and fused front-end) under torch.compile(fullgraph=True), CUDA-graph
capture and replay of a full forward+backward (also of the deterministic
backward, bit for bit), the mmcv / Deformable-DETR call shim, and batches
whose value tensor exceeds 2^28 elements (split into slices by the library),
for the plain and the fused operator."""

import pytest
import torch

from msda_cases import make_fused_inputs, make_inputs
from msda_triton_amd import MultiScaleDeformableAttnFunction, msda_fused_op, msda_op
from msda_triton_amd import multi_scale_deformable_attention as msda
from msda_triton_amd.fused import multi_scale_deformable_attention_fused as msda_fused

pytestmark = pytest.mark.gpu
DEVICE = "cuda"


def _case(dtype=torch.float32, **kw):
    args = dict(B=2, Q=40, M=4, D=32, shapes=[(12, 16), (6, 8)], K=4, dtype=dtype, device=DEVICE,
                loc_lo=-0.1, loc_hi=1.1)
    args.update(kw)
    return make_inputs(**args)


def _fwd_bwd(fn, value, shapes, starts, loc, attn):
    v, lo, a = (t.clone().requires_grad_(True) for t in (value, loc, attn))
    out = fn(v, shapes, starts, lo, a)
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(5)).to(out.device, out.dtype)
    out.backward(g)
    return [out.detach(), v.grad, lo.grad, a.grad]


def test_custom_op_matches_autograd_function():
    args = _case()
    ref = _fwd_bwd(msda, *args)
    got = _fwd_bwd(msda_op, *args)
    for r, x in zip(ref, got):
        torch.testing.assert_close(x, r, rtol=1e-5, atol=1e-5)


def test_custom_op_compiles_fullgraph():
    args = _case()
    value, shapes, starts, loc, attn = args

    def layer(v, lo, a):
        return (msda_op(v, shapes, starts, lo, a) * 2.0).sum()

    compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
    grads = []
    for fn in (layer, compiled):
        v, lo, a = (t.clone().requires_grad_(True) for t in (value, loc, attn))
        y = fn(v, lo, a)
        y.backward()
        grads.append([y.detach(), v.grad, lo.grad, a.grad])
    for r, x in zip(*grads):
        torch.testing.assert_close(x, r, rtol=1e-5, atol=1e-5)


def test_mmcv_shim_matches_operator():
    args = _case(torch.bfloat16)
    ref = _fwd_bwd(msda, *args)
    got = _fwd_bwd(lambda v, s, st, lo, a: MultiScaleDeformableAttnFunction.apply(v, s, st, lo, a, 64),
                   *args)
    for r, x in zip(ref, got):
        torch.testing.assert_close(x.float(), r.float(), rtol=2e-2, atol=2e-2)


def test_cuda_graph_replays_forward_backward():
    """A captured fwd+bwd (library zero-fill is a kernel, not a memset)
    replays correctly several times, with eager work between the replays."""
    value, shapes, starts, loc, attn = _case(torch.bfloat16)
    v, lo, a = (t.clone().requires_grad_(True) for t in (value, loc, attn))
    g = torch.randn(2, 40, 128, generator=torch.Generator().manual_seed(6)).to(DEVICE, torch.bfloat16)
    msda(v, shapes, starts, lo, a, fp32_grad_accum=True).backward(g)
    eager = [None, v.grad.clone(), lo.grad.clone(), a.grad.clone()]

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
    ref = msda(value, shapes, starts, loc, attn)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(out.detach().float(), ref.float(), rtol=0, atol=0)
        # v.grad, lo.grad, a.grad are the graph's own buffers, rewritten by each
        # replay; grad_value may differ from eager in the last bit (atomic order)
        for r, x in zip(eager[1:], (v.grad, lo.grad, a.grad)):
            torch.testing.assert_close(x.float(), r.float(), rtol=1e-2, atol=1e-2)
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
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(5)).to(out.device, out.dtype)
    out.backward(g)
    return [out.detach()] + [t.grad for t in leaves]


def test_fused_custom_op_matches_function_and_compiles():
    args = _fused_case()
    value, shapes, starts, ref, off, logits = args
    want = _fused_fwd_bwd(msda_fused, *args)
    got = _fused_fwd_bwd(msda_fused_op, *args)
    for r, x in zip(want, got):
        torch.testing.assert_close(x, r, rtol=1e-5, atol=1e-5)

    def layer(v, rp, o, lg):
        return (msda_fused_op(v, shapes, starts, rp, o, lg) * 2.0).sum()

    compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
    res = []
    for fn in (layer, compiled):
        leaves = [t.clone().requires_grad_(True) for t in (value, ref, off, logits)]
        y = fn(*leaves)
        y.backward()
        res.append([y.detach()] + [t.grad for t in leaves])
    for r, x in zip(*res):
        torch.testing.assert_close(x, r, rtol=1e-5, atol=1e-5)


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
