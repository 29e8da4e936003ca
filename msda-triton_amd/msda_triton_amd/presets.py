"""Benchmark presets and their seeded synthetic inputs.

The configurations are the operator's benchmark workloads (decoder and
encoder presets as in the reference's benchmarks/modal_benchmark.py:73-98,
the decoder also in fp16 and fp32, plus a tiny CPU-checkable case, a
high-contention backward case and a Mask2Former-style pixel decoder).  Inputs are drawn on the CPU with a seeded
``torch.Generator`` in fp32 -- value, then locations, then attention logits
(then grad_out, from its own seed) -- rounded to the preset dtype and only
then moved to the device, so the GPU kernels and any CPU check see identical
bits.
"""

from __future__ import annotations

import torch


def pyramid(height: int, width: int, levels: int = 4, stride0: int = 8):
    """Feature-pyramid (H, W) at strides 8, 16, 32, ... (ceil division), as
    the reference's benchmark builds them (benchmarks/modal_benchmark.py:76-82)."""
    return [((height + (stride0 << i) - 1) // (stride0 << i),
             (width + (stride0 << i) - 1) // (stride0 << i)) for i in range(levels)]


PRESETS = {
    # Tiny fp32 forward+backward, checkable on the CPU oracle.
    "tiny": dict(B=1, Q=100, M=8, D=32, K=4, shapes=[(32, 32), (16, 16), (8, 8), (4, 4)],
                 dtype=torch.float32, loc="uniform"),
    # Deformable-DETR decoder cross-attention on an 800x1333 image (headline).
    "decoder": dict(B=4, Q=300, M=8, D=32, K=4, shapes=pyramid(800, 1333),
                    dtype=torch.bfloat16, loc="uniform"),
    # The headline decoder in the reference's other two dtypes (its README
    # tables all three, README.md:121-124).
    "decoder_fp16": dict(B=4, Q=300, M=8, D=32, K=4, shapes=pyramid(800, 1333),
                         dtype=torch.float16, loc="uniform"),
    "decoder_fp32": dict(B=4, Q=300, M=8, D=32, K=4, shapes=pyramid(800, 1333),
                         dtype=torch.float32, loc="uniform"),
    # Encoder self-attention: one query per feature pixel.
    "encoder": dict(B=2, Q=None, M=8, D=32, K=4, shapes=pyramid(800, 1333),
                    dtype=torch.float16, loc="refpoint", sigma=0.02, clamp=(-0.1, 1.1)),
    # Decoder shapes, every sample near the image centre.
    "high_contention": dict(B=4, Q=300, M=8, D=32, K=4, shapes=pyramid(800, 1333),
                            dtype=torch.bfloat16, loc="normal", mean=0.5, sigma=0.005),
    # Mask2Former pixel decoder on a 1024x1024 image, 3 levels.
    "mask2former_fp32": dict(B=2, Q=None, M=8, D=32, K=4, shapes=pyramid(1024, 1024, 3),
                             dtype=torch.float32, loc="refpoint", sigma=0.05, clamp=None),
    "mask2former_bf16": dict(B=2, Q=None, M=8, D=32, K=4, shapes=pyramid(1024, 1024, 3),
                             dtype=torch.bfloat16, loc="refpoint", sigma=0.05, clamp=None),
}


def preset_dims(name: str) -> dict:
    cfg = dict(PRESETS[name])
    S = sum(h * w for h, w in cfg["shapes"])
    if cfg["Q"] is None:
        cfg["Q"] = S
    cfg["S"] = S
    cfg["L"] = len(cfg["shapes"])
    return cfg


def reference_points(shapes) -> torch.Tensor:
    """(S, 2) normalised pixel centres ((j + 0.5) / W, (i + 0.5) / H) of every
    pixel of every level, level by level, row-major: the reference point of
    the query that sits on that pixel."""
    pts = []
    for h, w in shapes:
        ys, xs = torch.meshgrid(torch.arange(h, dtype=torch.float32),
                                torch.arange(w, dtype=torch.float32), indexing="ij")
        pts.append(torch.stack([(xs.reshape(-1) + 0.5) / w, (ys.reshape(-1) + 0.5) / h], -1))
    return torch.cat(pts, 0)


def make_preset_inputs(name: str, device="cpu", seed: int = 0):
    """Seeded inputs of a preset: (value, spatial_shapes, level_start_index,
    sampling_locations, attention_weights)."""
    c = preset_dims(name)
    B, Q, M, D, K, L, S = c["B"], c["Q"], c["M"], c["D"], c["K"], c["L"], c["S"]
    dtype = c["dtype"]
    gen = torch.Generator().manual_seed(seed)
    value = torch.randn(B, S, M, D, generator=gen)
    if c["loc"] == "uniform":
        loc = torch.rand(B, Q, M, L, K, 2, generator=gen)
    elif c["loc"] == "normal":
        loc = c["mean"] + c["sigma"] * torch.randn(B, Q, M, L, K, 2, generator=gen)
    else:  # reference point of the query's own pixel + Gaussian offsets
        ref = reference_points(c["shapes"])[:Q]
        loc = ref[None, :, None, None, None, :] + c["sigma"] * torch.randn(
            B, Q, M, L, K, 2, generator=gen)
        if c.get("clamp"):
            loc = loc.clamp(*c["clamp"])
    logits = torch.randn(B, Q, M, L * K, generator=gen)
    attn = logits.softmax(-1).view(B, Q, M, L, K)
    shapes = torch.tensor(c["shapes"], dtype=torch.int64)
    hw = shapes.prod(-1)
    starts = torch.cat([hw.new_zeros(1), hw.cumsum(0)[:-1]])
    return (value.to(dtype).to(device), shapes.to(device), starts.to(device),
            loc.to(dtype).to(device), attn.to(dtype).to(device))


def make_fused_preset_inputs(name: str, device="cpu", seed: int = 0, offset_sigma: float = 2.0):
    """Inputs of the fused front-end on a preset's shapes: (value,
    spatial_shapes, level_start_index, reference_points (B, Q, L, 2) ~ U[0, 1),
    sampling_offsets ~ N(0, offset_sigma) level pixels, attention_logits
    (B, Q, M, L, K) ~ N(0, 1)); the value tensor is the preset's own draw."""
    c = preset_dims(name)
    B, Q, M, D, K, L, S = c["B"], c["Q"], c["M"], c["D"], c["K"], c["L"], c["S"]
    dtype = c["dtype"]
    gen = torch.Generator().manual_seed(seed)
    value = torch.randn(B, S, M, D, generator=gen)
    ref = torch.rand(B, Q, L, 2, generator=gen)
    off = offset_sigma * torch.randn(B, Q, M, L, K, 2, generator=gen)
    logits = torch.randn(B, Q, M, L, K, generator=gen)
    shapes = torch.tensor(c["shapes"], dtype=torch.int64)
    hw = shapes.prod(-1)
    starts = torch.cat([hw.new_zeros(1), hw.cumsum(0)[:-1]])
    cast = lambda t: t.to(dtype).to(device)  # noqa: E731
    return (cast(value), shapes.to(device), starts.to(device), cast(ref), cast(off),
            cast(logits))


def make_grad_out(name: str, device="cpu", seed: int = 7) -> torch.Tensor:
    """Seeded N(0, 1) upstream gradient (B, Q, M*D) in the preset dtype."""
    c = preset_dims(name)
    gen = torch.Generator().manual_seed(seed)
    g = torch.randn(c["B"], c["Q"], c["M"] * c["D"], generator=gen)
    return g.to(c["dtype"]).to(device)


def algorithmic_bytes(name: str) -> tuple[int, int]:
    """(forward, backward) algorithmic bytes per call, by the reference's own
    accounting (labs/03_the_machine.py:232-251): every sample reads 4 corner
    rows of D elements and 3 parameters; every (b, q, m) writes one output
    row.  The backward adds the grad_out row, the 3 parameter gradients and
    the 4 scattered corner rows."""
    c = preset_dims(name)
    e = torch.finfo(c["dtype"]).bits // 8
    ns = c["B"] * c["Q"] * c["M"] * c["L"] * c["K"]
    nq = c["B"] * c["Q"] * c["M"]
    D = c["D"]
    fwd = ns * (4 * D * e + 3 * e) + nq * D * e
    bwd = ns * (8 * D * e + 6 * e) + nq * D * e
    return fwd, bwd
